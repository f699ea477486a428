// C ABI, CSR site requests with ghost atoms (include/mtpx.h,
// mtpx_compute_sites): the request of MTPGpuBatchRequest / MTPGpuComputeRequest
// (runtime/mtp/gpu-direct/mtp_gpu_direct.h:359-440, :455-517) that the LAMMPS
// pair style mlip/gpudirect fills (LAMMPS/USER-MLIP/pair_MLIP_gpu_direct.cpp:
// 577-603), with the semantics of its CPU counterpart MLIPCore::compute
// (runtime/mtp/mlip.cpp:907-1191).  Host code; no exceptions escape.
//
// The request's topology is packed once into its own device CSR (centres of
// negative type dropped, neighbour indices masked), kept for reuse_topology,
// and every call refreshes the atom types and positions, forms the entry
// geometry on the device (site_prepare_kernel), runs the E/F/S kernel with
// forces sized to all owned and ghost atoms, and finishes either with
// atomics (fast) or with an ordered gather over every atom (deterministic).
#include "context.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace {

// Packs and uploads the request's topology into ctx->sites.
int upload_topology(mtpx_context *ctx, const mtpx_site_request &r, const std::vector<int> &rows)
{
    auto &S = ctx->sites;
    S.valid = false;
    const int mask = r.neighbor_index_mask;
    const int nr = (int)rows.size();
    std::vector<int> off((size_t)nr + 1, 0), atom(nr), idx;
    std::vector<int> atom_row((size_t)r.ntotal, -1);
    int64_t P = 0;
    for (int k = 0; k < nr; ++k)
        P += r.offsets[rows[k] + 1] - r.offsets[rows[k]];
    if (P > INT32_MAX)
        return set_error(ctx, MTPX_E_CAPACITY, "more than 2^31 - 1 neighbour entries");
    idx.reserve((size_t)P);
    for (int k = 0; k < nr; ++k) {
        const int c = rows[k];
        atom[k] = r.centers ? r.centers[c] : c;
        if (atom_row[atom[k]] >= 0)
            return set_error(ctx, MTPX_E_INVALID, "atom " + std::to_string(atom[k]) +
                                                      " is listed as a centre twice");
        atom_row[atom[k]] = k;
        for (int p = r.offsets[c]; p < r.offsets[c + 1]; ++p)
            idx.push_back(r.neighbors[p] & mask);
        off[k + 1] = (int)idx.size();
    }
    // ordered reverse index over every atom (deterministic assembly)
    std::vector<int> roff((size_t)r.ntotal + 1, 0), rp(std::max<size_t>(idx.size(), 1));
    for (int j : idx)
        roff[(size_t)j + 1]++;
    for (int k = 0; k < r.ntotal; ++k)
        roff[k + 1] += roff[k];
    std::vector<int> cur(roff.begin(), roff.end() - 1);
    for (size_t p = 0; p < idx.size(); ++p)
        rp[(size_t)cur[idx[p]]++] = (int)p;
    hipStream_t s = ctx->stream;
    HIP_TRY(upload(S.nb.offsets, off, s), "upload site topology");
    HIP_TRY(upload(S.nb.idx, idx, s), "upload site topology");
    HIP_TRY(upload(S.center_atom, atom, s), "upload site topology");
    HIP_TRY(upload(S.atom_row, atom_row, s), "upload site topology");
    HIP_TRY(upload(S.rev_offsets, roff, s), "upload site topology");
    HIP_TRY(upload(S.rev_pairs, rp, s), "upload site topology");
    const size_t Pz = std::max<size_t>(idx.size(), 1);
    HIP_TRY(S.nb.type.ensure(sizeof(int) * Pz), "allocate site lists");
    HIP_TRY(S.nb.x.ensure(sizeof(double) * Pz), "allocate site lists");
    HIP_TRY(S.nb.y.ensure(sizeof(double) * Pz), "allocate site lists");
    HIP_TRY(S.nb.z.ensure(sizeof(double) * Pz), "allocate site lists");
    HIP_TRY(S.nb.d.ensure(sizeof(double) * Pz), "allocate site lists");
    HIP_TRY(S.nb.center_type.ensure(sizeof(int) * std::max(nr, 1)), "allocate site lists");
    HIP_TRY(hipStreamSynchronize(s), "upload site topology");
    S.nb.n = nr;
    S.nb.P = (int64_t)idx.size();
    S.center_count = r.center_count;
    S.nlocal = r.nlocal;
    S.ntotal = r.ntotal;
    S.rows = nr;
    S.P_in = r.center_count > 0 ? r.offsets[r.center_count] : 0;
    S.row_src = rows;
    S.row_atom = atom;
    S.valid = true;
    return MTPX_OK;
}

// Argument checks of a request (types, centres, offsets, indices); the kept
// centre rows (non-negative type) go to rows.
int check_request(mtpx_context *ctx, const mtpx_site_request &r, bool check_topology,
                  std::vector<int> &rows)
{
    const int Z = ctx->model.Z;
    if (r.center_count < 0 || r.nlocal < 0 || r.ntotal < r.nlocal ||
        (r.center_count > 0 && !r.offsets) || (r.ntotal > 0 && !r.type))
        return set_error(ctx, MTPX_E_INVALID, "invalid site request sizes");
    if (r.center_count > r.nlocal)
        return set_error(ctx, MTPX_E_INVALID, "more centres than owned atoms");
    for (int k = 0; k < r.ntotal; ++k)
        if (r.type[k] >= Z)
            return set_error(ctx, MTPX_E_INVALID, "atom " + std::to_string(k) + " has species " +
                                                      std::to_string(r.type[k]) +
                                                      " but the model has " + std::to_string(Z));
    rows.clear();
    for (int c = 0; c < r.center_count; ++c) {
        const int a = r.centers ? r.centers[c] : c;
        if (a < 0 || a >= r.nlocal)
            return set_error(ctx, MTPX_E_INVALID, "centre atom out of range");
        if (r.type[a] >= 0)
            rows.push_back(c);
    }
    const int64_t P = r.center_count > 0 ? r.offsets[r.center_count] : 0;
    if (check_topology) {
        if (r.center_count > 0 && r.offsets[0] != 0)
            return set_error(ctx, MTPX_E_INVALID, "offsets must start at 0");
        for (int c = 0; c < r.center_count; ++c)
            if (r.offsets[c + 1] < r.offsets[c])
                return set_error(ctx, MTPX_E_INVALID, "offsets must be non-decreasing");
        if (P > 0 && !r.neighbors)
            return set_error(ctx, MTPX_E_INVALID, "missing neighbour indices");
        for (int64_t p = 0; p < P; ++p) {
            const int j = r.neighbors[p] & r.neighbor_index_mask;
            if (j < 0 || j >= r.ntotal)
                return set_error(ctx, MTPX_E_INVALID, "neighbour index out of range");
        }
    }
    if (P > 0 && !r.neighbor_vectors && !r.x)
        return set_error(ctx, MTPX_E_INVALID, "site request needs positions or vectors");
    if (r.x && !all_finite(r.x, 3 * (size_t)r.ntotal))
        return set_error(ctx, MTPX_E_INVALID, "non-finite position");
    if (r.neighbor_vectors && !all_finite(r.neighbor_vectors, 3 * (size_t)P))
        return set_error(ctx, MTPX_E_INVALID, "non-finite neighbour vector");
    return MTPX_OK;
}

}  // namespace

extern "C" {

int mtpx_compute_sites(mtpx_context *ctx, const mtpx_site_request *req)
{
    if (!ctx || !req)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    // atom types through the species map; species -1 is skipped below
    mtpx_site_request mapped = *req;
    std::vector<int> tbuf;
    if (req->ntotal > 0 && req->type)
        if (int rc = map_species(ctx, req->type, (size_t)req->ntotal, true, tbuf, mapped.type))
            return rc;
    const mtpx_site_request &r = mapped;
    auto &S = ctx->sites;
    const int64_t P_in = r.center_count > 0 && r.offsets ? r.offsets[r.center_count] : 0;
    // reuse_topology: the same counts (the reference rebuilds when atom or
    // entry counts change, mtp_gpu_direct.h:424-426)
    const bool reuse = r.reuse_topology && S.valid && S.center_count == r.center_count &&
                       S.ntotal == r.ntotal && S.nlocal == r.nlocal && S.P_in == P_in;
    std::vector<int> rows;
    if (int rc = check_request(ctx, r, !reuse, rows))
        return rc;
    // the kept centres changed: the topology is packed again from the
    // caller's offsets and neighbours, which are then checked in full
    if (reuse && rows != S.row_src)
        if (int rc = check_request(ctx, r, true, rows))
            return rc;
    (void)hipSetDevice(ctx->device);
    if (!reuse || rows != S.row_src)
        if (int rc = upload_topology(ctx, r, rows))
            return rc;
    hipStream_t s = ctx->stream;
    const int nr = S.rows, ntot = r.ntotal;
    const int64_t P = S.nb.P;
    // types and positions (or the kept rows' vectors), every call
    HIP_TRY(S.atom_type.ensure(sizeof(int) * std::max(ntot, 1)), "allocate site inputs");
    if (ntot > 0)
        HIP_TRY(hipMemcpyAsync(S.atom_type.p, r.type, sizeof(int) * ntot, hipMemcpyHostToDevice,
                               s),
                "upload types");
    const double *dpos = nullptr, *dvec = nullptr;
    std::vector<double> vec;
    if (r.neighbor_vectors) {
        vec.reserve(3 * (size_t)P);
        for (int k = 0; k < nr; ++k) {
            const int c = S.row_src[k];
            vec.insert(vec.end(), r.neighbor_vectors + 3 * (size_t)r.offsets[c],
                       r.neighbor_vectors + 3 * (size_t)r.offsets[c + 1]);
        }
        HIP_TRY(upload(S.vec, vec, s), "upload neighbour vectors");
        dvec = S.vec.as<double>();
    } else {
        HIP_TRY(S.pos.ensure(sizeof(double) * 3 * std::max(ntot, 1)), "allocate positions");
        if (ntot > 0)
            HIP_TRY(hipMemcpyAsync(S.pos.p, r.x, sizeof(double) * 3 * ntot,
                                   hipMemcpyHostToDevice, s),
                    "upload positions");
        dpos = S.pos.as<double>();
    }
    HIP_TRY(launch_site_prepare(nr, S.nb.offsets.as<int>(), S.center_atom.as<int>(),
                                S.nb.idx.as<int>(), S.atom_type.as<int>(), dpos, dvec,
                                ctx->model.rmax * ctx->model.rmax, S.nb.center_type.as<int>(),
                                S.nb.type.as<int>(), S.nb.x.as<double>(), S.nb.y.as<double>(),
                                S.nb.z.as<double>(), S.nb.d.as<double>(), s),
            "launch site geometry");

    const bool det = r.deterministic != 0;
    const bool want_v6 = r.site_virial != nullptr;
    EfsLaunch cfg;
    if (!efs_configure(ctx->dm, nr, ctx->num_cus, 0, ctx->lds_limit, cfg))
        return set_error(ctx, MTPX_E_CAPACITY, "model needs more LDS than a CU provides");
    HIP_TRY(S.forces.ensure(sizeof(double) * 3 * std::max(ntot, 1)), "allocate forces");
    HIP_TRY(S.site_energy.ensure(sizeof(double) * std::max(nr, 1)), "allocate site energies");
    HIP_TRY(S.partial.ensure(sizeof(double) * 10 * cfg.rows), "allocate partials");
    HIP_TRY(S.out10.ensure(sizeof(double) * 10), "allocate outputs");
    if (want_v6)
        HIP_TRY(S.site_virial6.ensure(sizeof(double) * 6 * std::max(ntot, 1)),
                "allocate site virials");
    if (det)
        HIP_TRY(S.pair_ders.ensure(sizeof(double) * 3 * std::max<int64_t>(P, 1)),
                "allocate pair derivatives");
    DevNeighbors nb;
    nb.n = nr;
    nb.P = P;
    nb.offsets = S.nb.offsets.as<int>();
    nb.idx = S.nb.idx.as<int>();
    nb.type = S.nb.type.as<int>();
    nb.x = S.nb.x.as<double>();
    nb.y = S.nb.y.as<double>();
    nb.z = S.nb.z.as<double>();
    nb.d = S.nb.d.as<double>();
    nb.center_type = S.nb.center_type.as<int>();
    nb.center = S.center_atom.as<int>();
    EfsOut out;
    out.forces = S.forces.as<double>();
    out.site_energy = S.site_energy.as<double>();
    out.partial = S.partial.as<double>();
    out.pair_ders = det ? S.pair_ders.as<double>() : nullptr;
    out.site_virial = nullptr;
    out.site_virial6 = want_v6 ? S.site_virial6.as<double>() : nullptr;
    if (!det && ntot > 0) {
        HIP_TRY(hipMemsetAsync(out.forces, 0, sizeof(double) * 3 * ntot, s), "clear forces");
        if (want_v6)
            HIP_TRY(hipMemsetAsync(out.site_virial6, 0, sizeof(double) * 6 * ntot, s),
                    "clear site virials");
    }
    if (nr > 0) {
        HIP_TRY(launch_efs(ctx->dm, nb, out, cfg, det ? kEfsDeterministic : 0, s),
                "launch efs kernel");
        HIP_TRY(launch_efs_finish(nb, out, cfg.rows, false, nullptr, nullptr,
                                  S.out10.as<double>(), s),
                "launch efs reductions");
        if (det)
            HIP_TRY(launch_site_gather(nb, ntot, S.atom_row.as<int>(), out.pair_ders,
                                       S.rev_offsets.as<int>(), S.rev_pairs.as<int>(),
                                       out.forces, out.site_virial6, s),
                    "launch site assembly");
    } else {
        HIP_TRY(hipMemsetAsync(S.out10.p, 0, sizeof(double) * 10, s), "clear outputs");
        if (det && ntot > 0) {
            HIP_TRY(hipMemsetAsync(out.forces, 0, sizeof(double) * 3 * ntot, s), "clear forces");
            if (want_v6)
                HIP_TRY(hipMemsetAsync(out.site_virial6, 0, sizeof(double) * 6 * ntot, s),
                        "clear site virials");
        }
    }
    HIP_TRY(hipStreamSynchronize(s), "site request");

    double o10[10];
    HIP_TRY(hipMemcpy(o10, S.out10.p, sizeof o10, hipMemcpyDeviceToHost), "copy outputs");
    if (r.total_energy)
        *r.total_energy = o10[0];
    if (r.global_virial) {
        const double *St = o10 + 1;  // row-major 3x3, -sum D r^T
        r.global_virial[0] = St[0];
        r.global_virial[1] = St[4];
        r.global_virial[2] = St[8];
        r.global_virial[3] = 0.5 * (St[1] + St[3]);
        r.global_virial[4] = 0.5 * (St[2] + St[6]);
        r.global_virial[5] = 0.5 * (St[5] + St[7]);
    }
    if (r.force)
        if (int rc = copy_out(ctx, r.force, S.forces.p, 3 * (size_t)ntot,
                              r.accumulate_force != 0, "copy forces"))
            return rc;
    if (r.site_energy && r.nlocal > 0) {
        std::vector<double> se((size_t)std::max(nr, 1));
        if (nr > 0)
            HIP_TRY(hipMemcpy(se.data(), S.site_energy.p, sizeof(double) * nr,
                              hipMemcpyDeviceToHost),
                    "copy site energies");
        std::fill(r.site_energy, r.site_energy + r.nlocal, 0.0);
        for (int k = 0; k < nr; ++k)
            r.site_energy[S.row_atom[k]] = se[k];
    }
    if (want_v6)
        if (int rc = copy_out(ctx, r.site_virial, S.site_virial6.p, 6 * (size_t)ntot, false,
                              "copy site virials"))
            return rc;
    return MTPX_OK;
}

}  // extern "C"
