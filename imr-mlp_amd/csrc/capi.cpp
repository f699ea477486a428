// C ABI (include/mtpx.h): context, device-resident model and neighbour lists,
// E/F/S launches.  Host code; no exceptions escape.
#include "context.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>

namespace {

// Upload coefficient-dependent arrays: radial, species, moment coefficients
// and the adjoint seeds (sum of the moment coefficients mapped to a moment,
// accumulated in scalar order as potential_mtp.cpp:2974-2977 does).  With an
// MTP-M head the seeds depend on the atom: the head tables go up instead --
// the distinct moments the scalars map to, in first-appearance order, the
// moment coefficients of each descriptor summed per distinct moment in
// scalar order (the projection of Cpu::Executor, runtime/mtp/cpu/
// mtp_cpu.cpp:138-157), the descriptor species and the head coefficients.
int upload_coeffs(mtpx_context *ctx)
{
    const Model &m = ctx->model;
    const size_t sp = (size_t)m.nradial(), mo = sp + (size_t)m.nspecies();
    std::vector<double> radial(m.coef.begin(), m.coef.begin() + sp);
    std::vector<double> species(m.coef.begin() + sp, m.coef.begin() + sp + m.Z);
    std::vector<double> moment(m.coef.begin() + mo, m.coef.begin() + mo + m.S);
    std::vector<double> seed((size_t)m.K, 0.0);
    if (m.linear())
        for (int s = 0; s < m.S; ++s)
            seed[m.map[s]] += moment[s];
    HIP_TRY(upload(ctx->radial, radial, ctx->stream), "upload radial coefficients");
    HIP_TRY(upload(ctx->species, species, ctx->stream), "upload species coefficients");
    HIP_TRY(upload(ctx->moment, moment, ctx->stream), "upload moment coefficients");
    HIP_TRY(upload(ctx->seed, seed, ctx->stream), "upload adjoint seeds");
    ctx->dm.hd = nullptr;
    if (!m.linear()) {
        const int P = m.head.P;
        std::vector<int> compact((size_t)m.K, -1), ids;
        for (int s = 0; s < m.S; ++s)
            if (compact[m.map[s]] < 0) {
                compact[m.map[s]] = (int)ids.size();
                ids.push_back(m.map[s]);
            }
        const size_t NS = ids.size();
        std::vector<double> proj((size_t)P * NS, 0.0);
        for (int p = 0; p < P; ++p)
            for (int s = 0; s < m.S; ++s)
                proj[p * NS + compact[m.map[s]]] += m.coef[mo + (size_t)p * m.S + s];
        std::vector<double> dsp(m.coef.begin() + sp + m.Z, m.coef.begin() + mo);
        std::vector<double> hc(m.coef.begin() + mo + m.nmoment(), m.coef.end());
        // a head without coefficients (mtp_m_li) still gets a valid pointer
        if (ids.empty())
            ids.push_back(0);
        if (proj.empty())
            proj.push_back(0.0);
        if (hc.empty())
            hc.push_back(0.0);
        HIP_TRY(upload(ctx->head_ids, ids, ctx->stream), "upload head tables");
        HIP_TRY(upload(ctx->head_proj, proj, ctx->stream), "upload head tables");
        HIP_TRY(upload(ctx->head_dsp, dsp, ctx->stream), "upload head tables");
        HIP_TRY(upload(ctx->head_coef, hc, ctx->stream), "upload head tables");
        DevHead h{};
        h.kind = m.head.kind;
        h.P = P;
        h.NS = (int)NS;
        h.h1 = m.head.h1;
        h.h2 = m.head.h2;
        h.act = m.head.act;
        h.Z = m.Z;
        h.K = m.K;
        h.ids = ctx->head_ids.as<int>();
        h.proj = ctx->head_proj.as<double>();
        h.dsp = ctx->head_dsp.as<double>();
        h.c = ctx->head_coef.as<double>();
        HIP_TRY(ctx->head_params.ensure(sizeof h), "upload head tables");
        HIP_TRY(hipMemcpyAsync(ctx->head_params.p, &h, sizeof h, hipMemcpyHostToDevice,
                               ctx->stream),
                "upload head tables");
        ctx->dm.hd = static_cast<const DevHead *>(ctx->head_params.p);
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "upload coefficients");
    ctx->dm.radial = ctx->radial.as<double>();
    ctx->dm.species = ctx->species.as<double>();
    ctx->dm.moment = ctx->moment.as<double>();
    ctx->dm.seed = ctx->seed.as<double>();
    return MTPX_OK;
}

// Sizes and work-space offsets of the device view (no device pointers).
void fill_model_sizes(const Model &M, const Plan &P, DevModel &dm)
{
    dm.Z = M.Z;
    dm.M = M.M;
    dm.R = M.R;
    dm.K = M.K;
    dm.B = M.B;
    dm.T = M.T;
    dm.S = M.S;
    dm.nslots = P.nslots;
    dm.rmin = M.rmin;
    dm.rmax = M.rmax;
    dm.scaling = M.scaling;
    // RBasis_Chebyshev::setup (basis/basis.cpp:119-125)
    dm.mult = 2.0 / (M.rmax - M.rmin);
    dm.su = M.rmax - M.rmin;
    dm.pu = M.rmax + M.rmin;
    for (int mu = 0; mu < kMaxMu; ++mu)
        dm.numax[mu] = P.numax[mu];
    dm.numax_all = P.numax_all;
    dm.ndup = (int)P.dup.size() / 2;
    dm.nfwd = (int)P.fwd_level_step.size() - 1;
    dm.nbwd = (int)P.bwd_level_step.size() - 1;
    dm.max_partials = P.max_partials;
    dm.K4 = P.K4;
    dm.dummy = P.dummy;
    dm.part0 = P.part0;
    dm.red0 = P.red0;
    dm.priv_doubles = P.priv_doubles;
    dm.efs_red = P.efs_red;
    dm.efs_stage = P.efs_stage;
    dm.efs_acc = P.efs_acc;
    dm.efs_head = P.efs_head;
    dm.head = M.head.kind;
    dm.hd = nullptr;
    dm.tr_red1 = P.tr_red1;
    dm.tr_red4 = P.tr_red4;
    dm.tr_stage = P.tr_stage;
    dm.tr_grad = P.tr_grad;
    dm.tr_ctype = P.tr_ctype;
    dm.tr_priv = P.tr_priv;
    dm.nradial = M.nradial();
    dm.ncoef = M.ncoef();
    dm.rb_general = M.general_basis() ? 1 : 0;
    dm.rb_table = nullptr;
    std::memcpy(dm.slot_base, P.slot_base, sizeof dm.slot_base);
    dm.fwd_nsteps = (int)(P.fwd_steps.size() / (2 * kWave));
    dm.bwd_nsteps = (int)(P.bwd_steps.size() / (2 * kWave));
}

int install_model(mtpx_context *ctx, Model &&m)
{
    std::string err;
    if (!validate_model(m, err))
        return set_error(ctx, MTPX_E_MODEL, err);
    Plan p;
    if (!build_plan(m, p, err))
        return set_error(ctx, MTPX_E_MODEL, err);
    // Sizes first, in a local view: a model whose work space does not fit a
    // CU's LDS is refused before anything of the context changes.
    DevModel dm{};
    fill_model_sizes(m, p, dm);
    EfsLaunch probe;
    if (!efs_configure(dm, 1, 1, 0, ctx->lds_limit, probe))
        return set_error(ctx, MTPX_E_CAPACITY, "model needs more LDS than a CU provides");
    // From here on the old model is gone: until every upload has succeeded the
    // context holds no model (a failed upload leaves MTPX_E_NO_MODEL behind,
    // never tables of two models).
    ctx->has_model = false;
    ctx->has_lin = false;
    ctx->has_batch_out = false;
    ctx->has_adjoints = false;
    ctx->model = std::move(m);
    ctx->plan = std::move(p);
    const Model &M = ctx->model;
    const Plan &P = ctx->plan;
    hipStream_t s = ctx->stream;
    HIP_TRY(upload(ctx->map, M.map, s), "upload model");
    HIP_TRY(upload(ctx->slot_basic, P.slot_basic, s), "upload model");
    HIP_TRY(upload(ctx->slot_abc, P.slot_abc, s), "upload model");
    HIP_TRY(upload(ctx->dup, P.dup, s), "upload model");
    HIP_TRY(upload(ctx->fwd_level, P.fwd_level_step, s), "upload model");
    HIP_TRY(upload(ctx->fwd_steps, P.fwd_steps, s), "upload model");
    HIP_TRY(upload(ctx->bwd_level, P.bwd_level_step, s), "upload model");
    HIP_TRY(upload(ctx->bwd_steps, P.bwd_steps, s), "upload model");
    HIP_TRY(upload(ctx->fwd_lcomb, P.fwd_level_comb, s), "upload model");
    HIP_TRY(upload(ctx->fwd_comb, P.fwd_comb, s), "upload model");
    HIP_TRY(upload(ctx->bwd_lcomb, P.bwd_level_comb, s), "upload model");
    HIP_TRY(upload(ctx->bwd_comb, P.bwd_comb, s), "upload model");
    if (dm.rb_general) {
        // per ordered pair: kind, min, max, scaling and the setup constants
        // of the basis (basis/basis.cpp setup(): mult, su, pu, pi / max,
        // and b, 1 / su for Poly4 / Poly5; the configurable basis's cutoff
        // and shift with their parameters and normalisations)
        std::vector<double> t((size_t)M.Z * M.Z * kRbStride, 0.0);
        for (int q = 0; q < M.Z * M.Z; ++q) {
            const RadialBasis &b = M.pair_basis(q / M.Z, q % M.Z);
            double *r = &t[(size_t)q * kRbStride];
            const double su = b.rmax - b.rmin;
            r[0] = b.kind;
            r[1] = b.rmin;
            r[2] = b.rmax;
            r[3] = b.scaling;
            if (b.kind == kRBChebyshevConfigurable) {
                r[4] = b.cut;
                r[5] = b.shift;
                r[6] = b.one_minus ? 1.0 : 0.0;
                r[7] = b.cut_b;
                r[8] = b.cut_r1;
                r[9] = b.cut_r2;
                r[10] = b.lambda;
                r[11] = b.scale_lambda;
                r[12] = 1.0 / su;
                r[13] = std::expm1(b.lambda);
                r[14] = std::tanh(b.scale_lambda);
                continue;
            }
            r[4] = 2.0 / (b.rmax - b.rmin);
            r[5] = su;
            r[6] = b.rmax + b.rmin;
            r[7] = M_PI / b.rmax;
            r[8] = b.b;
            r[9] = 1.0 / su;
        }
        HIP_TRY(upload(ctx->rb_table, t, s), "upload model");
        dm.rb_table = ctx->rb_table.as<double>();
    }
    dm.map = ctx->map.as<int>();
    dm.slot_basic = ctx->slot_basic.as<int>();
    dm.slot_abc = ctx->slot_abc.as<int>();
    dm.dup = ctx->dup.as<int>();
    dm.fwd_level_step = ctx->fwd_level.as<int>();
    dm.fwd_steps = ctx->fwd_steps.as<int2>();
    dm.bwd_level_step = ctx->bwd_level.as<int>();
    dm.bwd_steps = ctx->bwd_steps.as<int2>();
    dm.fwd_level_comb = ctx->fwd_lcomb.as<int>();
    dm.fwd_comb = ctx->fwd_comb.as<int4>();
    dm.bwd_level_comb = ctx->bwd_lcomb.as<int>();
    dm.bwd_comb = ctx->bwd_comb.as<int4>();
    // linear-fit plan: optional (the linear entry points report its error)
    const bool lin_ok = build_lin_plan(M, P, ctx->lin, ctx->lin_err);
    if (lin_ok) {
        const LinPlan &lp = ctx->lin;
        HIP_TRY(upload(ctx->lin_level, lp.level_step, s), "upload model");
        HIP_TRY(upload(ctx->lin_steps, lp.steps, s), "upload model");
        HIP_TRY(upload(ctx->lin_lcomb, lp.level_comb, s), "upload model");
        HIP_TRY(upload(ctx->lin_comb, lp.comb, s), "upload model");
        HIP_TRY(upload(ctx->lin_ent, lp.slot_L, s), "upload model");
        HIP_TRY(upload(ctx->lin_estart, lp.slot_mask, s), "upload model");
        HIP_TRY(upload(ctx->lin_chunk, lp.chunk_s0, s), "upload model");
        HIP_TRY(upload(ctx->lin_cscal, lp.chunk_scalar, s), "upload model");
        HIP_TRY(upload(ctx->lin_maskw, lp.maskw, s), "upload model");
        HIP_TRY(upload(ctx->lin_clist, lp.clist, s), "upload model");
        HIP_TRY(upload(ctx->lin_walk, lp.walk, s), "upload model");
        HIP_TRY(upload(ctx->lin_walk_off, lp.walk_off, s), "upload model");
        HIP_TRY(upload(ctx->lin_flevel, lp.fwd_level_step, s), "upload model");
        HIP_TRY(upload(ctx->lin_fsteps, lp.fwd_steps, s), "upload model");
        HIP_TRY(upload(ctx->lin_flcomb, lp.fwd_level_comb, s), "upload model");
        HIP_TRY(upload(ctx->lin_fcomb, lp.fwd_comb, s), "upload model");
        DevLin &L = ctx->dl;
        L.dummy = lp.dummy;
        L.red0 = lp.red0;
        L.nfwd = (int)lp.fwd_level_step.size() - 1;
        L.fwd_level_step = ctx->lin_flevel.as<int>();
        L.fwd_level_comb = ctx->lin_flcomb.as<int>();
        L.fwd_steps = ctx->lin_fsteps.as<int2>();
        L.fwd_comb = ctx->lin_fcomb.as<int4>();
        L.nL = lp.nL;
        L.one = lp.one;
        L.L0 = lp.L0;
        L.part0 = lp.part0;
        L.acc = lp.acc;
        L.priv = lp.priv;
        L.CH = lp.CH;
        L.nchunks = lp.nchunks;
        L.nlev = (int)lp.level_step.size() - 1;
        L.level_step = ctx->lin_level.as<int>();
        L.level_comb = ctx->lin_lcomb.as<int>();
        L.steps = ctx->lin_steps.as<int2>();
        L.comb = ctx->lin_comb.as<int4>();
        L.slot_L = ctx->lin_ent.as<int>();
        L.slot_mask = ctx->lin_estart.as<int>();
        L.chunk_s0 = ctx->lin_chunk.as<int>();
        L.chunk_scalar = ctx->lin_cscal.as<int>();
        L.maskw = ctx->lin_maskw.as<int>();
        L.clist = ctx->lin_clist.as<int>();
        L.walk = ctx->lin_walk.as<int>();
        L.walk_off = ctx->lin_walk_off.as<int>();
        L.nwalk = lp.walk_off.back();
        L.max_walk = 0;
        for (int c = 0; c < lp.nchunks; ++c)
            L.max_walk = std::max(L.max_walk, lp.walk_off[c + 1] - lp.walk_off[c]);
        L.lane_walk = lp.lane_walk ? 1 : 0;
        // MTPX_LIN_WALK=runtime (tuning): keep the run-time walk
        static const bool runtime_walk = [] {
            const char *e = getenv("MTPX_LIN_WALK");
            return e && std::string(e) == "runtime";
        }();
        L.compiled_walk = !runtime_walk && lin_walk_compiled(lp, P.nslots) ? 1 : 0;
    }
    ctx->dm = dm;
    int rc = upload_coeffs(ctx);
    if (rc != MTPX_OK)
        return rc;
    // a new model starts with the identity species map over [0, Z)
    ctx->spmap.resize((size_t)M.Z);
    for (int t = 0; t < M.Z; ++t)
        ctx->spmap[t] = t;
    ctx->max_type = M.Z;
    ctx->spmap_set = false;
    ctx->has_lin = lin_ok;
    ctx->has_model = true;
    return MTPX_OK;
}

}  // namespace

namespace mtpx {

// Every value finite (no exponent of all ones); branch-free, so the
// compiler vectorises the pass over the positions.
bool all_finite(const double *v, size_t n)
{
    uint64_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        uint64_t b;
        std::memcpy(&b, v + i, sizeof b);
        bad |= (uint64_t)((b & 0x7ff0000000000000ull) == 0x7ff0000000000000ull);
    }
    return bad == 0;
}

// Every species in [0, Z); *maxs receives the largest (-1 for none).
bool species_in_range(const int *t, size_t n, int Z, int &maxs)
{
    unsigned bad = 0;
    int m = -1;
    for (size_t i = 0; i < n; ++i) {
        bad |= (unsigned)((unsigned)t[i] >= (unsigned)Z);
        m = t[i] > m ? t[i] : m;
    }
    maxs = m;
    return bad == 0;
}

int map_species(mtpx_context *ctx, const int *types, size_t n, bool allow_unmapped,
                std::vector<int> &buf, const int *&out)
{
    out = types;
    if (!ctx->has_model || !ctx->spmap_set || n == 0)
        return MTPX_OK;
    buf.resize(n);
    for (size_t i = 0; i < n; ++i) {
        const int t = types[i];
        // the requests' type checks (mtp_gpu_direct.cu:9454, 9510)
        if (t < 0 || t >= ctx->max_type)
            return set_error(ctx, MTPX_E_INVALID, "atom type is outside the species-map range");
        const int sp = ctx->spmap[t];
        if (sp < 0 && !allow_unmapped)
            return set_error(ctx, MTPX_E_INVALID,
                             "atom type " + std::to_string(t) +
                                 " maps to species -1; only site requests skip such atoms");
        buf[i] = sp;
    }
    out = buf.data();
    return MTPX_OK;
}

DevNeighbors dev_neighbors(const mtpx_context *ctx)
{
    DevNeighbors nb;
    nb.n = ctx->n;
    nb.P = ctx->P;
    nb.offsets = ctx->offsets.as<int>();
    nb.idx = ctx->idx.as<int>();
    nb.type = ctx->type.as<int>();
    nb.x = ctx->x.as<double>();
    nb.y = ctx->y.as<double>();
    nb.z = ctx->z.as<double>();
    nb.d = ctx->d.as<double>();
    nb.center_type = ctx->center_type.as<int>();
    nb.center = nullptr;
    nb.mirror = ctx->nbh.has_mirror ? ctx->nbh.mirror.as<int>() : nullptr;
    return nb;
}

// Ordered reverse index: for each atom k, the pairs p with idx[p] == k, in
// ascending p (the deterministic force gather and the linear-fit gather);
// also keeps the list offsets on the host.
int ensure_reverse_index(mtpx_context *ctx)
{
    if (ctx->rev_ready)
        return MTPX_OK;
    std::vector<int> idx_host((size_t)std::max<int64_t>(ctx->P, 1));
    ctx->offsets_host.assign((size_t)ctx->n + 1, 0);
    if (ctx->P > 0)
        HIP_TRY(hipMemcpy(idx_host.data(), ctx->idx.p, sizeof(int) * ctx->P,
                          hipMemcpyDeviceToHost),
                "copy neighbour indices");
    if (ctx->n > 0)
        HIP_TRY(hipMemcpy(ctx->offsets_host.data(), ctx->offsets.p, sizeof(int) * (ctx->n + 1),
                          hipMemcpyDeviceToHost),
                "copy neighbour offsets");
    std::vector<int> roff((size_t)ctx->n + 1, 0), rp((size_t)std::max<int64_t>(ctx->P, 1));
    for (int64_t p = 0; p < ctx->P; ++p)
        roff[(size_t)idx_host[p] + 1]++;
    for (int k = 0; k < ctx->n; ++k)
        roff[k + 1] += roff[k];
    std::vector<int> cur(roff.begin(), roff.end() - 1);
    for (int64_t p = 0; p < ctx->P; ++p)
        rp[(size_t)cur[idx_host[p]]++] = (int)p;
    HIP_TRY(upload(ctx->rev_offsets, roff, ctx->stream), "upload reverse index");
    HIP_TRY(upload(ctx->rev_pairs, rp, ctx->stream), "upload reverse index");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "upload reverse index");
    ctx->rev_ready = true;
    return MTPX_OK;
}

int set_single_structure(mtpx_context *ctx)
{
    ctx->has_batch_out = false;
    ctx->has_adjoints = false;
    ctx->has_labels = false;
    // the device tables of one structure of n atoms are still in place
    if (ctx->single_n == ctx->n && ctx->nconf == 1)
        return MTPX_OK;
    ctx->single_n = -1;
    ctx->nconf = 1;
    ctx->soff_host = {0, ctx->n};
    HIP_TRY(upload(ctx->soff, ctx->soff_host, ctx->stream), "upload structure offsets");
    HIP_TRY(ctx->center_structure.ensure(sizeof(int) * std::max(ctx->n, 1)),
            "allocate structure index");
    HIP_TRY(hipMemsetAsync(ctx->center_structure.p, 0, sizeof(int) * std::max(ctx->n, 1),
                           ctx->stream),
            "clear structure index");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "upload structure offsets");
    ctx->single_n = ctx->n;
    return MTPX_OK;
}

int copy_out(mtpx_context *ctx, double *dst, const void *src, size_t count, bool add,
             const char *what)
{
    if (!count)
        return MTPX_OK;
    if (!add) {
        HIP_TRY(hipMemcpy(dst, src, sizeof(double) * count, hipMemcpyDeviceToHost), what);
        return MTPX_OK;
    }
    std::vector<double> tmp(count);
    HIP_TRY(hipMemcpy(tmp.data(), src, sizeof(double) * count, hipMemcpyDeviceToHost), what);
    for (size_t k = 0; k < count; ++k)
        dst[k] += tmp[k];
    return MTPX_OK;
}

int check_species(mtpx_context *ctx)
{
    if (ctx->max_species >= ctx->model.Z)
        return set_error(ctx, MTPX_E_INVALID,
                         "neighbour lists hold species " + std::to_string(ctx->max_species) +
                             " but the model has " + std::to_string(ctx->model.Z));
    return MTPX_OK;
}

int run_efs(mtpx_context *ctx, bool deterministic, bool site_virial, bool energy_only)
{
    if (energy_only)
        deterministic = false;
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no neighbour lists");
    if (int rc = check_species(ctx))
        return rc;
    // Lists built here carry each entry's mirror: the forces are then
    // assembled without atomics (per-entry derivatives, each atom's own force
    // stored, the reactions gathered by the mirrors), which is also the
    // ordered assembly.  Lists handed over take the reaction atomics, or the
    // reverse index when an ordered assembly is asked for.
    const bool mirror = ctx->nbh.has_mirror && !energy_only;
    if (mirror)
        deterministic = true;
    else if (deterministic)
        if (int rc = ensure_reverse_index(ctx))
            return rc;
    const int n = ctx->n;
    hipStream_t s = ctx->stream;
    // MTPX_EFS_WAVES (tuning): cap on the waves per workgroup
    static const int max_waves = [] {
        const char *e = getenv("MTPX_EFS_WAVES");
        return e ? atoi(e) : 0;
    }();
    // MTPX_EFS_TABLES (tuning): "lds" or "global" step-table placement
    static const int table_pref = [] {
        const char *e = getenv("MTPX_EFS_TABLES");
        return !e ? -1 : std::string(e) == "lds" ? 1 : std::string(e) == "global" ? 0 : -1;
    }();
    EfsLaunch cfg;
    if (!efs_configure(ctx->dm, n, ctx->num_cus, max_waves, ctx->lds_limit, cfg, table_pref))
        return set_error(ctx, MTPX_E_CAPACITY, "model needs more LDS than a CU provides");
    ctx->launch = cfg;
    HIP_TRY(ctx->forces.ensure(sizeof(double) * 3 * std::max(n, 1)), "allocate forces");
    HIP_TRY(ctx->site_energy.ensure(sizeof(double) * std::max(n, 1)), "allocate site energies");
    HIP_TRY(ctx->partial.ensure(sizeof(double) * 10 * cfg.rows), "allocate partials");
    HIP_TRY(ctx->out10.ensure(sizeof(double) * 10), "allocate outputs");
    if (deterministic)
        HIP_TRY(ctx->pair_ders.ensure(sizeof(double) * 3 * std::max<int64_t>(ctx->P, 1)),
                "allocate pair derivatives");
    EfsOut out;
    out.forces = ctx->forces.as<double>();
    out.site_energy = ctx->site_energy.as<double>();
    out.partial = ctx->partial.as<double>();
    out.pair_ders = deterministic ? ctx->pair_ders.as<double>() : nullptr;
    out.site_virial = nullptr;
    out.site_virial6 = nullptr;
    if (site_virial) {
        HIP_TRY(ctx->site_virial.ensure(sizeof(double) * 9 * std::max(n, 1)),
                "allocate site virials");
        out.site_virial = ctx->site_virial.as<double>();
    }
    DevNeighbors nb = dev_neighbors(ctx);
    if (!deterministic && !energy_only && n > 0)
        HIP_TRY(launch_fill_zero(out.forces, 3 * (size_t)n, s), "clear forces");
    const bool timed = ctx->timings_on;
    if (timed)
        HIP_TRY(hipEventRecord(ctx->ev[0], s), "record event");
    if (n > 0)
        HIP_TRY(launch_efs(ctx->dm, nb, out, cfg,
                           (deterministic ? kEfsDeterministic : 0) |
                               (energy_only ? kEfsEnergyOnly : 0) | (mirror ? kEfsOwnForce : 0),
                           s),
                "launch efs kernel");
    if (timed)
        HIP_TRY(hipEventRecord(ctx->ev[1], s), "record event");
    if (n > 0)
        HIP_TRY(launch_efs_finish(nb, out, cfg.rows, deterministic, ctx->rev_offsets.as<int>(),
                                  ctx->rev_pairs.as<int>(), ctx->out10.as<double>(), s),
                "launch efs reductions");
    else
        HIP_TRY(hipMemsetAsync(ctx->out10.p, 0, sizeof(double) * 10, s), "clear outputs");
    float t01 = 0, t12 = 0, t02 = 0;
    if (timed) {
        HIP_TRY(hipEventRecord(ctx->ev[2], s), "record event");
        HIP_TRY(hipEventSynchronize(ctx->ev[2]), "efs");
        (void)hipEventElapsedTime(&t01, ctx->ev[0], ctx->ev[1]);
        (void)hipEventElapsedTime(&t12, ctx->ev[1], ctx->ev[2]);
        (void)hipEventElapsedTime(&t02, ctx->ev[0], ctx->ev[2]);
    } else {
        HIP_TRY(hipStreamSynchronize(s), "efs");
    }
    ctx->timings[0] = t02;
    ctx->timings[1] = t01;
    ctx->timings[2] = t12;
    ctx->timings[3] = 0;
    return MTPX_OK;
}

}  // namespace mtpx

extern "C" {

const char *mtpx_version(void)
{
    return "mtpx 0.1 gfx950 fp64 (efs variants: M4/nu6/R8, M5/nu8/R10, M8/nu8/R16)";
}

int mtpx_create(int device, mtpx_context **out)
{
    if (!out)
        return MTPX_E_INVALID;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
        return MTPX_E_DEVICE;
    mtpx_context *ctx = new (std::nothrow) mtpx_context();
    if (!ctx)
        return MTPX_E_ALLOC;
    ctx->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreate(&ctx->stream) != hipSuccess) {
        delete ctx;
        return MTPX_E_DEVICE;
    }
    for (auto &e : ctx->ev)
        if (hipEventCreate(&e) != hipSuccess) {
            delete ctx;
            return MTPX_E_DEVICE;
        }
    // the allocation-free entry point's scratch: this device's copy
    if (noalloc_scratch_address(&ctx->noalloc_scratch) != hipSuccess || !ctx->noalloc_scratch) {
        delete ctx;
        return MTPX_E_DEVICE;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0) {
        ctx->num_cus = prop.multiProcessorCount;
        if (prop.sharedMemPerBlock > 0)
            ctx->lds_limit = std::min<size_t>(ctx->lds_limit, prop.sharedMemPerBlock);
    }
    *out = ctx;
    return MTPX_OK;
}

void mtpx_destroy(mtpx_context *ctx)
{
    if (!ctx)
        return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream)
        (void)hipStreamSynchronize(ctx->stream);
    delete ctx;
}

const char *mtpx_last_error(const mtpx_context *ctx)
{
    return ctx ? ctx->err.c_str() : "null context";
}

int mtpx_load_model(mtpx_context *ctx, const mtpx_model_view *v)
{
    if (!ctx || !v)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    Model m;
    std::vector<int> spmap;
    int code = MTPX_OK;
    std::string err;
    if (!model_from_view(*v, m, spmap, code, err))
        return set_error(ctx, code, err);
    (void)hipSetDevice(ctx->device);
    if (int rc = install_model(ctx, std::move(m)))
        return rc;
    ctx->spmap = std::move(spmap);
    ctx->max_type = v->max_type;
    ctx->spmap_set = true;
    return MTPX_OK;
}

int mtpx_set_species_map(mtpx_context *ctx, int max_type, const int *spmap)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    const int Z = ctx->model.Z;
    if (!spmap) {
        ctx->spmap.resize((size_t)Z);
        for (int t = 0; t < Z; ++t)
            ctx->spmap[t] = t;
        ctx->max_type = Z;
        ctx->spmap_set = false;
        return MTPX_OK;
    }
    if (max_type <= 0)
        return set_error(ctx, MTPX_E_INVALID, "invalid max_type/spmap");
    for (int t = 0; t < max_type; ++t)
        if (spmap[t] < -1 || spmap[t] >= Z)
            return set_error(ctx, MTPX_E_INVALID, "species mapping is outside [-1, species_count)");
    ctx->spmap.assign(spmap, spmap + max_type);
    ctx->max_type = max_type;
    ctx->spmap_set = true;
    return MTPX_OK;
}

int mtpx_load_model_text(mtpx_context *ctx, const char *text)
{
    if (!ctx || !text)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    Model m;
    std::string err;
    if (!parse_mtp(text, m, err))
        return set_error(ctx, MTPX_E_MODEL, err);
    (void)hipSetDevice(ctx->device);
    return install_model(ctx, std::move(m));
}

int mtpx_parse_model_text(const char *text, int out8[8], double *coeffs, char *err, int errlen)
{
    if (!text)
        return MTPX_E_INVALID;
    Model m;
    std::string e;
    if (!parse_mtp(text, m, e)) {
        if (err && errlen > 0) {
            std::strncpy(err, e.c_str(), (size_t)errlen - 1);
            err[errlen - 1] = 0;
        }
        return MTPX_E_MODEL;
    }
    if (out8) {
        const int v[8] = {m.Z, m.M, m.R, m.K, m.B, m.T, m.S, m.ncoef()};
        std::memcpy(out8, v, sizeof v);
    }
    if (coeffs)
        std::memcpy(coeffs, m.coef.data(), sizeof(double) * m.coef.size());
    return MTPX_OK;
}

namespace {
int copy_text(const std::string &t, char *buf, size_t cap, size_t *len)
{
    if (len)
        *len = t.size();
    if (!buf)
        return MTPX_OK;
    if (cap <= t.size())
        return MTPX_E_CAPACITY;
    std::memcpy(buf, t.c_str(), t.size() + 1);
    return MTPX_OK;
}
}  // namespace

int mtpx_save_model_text(const mtpx_context *ctx, char *buf, size_t cap, size_t *len)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    return copy_text(save_mtp(ctx->model), buf, cap, len);
}

namespace {
void copy_err(const std::string &e, char *err, int errlen)
{
    if (err && errlen > 0) {
        std::strncpy(err, e.c_str(), (size_t)errlen - 1);
        err[errlen - 1] = 0;
    }
}

int copy_bytes(const std::string &b, void *buf, size_t cap, size_t *len)
{
    if (len)
        *len = b.size();
    if (!buf)
        return MTPX_OK;
    if (cap < b.size())
        return MTPX_E_CAPACITY;
    std::memcpy(buf, b.data(), b.size());
    return MTPX_OK;
}

// A bundle's model: its .mtp text parsed, each radial basis given its own
// scaling (read_mtp, potentials/gpm_codec.cpp:370-382).
bool model_from_gpm(const void *bytes, size_t n, Model &m, std::string &e)
{
    std::string text;
    std::vector<double> scalings;
    if (!gpm_read(bytes, n, text, scalings, e) || !parse_mtp(text, m, e))
        return false;
    if (scalings.size() != m.bases.size()) {
        e = "GPM: radial bases do not match the model";
        return false;
    }
    for (size_t i = 0; i < scalings.size(); ++i)
        m.bases[i].scaling = scalings[i];
    m.scaling = scalings[0];
    return validate_model(m, e);
}
}  // namespace

int mtpx_load_model_gpm(mtpx_context *ctx, const void *bytes, size_t n)
{
    if (!ctx || !bytes)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    Model m;
    std::string err;
    if (!model_from_gpm(bytes, n, m, err))
        return set_error(ctx, MTPX_E_MODEL, err);
    (void)hipSetDevice(ctx->device);
    return install_model(ctx, std::move(m));
}

int mtpx_save_model_gpm(const mtpx_context *ctx, int zstd_level, void *buf, size_t cap,
                        size_t *len)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    std::string out, err;
    if (!gpm_write(ctx->model, zstd_level, out, err))
        return MTPX_E_MODEL;
    return copy_bytes(out, buf, cap, len);
}

int mtpx_gpm_to_text(const void *bytes, size_t n, char *buf, size_t cap, size_t *len, char *err,
                     int errlen)
{
    if (!bytes)
        return MTPX_E_INVALID;
    std::string text, e;
    std::vector<double> scalings;
    if (!gpm_read(bytes, n, text, scalings, e)) {
        copy_err(e, err, errlen);
        return MTPX_E_MODEL;
    }
    return copy_text(text, buf, cap, len);
}

int mtpx_gpm_from_text(const char *text, int zstd_level, void *buf, size_t cap, size_t *len,
                       char *err, int errlen)
{
    if (!text)
        return MTPX_E_INVALID;
    Model m;
    std::string out, e;
    if (!parse_mtp(text, m, e) || !gpm_write(m, zstd_level, out, e)) {
        copy_err(e, err, errlen);
        return MTPX_E_MODEL;
    }
    return copy_bytes(out, buf, cap, len);
}

int mtpx_parse_model_gpm(const void *bytes, size_t n, int out8[8], double *coeffs, char *err,
                         int errlen)
{
    if (!bytes)
        return MTPX_E_INVALID;
    Model m;
    std::string e;
    if (!model_from_gpm(bytes, n, m, e)) {
        copy_err(e, err, errlen);
        return MTPX_E_MODEL;
    }
    if (out8) {
        const int v[8] = {m.Z, m.M, m.R, m.K, m.B, m.T, m.S, m.ncoef()};
        std::memcpy(out8, v, sizeof v);
    }
    if (coeffs)
        std::memcpy(coeffs, m.coef.data(), sizeof(double) * m.coef.size());
    return MTPX_OK;
}

int mtpx_format_model_text(const char *text, char *buf, size_t cap, size_t *len, char *err,
                           int errlen)
{
    if (!text)
        return MTPX_E_INVALID;
    Model m;
    std::string e;
    if (!parse_mtp(text, m, e)) {
        if (err && errlen > 0) {
            std::strncpy(err, e.c_str(), (size_t)errlen - 1);
            err[errlen - 1] = 0;
        }
        return MTPX_E_MODEL;
    }
    return copy_text(save_mtp(m), buf, cap, len);
}

int mtpx_model_cutoff(const mtpx_context *ctx, double *cutoff)
{
    if (!ctx || !cutoff)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    *cutoff = ctx->model.rmax;
    return MTPX_OK;
}

int mtpx_model_info(const mtpx_context *ctx, int out8[8])
{
    if (!ctx || !out8)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    const Model &m = ctx->model;
    const int v[8] = {m.Z, m.M, m.R, m.K, m.B, m.T, m.S, m.ncoef()};
    std::memcpy(out8, v, sizeof v);
    return MTPX_OK;
}

int mtpx_model_head(const mtpx_context *ctx, int out6[6])
{
    if (!ctx || !out6)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    const Head &h = ctx->model.head;
    const int v[6] = {h.kind, h.P, h.h1, h.h2, h.act, h.Mc};
    std::memcpy(out6, v, sizeof v);
    return MTPX_OK;
}

int mtpx_parse_model_head(const char *text, int out6[6], char *err, int errlen)
{
    if (!text || !out6)
        return MTPX_E_INVALID;
    Model m;
    std::string e;
    if (!parse_mtp(text, m, e)) {
        if (err && errlen > 0) {
            std::strncpy(err, e.c_str(), (size_t)errlen - 1);
            err[errlen - 1] = 0;
        }
        return MTPX_E_MODEL;
    }
    const Head &h = m.head;
    const int v[6] = {h.kind, h.P, h.h1, h.h2, h.act, h.Mc};
    std::memcpy(out6, v, sizeof v);
    return MTPX_OK;
}

int mtpx_get_coeffs(const mtpx_context *ctx, double *coeffs)
{
    if (!ctx || !coeffs)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    std::memcpy(coeffs, ctx->model.coef.data(), sizeof(double) * ctx->model.coef.size());
    return MTPX_OK;
}

int mtpx_set_coeffs(mtpx_context *ctx, const double *coeffs)
{
    if (!ctx || !coeffs)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    std::memcpy(ctx->model.coef.data(), coeffs, sizeof(double) * ctx->model.coef.size());
    (void)hipSetDevice(ctx->device);
    ctx->has_batch_out = false;
    ctx->has_adjoints = false;
    return upload_coeffs(ctx);
}

int mtpx_set_neighbors(mtpx_context *ctx, int n, const int *offsets, const int *indices,
                       const int *types, const double *vecs, const double *dists,
                       const int *center_types)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (n < 0 || !offsets || (n > 0 && !center_types))
        return set_error(ctx, MTPX_E_INVALID, "invalid neighbour arrays");
    if (offsets[0] != 0)
        return set_error(ctx, MTPX_E_INVALID, "offsets must start at 0");
    for (int i = 0; i < n; ++i)
        if (offsets[i + 1] < offsets[i])
            return set_error(ctx, MTPX_E_INVALID, "offsets must be non-decreasing");
    const int64_t P = offsets[n];
    if (P > 0 && (!indices || !types || !vecs || !dists))
        return set_error(ctx, MTPX_E_INVALID, "invalid neighbour arrays");
    std::vector<int> tbuf, cbuf;
    if (int rc = map_species(ctx, types, (size_t)P, false, tbuf, types))
        return rc;
    if (int rc = map_species(ctx, center_types, (size_t)n, false, cbuf, center_types))
        return rc;
    int Z = ctx->has_model ? ctx->model.Z : 1 << 30;
    for (int64_t p = 0; p < P; ++p) {
        if (indices[p] < 0 || indices[p] >= n)
            return set_error(ctx, MTPX_E_INVALID, "neighbour index out of range");
        if (types[p] < 0 || types[p] >= Z)
            return set_error(ctx, MTPX_E_INVALID, "neighbour species out of range");
    }
    int maxs = -1;
    for (int i = 0; i < n; ++i) {
        if (center_types[i] < 0 || center_types[i] >= Z)
            return set_error(ctx, MTPX_E_INVALID, "centre species out of range");
        maxs = std::max(maxs, center_types[i]);
    }
    for (int64_t p = 0; p < P; ++p)
        maxs = std::max(maxs, types[p]);
    (void)hipSetDevice(ctx->device);
    ctx->has_nbh = false;
    ctx->rev_ready = false;
    ctx->nbh.has_mirror = false;  // lists handed over carry no mirror entries
    std::vector<double> xs((size_t)P), ys((size_t)P), zs((size_t)P);
    for (int64_t p = 0; p < P; ++p) {
        xs[p] = vecs[3 * p];
        ys[p] = vecs[3 * p + 1];
        zs[p] = vecs[3 * p + 2];
    }
    hipStream_t s = ctx->stream;
    HIP_TRY(upload(ctx->offsets, std::vector<int>(offsets, offsets + n + 1), s), "upload lists");
    HIP_TRY(upload(ctx->idx, std::vector<int>(indices, indices + P), s), "upload lists");
    HIP_TRY(upload(ctx->type, std::vector<int>(types, types + P), s), "upload lists");
    HIP_TRY(upload(ctx->x, xs, s), "upload lists");
    HIP_TRY(upload(ctx->y, ys, s), "upload lists");
    HIP_TRY(upload(ctx->z, zs, s), "upload lists");
    HIP_TRY(upload(ctx->d, std::vector<double>(dists, dists + P), s), "upload lists");
    HIP_TRY(upload(ctx->center_type, std::vector<int>(center_types, center_types + n), s),
            "upload lists");
    HIP_TRY(hipStreamSynchronize(s), "upload lists");
    ctx->n = n;
    ctx->P = P;
    ctx->max_species = maxs;
    ctx->has_nbh = true;
    return set_single_structure(ctx);
}

int mtpx_build_neighbors(mtpx_context *ctx, const double cell[9], const int pbc[3], int n,
                         const double *pos, const int *types, double cutoff)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!cell || !pbc || n < 0 || (n > 0 && (!pos || !types)) || !(cutoff > 0) ||
        !std::isfinite(cutoff))
        return set_error(ctx, MTPX_E_INVALID, "invalid neighbour-build arguments");
    for (int i = 0; i < 9; ++i)
        if (!std::isfinite(cell[i]))
            return set_error(ctx, MTPX_E_INVALID, "non-finite cell");
    if (!all_finite(pos, 3 * (size_t)n))
        return set_error(ctx, MTPX_E_INVALID, "non-finite position");
    std::vector<int> tbuf;
    if (int rc = map_species(ctx, types, (size_t)n, false, tbuf, types))
        return rc;
    const int Z = ctx->has_model ? ctx->model.Z : 1 << 30;
    int maxs = -1;
    if (!species_in_range(types, (size_t)n, Z, maxs))
        return set_error(ctx, MTPX_E_INVALID, "species out of range");
    (void)hipSetDevice(ctx->device);
    ctx->has_nbh = false;
    ctx->rev_ready = false;
    std::string err;
    int rc = build_neighbors_gpu(cell, pbc, n, pos, types, cutoff, ctx->stream, ctx->nbh,
                                 ctx->scratch, err);
    if (rc != MTPX_OK)
        return set_error(ctx, rc, err);
    ctx->max_species = maxs;
    ctx->has_nbh = true;
    return set_single_structure(ctx);
}

int mtpx_neighbor_count(const mtpx_context *ctx, int64_t *entries, int *centers)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_nbh)
        return MTPX_E_NO_TOPOLOGY;
    if (entries)
        *entries = ctx->P;
    if (centers)
        *centers = ctx->n;
    return MTPX_OK;
}

int mtpx_get_neighbors(const mtpx_context *ctx_c, int *offsets, int *indices, int *types,
                       double *vecs, double *dists, int *center_types)
{
    mtpx_context *ctx = const_cast<mtpx_context *>(ctx_c);
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no neighbour lists");
    (void)hipSetDevice(ctx->device);
    const int n = ctx->n;
    const int64_t P = ctx->P;
    auto d2h = [&](void *dst, const DBuf &src, size_t bytes) {
        return bytes ? hipMemcpy(dst, src.p, bytes, hipMemcpyDeviceToHost) : hipSuccess;
    };
    if (offsets)
        HIP_TRY(d2h(offsets, ctx->offsets, sizeof(int) * (n + 1)), "copy lists");
    if (indices)
        HIP_TRY(d2h(indices, ctx->idx, sizeof(int) * P), "copy lists");
    if (types)
        HIP_TRY(d2h(types, ctx->type, sizeof(int) * P), "copy lists");
    if (dists)
        HIP_TRY(d2h(dists, ctx->d, sizeof(double) * P), "copy lists");
    if (center_types)
        HIP_TRY(d2h(center_types, ctx->center_type, sizeof(int) * n), "copy lists");
    if (vecs) {
        std::vector<double> c((size_t)P);
        for (int a = 0; a < 3; ++a) {
            const DBuf &b = a == 0 ? ctx->x : a == 1 ? ctx->y : ctx->z;
            HIP_TRY(d2h(c.data(), b, sizeof(double) * P), "copy lists");
            for (int64_t p = 0; p < P; ++p)
                vecs[3 * p + a] = c[p];
        }
    }
    return MTPX_OK;
}

int mtpx_efs_device(mtpx_context *ctx, int deterministic)
{
    if (!ctx)
        return MTPX_E_INVALID;
    (void)hipSetDevice(ctx->device);
    return run_efs(ctx, deterministic != 0);
}

int mtpx_efs(mtpx_context *ctx, int deterministic, double *energy, double *forces, double *stress,
             double *site_energies)
{
    if (!ctx)
        return MTPX_E_INVALID;
    (void)hipSetDevice(ctx->device);
    int rc = run_efs(ctx, deterministic != 0);
    if (rc != MTPX_OK)
        return rc;
    const bool add = ctx->add_efs;
    double o10[10];
    HIP_TRY(hipMemcpy(o10, ctx->out10.p, sizeof o10, hipMemcpyDeviceToHost), "copy outputs");
    if (energy)
        *energy = add ? *energy + o10[0] : o10[0];
    if (stress)
        for (int k = 0; k < 9; ++k)
            stress[k] = add ? stress[k] + o10[1 + k] : o10[1 + k];
    if (forces)
        if (int rc2 = copy_out(ctx, forces, ctx->forces.p, 3 * (size_t)ctx->n, add, "copy forces"))
            return rc2;
    if (site_energies)
        if (int rc2 = copy_out(ctx, site_energies, ctx->site_energy.p, (size_t)ctx->n, add,
                               "copy site energies"))
            return rc2;
    return MTPX_OK;
}

int mtpx_efs_noalloc(mtpx_context *ctx, double *forces, double *site_energies,
                     double *energy_stress)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no neighbour lists");
    if (int rc = check_species(ctx))
        return rc;
    const int n = ctx->n;
    if (!energy_stress || (n > 0 && (!forces || !site_energies)))
        return set_error(ctx, MTPX_E_INVALID, "null device output");
    if (!ctx->noalloc_scratch)
        return set_error(ctx, MTPX_E_DEVICE, "no scratch address for this device");
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->stream;
    EfsLaunch cfg;
    if (!efs_configure(ctx->dm, n, ctx->num_cus, 0, ctx->lds_limit, cfg))
        return set_error(ctx, MTPX_E_CAPACITY, "model needs more LDS than a CU provides");
    // the per-wave partial rows must fit the scratch: fewer workgroups walk
    // the atoms with a longer stride when they would not
    const int cap_rows = (int)(kNoAllocScratchDoubles / 10);
    if (cfg.waves > cap_rows)
        return set_error(ctx, MTPX_E_CAPACITY,
                         "per-wave partial rows exceed the allocation-free scratch");
    cfg.grid = std::min(cfg.grid, cap_rows / cfg.waves);
    cfg.rows = cfg.grid * cfg.waves;
    if (n > 0) {
        EfsOut out;
        out.forces = forces;
        out.site_energy = site_energies;
        out.partial = ctx->noalloc_scratch;
        out.pair_ders = nullptr;
        out.site_virial = nullptr;
        out.site_virial6 = nullptr;
        const DevNeighbors nb = dev_neighbors(ctx);
        HIP_TRY(launch_fill_zero(forces, 3 * (size_t)n, s), "clear forces");
        HIP_TRY(launch_efs(ctx->dm, nb, out, cfg, 0, s), "launch efs kernel");
        HIP_TRY(launch_efs_finish(nb, out, cfg.rows, false, nullptr, nullptr, energy_stress, s),
                "launch efs reduction");
    } else {
        HIP_TRY(launch_fill_zero(energy_stress, 10, s), "clear outputs");
    }
    HIP_TRY(hipStreamSynchronize(s), "efs");
    return MTPX_OK;
}

int mtpx_set_add_efs(mtpx_context *ctx, int add_efs)
{
    if (!ctx)
        return MTPX_E_INVALID;
    ctx->add_efs = add_efs != 0;
    return MTPX_OK;
}

int mtpx_energy(mtpx_context *ctx, double *energies, double *site_energies)
{
    if (!ctx)
        return MTPX_E_INVALID;
    (void)hipSetDevice(ctx->device);
    int rc = run_efs(ctx, false, false, true);
    if (rc != MTPX_OK)
        return rc;
    const int nc = ctx->nconf, n = ctx->n;
    if (energies && nc > 0) {
        HIP_TRY(ctx->benergy.ensure(sizeof(double) * nc), "allocate energies");
        if (n > 0)
            HIP_TRY(launch_structure_reduce(ctx->soff.as<int>(), nc, ctx->site_energy.as<double>(),
                                            nullptr, ctx->benergy.as<double>(), nullptr,
                                            ctx->stream),
                    "launch structure reduction");
        else
            HIP_TRY(hipMemsetAsync(ctx->benergy.p, 0, sizeof(double) * nc, ctx->stream), "clear");
        HIP_TRY(hipMemcpyAsync(energies, ctx->benergy.p, sizeof(double) * nc,
                               hipMemcpyDeviceToHost, ctx->stream),
                "copy energies");
    }
    if (site_energies && n > 0)
        HIP_TRY(hipMemcpyAsync(site_energies, ctx->site_energy.p, sizeof(double) * n,
                               hipMemcpyDeviceToHost, ctx->stream),
                "copy site energies");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "energy");
    ctx->has_batch_out = false;
    return MTPX_OK;
}

int mtpx_last_timings(const mtpx_context *ctx, double out_ms[4])
{
    if (!ctx || !out_ms)
        return MTPX_E_INVALID;
    std::memcpy(out_ms, ctx->timings, sizeof ctx->timings);
    return MTPX_OK;
}

int mtpx_set_timings(mtpx_context *ctx, int enabled)
{
    if (!ctx)
        return MTPX_E_INVALID;
    ctx->timings_on = enabled != 0;
    return MTPX_OK;
}

}  // extern "C"
