// Fused MTP energy/force/stress kernel for gfx950 (CDNA4), fp64.
//
// Reference semantics: PotMTP::CalcSiteEFS + getEFS
// (potentials/potential_mtp.cpp:2813-2984, :1899-1933).  The arithmetic is
// reorganised for a wave64; results agree with the reference to rounding.
//
// A workgroup holds up to twelve wave64s (level 16: three per SIMD) that
// share one LDS copy of the model tables (radial coefficients, adjoint seeds,
// moment coefficients, slot tables and, when that costs no waves, the
// product-rule step tables).  Each wave owns a private LDS work space (the
// transpose buffer lies over the adjoint block, the force pass's adjoints
// over the moments) and works through its own atoms (grid-stride), so the
// waves synchronise only at wavefront scope.  Per atom:
//   1. lanes over neighbours: Chebyshev basis Q_k(d), radial functions
//      f_mu = sum_k c[ti,tj,mu,k] Q_k (coefficients staged in LDS), unit
//      vector u = r/d.  Every basic moment (mu, a, b, c) equals
//      sum_j f_mu(d_j) * Y_abc(u_j) with Y_abc = ux^a uy^b uz^c, so the basics
//      are produced shell by shell (degree nu = a+b+c, compile-time unrolled)
//      in registers and summed over neighbours through a padded LDS
//      transpose, 16 slots at a time.
//   2. the product rules run lane-parallel from lane-major step tables of
//      8-byte entries, one dependency level at a time (forward values, then
//      reverse adjoints).
//   3. lanes over neighbours again: dE_i/dr_j from the closed form
//      grad_r[f Y] = (f' - nu f/d) Y u + (f/d) grad_u Y, with the basic
//      adjoints read as LDS broadcasts.
//   4. F_i += sum_j D_j, F_idx(j) -= D_j, S_ab -= D_ja r_jb.  Fast mode uses
//      fp64 atomics for the neighbour reactions; deterministic mode stores D
//      per pair for an ordered gather.  Each atom's energy and virial are
//      summed over the lanes (lane swaps and DPP moves) into the wave's
//      sums in LDS, which a single ordered pass finishes.
//
// Kernel variants: a "shell profile" fixes, per radial function mu, the
// highest angular degree of its basic moments.  The level-10/16/20 template
// profiles are compile-time constants (every (nu, mu) guard folds away); the
// generic variants read the profile at run time.
#include "mtp_device.hpp"

#include <algorithm>

namespace mtpx {

namespace {

template <class P, bool kTabLds, int kMaxWaves, bool kHead>
__global__ __launch_bounds__(kWave *kMaxWaves) void efs_kernel(DevModel m, DevNeighbors nb,
                                                               EfsOut out, int flags)
{
    const bool deterministic = flags & kEfsDeterministic;
    extern __shared__ double lds[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nwaves = blockDim.x / kWave;
    const Shared L = shared_layout(m, lds);
    double *ws = lds + shared_doubles(m, kTabLds) + (size_t)wave * m.priv_doubles;
    double *mom = ws, *A = ws + m.K4, *red = ws + m.efs_red;
    double *As = ws + m.efs_stage;  // slot-ordered adjoints (force pass)
    double *sums = ws + m.efs_acc;  // the wave's energy and virial[9] (lane 0)

    // model tables the per-atom phases index, staged once per workgroup
    stage_shared(m, L, kTabLds, tid, blockDim.x);
    // the dummy slot and the partial sums start at zero; the rule phases
    // leave them zero
    for (int k = m.dummy + lane; k < m.red0; k += kWave)
        ws[k] = 0.0;
    if (lane < 10)
        sums[lane] = 0.0;
    __syncthreads();
    const int2 *fwd_tab = kTabLds ? L.fwd_steps : m.fwd_steps;
    const int2 *bwd_tab = kTabLds ? L.bwd_steps : m.bwd_steps;

    const int row = blockIdx.x * nwaves + wave;
    for (int i = row; i < nb.n; i += gridDim.x * nwaves) {
        const int ti = nb.center_type[i];
        const int ai = nb.center ? nb.center[i] : i;  // the centre's atom
        const int beg = nb.offsets[i];
        const int n = nb.offsets[i + 1] - beg;
        for (int k = lane; k < m.K; k += kWave)
            mom[k] = 0.0;
        wave_sync();

        // ---- basic moments -------------------------------------------------
        for (int base = 0; base < n; base += kWave) {
            FwdCtx cx{red, mom, L.slot_basic, lane, 0};
            Nbr<P::M> q;
            const bool valid = lane < n - base;
            load_neighbor<P>(m, nb, L.coef, ti, beg + base + lane, valid, q);
            fwd_shells<0, P>(m, cx, q, nullptr);
            const int rest = cx.slot % kChunk;
            if (rest)
                reduce_chunk(red, rest, cx.slot - rest, L.slot_basic, mom, lane);
        }
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                mom[m.dup[2 * k]] = mom[m.dup[2 * k + 1]];
        // the zero slot and the partial sums may lie under the transpose buffer
        for (int k = m.dummy + lane; k < m.red0; k += kWave)
            ws[k] = 0.0;
        wave_sync();

        run_rules<false, false>(fwd_tab, m.fwd_level_step, m.fwd_level_comb, m.fwd_comb, m.nfwd, ws, lane);

        // ---- site energy (potential_mtp.cpp:2966-2970) and adjoint seed ----
        // (an MTP-M head: the head of the descriptors, its seeds per atom)
        double e = 0.0;
        const bool energy_only = flags & kEfsEnergyOnly;
        if constexpr (kHead) {
            const int w0 = (int)(ws - lds);
            e = head_site(m.hd, ti, w0, w0 + m.efs_head, w0 + m.K4, lane, !energy_only);
        } else {
            for (int s = lane; s < m.S; s += kWave)
                e += L.moment[s] * mom[L.map[s]];
            e = wave_sum(e);
        }
        const double site_energy = m.species[ti] + e;
        if (lane == 0) {
            out.site_energy[i] = site_energy;
            sums[0] += site_energy;
        }
        if (energy_only)  // getE (potential_mtp.cpp:2604-2621): no gradient
            continue;
        if constexpr (!kHead)  // (a head has written its seeds)
            for (int k = lane; k < m.K; k += kWave)
                A[k] = L.seed[k];
        wave_sync();

        run_rules<false, true>(bwd_tab, m.bwd_level_step, m.bwd_level_comb, m.bwd_comb, m.nbwd, ws, lane);
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                A[m.dup[2 * k + 1]] += A[m.dup[2 * k]];
        wave_sync();
        // slot-ordered adjoints
        for (int s = lane; s < m.nslots; s += kWave) {
            const int b = L.slot_basic[s];
            As[s] = b >= 0 ? A[b] : 0.0;
        }
        wave_sync();

        // ---- forces and virial ---------------------------------------------
        double fi0 = 0, fi1 = 0, fi2 = 0;
        double vs[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};  // this lane's share of the virial
        for (int base = 0; base < n; base += kWave) {
            const bool valid = lane < n - base;
            const int64_t p = beg + base + lane;
            Nbr<P::M> q;
            load_neighbor<P>(m, nb, L.coef, ti, p, valid, q);
            BwdAcc acc{0, 0, 0, 0};
            int slot = 0;
            bwd_shells<0, P>(m, As, slot, q, nullptr, acc);
            const double D0 = acc.s * q.ux + acc.gx * q.invd;
            const double D1 = acc.s * q.uy + acc.gy * q.invd;
            const double D2 = acc.s * q.uz + acc.gz * q.invd;
            const double r[3] = {q.x, q.y, q.z}, D[3] = {D0, D1, D2};
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int bq = 0; bq < 3; ++bq)
                    vs[3 * a + bq] -= D[a] * r[bq];
            fi0 += D0;
            fi1 += D1;
            fi2 += D2;
            if (valid) {
                if (deterministic) {
                    // with the mirror assembly D goes to the slot of the
                    // entry's mirror, so the gather reads each list's
                    // reactions in order
                    const int64_t w = (flags & kEfsOwnForce) ? (int64_t)nb.mirror[p] : p;
                    out.pair_ders[3 * w + 0] = D0;
                    out.pair_ders[3 * w + 1] = D1;
                    out.pair_ders[3 * w + 2] = D2;
                } else {
                    const int j = nb.idx[p];
                    atomicAdd(&out.forces[3 * j + 0], -D0);
                    atomicAdd(&out.forces[3 * j + 1], -D1);
                    atomicAdd(&out.forces[3 * j + 2], -D2);
                    if (out.site_virial6) {
                        // the neighbour's half (runtime/mtp/mlip.cpp:1181-1189)
                        double *v = out.site_virial6 + 6 * (size_t)j;
                        atomicAdd(v + 0, -0.5 * D0 * q.x);
                        atomicAdd(v + 1, -0.5 * D1 * q.y);
                        atomicAdd(v + 2, -0.5 * D2 * q.z);
                        atomicAdd(v + 3, -0.25 * (D1 * q.x + D0 * q.y));
                        atomicAdd(v + 4, -0.25 * (D2 * q.x + D0 * q.z));
                        atomicAdd(v + 5, -0.25 * (D2 * q.y + D1 * q.z));
                    }
                }
            }
        }
        // this atom's force (its own entries) and virial, summed over the
        // lanes in one pass: lane 16 r + k (k < 3) ends with one total
        double fv[12] = {fi0, fi1, fi2, vs[0], vs[1], vs[2], vs[3], vs[4], vs[5], vs[6], vs[7],
                         vs[8]};
        int vi;
        const double tot = wave_reduce_scatter<12>(fv, lane, vi);
        if (vi >= 0 && vi < 3) {
            if (!deterministic)
                atomicAdd(&out.forces[3 * ai + vi], tot);
            else if (flags & kEfsOwnForce)
                out.forces[3 * ai + vi] = tot;
        } else if (vi >= 3) {
            sums[vi - 2] += tot;  // the wave's virial sums, sums[1 .. 9]
            if (out.site_virial)
                out.site_virial[9 * (size_t)i + vi - 3] = tot;
        }
        if (out.site_virial6 && !deterministic) {
            // the centre's half of its entries (mlip.cpp:1164-1180), from the
            // nine totals gathered through the (idle) transpose buffer
            if (vi >= 3)
                red[vi - 3] = tot;
            wave_sync();
            if (lane == 0) {
                double *v = out.site_virial6 + 6 * (size_t)ai;
                atomicAdd(v + 0, 0.5 * red[0]);
                atomicAdd(v + 1, 0.5 * red[4]);
                atomicAdd(v + 2, 0.5 * red[8]);
                atomicAdd(v + 3, 0.25 * (red[3] + red[1]));
                atomicAdd(v + 4, 0.25 * (red[6] + red[2]));
                atomicAdd(v + 5, 0.25 * (red[7] + red[5]));
            }
        }
        wave_sync();
    }
    // per-wave partials: energy, stress[9]
    wave_sync();
    if (lane < 10)
        out.partial[10 * row + lane] = sums[lane];
}

// Ordered reduction of the per-wave partials (one workgroup of 256).
__device__ __forceinline__ void partial_reduce(const double *partial, int nrows, double *out10)
{
    __shared__ double buf[256][10];
    const int t = threadIdx.x;
    double acc[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = t; b < nrows; b += 256)
#pragma unroll
        for (int k = 0; k < 10; ++k)
            acc[k] += partial[10 * b + k];
#pragma unroll
    for (int k = 0; k < 10; ++k)
        buf[t][k] = acc[k];
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if (t < w)
#pragma unroll
            for (int k = 0; k < 10; ++k)
                buf[t][k] += buf[t + w][k];
        __syncthreads();
    }
    if (t < 10)
        out10[t] = buf[0][t];
}

__global__ __launch_bounds__(256) void partial_reduce_kernel(const double *partial, int nrows,
                                                             double *out10)
{
    partial_reduce(partial, nrows, out10);
}

// Deterministic force assembly: F_k = sum_{p in list(k)} D_p - sum_{p : idx_p = k} D_p,
// both sums in ascending pair order.
__global__ __launch_bounds__(256) void force_gather_kernel(DevNeighbors nb, const double *D,
                                                           const int *rev_offsets,
                                                           const int *rev_pairs, double *forces)
{
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= nb.n)
        return;
    double f0 = 0, f1 = 0, f2 = 0;
    for (int p = nb.offsets[k]; p < nb.offsets[k + 1]; ++p) {
        f0 += D[3 * (int64_t)p];
        f1 += D[3 * (int64_t)p + 1];
        f2 += D[3 * (int64_t)p + 2];
    }
    for (int q = rev_offsets[k]; q < rev_offsets[k + 1]; ++q) {
        const int64_t p = rev_pairs[q];
        f0 -= D[3 * p];
        f1 -= D[3 * p + 1];
        f2 -= D[3 * p + 2];
    }
    forces[3 * k] = f0;
    forces[3 * k + 1] = f1;
    forces[3 * k + 2] = f2;
}

// The reactions: F_a -= sum over a's entries q of Dm[q], the derivative of
// q's mirror entry (the E/F/S kernel stored each entry's derivative at its
// mirror's slot), onto the own force the kernel stored.  Sixteen lanes per
// atom stride over its entries (contiguous reads) and sum over their row
// (DPP), so the order is fixed and the result repeatable.
// The first workgroup reduces the per-wave partials instead (one launch for
// both; dispatched first, its dependent loads overlap the gather).
__global__ __launch_bounds__(256) void mirror_gather_kernel(DevNeighbors nb, const double *Dm,
                                                            double *forces, const double *partial,
                                                            int nrows, double *out10)
{
    if (blockIdx.x == 0) {
        partial_reduce(partial, nrows, out10);
        return;
    }
    const int t = (blockIdx.x - 1) * blockDim.x + threadIdx.x;
    const int a = t >> 4, l = t & 15;
    double f0 = 0.0, f1 = 0.0, f2 = 0.0;
    if (a < nb.n) {
        const int e = nb.offsets[a + 1];
        for (int64_t q = nb.offsets[a] + l; q < e; q += 16) {
            f0 += Dm[3 * q];
            f1 += Dm[3 * q + 1];
            f2 += Dm[3 * q + 2];
        }
    }
    f0 = row16_sum(f0);
    f1 = row16_sum(f1);
    f2 = row16_sum(f2);
    if (a < nb.n && l < 3)
        forces[3 * (int64_t)a + l] -= l == 0 ? f0 : l == 1 ? f1 : f2;
}

// -1/2 D r^T, symmetrised off the diagonal, as (xx, yy, zz, xy, xz, yz): one
// endpoint's share of an entry in the LAMMPS per-atom virial
// (runtime/mtp/mlip.cpp:1164-1190).
__device__ __forceinline__ void half_virial(const double *D, double rx, double ry, double rz,
                                            double v[6])
{
    v[0] += -0.5 * D[0] * rx;
    v[1] += -0.5 * D[1] * ry;
    v[2] += -0.5 * D[2] * rz;
    v[3] += -0.25 * (D[1] * rx + D[0] * ry);
    v[4] += -0.25 * (D[2] * rx + D[0] * rz);
    v[5] += -0.25 * (D[2] * ry + D[1] * rz);
}

// Deterministic assembly of a site request over every atom k (owned and
// ghost): F_k = sum over k's own entries (when k is a centre) of D minus the
// sum over the entries whose neighbour is k, both in ascending entry order;
// the per-atom virial takes half of each of those entries.
__global__ __launch_bounds__(256) void site_gather_kernel(DevNeighbors nb, int ntotal,
                                                          const int *atom_row, const double *D,
                                                          const int *rev_offsets,
                                                          const int *rev_pairs, double *forces,
                                                          double *site_virial6)
{
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= ntotal)
        return;
    double f[3] = {0, 0, 0}, v[6] = {0, 0, 0, 0, 0, 0};
    const int row = atom_row[k];
    if (row >= 0)
        for (int p = nb.offsets[row]; p < nb.offsets[row + 1]; ++p) {
            const double *Dp = D + 3 * (int64_t)p;
            f[0] += Dp[0];
            f[1] += Dp[1];
            f[2] += Dp[2];
            if (site_virial6)
                half_virial(Dp, nb.x[p], nb.y[p], nb.z[p], v);
        }
    for (int q = rev_offsets[k]; q < rev_offsets[k + 1]; ++q) {
        const int64_t p = rev_pairs[q];
        const double *Dp = D + 3 * p;
        f[0] -= Dp[0];
        f[1] -= Dp[1];
        f[2] -= Dp[2];
        if (site_virial6)
            half_virial(Dp, nb.x[p], nb.y[p], nb.z[p], v);
    }
    if (forces) {
        forces[3 * (int64_t)k] = f[0];
        forces[3 * (int64_t)k + 1] = f[1];
        forces[3 * (int64_t)k + 2] = f[2];
    }
    if (site_virial6)
        for (int c = 0; c < 6; ++c)
            site_virial6[6 * (int64_t)k + c] = v[c];
}

// Scratch of the allocation-free entry point: the per-wave partial rows.
// Host code never names this array; it takes the device address from
// noalloc_scratch_address once per device.
static __device__ __align__(256) double scratch[kNoAllocScratchDoubles];

__global__ __launch_bounds__(256) void fill_zero_kernel(double *p, size_t count)
{
    for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < count;
         k += (size_t)gridDim.x * blockDim.x)
        p[k] = 0.0;
}

// Kernel variants: shell profile x table placement.  The profiles whose
// kernels fit 256 registers run eight waves per workgroup, the larger ones four.
template <class P>
struct VariantWaves {
    static constexpr int value = 12;
};
template <>
struct VariantWaves<ProfLevel20> {
    static constexpr int value = 8;
};
template <>
struct VariantWaves<ProfGeneric> {
    static constexpr int value = 4;
};

template <class P>
void launch_variant(const DevModel &m, const DevNeighbors &nb, const EfsOut &out,
                    const EfsLaunch &cfg, int det, hipStream_t s)
{
    // MTP-M heads get kernels of their own: a linear model's kernel holds no
    // call of the out-of-line head (a call site costs registers and a stack)
    constexpr int W = VariantWaves<P>::value;
    const dim3 grid(cfg.grid), block(kWave * cfg.waves);
    if (m.head) {
        if (cfg.lds_tables)
            hipLaunchKernelGGL((efs_kernel<P, true, W, true>), grid, block, cfg.lds_bytes, s, m,
                               nb, out, det);
        else
            hipLaunchKernelGGL((efs_kernel<P, false, W, true>), grid, block, cfg.lds_bytes, s, m,
                               nb, out, det);
    } else if (cfg.lds_tables) {
        hipLaunchKernelGGL((efs_kernel<P, true, W, false>), grid, block, cfg.lds_bytes, s, m, nb,
                           out, det);
    } else {
        hipLaunchKernelGGL((efs_kernel<P, false, W, false>), grid, block, cfg.lds_bytes, s, m, nb,
                           out, det);
    }
}

int variant_max_waves(int v)
{
    switch (v) {
    case 0: return VariantWaves<ProfLevel16>::value;
    case 1: return VariantWaves<ProfLevel20>::value;
    case 2: return VariantWaves<ProfLevel10>::value;
    case 3: return VariantWaves<ProfSmall>::value;
    default: return VariantWaves<ProfGeneric>::value;
    }
}

}  // namespace

bool efs_configure(const DevModel &m, int n, int num_cus, int max_waves, size_t lds_limit,
                   EfsLaunch &cfg, int table_pref)
{
    const int vmax = variant_max_waves(efs_variant(m, m.R));
    const int wcap = max_waves > 0 ? std::min(vmax, max_waves) : vmax;
    return configure_launch(m, n, num_cus, wcap, lds_limit, m.priv_doubles, cfg, table_pref);
}

// 0: level-16 profile, 1: level-20, 2: level-10 (each with its template's
// radial basis size), 3: small runtime, 4: generic
int efs_variant(const DevModel &m, int R)
{
    // general radial bases are evaluated by the run-time profiles only
    if (m.rb_general)
        return m.M <= 4 && m.numax_all <= 6 && R <= 8 ? 3 : 4;
    if (profile_is<6, 4, 2, 0>(m) && R == 8)
        return 0;
    if (profile_is<8, 6, 4, 2, 0>(m) && R == 10)
        return 1;
    if (profile_is<3, 1, 0>(m) && R == 8)
        return 2;
    if (m.M <= 4 && m.numax_all <= 6 && R <= 8)
        return 3;
    return 4;
}

hipError_t launch_efs(const DevModel &m, const DevNeighbors &nb, const EfsOut &out,
                      const EfsLaunch &cfg, int flags, hipStream_t s)
{
    const int det = flags;
    switch (efs_variant(m, m.R)) {
    case 0: launch_variant<ProfLevel16>(m, nb, out, cfg, det, s); break;
    case 1: launch_variant<ProfLevel20>(m, nb, out, cfg, det, s); break;
    case 2: launch_variant<ProfLevel10>(m, nb, out, cfg, det, s); break;
    case 3: launch_variant<ProfSmall>(m, nb, out, cfg, det, s); break;
    default: launch_variant<ProfGeneric>(m, nb, out, cfg, det, s); break;
    }
    return hipGetLastError();
}

hipError_t noalloc_scratch_address(double **ptr)
{
    return hipGetSymbolAddress(reinterpret_cast<void **>(ptr), HIP_SYMBOL(scratch));
}

hipError_t launch_fill_zero(double *p, size_t count, hipStream_t s)
{
    if (count)
        hipLaunchKernelGGL(fill_zero_kernel,
                           dim3((unsigned)std::min<size_t>((count + 255) / 256, 4096)), dim3(256),
                           0, s, p, count);
    return hipGetLastError();
}

hipError_t launch_site_gather(const DevNeighbors &nb, int ntotal, const int *atom_row,
                              const double *pair_ders, const int *rev_offsets,
                              const int *rev_pairs, double *forces, double *site_virial6,
                              hipStream_t s)
{
    if (ntotal > 0)
        hipLaunchKernelGGL(site_gather_kernel, dim3((ntotal + 255) / 256), dim3(256), 0, s, nb,
                           ntotal, atom_row, pair_ders, rev_offsets, rev_pairs, forces,
                           site_virial6);
    return hipGetLastError();
}

hipError_t launch_efs_finish(const DevNeighbors &nb, const EfsOut &out, int rows,
                             bool deterministic, const int *rev_offsets, const int *rev_pairs,
                             double *energy_stress10, hipStream_t s)
{
    if (deterministic && nb.n > 0 && nb.mirror) {
        const unsigned gather = (unsigned)(((int64_t)nb.n * 16 + 255) / 256);
        hipLaunchKernelGGL(mirror_gather_kernel, dim3(gather + 1), dim3(256), 0, s, nb,
                           out.pair_ders, out.forces, out.partial, rows, energy_stress10);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(partial_reduce_kernel, dim3(1), dim3(256), 0, s, out.partial, rows,
                       energy_stress10);
    if (deterministic && nb.n > 0)
        hipLaunchKernelGGL(force_gather_kernel, dim3((nb.n + 255) / 256), dim3(256), 0, s, nb,
                           out.pair_ders, rev_offsets, rev_pairs, out.forces);
    return hipGetLastError();
}

}  // namespace mtpx
