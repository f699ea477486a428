// Fused MTP energy/force/stress kernel for gfx950 (CDNA4), fp64.
//
// Reference semantics: PotMTP::CalcSiteEFS + getEFS
// (potentials/potential_mtp.cpp:2813-2984, :1899-1933).  The arithmetic is
// reorganised for a wave64; results agree with the reference to rounding.
//
// A workgroup holds up to eight wave64s that share one LDS copy of the model
// tables (radial coefficients, adjoint seeds, moment coefficients, slot
// tables and, when they fit, the product-rule step tables).  Each wave owns a
// private LDS work space and works through its own atoms (grid-stride), so the
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
//      per pair for an ordered gather.  Energy and virial are reduced per
//      wave and finished by a single ordered pass.
//
// Kernel variants: a "shell profile" fixes, per radial function mu, the
// highest angular degree of its basic moments.  The level-10/16/20 template
// profiles are compile-time constants (every (nu, mu) guard folds away); the
// generic variants read the profile at run time.
#include "mtpx_internal.hpp"

#include <algorithm>

namespace mtpx {

namespace {

constexpr int shell_size(int nu) { return (nu + 1) * (nu + 2) / 2; }

// Position of (a, b, c = nu-a-b) in the shell enumeration a = nu..0, b = nu-a..0.
constexpr int shell_index(int nu, int a, int b)
{
    int pos = 0;
    for (int ap = nu; ap > a; --ap)
        pos += nu - ap + 1;
    return pos + (nu - a - b);
}

// ---- shell profiles ---------------------------------------------------
template <int MM, int NN, int RR, int... NM>
struct ExactProfile {
    static constexpr bool exact = true;
    static constexpr int M = MM, NUMAX = NN, RMAX = RR;
    static constexpr int nm[MM] = {NM...};
    static __device__ __forceinline__ bool active(const DevModel &, int mu, int nu)
    {
        return nm[mu] >= nu;
    }
    static __device__ __forceinline__ bool deeper(const DevModel &, int nu) { return nu < NN; }
};
template <int MM, int NN, int RR>
struct RuntimeProfile {
    static constexpr bool exact = false;
    static constexpr int M = MM, NUMAX = NN, RMAX = RR;
    static __device__ __forceinline__ bool active(const DevModel &m, int mu, int nu)
    {
        return mu < m.M && m.numax[mu] >= nu;
    }
    static __device__ __forceinline__ bool deeper(const DevModel &m, int nu)
    {
        return nu < m.numax_all;
    }
};
using ProfLevel10 = ExactProfile<3, 3, 8, 3, 1, 0>;
using ProfLevel16 = ExactProfile<4, 6, 8, 6, 4, 2, 0>;
using ProfLevel20 = ExactProfile<5, 8, 10, 8, 6, 4, 2, 0>;
using ProfSmall = RuntimeProfile<4, 6, 8>;
using ProfGeneric = RuntimeProfile<kMaxMu, kMaxNu, kMaxR>;

// v[l] + v[l ^ 32] and v[l] + v[l ^ 16] with the gfx950 lane swaps (VALU, no
// LDS crossbar): permlane32_swap exchanges the wave halves, permlane16_swap
// the odd and even rows of 16 lanes.
__device__ __forceinline__ double xor32_sum(double v)
{
    const unsigned lo = __double2loint(v), hi = __double2hiint(v);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return __hiloint2double(h[0], l[0]) + __hiloint2double(h[1], l[1]);
}
__device__ __forceinline__ double xor16_sum(double v)
{
    const unsigned lo = __double2loint(v), hi = __double2hiint(v);
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return __hiloint2double(h[0], l[0]) + __hiloint2double(h[1], l[1]);
}

__device__ __forceinline__ double wave_sum(double v)
{
    v = xor32_sum(v);
    v = xor16_sum(v);
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1)
        v += __shfl_xor(v, off, kWave);
    return v;
}

// Orders the LDS accesses of one wave: a wave's LDS operations complete in
// issue order, so a compiler-level fence at wavefront scope is all that is
// needed between a lane's store and another lane's load.
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int MMAX>
struct Nbr {
    double x, y, z, d, invd, ux, uy, uz;
    double f[MMAX], fd[MMAX];
};

// Neighbour data of list entry p; lanes without an entry keep zeros, so
// they contribute nothing to the sums below.
template <class P>
__device__ __forceinline__ void load_neighbor(const DevModel &m, const DevNeighbors &nb,
                                              const double *coef_lds, int ti, int64_t p,
                                              bool valid, Nbr<P::M> &q)
{
    constexpr int RMAX = P::RMAX;
    q.x = valid ? nb.x[p] : 0.0;
    q.y = valid ? nb.y[p] : 0.0;
    q.z = valid ? nb.z[p] : 0.0;
    const double dd = valid ? nb.d[p] : m.rmax;
    const int tj = valid ? nb.type[p] : 0;
    // potential_mtp.cpp:2842 -- entries beyond the cutoff are skipped, r == cutoff kept
    const bool in_cutoff = valid && !(dd > m.rmax);
    const double d = in_cutoff ? dd : m.rmax;
    q.d = d;
    q.invd = 1.0 / d;
    q.ux = q.x * q.invd;
    q.uy = q.y * q.invd;
    q.uz = q.z * q.invd;
    // RBasis_Chebyshev::calc_der (basis/basis.cpp:148-164)
    double Q[RMAX], dQ[RMAX];
    const double ksi = (2 * d - m.pu) / m.su;
    const double ru = d - m.rmax;
    Q[0] = m.scaling * (ru * ru);
    dQ[0] = m.scaling * (2 * ru);
    if (RMAX > 1) {
        Q[1] = m.scaling * (ksi * ru * ru);
        dQ[1] = m.scaling * (m.mult * ru * ru + 2 * ksi * ru);
    }
#pragma unroll
    for (int k = 2; k < RMAX; ++k) {
        Q[k] = 2 * ksi * Q[k - 1] - Q[k - 2];
        dQ[k] = 2 * (m.mult * Q[k - 1] + ksi * dQ[k - 1]) - dQ[k - 2];
    }
    const double w = in_cutoff ? 1.0 : 0.0;
    const double *c = coef_lds + (ti * m.Z + tj) * m.M * m.R;
#pragma unroll
    for (int mu = 0; mu < P::M; ++mu) {
        double f = 0, fd = 0;
        if (P::exact || mu < m.M) {
            const double *cm = c + mu * m.R;
#pragma unroll
            for (int k = 0; k < RMAX; ++k)
                if (k < m.R) {
                    f += cm[k] * Q[k];
                    fd += cm[k] * dQ[k];
                }
        }
        q.f[mu] = f * w;
        q.fd[mu] = fd * w;
    }
}

template <int NU, int MMAX>
__device__ __forceinline__ void next_shell(const double *prev, double *cur, const Nbr<MMAX> &q)
{
#pragma unroll
    for (int a = NU; a >= 0; --a)
#pragma unroll
        for (int b = NU - a; b >= 0; --b) {
            const int i = shell_index(NU, a, b);
            if (a > 0)
                cur[i] = prev[shell_index(NU - 1, a - 1, b)] * q.ux;
            else if (b > 0)
                cur[i] = prev[shell_index(NU - 1, 0, b - 1)] * q.uy;
            else
                cur[i] = prev[shell_index(NU - 1, 0, 0)] * q.uz;
        }
}

// Sum `nrows` slots of the transpose buffer over the neighbour columns and
// add the sums to the moment array.  Rows hold 64 columns; columns of lanes
// without a neighbour hold zeros.
__device__ __forceinline__ void reduce_chunk(const double *red, int nrows, int slot0,
                                             const int *slot_basic, double *mom, int lane)
{
    wave_sync();
    const int s = lane & (kChunk - 1), qq = lane >> 4;
    const double2 *row = reinterpret_cast<const double2 *>(red + s * kRedStride + qq * 16);
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        const double2 v = row[jj];
        a0 += v.x;
        a1 += v.y;
    }
    double acc = xor16_sum(xor32_sum(a0 + a1));
    if (lane < nrows) {
        const int b = slot_basic[slot0 + lane];
        if (b >= 0)
            mom[b] += acc;
    }
    wave_sync();
}

struct FwdCtx {
    double *red, *mom;
    const int *slot_basic;
    int lane, slot;  // slots written so far; rows are packed across (nu, mu) blocks
};

template <int NU, class P>
__device__ __forceinline__ void fwd_shells(const DevModel &m, FwdCtx &cx, const Nbr<P::M> &q,
                                           const double *prev)
{
    double cur[shell_size(NU)];
    if constexpr (NU == 0)
        cur[0] = 1.0;
    else
        next_shell<NU, P::M>(prev, cur, q);
#pragma unroll
    for (int mu = 0; mu < P::M; ++mu) {
        if (P::active(m, mu, NU)) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < shell_size(NU); ++i) {
                cx.red[(cx.slot % kChunk) * kRedStride + cx.lane] = q.f[mu] * cur[i];
                ++cx.slot;
                if (cx.slot % kChunk == 0)
                    reduce_chunk(cx.red, kChunk, cx.slot - kChunk, cx.slot_basic, cx.mom,
                                 cx.lane);
            }
        }
    }
    if constexpr (NU < P::NUMAX) {
        if (P::deeper(m, NU))
            fwd_shells<NU + 1, P>(m, cx, q, cur);
    }
}

struct BwdAcc {
    double s, gx, gy, gz;
};

template <int NU, class P>
__device__ __forceinline__ void bwd_shells(const DevModel &m, const double4 *A4, int &slot,
                                           const Nbr<P::M> &q, const double *prev, BwdAcc &acc)
{
    double cur[shell_size(NU)];
    if constexpr (NU == 0)
        cur[0] = 1.0;
    else
        next_shell<NU, P::M>(prev, cur, q);
#pragma unroll
    for (int mu = 0; mu < P::M; ++mu) {
        if (P::active(m, mu, NU)) {
            // keep the adjoint loads of one (nu, mu) block from being hoisted
            // into the previous one: bounds the live registers
            __builtin_amdgcn_sched_barrier(0);
            double u = 0, Gx = 0, Gy = 0, Gz = 0;
#pragma unroll
            for (int a = NU; a >= 0; --a)
#pragma unroll
                for (int b = NU - a; b >= 0; --b) {
                    const int i = shell_index(NU, a, b);
                    const double4 w = A4[slot + i];  // {A, aA, bA, cA}, LDS broadcast
                    u += w.x * cur[i];
                    if constexpr (NU > 0) {
                        if (a > 0)
                            Gx += w.y * prev[shell_index(NU - 1, a - 1, b)];
                        if (b > 0)
                            Gy += w.z * prev[shell_index(NU - 1, a, b - 1)];
                        if (NU - a - b > 0)
                            Gz += w.w * prev[shell_index(NU - 1, a, b)];
                    }
                }
            const double h = q.fd[mu] - NU * q.f[mu] * q.invd;
            acc.s += h * u;
            acc.gx += q.f[mu] * Gx;
            acc.gy += q.f[mu] * Gy;
            acc.gz += q.f[mu] * Gz;
            slot += shell_size(NU);
        }
    }
    if constexpr (NU < P::NUMAX) {
        if (P::deeper(m, NU))
            bwd_shells<NU + 1, P>(m, A4, slot, q, cur, acc);
    }
}

// Product rules from a lane-major step table (forward: potential_mtp.cpp:
// 2918-2924; reverse: backpropagate_moments, :3292-3305), one dependency
// level at a time.  Steps are taken in groups of four: the entries of the
// next group are loaded while the current one runs, and every operand of a
// group is read before any of its results is written (a level never reads
// what it writes).
__device__ __forceinline__ void run_rules(const int2 *tab, const int *level_step,
                                          const int *level_comb, const int4 *comb, int nlev,
                                          double *ws, int lane)
{
    for (int L = 0; L < nlev; ++L) {
        const int s0 = level_step[L], s1 = level_step[L + 1];
        double acc = 0.0;
        if (s1 > s0) {
            const int2 *t = tab + (size_t)s0 * kWave + lane;
            int2 e[4] = {t[0], t[kWave], t[2 * kWave], t[3 * kWave]};
            for (int st = s0; st < s1; st += 4) {
                int2 nx[4] = {e[0], e[1], e[2], e[3]};
                if (st + 4 < s1) {
                    const int2 *u = t + (size_t)(st + 4 - s0) * kWave;
                    nx[0] = u[0];
                    nx[1] = u[kWave];
                    nx[2] = u[2 * kWave];
                    nx[3] = u[3 * kWave];
                }
                double ml[4], mr[4], init[4], v[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    ml[k] = ws[e[k].x & 0xffff];
                    mr[k] = ws[(unsigned)e[k].x >> 16];
                    init[k] = ws[e[k].y & 0xffff];
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const double c = (double)(e[k].y >> 17);
                    acc = fma(c * ml[k], mr[k], (e[k].y & 0x10000) ? init[k] : acc);
                    v[k] = acc;
                }
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    ws[e[k].y & 0xffff] = v[k];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    e[k] = nx[k];
            }
        }
        const int c0 = level_comb[L], c1 = level_comb[L + 1];
        if (c1 > c0) {
            wave_sync();
            for (int c = c0 + lane; c < c1; c += kWave) {
                const int4 q = comb[c];
                double sum = ws[q.x];
                for (int k = 0; k < q.z; ++k) {
                    sum += ws[q.y + k];
                    ws[q.y + k] = 0.0;
                }
                ws[q.x] = sum;
            }
        }
        wave_sync();
    }
}

// Block-shared LDS tables, in this order (doubles, then ints, then the
// optional step tables; every part a multiple of 32 bytes).
struct Shared {
    double *coef, *seed, *moment;
    int *map, *slot_basic, *slot_abc;
    int2 *fwd_steps, *bwd_steps;
};

__device__ __host__ __forceinline__ size_t shared_doubles(const DevModel &m, bool tables)
{
    const size_t r4c = ((size_t)m.Z * m.Z * m.M * m.R + 3) & ~size_t(3);
    const size_t S4 = (m.S + 3) & ~3, N4 = (m.nslots + 3) & ~3;
    size_t d = r4c + m.K4 + S4 + (S4 + 2 * N4) / 2;
    if (tables)
        d += (size_t)(m.fwd_nsteps + m.bwd_nsteps) * kWave;
    return (d + 3) & ~size_t(3);
}

__device__ __forceinline__ Shared shared_layout(const DevModel &m, double *base)
{
    const int r4c = (m.Z * m.Z * m.M * m.R + 3) & ~3;
    const int S4 = (m.S + 3) & ~3, N4 = (m.nslots + 3) & ~3;
    Shared L;
    L.coef = base;
    L.seed = L.coef + r4c;
    L.moment = L.seed + m.K4;
    L.map = reinterpret_cast<int *>(L.moment + S4);
    L.slot_basic = L.map + S4;
    L.slot_abc = L.slot_basic + N4;
    L.fwd_steps = reinterpret_cast<int2 *>(L.slot_abc + N4);
    L.bwd_steps = L.fwd_steps + (size_t)m.fwd_nsteps * kWave;
    return L;
}

template <class P, bool kTabLds, int kMaxWaves>
__global__ __launch_bounds__(kWave *kMaxWaves) void efs_kernel(DevModel m, DevNeighbors nb,
                                                               EfsOut out, int deterministic)
{
    extern __shared__ double lds[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nwaves = blockDim.x / kWave;
    const Shared L = shared_layout(m, lds);
    double *ws = lds + shared_doubles(m, kTabLds) + (size_t)wave * m.priv_doubles;
    double *mom = ws, *A = ws + m.K4, *red = ws + m.red0;
    const double4 *A4 = reinterpret_cast<const double4 *>(red);

    // model tables the per-atom phases index, staged once per workgroup
    const int ncoef_r = m.Z * m.Z * m.M * m.R;
    for (int k = tid; k < ncoef_r; k += blockDim.x)
        L.coef[k] = m.radial[k];
    for (int k = tid; k < m.K; k += blockDim.x)
        L.seed[k] = m.seed[k];
    for (int k = tid; k < m.S; k += blockDim.x) {
        L.moment[k] = m.moment[k];
        L.map[k] = m.map[k];
    }
    for (int k = tid; k < m.nslots; k += blockDim.x) {
        L.slot_basic[k] = m.slot_basic[k];
        L.slot_abc[k] = m.slot_abc[k];
    }
    if constexpr (kTabLds) {
        for (int k = tid; k < m.fwd_nsteps * kWave; k += blockDim.x)
            L.fwd_steps[k] = m.fwd_steps[k];
        for (int k = tid; k < m.bwd_nsteps * kWave; k += blockDim.x)
            L.bwd_steps[k] = m.bwd_steps[k];
    }
    // the dummy slot and the partial sums start at zero; the rule phases
    // leave them zero
    for (int k = m.dummy + lane; k < m.red0; k += kWave)
        ws[k] = 0.0;
    __syncthreads();
    const int2 *fwd_tab = kTabLds ? L.fwd_steps : m.fwd_steps;
    const int2 *bwd_tab = kTabLds ? L.bwd_steps : m.bwd_steps;

    double e_acc = 0.0;  // this lane's share of the wave's energy and virial
    double v_acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};

    const int row = blockIdx.x * nwaves + wave;
    for (int i = row; i < nb.n; i += gridDim.x * nwaves) {
        const int ti = nb.center_type[i];
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
        wave_sync();

        run_rules(fwd_tab, m.fwd_level_step, m.fwd_level_comb, m.fwd_comb, m.nfwd, ws, lane);

        // ---- site energy (potential_mtp.cpp:2966-2970) and adjoint seed ----
        double e = 0.0;
        for (int s = lane; s < m.S; s += kWave)
            e += L.moment[s] * mom[L.map[s]];
        e = wave_sum(e);
        const double site_energy = m.species[ti] + e;
        if (lane == 0) {
            out.site_energy[i] = site_energy;
            e_acc += site_energy;
        }
        for (int k = lane; k < m.K; k += kWave)
            A[k] = L.seed[k];
        wave_sync();

        run_rules(bwd_tab, m.bwd_level_step, m.bwd_level_comb, m.bwd_comb, m.nbwd, ws, lane);
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                A[m.dup[2 * k + 1]] += A[m.dup[2 * k]];
        wave_sync();
        // slot-ordered adjoints {A, aA, bA, cA}
        for (int s = lane; s < m.nslots; s += kWave) {
            const int b = L.slot_basic[s];
            double4 w = {0, 0, 0, 0};
            if (b >= 0) {
                const double a = A[b];
                const int abc = L.slot_abc[s];
                w = {a, a * (abc & 0xff), a * ((abc >> 8) & 0xff), a * ((abc >> 16) & 0xff)};
            }
            reinterpret_cast<double4 *>(red)[s] = w;
        }
        wave_sync();

        // ---- forces and virial ---------------------------------------------
        double fi0 = 0, fi1 = 0, fi2 = 0;
        for (int base = 0; base < n; base += kWave) {
            const bool valid = lane < n - base;
            const int64_t p = beg + base + lane;
            Nbr<P::M> q;
            load_neighbor<P>(m, nb, L.coef, ti, p, valid, q);
            BwdAcc acc{0, 0, 0, 0};
            int slot = 0;
            bwd_shells<0, P>(m, A4, slot, q, nullptr, acc);
            const double D0 = acc.s * q.ux + acc.gx * q.invd;
            const double D1 = acc.s * q.uy + acc.gy * q.invd;
            const double D2 = acc.s * q.uz + acc.gz * q.invd;
            fi0 += D0;
            fi1 += D1;
            fi2 += D2;
            const double r[3] = {q.x, q.y, q.z}, D[3] = {D0, D1, D2};
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int bq = 0; bq < 3; ++bq)
                    v_acc[3 * a + bq] -= D[a] * r[bq];
            if (valid) {
                if (deterministic) {
                    out.pair_ders[3 * p + 0] = D0;
                    out.pair_ders[3 * p + 1] = D1;
                    out.pair_ders[3 * p + 2] = D2;
                } else {
                    const int j = nb.idx[p];
                    atomicAdd(&out.forces[3 * j + 0], -D0);
                    atomicAdd(&out.forces[3 * j + 1], -D1);
                    atomicAdd(&out.forces[3 * j + 2], -D2);
                }
            }
        }
        if (!deterministic) {
            fi0 = wave_sum(fi0);
            fi1 = wave_sum(fi1);
            fi2 = wave_sum(fi2);
            if (lane == 0) {
                atomicAdd(&out.forces[3 * i + 0], fi0);
                atomicAdd(&out.forces[3 * i + 1], fi1);
                atomicAdd(&out.forces[3 * i + 2], fi2);
            }
        }
        wave_sync();
    }
    // per-wave partials: energy, stress[9]
    e_acc = wave_sum(e_acc);
#pragma unroll
    for (int k = 0; k < 9; ++k)
        v_acc[k] = wave_sum(v_acc[k]);
    if (lane == 0) {
        out.partial[10 * row] = e_acc;
#pragma unroll
        for (int k = 0; k < 9; ++k)
            out.partial[10 * row + 1 + k] = v_acc[k];
    }
}

// Ordered reduction of the per-wave partials (one workgroup).
__global__ __launch_bounds__(256) void partial_reduce_kernel(const double *partial, int nrows,
                                                             double *out10)
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

template <int... NM>
bool profile_is(const DevModel &m)
{
    constexpr int nm[] = {NM...};
    constexpr int M = sizeof...(NM);
    if (m.M != M)
        return false;
    for (int mu = 0; mu < M; ++mu)
        if (m.numax[mu] != nm[mu])
            return false;
    return true;
}

// Kernel variants: shell profile x table placement.  The profiles whose
// kernels fit 256 registers run eight waves per workgroup, the larger ones four.
template <class P>
struct VariantWaves {
    static constexpr int value = 8;
};
template <>
struct VariantWaves<ProfLevel20> {
    static constexpr int value = 4;
};
template <>
struct VariantWaves<ProfGeneric> {
    static constexpr int value = 4;
};

template <class P>
void launch_variant(const DevModel &m, const DevNeighbors &nb, const EfsOut &out,
                    const EfsLaunch &cfg, int det, hipStream_t s)
{
    constexpr int W = VariantWaves<P>::value;
    if (cfg.lds_tables)
        hipLaunchKernelGGL((efs_kernel<P, true, W>), dim3(cfg.grid), dim3(kWave * cfg.waves),
                           cfg.lds_bytes, s, m, nb, out, det);
    else
        hipLaunchKernelGGL((efs_kernel<P, false, W>), dim3(cfg.grid), dim3(kWave * cfg.waves),
                           cfg.lds_bytes, s, m, nb, out, det);
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
                   EfsLaunch &cfg)
{
    const size_t kLdsPerCu = lds_limit;
    const size_t priv = (size_t)m.priv_doubles * sizeof(double);
    const int vmax = variant_max_waves(efs_variant(m, m.R));
    const int wcap = max_waves > 0 ? std::min(vmax, max_waves) : vmax;
    auto fit = [&](bool tables) {
        const size_t sh = shared_doubles(m, tables) * sizeof(double);
        if (sh + priv > kLdsPerCu)
            return 0;
        return (int)std::min<size_t>(wcap, (kLdsPerCu - sh) / priv);
    };
    const int wt = fit(true), wg = fit(false);
    if (wg == 0)
        return false;
    // rule tables in LDS unless that costs more than half the waves
    cfg.lds_tables = wt > 0 && 2 * wt >= wg;
    cfg.waves = cfg.lds_tables ? wt : wg;
    cfg.lds_bytes = shared_doubles(m, cfg.lds_tables) * sizeof(double) + cfg.waves * priv;
    const int per_cu = std::max<int>(1, (int)(kLdsPerCu / cfg.lds_bytes));
    const int need = (std::max(n, 1) + cfg.waves - 1) / cfg.waves;
    cfg.grid = std::max(1, std::min(need, num_cus * per_cu));
    cfg.rows = cfg.grid * cfg.waves;
    return true;
}

// 0: level-16 profile, 1: level-20, 2: level-10, 3: small runtime, 4: generic
int efs_variant(const DevModel &m, int R)
{
    if (profile_is<6, 4, 2, 0>(m) && R <= 8)
        return 0;
    if (profile_is<8, 6, 4, 2, 0>(m) && R <= 10)
        return 1;
    if (profile_is<3, 1, 0>(m) && R <= 8)
        return 2;
    if (m.M <= 4 && m.numax_all <= 6 && R <= 8)
        return 3;
    return 4;
}

hipError_t launch_efs(const DevModel &m, const DevNeighbors &nb, const EfsOut &out,
                      const EfsLaunch &cfg, bool deterministic, hipStream_t s)
{
    const int det = deterministic ? 1 : 0;
    switch (efs_variant(m, m.R)) {
    case 0: launch_variant<ProfLevel16>(m, nb, out, cfg, det, s); break;
    case 1: launch_variant<ProfLevel20>(m, nb, out, cfg, det, s); break;
    case 2: launch_variant<ProfLevel10>(m, nb, out, cfg, det, s); break;
    case 3: launch_variant<ProfSmall>(m, nb, out, cfg, det, s); break;
    default: launch_variant<ProfGeneric>(m, nb, out, cfg, det, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_efs_finish(const DevNeighbors &nb, const EfsOut &out, int rows,
                             bool deterministic, const int *rev_offsets, const int *rev_pairs,
                             double *energy_stress10, hipStream_t s)
{
    hipLaunchKernelGGL(partial_reduce_kernel, dim3(1), dim3(256), 0, s, out.partial, rows,
                       energy_stress10);
    if (deterministic && nb.n > 0)
        hipLaunchKernelGGL(force_gather_kernel, dim3((nb.n + 255) / 256), dim3(256), 0, s, nb,
                           out.pair_ders, rev_offsets, rev_pairs, out.forces);
    return hipGetLastError();
}

}  // namespace mtpx
