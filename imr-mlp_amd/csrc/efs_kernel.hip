// Fused MTP energy/force/stress kernel for gfx950 (CDNA4), fp64.
//
// Reference semantics: PotMTP::CalcSiteEFS + getEFS
// (potentials/potential_mtp.cpp:2813-2984, :1899-1933).  The arithmetic is
// reorganised for a wave64; results agree with the reference to rounding.
//
// One workgroup = one wave64, grid-stride over atoms.  Per atom:
//   1. lanes over neighbours: Chebyshev basis Q_k(d), radial functions
//      f_mu = sum_k c[ti,tj,mu,k] Q_k (coefficients staged in LDS), unit
//      vector u = r/d.  Every basic moment (mu, a, b, c) equals
//      sum_j f_mu(d_j) * Y_abc(u_j) with Y_abc = ux^a uy^b uz^c, so the basics
//      are produced shell by shell (degree nu = a+b+c, compile-time unrolled)
//      in registers and summed over neighbours through a padded LDS
//      transpose, 16 slots at a time.
//   2. the product rules run lane-parallel from lane-major step tables, one
//      dependency level at a time (forward values, then reverse adjoints).
//   3. lanes over neighbours again: dE_i/dr_j from the closed form
//      grad_r[f Y] = (f' - nu f/d) Y u + (f/d) grad_u Y, with the basic
//      adjoints read as LDS broadcasts.
//   4. F_i += sum_j D_j, F_idx(j) -= D_j, S_ab -= D_ja r_jb.  Fast mode uses
//      fp64 atomics for the neighbour reactions; deterministic mode stores D
//      per pair for an ordered gather.  Energy and virial are reduced per
//      workgroup and finished by a single ordered pass.
//
// Kernel variants: a "shell profile" fixes, per radial function mu, the
// highest angular degree of its basic moments.  The level-10/16/20 template
// profiles are compile-time constants (every (nu, mu) guard folds away); the
// generic variants read the profile at run time.
#include "mtpx_internal.hpp"

#include <cstdlib>

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
    __syncthreads();
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
    __syncthreads();
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

// One level of a lane-major step table; entries are prefetched four steps
// ahead so every step costs one coalesced, already-resident int4.
template <class Step>
__device__ __forceinline__ void run_steps(const int4 *steps, int s0, int s1, int lane, Step step)
{
    if (s1 <= s0)
        return;
    const int4 *tab = steps + (size_t)s0 * kWave + lane;
    int4 e0 = tab[0], e1 = tab[kWave], e2 = tab[2 * kWave], e3 = tab[3 * kWave];
    for (int st = s0; st < s1; st += 4) {
        int4 n0 = e0, n1 = e1, n2 = e2, n3 = e3;
        if (st + 4 < s1) {
            const int4 *nt = tab + (size_t)(st + 4 - s0) * kWave;
            n0 = nt[0];
            n1 = nt[kWave];
            n2 = nt[2 * kWave];
            n3 = nt[3 * kWave];
        }
        step(e0);
        step(e1);
        step(e2);
        step(e3);
        e0 = n0;
        e1 = n1;
        e2 = n2;
        e3 = n3;
    }
}

// Product rules, forward (potential_mtp.cpp:2918-2924): one level at a time.
__device__ __forceinline__ void rules_forward(const DevModel &m, double *mom, double *partial,
                                              int lane)
{
    for (int L = 0; L < m.nfwd; ++L) {
        double acc = 0.0;
        run_steps(m.fwd_steps, m.fwd_level_step[L], m.fwd_level_step[L + 1], lane,
                  [&](const int4 &e) {
                      acc += (double)e.z * mom[e.x] * mom[e.y];
                      if (e.w != -1) {
                          if (e.w >= 0)
                              mom[e.w] = acc;
                          else
                              partial[-e.w - 2] = acc;
                          acc = 0.0;
                      }
                  });
        const int c0 = m.fwd_level_comb[L], c1 = m.fwd_level_comb[L + 1];
        if (c1 > c0) {
            __syncthreads();
            for (int c = c0 + lane; c < c1; c += kWave) {
                const int4 t = m.fwd_comb[c];
                double sum = 0.0;
                for (int k = 0; k < t.z; ++k)
                    sum += partial[t.y + k];
                mom[t.x] = sum;
            }
        }
        __syncthreads();
    }
}

// Product rules, reverse (backpropagate_moments, potential_mtp.cpp:3292-3305).
__device__ __forceinline__ void rules_reverse(const DevModel &m, const double *mom, double *A,
                                              double *partial, int lane)
{
    for (int L = 0; L < m.nbwd; ++L) {
        double acc = 0.0;
        run_steps(m.bwd_steps, m.bwd_level_step[L], m.bwd_level_step[L + 1], lane,
                  [&](const int4 &e) {
                      acc += (double)e.z * A[e.x] * mom[e.y];
                      if (e.w != -1) {
                          if (e.w >= 0)
                              A[e.w] += acc;
                          else
                              partial[-e.w - 2] = acc;
                          acc = 0.0;
                      }
                  });
        const int c0 = m.bwd_level_comb[L], c1 = m.bwd_level_comb[L + 1];
        if (c1 > c0) {
            __syncthreads();
            for (int c = c0 + lane; c < c1; c += kWave) {
                const int4 t = m.bwd_comb[c];
                double sum = 0.0;
                for (int k = 0; k < t.z; ++k)
                    sum += partial[t.y + k];
                A[t.x] += sum;
            }
        }
        __syncthreads();
    }
}

struct Lds {
    double *coef, *mom, *A, *red, *seed, *moment, *partial;
    int *map, *slot_basic, *slot_abc;
};

__device__ __forceinline__ Lds lds_layout(const DevModel &m, double *base)
{
    const int ncoef_r = m.Z * m.Z * m.M * m.R;
    const int K4 = (m.K + 3) & ~3, S4 = (m.S + 3) & ~3, N4 = (m.nslots + 3) & ~3;
    const int P4 = (m.max_partials + 3) & ~3;
    Lds L;
    L.coef = base;
    L.mom = L.coef + ((ncoef_r + 3) & ~3);
    L.A = L.mom + K4;
    L.red = L.A + K4;
    L.seed = L.red + max(kChunk * kRedStride, 4 * N4);
    L.moment = L.seed + K4;
    L.partial = L.moment + S4;
    L.map = reinterpret_cast<int *>(L.partial + P4);
    L.slot_basic = L.map + S4;
    L.slot_abc = L.slot_basic + N4;
    return L;
}

template <class P, int WPE>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(WPE))) void efs_kernel(
    DevModel m, DevNeighbors nb, EfsOut out, int deterministic)
{
    extern __shared__ double lds[];
    const int lane = threadIdx.x;
    const Lds L = lds_layout(m, lds);
    const double4 *A4 = reinterpret_cast<const double4 *>(L.red);

    // model tables the per-atom phases index, staged once per workgroup
    const int ncoef_r = m.Z * m.Z * m.M * m.R;
    for (int k = lane; k < ncoef_r; k += kWave)
        L.coef[k] = m.radial[k];
    for (int k = lane; k < m.K; k += kWave)
        L.seed[k] = m.seed[k];
    for (int k = lane; k < m.S; k += kWave) {
        L.moment[k] = m.moment[k];
        L.map[k] = m.map[k];
    }
    for (int k = lane; k < m.nslots; k += kWave) {
        L.slot_basic[k] = m.slot_basic[k];
        L.slot_abc[k] = m.slot_abc[k];
    }
    __syncthreads();

    double e_acc = 0.0;  // this lane's share of the block's energy and virial
    double v_acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};

    for (int i = blockIdx.x; i < nb.n; i += gridDim.x) {
        const int ti = nb.center_type[i];
        const int beg = nb.offsets[i];
        const int n = nb.offsets[i + 1] - beg;
        for (int k = lane; k < m.K; k += kWave)
            L.mom[k] = 0.0;
        __syncthreads();

        // ---- basic moments -------------------------------------------------
        for (int base = 0; base < n; base += kWave) {
            FwdCtx cx{L.red, L.mom, L.slot_basic, lane, 0};
            Nbr<P::M> q;
            const bool valid = lane < n - base;
            load_neighbor<P>(m, nb, L.coef, ti, beg + base + lane, valid, q);
            fwd_shells<0, P>(m, cx, q, nullptr);
            const int rest = cx.slot % kChunk;
            if (rest)
                reduce_chunk(L.red, rest, cx.slot - rest, L.slot_basic, L.mom, lane);
        }
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                L.mom[m.dup[2 * k]] = L.mom[m.dup[2 * k + 1]];
        __syncthreads();

        rules_forward(m, L.mom, L.partial, lane);

        // ---- site energy (potential_mtp.cpp:2966-2970) and adjoint seed ----
        double e = 0.0;
        for (int s = lane; s < m.S; s += kWave)
            e += L.moment[s] * L.mom[L.map[s]];
        e = wave_sum(e);
        const double site_energy = m.species[ti] + e;
        if (lane == 0) {
            out.site_energy[i] = site_energy;
            e_acc += site_energy;
        }
        for (int k = lane; k < m.K; k += kWave)
            L.A[k] = L.seed[k];
        __syncthreads();

        rules_reverse(m, L.mom, L.A, L.partial, lane);
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                L.A[m.dup[2 * k + 1]] += L.A[m.dup[2 * k]];
        __syncthreads();
        // slot-ordered adjoints {A, aA, bA, cA}
        for (int s = lane; s < m.nslots; s += kWave) {
            const int b = L.slot_basic[s];
            double4 w = {0, 0, 0, 0};
            if (b >= 0) {
                const double a = L.A[b];
                const int abc = L.slot_abc[s];
                w = {a, a * (abc & 0xff), a * ((abc >> 8) & 0xff), a * ((abc >> 16) & 0xff)};
            }
            reinterpret_cast<double4 *>(L.red)[s] = w;
        }
        __syncthreads();

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
        __syncthreads();
    }
    // block partials: energy, stress[9]
    e_acc = wave_sum(e_acc);
#pragma unroll
    for (int k = 0; k < 9; ++k)
        v_acc[k] = wave_sum(v_acc[k]);
    if (lane == 0) {
        out.partial[10 * blockIdx.x] = e_acc;
#pragma unroll
        for (int k = 0; k < 9; ++k)
            out.partial[10 * blockIdx.x + 1 + k] = v_acc[k];
    }
}

// Ordered reduction of the per-workgroup partials (one workgroup).
__global__ __launch_bounds__(256) void partial_reduce_kernel(const double *partial, int nblocks,
                                                             double *out10)
{
    __shared__ double buf[256][10];
    const int t = threadIdx.x;
    double acc[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = t; b < nblocks; b += 256)
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

}  // namespace

size_t efs_lds_bytes(const DevModel &m)
{
    auto r4 = [](size_t v) { return (v + 3) & ~size_t(3); };
    const size_t ncoef_r = (size_t)m.Z * m.Z * m.M * m.R;
    const size_t red = std::max<size_t>((size_t)kChunk * kRedStride, 4 * r4((size_t)m.nslots));
    const size_t dbl = r4(ncoef_r) + 3 * r4((size_t)m.K) + red + r4((size_t)m.S) +
                       r4((size_t)m.max_partials);
    const size_t ints = r4((size_t)m.S) + 2 * r4((size_t)m.nslots);
    return dbl * sizeof(double) + ints * sizeof(int);
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

hipError_t launch_efs(const DevModel &m, const DevNeighbors &nb, const EfsOut &out, int grid,
                      bool deterministic, hipStream_t s)
{
    const size_t lds = efs_lds_bytes(m);
    const int det = deterministic ? 1 : 0;
    // MTPX_EFS_WAVES_PER_EU (tuning): occupancy the level-16 kernel is
    // register-allocated for (1 = compiler's choice, 3)
    static const int wpe = [] {
        const char *e = getenv("MTPX_EFS_WAVES_PER_EU");
        return e ? atoi(e) : 1;
    }();
    switch (efs_variant(m, m.R)) {
    case 0:
        if (wpe == 3)
            hipLaunchKernelGGL((efs_kernel<ProfLevel16, 3>), dim3(grid), dim3(kWave), lds, s, m, nb,
                               out, det);
        else
            hipLaunchKernelGGL((efs_kernel<ProfLevel16, 1>), dim3(grid), dim3(kWave), lds, s, m, nb,
                               out, det);
        break;
    case 1:
        hipLaunchKernelGGL((efs_kernel<ProfLevel20, 1>), dim3(grid), dim3(kWave), lds, s, m, nb,
                           out, det);
        break;
    case 2:
        hipLaunchKernelGGL((efs_kernel<ProfLevel10, 1>), dim3(grid), dim3(kWave), lds, s, m, nb,
                           out, det);
        break;
    case 3:
        hipLaunchKernelGGL((efs_kernel<ProfSmall, 1>), dim3(grid), dim3(kWave), lds, s, m, nb, out,
                           det);
        break;
    default:
        hipLaunchKernelGGL((efs_kernel<ProfGeneric, 1>), dim3(grid), dim3(kWave), lds, s, m, nb,
                           out, det);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_efs_finish(const DevNeighbors &nb, const EfsOut &out, int grid,
                             bool deterministic, const int *rev_offsets, const int *rev_pairs,
                             double *energy_stress10, hipStream_t s)
{
    hipLaunchKernelGGL(partial_reduce_kernel, dim3(1), dim3(256), 0, s, out.partial, grid,
                       energy_stress10);
    if (deterministic && nb.n > 0)
        hipLaunchKernelGGL(force_gather_kernel, dim3((nb.n + 255) / 256), dim3(256), 0, s, nb,
                           out.pair_ders, rev_offsets, rev_pairs, out.forces);
    return hipGetLastError();
}

}  // namespace mtpx
