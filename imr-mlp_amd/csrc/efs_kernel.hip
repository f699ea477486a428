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
//      in registers and reduced over neighbours through a padded LDS
//      transpose, 16 slots at a time.
//   2. the product rules run lane-parallel, one output per lane and level
//      (forward) and one destination per lane and level (reverse adjoint).
//   3. lanes over neighbours again: dE_i/dr_j from the closed form
//      grad_r[f Y] = (f' - nu f/d) Y u + (f/d) grad_u Y, with the basic
//      adjoints read as LDS broadcasts.
//   4. F_i += sum_j D_j, F_idx(j) -= D_j, S_ab -= D_ja r_jb.  Fast mode uses
//      fp64 atomics for the neighbour reactions; deterministic mode stores D
//      per pair for an ordered gather.  Energy and virial are reduced per
//      workgroup and finished by a single ordered pass.
#include "mtpx_internal.hpp"

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

__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v += __shfl_xor(v, off, kWave);
    return v;
}

struct Nbr {
    double x, y, z, d, invd, ux, uy, uz;
    double f[kMaxMu], fd[kMaxMu];
    bool in_cutoff;
};

template <int MMAX, int RMAX>
__device__ __forceinline__ void load_neighbor(const DevModel &m, const DevNeighbors &nb,
                                              const double *coef_lds, int ti, int64_t p,
                                              Nbr &q)
{
    q.x = nb.x[p];
    q.y = nb.y[p];
    q.z = nb.z[p];
    q.d = nb.d[p];
    const int tj = nb.type[p];
    // potential_mtp.cpp:2842 -- entries beyond the cutoff are skipped, r == cutoff kept
    q.in_cutoff = !(q.d > m.rmax);
    const double d = q.in_cutoff ? q.d : m.rmax;
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
    const double *c = coef_lds + (ti * m.Z + tj) * m.M * m.R;
#pragma unroll
    for (int mu = 0; mu < MMAX; ++mu) {
        double f = 0, fd = 0;
        if (mu < m.M) {
            const double *cm = c + mu * m.R;
#pragma unroll
            for (int k = 0; k < RMAX; ++k)
                if (k < m.R) {
                    f += cm[k] * Q[k];
                    fd += cm[k] * dQ[k];
                }
        }
        const double w = q.in_cutoff ? 1.0 : 0.0;
        q.f[mu] = f * w;
        q.fd[mu] = fd * w;
    }
}

template <int NU>
__device__ __forceinline__ void next_shell(const double *prev, double *cur, const Nbr &q)
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

// Sum a chunk of `nrows` slots over the `ncols` neighbour columns of the
// transpose buffer and add the sums into the moment array.
__device__ __forceinline__ void reduce_chunk(double *red, int ncols, int nrows, int slot0,
                                             const int *slot_basic, double *mom, int lane)
{
    __syncthreads();
    const int s = lane & (kChunk - 1), qq = lane >> 4;
    double acc = 0.0;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
        const int j = qq * 16 + jj;
        if (j < ncols)
            acc += red[s * kRedStride + j];
    }
    acc += __shfl_xor(acc, 16, kWave);
    acc += __shfl_xor(acc, 32, kWave);
    if (lane < nrows) {
        const int b = slot_basic[slot0 + lane];
        if (b >= 0)
            mom[b] += acc;
    }
    __syncthreads();
}

struct FwdCtx {
    const DevModel *m;
    double *red, *mom;
    int ncols, lane;
    bool active;
    int slot;
};

template <int NU, int NUMAX, int MMAX>
__device__ __forceinline__ void fwd_shells(FwdCtx &cx, const Nbr &q, const double *prev)
{
    double cur[shell_size(NU)];
    if constexpr (NU == 0)
        cur[0] = 1.0;
    else
        next_shell<NU>(prev, cur, q);
    const DevModel &m = *cx.m;
#pragma unroll
    for (int mu = 0; mu < MMAX; ++mu) {
        if (mu < m.M && m.numax[mu] >= NU) {
            int row = 0;
#pragma unroll
            for (int i = 0; i < shell_size(NU); ++i) {
                if (cx.active)
                    cx.red[row * kRedStride + cx.lane] = q.f[mu] * cur[i];
                ++row;
                if (row == kChunk || i == shell_size(NU) - 1) {
                    reduce_chunk(cx.red, cx.ncols, row, cx.slot, m.slot_basic, cx.mom, cx.lane);
                    cx.slot += row;
                    row = 0;
                }
            }
        }
    }
    if constexpr (NU < NUMAX) {
        if (NU < m.numax_all)
            fwd_shells<NU + 1, NUMAX, MMAX>(cx, q, cur);
    }
}

struct BwdAcc {
    double s, gx, gy, gz;
};

template <int NU, int NUMAX, int MMAX>
__device__ __forceinline__ void bwd_shells(const DevModel &m, const double4 *A4, int &slot,
                                           const Nbr &q, const double *prev, BwdAcc &acc)
{
    double cur[shell_size(NU)];
    if constexpr (NU == 0)
        cur[0] = 1.0;
    else
        next_shell<NU>(prev, cur, q);
#pragma unroll
    for (int mu = 0; mu < MMAX; ++mu) {
        if (mu < m.M && m.numax[mu] >= NU) {
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
    if constexpr (NU < NUMAX) {
        if (NU < m.numax_all)
            bwd_shells<NU + 1, NUMAX, MMAX>(m, A4, slot, q, cur, acc);
    }
}

template <int MMAX, int NUMAX, int RMAX>
__global__ __launch_bounds__(kWave) void efs_kernel(DevModel m, DevNeighbors nb, EfsOut out,
                                                     int deterministic)
{
    extern __shared__ double lds[];
    const int lane = threadIdx.x;
    const int ncoef_r = m.Z * m.Z * m.M * m.R;
    // LDS: radial coefficients | moments | adjoints | transpose buffer, each
    // region a multiple of 4 doubles so the double4 view stays 32-byte aligned
    double *coef = lds;
    double *mom = coef + ((ncoef_r + 3) & ~3);
    double *A = mom + ((m.K + 3) & ~3);
    double *red = A + ((m.K + 3) & ~3);
    const double4 *A4 = reinterpret_cast<const double4 *>(red);

    for (int k = lane; k < ncoef_r; k += kWave)
        coef[k] = m.radial[k];
    __syncthreads();

    double e_acc = 0.0;  // this lane's share of the block's energy and virial
    double v_acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};

    for (int i = blockIdx.x; i < nb.n; i += gridDim.x) {
        const int ti = nb.center_type[i];
        const int beg = nb.offsets[i];
        const int n = nb.offsets[i + 1] - beg;
        for (int k = lane; k < m.K; k += kWave)
            mom[k] = 0.0;
        __syncthreads();

        // ---- basic moments -------------------------------------------------
        for (int base = 0; base < n; base += kWave) {
            const int ncols = min(kWave, n - base);
            FwdCtx cx{&m, red, mom, ncols, lane, lane < ncols, 0};
            Nbr q;
            if (cx.active)
                load_neighbor<MMAX, RMAX>(m, nb, coef, ti, beg + base + lane, q);
            else
                q = Nbr{};
            fwd_shells<0, NUMAX, MMAX>(cx, q, nullptr);
        }
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                mom[m.dup[2 * k]] = mom[m.dup[2 * k + 1]];
        __syncthreads();

        // ---- product rules, forward ----------------------------------------
        for (int L = 0; L < m.nfwd; ++L) {
            for (int t = m.fwd_level[L] + lane; t < m.fwd_level[L + 1]; t += kWave) {
                const int4 task = m.fwd_task[t];
                double acc = 0.0;
                for (int k = 0; k < task.z; ++k) {
                    const int lr = m.fwd_lr[task.y + k];
                    acc += m.fwd_c[task.y + k] * mom[lr & 0xffff] * mom[lr >> 16];
                }
                mom[task.x] = acc;
            }
            __syncthreads();
        }

        // ---- site energy (potential_mtp.cpp:2966-2970) and adjoint seed ----
        double e = 0.0;
        for (int s = lane; s < m.S; s += kWave)
            e += m.moment[s] * mom[m.map[s]];
        e = wave_sum(e);
        const double site_energy = m.species[ti] + e;
        if (lane == 0) {
            out.site_energy[i] = site_energy;
            e_acc += site_energy;
        }
        for (int k = lane; k < m.K; k += kWave)
            A[k] = m.seed[k];
        __syncthreads();

        // ---- product rules, reverse (backpropagate_moments) -----------------
        for (int L = 0; L < m.nbwd; ++L) {
            for (int t = m.bwd_level[L] + lane; t < m.bwd_level[L + 1]; t += kWave) {
                const int4 task = m.bwd_task[t];
                double acc = A[task.x];
                for (int k = 0; k < task.z; ++k) {
                    const int oo = m.bwd_oo[task.y + k];
                    acc += m.bwd_c[task.y + k] * A[oo & 0xffff] * mom[oo >> 16];
                }
                A[task.x] = acc;
            }
            __syncthreads();
        }
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                A[m.dup[2 * k + 1]] += A[m.dup[2 * k]];
        __syncthreads();
        // slot-ordered adjoints {A, aA, bA, cA}
        for (int s = lane; s < m.nslots; s += kWave) {
            const int b = m.slot_basic[s];
            double4 w = {0, 0, 0, 0};
            if (b >= 0) {
                const double a = A[b];
                const int abc = m.slot_abc[s];
                w = {a, a * (abc & 0xff), a * ((abc >> 8) & 0xff), a * ((abc >> 16) & 0xff)};
            }
            reinterpret_cast<double4 *>(red)[s] = w;
        }
        __syncthreads();

        // ---- forces and virial ---------------------------------------------
        double fi0 = 0, fi1 = 0, fi2 = 0;
        for (int base = 0; base < n; base += kWave) {
            const bool active = lane < n - base;
            if (active) {
                const int64_t p = beg + base + lane;
                Nbr q;
                load_neighbor<MMAX, RMAX>(m, nb, coef, ti, p, q);
                BwdAcc acc{0, 0, 0, 0};
                int slot = 0;
                bwd_shells<0, NUMAX, MMAX>(m, A4, slot, q, nullptr, acc);
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

}  // namespace

size_t efs_lds_bytes(const DevModel &m)
{
    const size_t ncoef_r = (size_t)m.Z * m.Z * m.M * m.R;
    const size_t red = std::max<size_t>((size_t)kChunk * kRedStride, 4 * (size_t)m.nslots);
    auto r4 = [](size_t v) { return (v + 3) & ~size_t(3); };
    return (r4(ncoef_r) + 2 * r4((size_t)m.K) + red) * sizeof(double);
}

int efs_variant(const DevModel &m, int R)
{
    if (m.M <= 4 && m.numax_all <= 6 && R <= 8)
        return 0;
    if (m.M <= 5 && m.numax_all <= 8 && R <= 10)
        return 1;
    return 2;
}

hipError_t launch_efs(const DevModel &m, const DevNeighbors &nb, const EfsOut &out, int grid,
                      bool deterministic, hipStream_t s)
{
    const size_t lds = efs_lds_bytes(m);
    const int det = deterministic ? 1 : 0;
    switch (efs_variant(m, m.R)) {
    case 0:
        hipLaunchKernelGGL((efs_kernel<4, 6, 8>), dim3(grid), dim3(kWave), lds, s, m, nb, out, det);
        break;
    case 1:
        hipLaunchKernelGGL((efs_kernel<5, 8, 10>), dim3(grid), dim3(kWave), lds, s, m, nb, out,
                           det);
        break;
    default:
        hipLaunchKernelGGL((efs_kernel<kMaxMu, kMaxNu, kMaxR>), dim3(grid), dim3(kWave), lds, s, m,
                           nb, out, det);
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
