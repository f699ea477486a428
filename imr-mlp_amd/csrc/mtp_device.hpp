// Device building blocks shared by the E/F/S and training kernels (gfx950,
// fp64, one wave64 per atom).  See efs_kernel.hip for the phase structure.
#pragma once

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

// Sum of one row of a reduction chunk (kChunk = 16 rows of 64 columns,
// stride kRedStride): lane l sums row l & 15 over columns 16 (l >> 4) .. +15
// with 16-byte reads, then the four column groups are combined (lanes l ^ 32,
// l ^ 16); every lane of the row's group ends with the row total.
__device__ __forceinline__ double chunk_row_sum(const double *red, int lane)
{
    const double2 *row =
        reinterpret_cast<const double2 *>(red + (lane & (kChunk - 1)) * kRedStride + (lane >> 4) * 16);
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        const double2 v = row[jj];
        a0 += v.x;
        a1 += v.y;
    }
    return xor16_sum(xor32_sum(a0 + a1));
}

// v plus the value of the lane that the DPP control kCtrl selects within the
// lane's row of 16 (VALU lane move, no LDS crossbar).
template <int kCtrl>
__device__ __forceinline__ double dpp_add(double v)
{
    const int lo = __builtin_amdgcn_update_dpp(0, (int)__double2loint(v), kCtrl, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)__double2hiint(v), kCtrl, 0xf, 0xf, false);
    return v + __hiloint2double(hi, lo);
}

// Sum over the lane's row of 16, in every lane of the row (the last four
// steps of wave_sum below).
__device__ __forceinline__ double row16_sum(double v)
{
    v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);  // row_half_mirror
    v = dpp_add<0x140>(v);  // row_mirror
    return v;
}

// Sum over the whole wave, in every lane: the two lane swaps, then within
// each row of 16 the quad permutations [1,0,3,2] and [2,3,0,1], the
// half-row mirror and the row mirror (each pairs lanes holding disjoint
// partial sums).
__device__ __forceinline__ double wave_sum(double v)
{
    v = xor32_sum(v);
    v = xor16_sum(v);
    v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);  // row_half_mirror
    v = dpp_add<0x140>(v);  // row_mirror
    return v;
}

// Sums over the wave of NV values per lane (NV a multiple of 4) in one pass:
// the wave halves, then the rows, exchange half of their values (lane swaps;
// a lane keeps the half its position selects and adds its partner's), and
// each row of 16 sums its NV/4 values over its lanes (DPP).  Lane 16 r + k
// (k < NV/4) returns the total of value k + (NV/4) (r & 1) + (NV/2) (r >> 1)
// and sets idx to that index; the other lanes return 0 with idx = -1.
// About (NV/2 + NV/4) * 3 + (NV/4) * 12 instructions instead of NV * 18 for
// NV separate wave_sum calls.
template <int NV>
__device__ __forceinline__ double wave_reduce_scatter(const double (&v)[NV], int lane, int &idx)
{
    static_assert(NV % 4 == 0, "NV must be a multiple of 4");
    constexpr int H = NV / 2, Q = NV / 4;
    double u[H], w[Q];
#pragma unroll
    for (int k = 0; k < H; ++k) {
        // lanes < 32 keep value k, lanes >= 32 value k + H
        const unsigned alo = __double2loint(v[k]), ahi = __double2hiint(v[k]);
        const unsigned blo = __double2loint(v[k + H]), bhi = __double2hiint(v[k + H]);
        const auto lo = __builtin_amdgcn_permlane32_swap(alo, blo, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap(ahi, bhi, false, false);
        u[k] = __hiloint2double(hi[0], lo[0]) + __hiloint2double(hi[1], lo[1]);
    }
#pragma unroll
    for (int k = 0; k < Q; ++k) {
        // even rows keep value k, odd rows value k + Q
        const unsigned alo = __double2loint(u[k]), ahi = __double2hiint(u[k]);
        const unsigned blo = __double2loint(u[k + Q]), bhi = __double2hiint(u[k + Q]);
        const auto lo = __builtin_amdgcn_permlane16_swap(alo, blo, false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap(ahi, bhi, false, false);
        double x = __hiloint2double(hi[0], lo[0]) + __hiloint2double(hi[1], lo[1]);
        x = dpp_add<0xB1>(x);   // quad_perm [1,0,3,2]
        x = dpp_add<0x4E>(x);   // quad_perm [2,3,0,1]
        x = dpp_add<0x141>(x);  // row_half_mirror
        x = dpp_add<0x140>(x);  // row_mirror
        w[k] = x;
    }
    const int r = lane >> 4, k = lane & 15;
    double out = 0.0;
#pragma unroll
    for (int j = 0; j < Q; ++j)
        out = k == j ? w[j] : out;
    idx = k < Q ? k + Q * (r & 1) + H * (r >> 1) : -1;
    return out;
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

// The cutoff of the pair (ti, tj): the model's, or with general radial bases
// the pair basis's max_dist (cutoffs(itype, jtype), potential_mtp.cpp:2842).
template <bool kGeneral>
__device__ __forceinline__ double pair_cutoff(const DevModel &m, int ti, int tj)
{
    if constexpr (kGeneral)
        if (m.rb_general)
            return m.rb_table[(ti * m.Z + tj) * kRbStride + 2];
    return m.rmax;
}

// Geometry of list entry p; lanes without an entry keep zeros, so they
// contribute nothing to the sums below.  Returns 1 for an entry inside the
// cutoff and 0 otherwise (potential_mtp.cpp:2842 skips entries beyond the
// cutoff and keeps r == cutoff); such entries get d = cutoff.  kGeneral
// (run-time profiles) reads the pair's cutoff when the model has general
// radial bases.
template <int MMAX, bool kGeneral = false>
__device__ __forceinline__ double load_geometry(const DevModel &m, const DevNeighbors &nb,
                                                int64_t p, bool valid, Nbr<MMAX> &q, int &tj,
                                                int ti = 0)
{
    q.x = valid ? nb.x[p] : 0.0;
    q.y = valid ? nb.y[p] : 0.0;
    q.z = valid ? nb.z[p] : 0.0;
    tj = valid ? nb.type[p] : 0;
    const double rc = pair_cutoff<kGeneral>(m, ti, tj);
    const double dd = valid ? nb.d[p] : rc;
    const bool in_cutoff = valid && !(dd > rc);
    const double d = in_cutoff ? dd : rc;
    q.d = d;
    q.invd = 1.0 / d;
    q.ux = q.x * q.invd;
    q.uy = q.y * q.invd;
    q.uz = q.z * q.invd;
    return in_cutoff ? 1.0 : 0.0;
}

// RBasis_Chebyshev::calc_der (basis/basis.cpp:148-164): Q_k and dQ_k/dd.
template <int RMAX>
__device__ __forceinline__ void chebyshev(const DevModel &m, double d, double *Q, double *dQ)
{
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
}

// A general radial basis (basis/basis.cpp): Chebyshev polynomials of
// xi = (2d - (min + max)) / (max - min) times an envelope rc(d), by the same
// recurrence as RBChebyshev -- Q_0 = s rc, Q_1 = s xi rc,
// Q_k = 2 xi Q_(k-1) - Q_(k-2), and the derivative recurrence with
// mult = 2 / (max - min) -- for the envelopes
//   RBChebyshev       (d - max)^2                              (:148-164)
//   RBChebyCos        (1 + cos(pi d / max)) / 2                (:242-271)
//   RBChebyshevPoly4  (1 - x)^3 (1 + (3 + b) x), x = (d - min) / (max - min),
//                     zero outside [min, max]                  (:585-619)
//   RBChebyshevPoly5  (1 - x)^4 (1 + (4 + b) x), likewise      (:776-805)
// t is the pair's row of the basis table (kRbStride doubles).
//
// RBChebyshevConfigurable (basis/basis.cpp:931-1011): zero outside
// [min, max]; otherwise Q_k = s raw_k(x(r)) fc(r) with raw_k = T_k or, for
// one_minus_chebyshev, 1 - T_(k+1), the Chebyshev polynomials of the shift
// x(r) by T_k = 2 x T_(k-1) - T_(k-2).  The cutoff fc and the shift x with
// their derivatives are the closed forms of Cutoff::* (basis/cutoff.cpp)
// and XTransForm::* (basis/xtrans.cpp); table row {kind, min, max, s,
// cutoff, shift, one_minus, cutoff_b, r1, r2, lambda, scale_lambda,
// 1 / (max - min), expm1(lambda), tanh(scale_lambda)}.
__device__ __forceinline__ void configurable_cutoff(const double *t, double r, double &fc,
                                                    double &dfc)
{
    const double lo = t[1], hi = t[2], b = t[7], inv = t[12], pi = M_PI;
    const double tt = (r - lo) * inv, q = 1.0 - tt, a = pi * tt;
    switch ((int)t[4]) {
    case kCutQuadratic: {
        const double dl = r - hi;
        fc = dl * dl;
        dfc = 2.0 * dl;
        break;
    }
    case kCutNormalizedQuadratic:
        fc = q * q;
        dfc = -2.0 * q * inv;
        break;
    case kCutCosine: {
        const double freq = pi / (hi - lo), ph = (r - lo) * freq;
        fc = 0.5 * (1.0 + cos(ph));
        dfc = -0.5 * freq * sin(ph);
        break;
    }
    case kCutCosineLeft: {
        const double w = pi / hi, ph = w * r;
        fc = 0.5 * (1.0 + cos(ph));
        dfc = -0.5 * w * sin(ph);
        break;
    }
    case kCutCosineUnscaled:
        fc = 1.0 + cos(a);
        dfc = -sin(a) * pi * inv;
        break;
    case kCutCosineSquared: {
        const double g = 1.0 + cos(a), dg = -sin(a) * pi * inv;
        fc = g * g;
        dfc = 2.0 * g * dg;
        break;
    }
    case kCutSineSquared: {
        const double sn = sin(a);
        fc = sn * sn;
        dfc = 2.0 * sn * cos(a) * pi * inv;
        break;
    }
    case kCutPoly3: {
        const double p = 1.0 + (b + 2.0) * tt;
        fc = q * q * p;
        dfc = -2.0 * q * inv * p + q * q * (b + 2.0) * inv;
        break;
    }
    case kCutPoly4: {
        const double p = 1.0 + (b + 3.0) * tt;
        fc = q * q * q * p;
        dfc = -3.0 * q * q * inv * p + q * q * q * (b + 3.0) * inv;
        break;
    }
    case kCutPoly5: {
        const double sq = q * q;
        fc = sq * sq * (1.0 + (4.0 + b) * tt);
        dfc = -sq * q * (20.0 * tt + b * (5.0 * tt - 1.0)) * inv;
        break;
    }
    case kCutSmoothstep5: {
        const double q2 = q * q, q3 = q2 * q;
        fc = 6.0 * q3 * q2 - 15.0 * q2 * q2 + 10.0 * q3;
        dfc = -(30.0 * q2 * q2 - 60.0 * q3 + 30.0 * q2) * inv;
        break;
    }
    default: {  // smoothstep7
        const double r1 = t[8], r2 = t[9];
        if (r <= r1 || r >= r2) {
            const double dp = r <= r1 ? 1.0 / (r1 - lo) : 1.0 / (hi - r2);
            const double p = r <= r1 ? (r - lo) * dp : (r - r2) * dp;
            const double p2 = p * p, p3 = p2 * p, p4 = p2 * p2;
            const double v = 35.0 * p4 - 84.0 * p4 * p + 70.0 * p3 * p3 - 20.0 * p3 * p4;
            const double dv = (140.0 * p3 - 420.0 * p4 + 420.0 * p4 * p - 140.0 * p3 * p3) * dp;
            fc = r <= r1 ? v : 1.0 - v;
            dfc = r <= r1 ? dv : -dv;
        } else {
            fc = 1.0;
            dfc = 0.0;
        }
        break;
    }
    }
}

__device__ __forceinline__ void configurable_shift(const double *t, double r, double &x,
                                                   double &dx)
{
    const double lo = t[1], hi = t[2], lam = t[10], sl = t[11], inv = t[12], den = t[13];
    const double tt = (r - lo) * inv;
    switch ((int)t[5]) {
    case kShiftLinear: {
        const double slope = 2.0 / (hi - lo);
        x = -1.0 + slope * (r - lo);
        dx = slope;
        break;
    }
    case kShiftExponential:
        if (lam == 0.0) {
            x = -1.0 + 2.0 * (r - lo) * inv;
            dx = 2.0 * inv;
        } else {
            const double e = lam * (hi - r) * inv;
            x = 1.0 - 2.0 * expm1(e) / den;
            dx = 2.0 * lam * inv * exp(e) / den;
        }
        break;
    case kShiftExponentialLeft:
        if (lam == 0.0) {
            x = 2.0 * (r / hi) - 1.0;
            dx = 2.0 / hi;
        } else {
            const double e = exp(lam * (1.0 - r / hi));
            x = 1.0 - (2.0 / den) * (e - 1.0);
            dx = (2.0 / den) * e * lam / hi;
        }
        break;
    case kShiftI2: {
        const double k = (r - hi) * inv;
        x = 2.0 * k * k - 1.0;
        dx = 4.0 * k * inv;
        break;
    }
    default: {  // exponential_tanh
        double sh, dsh;
        if (lam == 0.0) {
            sh = 2.0 * tt - 1.0;
            dsh = 2.0 * inv;
        } else {
            const double e = exp(lam * (1.0 - tt));
            sh = 1.0 - (2.0 / den) * (e - 1.0);
            dsh = (2.0 / den) * e * lam * inv;
        }
        if (sl == 0.0) {
            x = sh;
            dx = dsh;
        } else {
            const double th = tanh(sl * sh), tsl = t[14];
            x = th / tsl;
            dx = (1.0 - th * th) * sl * dsh / tsl;
        }
        break;
    }
    }
}

template <int RMAX>
__device__ __forceinline__ void configurable_basis(const double *t, double d, double *Q,
                                                   double *dQ)
{
    const bool inside = !(d < t[1] || d > t[2]);
    double fc, dfc, x, dx;
    configurable_cutoff(t, d, fc, dfc);
    configurable_shift(t, d, x, dx);
    const double s = t[3];
    const bool om = t[6] != 0.0;
    double T[RMAX + 1], dT[RMAX + 1];
    T[0] = 1.0;
    dT[0] = 0.0;
    T[1] = x;
    dT[1] = dx;
#pragma unroll
    for (int k = 2; k <= RMAX; ++k) {
        T[k] = 2.0 * x * T[k - 1] - T[k - 2];
        dT[k] = 2.0 * (dx * T[k - 1] + x * dT[k - 1]) - dT[k - 2];
    }
#pragma unroll
    for (int k = 0; k < RMAX; ++k) {
        const double raw = om ? 1.0 - T[k + 1] : T[k];
        const double rawd = om ? -dT[k + 1] : dT[k];
        Q[k] = inside ? s * raw * fc : 0.0;
        dQ[k] = inside ? s * (rawd * fc + raw * dfc) : 0.0;
    }
}

template <int RMAX>
__device__ __forceinline__ void general_basis(const double *t, double d, double *Q, double *dQ)
{
    const int kind = (int)t[0];
    if (kind == kRBChebyshevConfigurable) {
        configurable_basis<RMAX>(t, d, Q, dQ);
        return;
    }
    const double rmin = t[1], rmax = t[2], s = t[3], mult = t[4], su = t[5], pu = t[6];
    const double ksi = (2 * d - pu) / su;
    double rc, drc;
    if (kind == kRBChebyshev) {
        const double ru = d - rmax;
        rc = ru * ru;
        drc = 2 * ru;
    } else if (kind == kRBChebyCos) {
        const double irpi = t[7];
        rc = 0.5 * (1.0 + cos(d * irpi));
        drc = -0.5 * irpi * sin(d * irpi);
    } else {
        const double b = t[8], dxdr = t[9];
        const bool inside = !(d < rmin || d > rmax);
        const double x = (d - rmin) / su;
        const double vx = 1.0 - x, vxx = vx * vx, vxxx = vxx * vx;
        if (kind == kRBChebyshevPoly4) {
            rc = vxxx * (1 + (3 + b) * x);
            drc = vxx * (b * (1. - 4.0 * x) - 12.0 * x) * dxdr;
        } else {
            rc = vxx * vxx * (1 + (4 + b) * x);
            drc = -vxxx * (20 * x + b * (5 * x - 1)) * dxdr;
        }
        rc = inside ? rc : 0.0;
        drc = inside ? drc : 0.0;
    }
    Q[0] = s * rc;
    dQ[0] = s * drc;
    if (RMAX > 1) {
        Q[1] = s * (ksi * rc);
        dQ[1] = s * (mult * rc + ksi * drc);
    }
#pragma unroll
    for (int k = 2; k < RMAX; ++k) {
        Q[k] = 2 * ksi * Q[k - 1] - Q[k - 2];
        dQ[k] = 2 * (mult * Q[k - 1] + ksi * dQ[k - 1]) - dQ[k - 2];
    }
}

// The radial basis of the pair (ti, tj) at distance d: the model's shared
// RBChebyshev basis, or (run-time profiles only) the pair's general basis.
template <class P>
__device__ __forceinline__ void radial_basis(const DevModel &m, int ti, int tj, double d,
                                             double *Q, double *dQ)
{
    if constexpr (!P::exact)
        if (m.rb_general) {
            general_basis<P::RMAX>(m.rb_table + (ti * m.Z + tj) * kRbStride, d, Q, dQ);
            return;
        }
    chebyshev<P::RMAX>(m, d, Q, dQ);
}

// The fields of list entry p that load_neighbor reads (zeros and type 0 for
// a lane without an entry), so that a kernel can fetch the next batch's
// entries ahead of their use; j is the neighbour's atom (-1 without entry).
struct EntryRaw {
    double x, y, z, d;
    int tj, j;
};
__device__ __forceinline__ EntryRaw fetch_entry(const DevNeighbors &nb, int64_t p, bool valid)
{
    EntryRaw e;
    e.x = valid ? nb.x[p] : 0.0;
    e.y = valid ? nb.y[p] : 0.0;
    e.z = valid ? nb.z[p] : 0.0;
    e.d = valid ? nb.d[p] : 0.0;
    e.tj = valid ? nb.type[p] : 0;
    e.j = valid ? nb.idx[p] : -1;
    return e;
}

// Geometry (as load_geometry) plus the radial functions
// f_mu = sum_k c[ti,tj,mu,k] Q_k and their derivatives (coefficients staged
// in LDS) of a fetched entry, zero beyond the cutoff.
template <class P>
__device__ __forceinline__ void neighbor_from(const DevModel &m, const double *coef_lds, int ti,
                                              const EntryRaw &e, bool valid, Nbr<P::M> &q)
{
    constexpr int RMAX = P::RMAX;
    const int tj = e.tj;
    q.x = e.x;
    q.y = e.y;
    q.z = e.z;
    const double rc = pair_cutoff<!P::exact>(m, ti, tj);
    const double dd = valid ? e.d : rc;
    const bool in_cutoff = valid && !(dd > rc);
    const double d = in_cutoff ? dd : rc;
    q.d = d;
    q.invd = 1.0 / d;
    q.ux = q.x * q.invd;
    q.uy = q.y * q.invd;
    q.uz = q.z * q.invd;
    const double w = in_cutoff ? 1.0 : 0.0;
    double Q[RMAX], dQ[RMAX];
    radial_basis<P>(m, ti, tj, q.d, Q, dQ);
    // exact profiles fix M and R at compile time
    const int R = P::exact ? RMAX : m.R;
    const double *c = coef_lds + (ti * m.Z + tj) * (P::exact ? P::M : m.M) * R;
#pragma unroll
    for (int mu = 0; mu < P::M; ++mu) {
        double f = 0, fd = 0;
        if (P::exact || mu < m.M) {
            const double *cm = c + mu * R;
#pragma unroll
            for (int k = 0; k < RMAX; ++k)
                if (P::exact || k < m.R) {
                    f += cm[k] * Q[k];
                    fd += cm[k] * dQ[k];
                }
        }
        q.f[mu] = f * w;
        q.fd[mu] = fd * w;
    }
}

// Geometry plus the radial functions of list entry p.
template <class P>
__device__ __forceinline__ void load_neighbor(const DevModel &m, const DevNeighbors &nb,
                                              const double *coef_lds, int ti, int64_t p,
                                              bool valid, Nbr<P::M> &q)
{
    constexpr int RMAX = P::RMAX;
    int tj;
    const double w = load_geometry<P::M, !P::exact>(m, nb, p, valid, q, tj, ti);
    double Q[RMAX], dQ[RMAX];
    radial_basis<P>(m, ti, tj, q.d, Q, dQ);
    // exact profiles fix M and R at compile time
    const int R = P::exact ? RMAX : m.R;
    const double *c = coef_lds + (ti * m.Z + tj) * (P::exact ? P::M : m.M) * R;
#pragma unroll
    for (int mu = 0; mu < P::M; ++mu) {
        double f = 0, fd = 0;
        if (P::exact || mu < m.M) {
            const double *cm = c + mu * R;
#pragma unroll
            for (int k = 0; k < RMAX; ++k)
                if (P::exact || k < m.R) {
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
// without a neighbour hold zeros.  Lanes 0 .. nrows-1 hold the row sums.
__device__ __forceinline__ void reduce_chunk(const double *red, int nrows, int slot0,
                                             const int *slot_basic, double *mom, int lane)
{
    wave_sync();
    const double acc = chunk_row_sum(red, lane);
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

// Force pass over the slots: u = sum A Y, G = sum (a A, b A, c A) . Y_{-1}
// with the slot-ordered adjoints A (an 8-byte LDS broadcast per slot; the
// integer factors are applied in registers).
template <int NU, class P>
__device__ __forceinline__ void bwd_shells(const DevModel &m, const double *As, int &slot,
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
                    const double w = As[slot + i];  // LDS broadcast
                    u += w * cur[i];
                    if constexpr (NU > 0) {
                        if (a > 0)
                            Gx += (w * a) * prev[shell_index(NU - 1, a - 1, b)];
                        if (b > 0)
                            Gy += (w * b) * prev[shell_index(NU - 1, a, b - 1)];
                        if (NU - a - b > 0)
                            Gz += (w * (NU - a - b)) * prev[shell_index(NU - 1, a, b)];
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
            bwd_shells<NU + 1, P>(m, As, slot, q, cur, acc);
    }
}

// One group of up to four steps of a level (cnt of them applied).
template <bool kInit>
__device__ __forceinline__ void rule_group(const int2 (&e)[4], int cnt, double *ws, double &acc)
{
    double ml[4], mr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int l = e[k].x & 0xffff, r = (unsigned)e[k].x >> 16;
        ml[k] = ws[l];
        mr[k] = ws[r];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k >= cnt)
            break;
        const double c = (double)(e[k].y >> 18);
        acc = fma(c * ml[k], mr[k], acc);
        if (e[k].y & 0x20000) {
            const int w = e[k].y & 0xffff;
            ws[w] = kInit ? ws[w] + acc : acc;
            acc = 0.0;
        }
    }
}

// The same over {value, dual} pairs.
template <bool kInit>
__device__ __forceinline__ void rule_group_dual(const int2 (&e)[4], int cnt, double2 *wp,
                                                double &acc, double &acd)
{
    double2 vl[4], vr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        vl[k] = wp[e[k].x & 0xffff];
        vr[k] = wp[(unsigned)e[k].x >> 16];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k >= cnt)
            break;
        const double c = (double)(e[k].y >> 18);
        acc = fma(c * vl[k].x, vr[k].x, acc);
        acd = fma(c * vl[k].x, vr[k].y, fma(c * vl[k].y, vr[k].x, acd));
        if (e[k].y & 0x20000) {
            const int w = e[k].y & 0xffff;
            if (kInit) {
                const double2 o = wp[w];
                wp[w] = double2{o.x + acc, o.y + acd};
            } else {
                wp[w] = double2{acc, acd};
            }
            acc = 0.0;
            acd = 0.0;
        }
    }
}

// Product rules from a lane-major step table (forward: potential_mtp.cpp:
// 2918-2924; reverse: backpropagate_moments, :3292-3305), one dependency
// level at a time.  Steps are taken in groups of four: the entries of the
// next group are loaded while the current one runs, and every operand of a
// group is read before any of its results is written (a level never reads
// what it writes).  A level's last group holds its last one to four steps;
// the entries it loads past the level (the next level's, or the padding
// after the last level) are read but not applied.  A task's sum starts
// from zero and is stored on the task's last entry: added to its target
// (kInit: adjoints, which start from their seeds) or written over it
// (outputs and partial sums, which start at zero).  No task reads or writes
// another task's target within a level.
//
// kDual carries a dual value beside every element: the work space holds
// pairs {x, x'} (element x's value in double 2x, its dual in 2x + 1; the
// tables' indices count pairs), read and written 16 bytes at a time, and
// for a step  x_w += c x_l x_r  it adds  c (x'_l x_r + x_l x'_r)  to x'_w.
// Forward entries then propagate tangents (Q_o += c (Q_l m_r + m_l Q_r));
// reverse entries, whose l is an adjoint and r a moment, propagate the
// adjoint of the tangent computation (G_x += c (G_o m_r + A_o Q_r)).
template <bool kDual, bool kInit>
__device__ __forceinline__ void run_rules(const int2 *tab, const int *level_step,
                                          const int *level_comb, const int4 *comb, int nlev,
                                          double *ws, int lane)
{
    double2 *wp = reinterpret_cast<double2 *>(ws);
    for (int L = 0; L < nlev; ++L) {
        const int s0 = level_step[L], s1 = level_step[L + 1];
        double acc = 0.0, acd = 0.0;
        auto group = [&](const int2(&e)[4], int cnt) {
            if constexpr (kDual)
                rule_group_dual<kInit>(e, cnt, wp, acc, acd);
            else
                rule_group<kInit>(e, cnt, ws, acc);
        };
        if (s1 > s0) {
            const int2 *t = tab + (size_t)s0 * kWave + lane;
            int2 e[4] = {t[0], t[kWave], t[2 * kWave], t[3 * kWave]};
            int st = s0;
            for (; st + 4 < s1; st += 4) {
                const int2 *u = t + (size_t)(st + 4 - s0) * kWave;
                const int2 nx[4] = {u[0], u[kWave], u[2 * kWave], u[3 * kWave]};
                group(e, 4);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    e[k] = nx[k];
            }
            group(e, s1 - st);
        }
        const int c0 = level_comb[L], c1 = level_comb[L + 1];
        if (c1 > c0) {
            wave_sync();
            for (int c = c0 + lane; c < c1; c += kWave) {
                const int4 q = comb[c];
                if constexpr (kDual) {
                    double2 sum = wp[q.x];
                    for (int k = 0; k < q.z; ++k) {
                        const double2 v = wp[q.y + k];
                        sum.x += v.x;
                        sum.y += v.y;
                        wp[q.y + k] = double2{0.0, 0.0};
                    }
                    wp[q.x] = sum;
                } else {
                    double sum = ws[q.x];
                    for (int k = 0; k < q.z; ++k) {
                        sum += ws[q.y + k];
                        ws[q.y + k] = 0.0;
                    }
                    ws[q.x] = sum;
                }
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

// The block-shared model tables in LDS: radial coefficients, the adjoint
// seeds (kernels that run the reverse rules from LDS), moment coefficients,
// map, slot tables and optionally the rule step tables.
__device__ __host__ __forceinline__ size_t shared_doubles(const DevModel &m, bool tables,
                                                          bool seeds = true)
{
    const size_t r4c = ((size_t)m.Z * m.Z * m.M * m.R + 3) & ~size_t(3);
    const size_t S4 = (m.S + 3) & ~3, N4 = (m.nslots + 3) & ~3;
    size_t d = r4c + (seeds ? m.K4 : 0) + S4 + (S4 + 2 * N4) / 2;
    if (tables)
        d += (size_t)(m.fwd_nsteps + m.bwd_nsteps) * kWave;
    return (d + 3) & ~size_t(3);
}

__device__ __forceinline__ Shared shared_layout(const DevModel &m, double *base,
                                                bool seeds = true)
{
    const int r4c = (m.Z * m.Z * m.M * m.R + 3) & ~3;
    const int S4 = (m.S + 3) & ~3, N4 = (m.nslots + 3) & ~3;
    Shared L;
    L.coef = base;
    L.seed = seeds ? L.coef + r4c : nullptr;
    L.moment = L.coef + r4c + (seeds ? m.K4 : 0);
    L.map = reinterpret_cast<int *>(L.moment + S4);
    L.slot_basic = L.map + S4;
    L.slot_abc = L.slot_basic + N4;
    L.fwd_steps = reinterpret_cast<int2 *>(L.slot_abc + N4);
    L.bwd_steps = L.fwd_steps + (size_t)m.fwd_nsteps * kWave;
    return L;
}

// Model tables every workgroup stages into its shared LDS region.
__device__ __forceinline__ void stage_shared(const DevModel &m, const Shared &L, bool tables,
                                             int tid, int nthreads)
{
    const int ncoef_r = m.Z * m.Z * m.M * m.R;
    for (int k = tid; k < ncoef_r; k += nthreads)
        L.coef[k] = m.radial[k];
    if (L.seed)
        for (int k = tid; k < m.K; k += nthreads)
            L.seed[k] = m.seed[k];
    for (int k = tid; k < m.S; k += nthreads) {
        L.moment[k] = m.moment[k];
        L.map[k] = m.map[k];
    }
    for (int k = tid; k < m.nslots; k += nthreads) {
        L.slot_basic[k] = m.slot_basic[k];
        L.slot_abc[k] = m.slot_abc[k];
    }
    if (tables) {
        for (int k = tid; k < m.fwd_nsteps * kWave; k += nthreads)
            L.fwd_steps[k] = m.fwd_steps[k];
        for (int k = tid; k < m.bwd_nsteps * kWave; k += nthreads)
            L.bwd_steps[k] = m.bwd_steps[k];
    }
}

// ---- MTP-M site heads -------------------------------------------------------
// The activations of the neural heads and their derivatives (runtime/mtp/cpu/
// mtp_cpu.cpp:21-45).
__device__ __forceinline__ double head_activate(double x, int act, double &der)
{
    if (act == kActTanh) {
        const double v = tanh(x);
        der = 1.0 - v * v;
        return v;
    }
    if (act == kActRelu) {
        der = x > 0.0 ? 1.0 : 0.0;
        return x > 0.0 ? x : 0.0;
    }
    if (act == kActSigmoid) {
        const double v = 1.0 / (1.0 + exp(-x));
        der = v * (1.0 - v);
        return v;
    }
    der = 1.0;
    return x;
}

// Descriptor-indexed sums run in chunks of this many independent
// accumulators per lane, so their loads overlap.
constexpr int kHeadChunk = 8;

// out[j] = sum over r in [0, n) of w[r * ld + j] * x[r] for j < nj
// (nj <= kHeadChunk), every lane taking rows lane, lane + 64, ..., then
// summed over the wave; the result is in every lane.
__device__ __forceinline__ void wave_matvec_chunk(const double *w, int ld, int nj,
                                                  const double *x, int n, int lane, double *out)
{
    double part[kHeadChunk];
#pragma unroll
    for (int j = 0; j < kHeadChunk; ++j)
        part[j] = 0.0;
    for (int r = lane; r < n; r += kWave) {
        const double v = x[r];
        const double *row = w + (size_t)r * ld;
#pragma unroll
        for (int j = 0; j < kHeadChunk; ++j)
            if (j < nj)
                part[j] += row[j] * v;
    }
#pragma unroll
    for (int j = 0; j < kHeadChunk; ++j)
        out[j] = j < nj ? wave_sum(part[j]) : 0.0;
}

// b + sum_k w[k * stride] x[k] for k < n, with four accumulators.
__device__ __forceinline__ double dot4(double b, const double *w, size_t stride, const double *x,
                                       int n)
{
    double a0 = b, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    int k = 0;
    for (; k + 4 <= n; k += 4) {
        a0 += w[k * stride] * x[k];
        a1 += w[(k + 1) * stride] * x[k + 1];
        a2 += w[(k + 2) * stride] * x[k + 2];
        a3 += w[(k + 3) * stride] * x[k + 3];
    }
    for (; k < n; ++k)
        a0 += w[k * stride] * x[k];
    return (a0 + a1) + (a2 + a3);
}

// The dynamic LDS of a launch (the same storage as the kernels' own
// extern __shared__ arrays), for device functions that are not inlined.
extern __shared__ double mtpx_lds[];

// The site energy of an MTP-M potential less its species term, for the
// centre species t, in every lane (Executor::evaluate_site and
// Executor::head, mtp_cpu.cpp:291-442).  The moments are at LDS offset
// mom; the descriptors Q_p = dspecies[p Z + t] + sum_a proj[p][a] m(ids[a])
// are wave sums over the distinct scalar moments, the hidden units run one
// per lane and dE/dQ is a wave sum over them.  With grad the adjoint seeds
// A(ids[a]) = sum_p proj[p][a] dE/dQ_p go to the block at LDS offset adj
// (zero elsewhere).  hs (an LDS offset) is the wave's head work space:
// Q [P], dE/dQ [P], first-layer activations and then responses [h1], their
// derivatives [h1], second-layer adjoints [h2].  The sums are ordered
// differently from the reference's loops (rounding only).  Out of line: the
// E/F/S kernel's register allocation stays that of the linear model.
__device__ __noinline__ double head_site(const DevHead *__restrict__ H, int t, int mom, int hs,
                                         int adj, int lane, bool grad)
{
    const int P = H->P, NS = H->NS, h1 = H->h1, h2 = H->h2, act = H->act, kind = H->kind;
    const int *ids = H->ids;
    const double *proj = H->proj, *c = H->c;
    const double *mv = mtpx_lds + mom;
    double *Q = mtpx_lds + hs, *dQ = Q + P, *a1 = dQ + P, *d1 = a1 + h1, *g2 = d1 + h1;
    double part[kHeadChunk];
    // proj is [P][NS]: over the distinct moments a, column j at stride NS
    for (int p0 = 0; p0 < P; p0 += kHeadChunk) {
        const int np = min(kHeadChunk, P - p0);
        double acc[kHeadChunk];
#pragma unroll
        for (int j = 0; j < kHeadChunk; ++j)
            acc[j] = 0.0;
        for (int a = lane; a < NS; a += kWave) {
            const double v = mv[ids[a]];
            const double *w = proj + (size_t)p0 * NS + a;
#pragma unroll
            for (int j = 0; j < kHeadChunk; ++j)
                if (j < np)
                    acc[j] += w[(size_t)j * NS] * v;
        }
#pragma unroll
        for (int j = 0; j < kHeadChunk; ++j)
            part[j] = j < np ? wave_sum(acc[j]) : 0.0;
        if (lane == 0)
#pragma unroll
            for (int j = 0; j < kHeadChunk; ++j)
                if (j < np)
                    Q[p0 + j] = H->dsp[(p0 + j) * H->Z + t] + part[j];
    }
    wave_sync();
    double e = 0.0;
    if (kind == kHeadLi) {
        e = Q[0];
        if (grad && lane == 0)
            dQ[0] = 1.0;
    } else if (kind == kHeadQ2) {
        const double x = Q[0], y = Q[1];
        e = c[0] * x + c[1] * y + c[2] * x * x + c[3] * y * y + c[4] * x * y;
        if (grad && lane == 0) {
            dQ[0] = c[0] + 2.0 * c[2] * x + c[4] * y;
            dQ[1] = c[1] + 2.0 * c[3] * y + c[4] * x;
        }
    } else if (kind == kHeadFs) {
        e = Q[0] + c[0] * asinh(Q[1]);
        if (grad && lane == 0) {
            dQ[0] = 1.0;
            dQ[1] = c[0] / sqrt(1.0 + Q[1] * Q[1]);
        }
    } else {
        // NN1: [W1 (h1 x P) | out (h1) | b1 (h1)]; NN2: [W1 | b1 | W2 (h2 x h1)
        // | b2 (h2) | out (h2)] (the coefficient order of mtp_cpu.cpp:334-337)
        const bool nn2 = kind == kHeadNn2;
        const double *b1 = c + P * h1 + (nn2 ? 0 : h1);
        const double *w2 = b1 + h1, *b2 = w2 + (size_t)h1 * h2;
        const double *out = nn2 ? b2 + h2 : c + P * h1;
        double sum = 0.0;
        for (int h = lane; h < h1; h += kWave) {
            double d;
            const double a = head_activate(dot4(b1[h], c + (size_t)h * P, 1, Q, P), act, d);
            a1[h] = a;
            d1[h] = d;
            if (!nn2)
                sum += out[h] * a;
        }
        wave_sync();
        if (nn2) {
            for (int k = lane; k < h2; k += kWave) {
                double d;
                sum += out[k] * head_activate(dot4(b2[k], w2 + (size_t)k * h1, 1, a1, h1), act, d);
                g2[k] = out[k] * d;
            }
            wave_sync();
        }
        e = wave_sum(sum);
        if (grad) {
            // responses over the activations they replace (each lane its own)
            for (int h = lane; h < h1; h += kWave) {
                const double r = nn2 ? dot4(0.0, w2 + h, (size_t)h1, g2, h2) : out[h];
                a1[h] = r * d1[h];
            }
            wave_sync();
            // dE/dQ_p = sum_h W1[h][p] r_h: W1 read as rows h of P entries
            for (int p0 = 0; p0 < P; p0 += kHeadChunk) {
                const int np = min(kHeadChunk, P - p0);
                wave_matvec_chunk(c + p0, P, np, a1, h1, lane, part);
                if (lane == 0)
#pragma unroll
                    for (int j = 0; j < kHeadChunk; ++j)
                        if (j < np)
                            dQ[p0 + j] = part[j];
            }
        }
    }
    wave_sync();
    if (grad) {
        double *A = mtpx_lds + adj;
        for (int k = lane; k < H->K; k += kWave)
            A[k] = 0.0;
        wave_sync();
        for (int a = lane; a < NS; a += kWave)
            A[ids[a]] = dot4(0.0, proj + a, (size_t)NS, dQ, P);
    }
    return e;
}

// Launch shape for a kernel whose waves each own `priv_doubles` of LDS work
// space next to the block-shared model tables: rule tables in LDS unless that
// costs waves; false if a single wave does not fit.
// table_pref: -1 chooses the step-table placement, 0 keeps the tables in
// global memory, 1 in LDS where they fit.
inline bool configure_launch(const DevModel &m, int n, int num_cus, int wcap, size_t lds_limit,
                             int priv_doubles, EfsLaunch &cfg, int table_pref = -1,
                             bool seeds = true)
{
    const size_t priv = (size_t)priv_doubles * sizeof(double);
    auto fit = [&](bool tables) {
        const size_t sh = shared_doubles(m, tables, seeds) * sizeof(double);
        if (sh + priv > lds_limit)
            return 0;
        return (int)std::min<size_t>(wcap, (lds_limit - sh) / priv);
    };
    const int wt = fit(true), wg = fit(false);
    if (wg == 0)
        return false;
    cfg.lds_tables = table_pref < 0 ? wt > 0 && wt >= wg : table_pref == 1 && wt > 0;
    cfg.waves = cfg.lds_tables ? wt : wg;
    cfg.lds_bytes = shared_doubles(m, cfg.lds_tables, seeds) * sizeof(double) + cfg.waves * priv;
    const int per_cu = std::max<int>(1, (int)(lds_limit / cfg.lds_bytes));
    const int need = (std::max(n, 1) + cfg.waves - 1) / cfg.waves;
    cfg.grid = std::max(1, std::min(need, num_cus * per_cu));
    cfg.rows = cfg.grid * cfg.waves;
    return true;
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
}  // namespace mtpx
