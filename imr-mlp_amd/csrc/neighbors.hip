// Device neighbour-list builder reproducing the reference BOXED builder
// (base/neighborhoods_base.h:31-266, base/neighborhood.cpp:77-146) bit for
// bit.  Compiled with -ffp-contract=off; every floating-point expression
// keeps the reference's operation order, and fp64 division and sqrt are
// IEEE correctly rounded on gfx950.
//
// Pipeline (all on one stream, every structure of a chunk in the same
// launches):
//   1. wrap (load_positions, only for fully periodic cells) and AABB min/max;
//   2. periodic images: the host walks the integer image triples in the
//      reference's lexicographic order (outermost = longest periodic axis),
//      keeps the triples whose translated box can reach the AABB +- cutoff,
//      and the device tests every (image, atom) pair; an exclusive scan over
//      the flattened (image-major, atom-minor) flags places the images in
//      the reference's append order;
//   3. boxes: box index by the reference's ceil formula and clamps, then a
//      counting sort with each box's points ranked by point index (the
//      reference's insertion order: originals by index, then images);
//   4. construct: each centre's processing rank is its position in the
//      lexicographic walk over the interior boxes; a centre enumerates its
//      qualifying (offset, slot) events in order, numbering them.  An event
//      appends (idx, r, d) to the centre's list and, if idx != centre, the
//      mirrored entry to list[idx].  Every entry carries the key
//      (processing rank, event number), which is the order in which the
//      reference appends it; lists are filled in any order and then ranked
//      by key.
#include "mtpx.h"
#include "mtpx_geometry.hpp"
#include "mtpx_internal.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace mtpx {

namespace {

struct Cell {
    double m[9];    // rows are lattice vectors
    double inv[9];  // Matrix3d::inverse
};

__device__ __forceinline__ void dev_row_times(const double *p, const double *M, double *out)
{
    double r[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const double a0 = p[0] * M[j], a1 = p[1] * M[3 + j], a2 = p[2] * M[6 + j];
        r[j] = (a0 + a1) + a2;
    }
    out[0] = r[0];
    out[1] = r[1];
    out[2] = r[2];
}

// Place each point at box_start[b] + (number of points of box b with a smaller
// index): the first pass drops points in any order, the second ranks them.
__global__ void box_place_kernel(const int *box, const int *npts, int *box_cur, int *items)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= *npts)
        return;
    const int q = atomicAdd(&box_cur[box[i]], 1);
    items[q] = i;
}

// One thread per point: its slot in its box is the number of the box's
// points with a smaller index (a box of a small cell can hold every point).
__global__ void box_rank_kernel(const int *box, const int *box_start, const int *npts,
                                const int *unsorted, int *items)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= *npts)
        return;
    const int b = box[i];
    const int s = box_start[b], e = box_start[b + 1];
    int r = 0;
    for (int u = s; u < e; ++u)
        r += unsorted[u] < i;
    items[s + r] = i;
}

// Rank every staged entry within its list by key and write it to its final
// slot (SoA); a staged entry is its key and its two points (neighbour,
// centre), from which the displacement and distance are formed again.  One
// wave per list: lanes take 64 entries at a time and count the list's
// smaller keys, read 64 at a time and broadcast lane by lane (keys within a
// list are distinct).  The staged entries of list l lie at its final offsets
// (cap == 0) or in its bin from l cap; with bins, a set overflow flag means
// the staging is incomplete and nothing is written.
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l)
{
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

__global__ __launch_bounds__(256) void list_rank_kernel(const int *offsets, int n, int cap,
                                                        const int *overflow, const uint64_t *key,
                                                        const int *st_nbr, const int *st_ctr,
                                                        const double *pts, const int *orig,
                                                        const int *types, int *idx, int *type,
                                                        double *x, double *y, double *z,
                                                        double *d, int *st_final)
{
    const int lane = threadIdx.x & 63;
    const int l = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (l >= n || (overflow && *overflow))
        return;  // uniform over the wave
    const int s = offsets[l], cnt = offsets[l + 1] - s;
    const int64_t sb = cap ? (int64_t)l * cap : s;  // the list's first staged entry
    for (int j0 = 0; j0 < cnt; j0 += 64) {
        const int j = j0 + lane;
        const int64_t q = sb + j;
        const uint64_t k = j < cnt ? key[q] : 0;
        int r = 0;
        for (int u0 = 0; u0 < cnt; u0 += 64) {
            const uint64_t ku = u0 + lane < cnt ? key[sb + u0 + lane] : 0;
            const int m = cnt - u0 < 64 ? cnt - u0 : 64;
            for (int u = 0; u < m; ++u)
                r += readlane_u64(ku, u) < k;
        }
        if (j < cnt) {
            const int64_t o = s + r;
            // the entry from its two points, by the operations construct
            // tested it with (the mirrored entry's vector is the exact
            // negation, its distance the same)
            const int pn = st_nbr[q], pc = st_ctr[q];
            const double r0 = pts[3 * (size_t)pn] - pts[3 * (size_t)pc];
            const double r1 = pts[3 * (size_t)pn + 1] - pts[3 * (size_t)pc + 1];
            const double r2 = pts[3 * (size_t)pn + 2] - pts[3 * (size_t)pc + 2];
            const int aj = orig[pn];
            idx[o] = aj;
            type[o] = types[aj];
            x[o] = r0;
            y[o] = r1;
            z[o] = r2;
            d[o] = sqrt(r0 * r0 + r1 * r1 + r2 * r2);
            st_final[q] = (int)o;
        }
    }
}

// mirror[final(q)] = final(mate(q)) for every staged entry q (the staging
// as list_rank_kernel reads it; nothing when a bin overflowed).
__global__ __launch_bounds__(256) void mirror_kernel(const int *offsets, int n, int cap,
                                                     const int *overflow, const int *mate,
                                                     const int *st_final, int *mirror)
{
    const int lane = threadIdx.x & 63;
    const int l = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (l >= n || (overflow && *overflow))
        return;  // uniform over the wave
    const int s = offsets[l], cnt = offsets[l + 1] - s;
    const int64_t sb = cap ? (int64_t)l * cap : s;
    for (int j = lane; j < cnt; j += 64) {
        const int64_t q = sb + j;
        mirror[st_final[q]] = st_final[mate[q]];
    }
}

// ---- exclusive scan of int32 (three passes) ---------------------------
constexpr int kScanBlock = 256, kScanItems = 8, kScanTile = kScanBlock * kScanItems;

// Every scan reads min(in[i], clamp): the per-list counts of a one-pass
// build are taken up to their bin size, which keeps the sums in int32 when
// a list has outgrown its bin (that build is then discarded).
__global__ __launch_bounds__(kScanBlock) void scan_tile_sums(const int *in, int64_t n, int clamp,
                                                             int *sums)
{
    __shared__ int buf[kScanBlock];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int s = 0;
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + (int64_t)k * kScanBlock + threadIdx.x;
        if (i < n)
            s += min(in[i], clamp);
    }
    buf[threadIdx.x] = s;
    __syncthreads();
    for (int w = kScanBlock / 2; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w)
            buf[threadIdx.x] += buf[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        sums[blockIdx.x] = buf[0];
}

__global__ __launch_bounds__(1024) void scan_sums(int *sums, int ntiles, int *total)
{
    __shared__ int buf[1024];
    __shared__ int carry;
    if (threadIdx.x == 0)
        carry = 0;
    __syncthreads();
    for (int base = 0; base < ntiles; base += 1024) {
        const int i = base + threadIdx.x;
        const int v = i < ntiles ? sums[i] : 0;
        buf[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int t = threadIdx.x >= (unsigned)off ? buf[threadIdx.x - off] : 0;
            __syncthreads();
            buf[threadIdx.x] += t;
            __syncthreads();
        }
        if (i < ntiles)
            sums[i] = carry + buf[threadIdx.x] - v;
        __syncthreads();
        if (threadIdx.x == 1023)
            carry += buf[1023];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        *total = carry;
}

__global__ __launch_bounds__(kScanBlock) void scan_tiles(const int *in, int64_t n, int clamp,
                                                          const int *sums, int *out, int *out2)
{
    __shared__ int buf[kScanBlock];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int v[kScanItems];
    int s = 0;
    for (int k = 0; k < kScanItems; ++k) {
        v[k] = base + k < n ? min(in[base + k], clamp) : 0;
        s += v[k];
    }
    buf[threadIdx.x] = s;
    __syncthreads();
    for (int off = 1; off < kScanBlock; off <<= 1) {
        const int t = threadIdx.x >= (unsigned)off ? buf[threadIdx.x - off] : 0;
        __syncthreads();
        buf[threadIdx.x] += t;
        __syncthreads();
    }
    int run = sums[blockIdx.x] + buf[threadIdx.x] - s;
    for (int k = 0; k < kScanItems; ++k) {
        if (base + k < n) {
            out[base + k] = run;
            if (out2)
                out2[base + k] = run;
        }
        run += v[k];
    }
}

// 64-bit sum of n non-negative ints into *total and their maximum into
// *largest (both zeroed by the caller): the list-length total, checked
// against the int32 entry indices before any offset is trusted, and the
// longest list, which sizes the bins of the next build.
__global__ __launch_bounds__(256) void sum64_kernel(const int *in, int64_t n,
                                                    unsigned long long *total, int *largest)
{
    __shared__ unsigned long long buf[256];
    __shared__ int big[256];
    unsigned long long s = 0;
    int mx = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        s += (unsigned)in[i];
        mx = max(mx, in[i]);
    }
    buf[threadIdx.x] = s;
    big[threadIdx.x] = mx;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) {
            buf[threadIdx.x] += buf[threadIdx.x + w];
            big[threadIdx.x] = max(big[threadIdx.x], big[threadIdx.x + w]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        atomicAdd(total, buf[0]);
        atomicMax(largest, big[0]);
    }
}

// Inclusive prefix sum over the 64 lanes of a wave: rows of 16 by DPP row
// shifts (lanes without a source add 0), then each row adds the totals of
// the rows before it (lane reads).
__device__ __forceinline__ int wave_incl_scan(int x, int lane)
{
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    const int t0 = __builtin_amdgcn_readlane(x, 15), t1 = __builtin_amdgcn_readlane(x, 31),
              t2 = __builtin_amdgcn_readlane(x, 47);
    const int r = lane >> 4;
    return x + (r >= 1 ? t0 : 0) + (r >= 2 ? t1 : 0) + (r >= 3 ? t2 : 0);
}

// One-workgroup scans use 1,024 threads (16 waves).
constexpr int kScan1Threads = 1024, kScan1Waves = kScan1Threads / 64;

// Exclusive prefix of one value per thread over such a workgroup (thread
// order); tot receives the workgroup's total.
__device__ __forceinline__ int block_excl_scan(int v, int *wsum, int &tot)
{
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int x = wave_incl_scan(v, lane);
    if (lane == 63)
        wsum[wv] = x;
    __syncthreads();
    int carry = 0;
    tot = 0;
    for (int k = 0; k < kScan1Waves; ++k) {
        const int w = wsum[k];
        carry += k < wv ? w : 0;
        tot += w;
    }
    return carry + x - v;
}

// Exclusive scan of up to kScanLdsMax values in one workgroup through LDS:
// the values go in with coalesced loads (slot i + i / 32, so that threads
// reading consecutive runs hit distinct banks), thread t scans the run
// [t m, (t+1) m) after the prefix of the runs before it, and the prefixes
// go out with coalesced stores.  Every value is read before any is written,
// so out and out2 may be in.  One launch instead of three.
constexpr int kScanLdsMax = 36864;

__host__ __device__ constexpr size_t scan_lds_bytes(int n)
{
    return sizeof(int) * ((size_t)n + (size_t)n / 32 + 1);
}

__global__ __launch_bounds__(kScan1Threads) void scan_one_block(const int *in, int n, int clamp,
                                                                int *out, int *out2, int *total)
{
    extern __shared__ int buf[];
    __shared__ int wsum[kScan1Waves];
    const int t = threadIdx.x;
#pragma unroll 8
    for (int i = t; i < n; i += kScan1Threads)
        buf[i + (i >> 5)] = min(in[i], clamp);
    __syncthreads();
    const int m = (n + kScan1Threads - 1) / kScan1Threads;
    const int b0 = min(n, t * m), b1 = min(n, b0 + m);
    int sum = 0;
    for (int i = b0; i < b1; ++i)
        sum += buf[i + (i >> 5)];
    int tot;
    int run = block_excl_scan(sum, wsum, tot);
    for (int i = b0; i < b1; ++i) {
        const int v = buf[i + (i >> 5)];
        buf[i + (i >> 5)] = run;
        run += v;
    }
    __syncthreads();
#pragma unroll 8
    for (int i = t; i < n; i += kScan1Threads) {
        const int v = buf[i + (i >> 5)];
        out[i] = v;
        if (out2)
            out2[i] = v;
    }
    if (t == 0)
        *total = tot;
}

// Exclusive scan into out (and out2 when given, which may be in: every
// value is read before its slot is written); *total receives the sum
// (device); returns the error.
hipError_t scan_exclusive(const int *in, int64_t n, int *out, DBuf &tmp, int *total,
                          hipStream_t s, int *out2 = nullptr, int clamp = INT_MAX)
{
    if (n <= kScanLdsMax) {
        hipLaunchKernelGGL(scan_one_block, dim3(1), dim3(kScan1Threads), scan_lds_bytes((int)n), s,
                           in, (int)n, clamp, out, out2, total);
        return hipGetLastError();
    }
    const int64_t ntiles = std::max<int64_t>(1, (n + kScanTile - 1) / kScanTile);
    hipError_t e = tmp.ensure(sizeof(int) * (size_t)ntiles);
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(scan_tile_sums, dim3((unsigned)ntiles), dim3(kScanBlock), 0, s, in, n,
                       clamp, tmp.as<int>());
    hipLaunchKernelGGL(scan_sums, dim3(1), dim3(1024), 0, s, tmp.as<int>(), (int)ntiles, total);
    hipLaunchKernelGGL(scan_tiles, dim3((unsigned)ntiles), dim3(kScanBlock), 0, s, in, n, clamp,
                       tmp.as<int>(), out, out2);
    return hipGetLastError();
}

inline unsigned blocks(int64_t n, int t) { return (unsigned)std::max<int64_t>(1, (n + t - 1) / t); }

#define DTRY(expr)                                                                         \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) {                                                            \
            err = std::string("neighbour build: ") + hipGetErrorString(e_);                \
            return e_ == hipErrorOutOfMemory ? MTPX_E_ALLOC : MTPX_E_DEVICE;               \
        }                                                                                  \
    } while (0)

// Candidate image translations in the reference's enumeration order
// (append_images, neighborhoods_base.h:31-99).  The reference bounds every
// integer range with a Householder QR back-substitution; this walk uses a
// wider range from the pseudo-inverse of the periodic basis and skips the
// triples whose translated AABB cannot meet [lo - rc, hi + rc].  Both walks
// visit the passing triples in the same order, so the appended images are
// identical.  Translations use Eigen's Matrix3d * Vector3d order: rows 0, 1
// summed left to right, row 2 as b0 + (b1 + b2).
int image_candidates(const double cell[9], const int pbc[3], const double lo[3],
                     const double hi[3], double cutoff, std::vector<double> &cand,
                     std::string &err)
{
    cand.clear();
    if (!pbc[0] && !pbc[1] && !pbc[2])
        return MTPX_OK;
    int axes[3] = {0, 1, 2};
    double nrm[3];
    for (int a = 0; a < 3; ++a)
        nrm[a] = cell[3 * a] * cell[3 * a] + cell[3 * a + 1] * cell[3 * a + 1] +
                 cell[3 * a + 2] * cell[3 * a + 2];
    std::stable_sort(axes, axes + 3, [&](int a, int b) { return nrm[a] < nrm[b]; });
    double basis[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    int dims = 0;
    for (int q = 0; q < 3; ++q)
        if (pbc[axes[q]]) {
            for (int r = 0; r < 3; ++r)
                basis[r * 3 + dims] = cell[axes[q] * 3 + r];
            dims++;
        }
    double ext[3];
    for (int d = 0; d < 3; ++d)
        ext[d] = hi[d] - lo[d] + cutoff;
    // pseudo-inverse of the 3 x dims basis
    double g[9] = {0}, gi[9] = {0};
    for (int a = 0; a < dims; ++a)
        for (int b = 0; b < dims; ++b) {
            double s = 0;
            for (int r = 0; r < 3; ++r)
                s += basis[r * 3 + a] * basis[r * 3 + b];
            g[a * dims + b] = s;
        }
    if (dims == 1) {
        gi[0] = 1.0 / g[0];
    } else if (dims == 2) {
        const double det = g[0] * g[3] - g[1] * g[2];
        if (det == 0) {
            err = "singular periodic cell";
            return MTPX_E_INVALID;
        }
        gi[0] = g[3] / det;
        gi[1] = -g[1] / det;
        gi[2] = -g[2] / det;
        gi[3] = g[0] / det;
    } else if (!cell_inverse(g, gi)) {
        err = "singular periodic cell";
        return MTPX_E_INVALID;
    }
    long rng[3] = {0, 0, 0};
    for (int k = 0; k < dims; ++k) {
        double bnd = 0;
        for (int r = 0; r < 3; ++r) {
            double pk = 0;
            for (int a = 0; a < dims; ++a)
                pk += gi[k * dims + a] * basis[r * 3 + a];
            bnd += std::fabs(pk) * ext[r];
        }
        if (!(bnd < 1e6)) {
            err = "Neighbor periodic image index exceeds integer range";
            return MTPX_E_RANGE;
        }
        rng[k] = (long)std::ceil(bnd) + 1;
    }
    long img[3];
    for (img[2] = dims > 2 ? -rng[2] : 0; img[2] <= (dims > 2 ? rng[2] : 0); ++img[2])
        for (img[1] = dims > 1 ? -rng[1] : 0; img[1] <= (dims > 1 ? rng[1] : 0); ++img[1])
            for (img[0] = -rng[0]; img[0] <= rng[0]; ++img[0]) {
                if (img[0] == 0 && img[1] == 0 && img[2] == 0)
                    continue;
                const double iv[3] = {(double)img[0], (double)img[1], (double)img[2]};
                double b[3][3];
                for (int r = 0; r < 3; ++r)
                    for (int c = 0; c < 3; ++c)
                        b[r][c] = basis[r * 3 + c] * iv[c];
                const double t[3] = {(b[0][0] + b[0][1]) + b[0][2], (b[1][0] + b[1][1]) + b[1][2],
                                     b[2][0] + (b[2][1] + b[2][2])};
                // a translated point lies in [lo + t, hi + t]; it can pass the
                // test only if that box meets [lo - rc, hi + rc]
                bool reach = true;
                for (int d = 0; d < 3; ++d)
                    if (hi[d] + t[d] < lo[d] - cutoff - 1e-9 * (1 + std::fabs(t[d])) ||
                        lo[d] + t[d] > hi[d] + cutoff + 1e-9 * (1 + std::fabs(t[d])))
                        reach = false;
                if (reach)
                    cand.insert(cand.end(), {t[0], t[1], t[2]});
            }
    return MTPX_OK;
}

}  // namespace

namespace {

// Entry geometry of a site request, one wave per centre row: r = x[j] - x[i]
// (or the caller's vector) and d = sqrt(r.r) as MLIPCore::compute forms them
// (runtime/mtp/mlip.cpp:949-968, no contraction in this file).  Entries the
// reference skips (r.r == 0, r.r >= cutoff^2, a neighbour of negative type)
// get d = +inf, beyond every cutoff, and type 0.
__global__ __launch_bounds__(256) void site_prepare_kernel(
    int nrows, const int *offsets, const int *center_atom, const int *idx, const int *atom_type,
    const double *pos, const double *vec, double cutoffsq, int *center_type, int *type,
    double *x, double *y, double *z, double *d)
{
    const int row = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (row >= nrows)
        return;
    const int ai = center_atom[row];
    if (lane == 0)
        center_type[row] = atom_type[ai];
    double xi0 = 0, xi1 = 0, xi2 = 0;
    if (!vec) {
        xi0 = pos[3 * (int64_t)ai];
        xi1 = pos[3 * (int64_t)ai + 1];
        xi2 = pos[3 * (int64_t)ai + 2];
    }
    for (int p = offsets[row] + lane; p < offsets[row + 1]; p += 64) {
        const int j = idx[p];
        double r0, r1, r2;
        if (vec) {
            r0 = vec[3 * (int64_t)p];
            r1 = vec[3 * (int64_t)p + 1];
            r2 = vec[3 * (int64_t)p + 2];
        } else {
            r0 = pos[3 * (int64_t)j] - xi0;
            r1 = pos[3 * (int64_t)j + 1] - xi1;
            r2 = pos[3 * (int64_t)j + 2] - xi2;
        }
        const double rr = r0 * r0 + r1 * r1 + r2 * r2;
        const int tj = atom_type[j];
        const bool keep = tj >= 0 && rr > 0.0 && rr < cutoffsq;
        x[p] = r0;
        y[p] = r1;
        z[p] = r2;
        d[p] = keep ? sqrt(rr) : __builtin_inf();
        type[p] = keep ? tj : 0;
    }
}

// Append one structure's lists (atoms from a0, entries from p0) to a batch.
__global__ void append_lists_kernel(const int *offsets, const int *idx, const int *mirror, int n,
                                    int64_t P, int a0, int64_t p0, int *out_offsets, int *out_idx,
                                    int *out_mirror)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k <= n)
        out_offsets[a0 + k] = (int)(p0 + offsets[k]);
    if (k < P) {
        out_idx[p0 + k] = a0 + idx[k];
        out_mirror[p0 + k] = (int)(p0 + mirror[k]);
    }
}

// Grows a device buffer to `need` bytes, keeping its first `keep` bytes.
hipError_t grow_keep(DBuf &b, size_t need, size_t keep, hipStream_t s)
{
    if (need <= b.bytes && b.p)
        return hipSuccess;
    size_t want = std::max<size_t>(need, 2 * b.bytes);
    void *np = nullptr;
    hipError_t e = hipMalloc(&np, want);
    if (e != hipSuccess)
        return e;
    if (keep && b.p)
        e = hipMemcpyAsync(np, b.p, keep, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        (void)hipFree(np);
        return e;
    }
    if (b.p)
        (void)hipFree(b.p);
    b.p = np;
    b.bytes = want;
    return hipSuccess;
}

}  // namespace

hipError_t launch_site_prepare(int nrows, const int *offsets, const int *center_atom,
                               const int *idx, const int *atom_type, const double *pos,
                               const double *vec, double cutoffsq, int *center_type, int *type,
                               double *x, double *y, double *z, double *d, hipStream_t s)
{
    if (nrows > 0)
        hipLaunchKernelGGL(site_prepare_kernel, dim3((nrows + 3) / 4), dim3(256), 0, s, nrows,
                           offsets, center_atom, idx, atom_type, pos, vec, cutoffsq, center_type,
                           type, x, y, z, d);
    return hipGetLastError();
}

// ---- the pipeline over a chunk of structures ----------------------------
//
// Every kernel runs over the concatenation of a chunk's structures with a
// table of per-structure offsets (atoms, points, image flags, image
// candidates, box counters with one closing counter each, interior boxes)
// and geometry; a thread finds its structure by binary search over the
// offsets.  Points are numbered structure by structure (originals, then
// images), atoms and list entries over the chunk, so the lists come out as
// the structures' own lists concatenated with chunk-wide atom indices.  A
// single structure is a chunk of one.  Two host synchronisations per chunk,
// the AABBs and the entry total (point counts and offsets stay on the
// device), and a third for the point total where the bound on the points
// would need large new buffers.
namespace {

struct SegGeom {      // per structure, after the AABB
    double lo[3], hi[3], xd[3], cutoff;
    int bl[3];
};

struct Seg {
    int nconf;
    const int *atom_off, *pt_off, *cand_off, *box_off, *int_off;  // [nconf + 1]
    const long long *flag_off;                                    // [nconf + 1]
    const Cell *cell;                                             // [nconf]
    const int *wrap;                                              // [nconf]
    const SegGeom *geo;                                           // [nconf]
    const double *cand;                                           // [3 * candidates]
};

// The segment holding k: off[c] <= k < off[c + 1] (the last such c when
// segments are empty).
template <class T>
__device__ __forceinline__ int seg_of(const T *off, int n, T k)
{
    int lo = 0, hi = n;  // off[lo] <= k < off[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= k)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

// load_positions (neighborhoods_base.h:113-127) and the AABB; the centres'
// species are copied on the way.  Workgroup k
// of structure c (B per structure) wraps the atoms [k m, (k+1) m) of it,
// m = ceil(n_c / B), into the cell if the structure is fully periodic, and
// writes their component-wise min and max (+inf / -inf for an empty range);
// the host takes the min / max of the B partials.  Min and max are exact.
__global__ __launch_bounds__(256) void wrap_minmax_kernel(Seg g, const double *pos,
                                                          const int *types, int B, double *wr,
                                                          double *part, int *center_type)
{
    __shared__ double lo[256][3], hi[256][3];
    const int c = blockIdx.x / B, k = blockIdx.x % B, t = threadIdx.x;
    const int a0 = g.atom_off[c], n = g.atom_off[c + 1] - a0;
    const int m = (n + B - 1) / B;
    const int i0 = min(n, k * m), i1 = min(n, i0 + m);
    const bool wrap = g.wrap[c] != 0;
    const Cell &cl = g.cell[c];
    double l[3] = {__builtin_inf(), __builtin_inf(), __builtin_inf()};
    double h[3] = {-__builtin_inf(), -__builtin_inf(), -__builtin_inf()};
    for (int i = i0 + t; i < i1; i += 256) {
        center_type[a0 + i] = types[a0 + i];
        const size_t q = 3 * (size_t)(a0 + i);
        double p[3] = {pos[q], pos[q + 1], pos[q + 2]};
        if (wrap) {
            double f[3];
            dev_row_times(p, cl.inv, f);
            f[0] -= floor(f[0]);
            f[1] -= floor(f[1]);
            f[2] -= floor(f[2]);
            dev_row_times(f, cl.m, p);
        }
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            wr[q + d] = p[d];
            l[d] = p[d] < l[d] ? p[d] : l[d];
            h[d] = p[d] > h[d] ? p[d] : h[d];
        }
    }
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        lo[t][d] = l[d];
        hi[t][d] = h[d];
    }
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if (t < w)
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                lo[t][d] = lo[t + w][d] < lo[t][d] ? lo[t + w][d] : lo[t][d];
                hi[t][d] = hi[t + w][d] > hi[t][d] ? hi[t + w][d] : hi[t][d];
            }
        __syncthreads();
    }
    if (t < 3) {
        part[6 * (size_t)blockIdx.x + t] = lo[0][t];
        part[6 * (size_t)blockIdx.x + 3 + t] = hi[0][t];
    }
}

// flag k = image q of atom i of structure c lies in [lo - rc, hi + rc]
// (append_images, neighborhoods_base.h:72-80); k - flag_off[c] = q n_c + i.
__device__ __forceinline__ int image_flag_at(const Seg &g, const double *wr, long long k)
{
    const int c = seg_of(g.flag_off, g.nconf, k);
    const int a0 = g.atom_off[c], n = g.atom_off[c + 1] - a0;
    const long long kk = k - g.flag_off[c];
    const int q = (int)(kk / n), i = (int)(kk % n);
    const double *t = g.cand + 3 * (size_t)(g.cand_off[c] + q);
    const double *w = wr + 3 * (size_t)(a0 + i);
    const SegGeom &b = g.geo[c];
    const double p0 = w[0] + t[0], p1 = w[1] + t[1], p2 = w[2] + t[2];
    const bool out = p0 < b.lo[0] - b.cutoff || p1 < b.lo[1] - b.cutoff ||
                     p2 < b.lo[2] - b.cutoff || p0 > b.hi[0] + b.cutoff ||
                     p1 > b.hi[1] + b.cutoff || p2 > b.hi[2] + b.cutoff;
    return out ? 0 : 1;
}

__global__ void image_flag_kernel(Seg g, const double *wr, long long total, int *flags)
{
    const long long k = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (k < total)
        flags[k] = image_flag_at(g, wr, k);
}

// The flags of one scan tile per workgroup (the tiles of scan_tile_sums)
// and the tile's sum, so the scan needs two more launches, not three.
__global__ __launch_bounds__(kScanBlock) void image_flag_tiles_kernel(Seg g, const double *wr,
                                                                      long long total,
                                                                      int *flags, int *sums)
{
    __shared__ int buf[kScanBlock];
    const long long base = (long long)blockIdx.x * kScanTile;
    int s = 0;
    for (int k = 0; k < kScanItems; ++k) {
        const long long i = base + (long long)k * kScanBlock + threadIdx.x;
        if (i < total) {
            const int f = image_flag_at(g, wr, i);
            flags[i] = f;
            s += f;
        }
    }
    buf[threadIdx.x] = s;
    __syncthreads();
    for (int w = kScanBlock / 2; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w)
            buf[threadIdx.x] += buf[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        sums[blockIdx.x] = buf[0];
}

// points of each structure: its atoms and its images (the flags' exclusive
// scan at its end less at its start); entry nconf is 0, so an exclusive scan
// gives the point offsets and the point total
__device__ __forceinline__ int point_count_of(const Seg &g, const int *flags, const int *scan,
                                              int c)
{
    if (c >= g.nconf)
        return 0;
    const long long f0 = g.flag_off[c], f1 = g.flag_off[c + 1];
    const int nimg = f1 == f0 ? 0 : scan[f1 - 1] + flags[f1 - 1] - scan[f0];
    return g.atom_off[c + 1] - g.atom_off[c] + nimg;
}

__global__ void point_count_kernel(Seg g, const int *flags, const int *scan, int *count)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c <= g.nconf)
        count[c] = point_count_of(g, flags, scan, c);
}

// The point offsets [nconf + 1] in one workgroup (nconf + 1 <= 8 x 1,024):
// thread t counts the structures [t m, (t+1) m) and the counts are scanned.
constexpr int kOffsetsPerThread = 8;

__global__ __launch_bounds__(kScan1Threads) void point_offsets_kernel(Seg g, const int *flags,
                                                                     const int *scan,
                                                                     int *pt_off)
{
    __shared__ int wsum[kScan1Waves];
    const int n = g.nconf + 1;
    const int m = (n + kScan1Threads - 1) / kScan1Threads;
    const int c0 = threadIdx.x * m;
    int v[kOffsetsPerThread], sum = 0;
#pragma unroll
    for (int j = 0; j < kOffsetsPerThread; ++j) {
        v[j] = j < m && c0 + j < n ? point_count_of(g, flags, scan, c0 + j) : 0;
        sum += v[j];
    }
    int tot;
    int run = block_excl_scan(sum, wsum, tot);
#pragma unroll
    for (int j = 0; j < kOffsetsPerThread; ++j)
        if (j < m && c0 + j < n) {
            pt_off[c0 + j] = run;
            run += v[j];
        }
}

// Thread k: the original point pt_off[c] + i = atom a0 + i (k < ntot) and
// the image of flag k when it is set (k < nflags); the grid also clears the
// box counters [nz1], the list counters [nz2], *z64 and z3[0 .. 3] for the
// launches after it (fewer launches than separate fills).
__global__ void points_kernel(Seg g, const double *wr, int ntot, long long nflags,
                              const int *flags, const int *scan, double *pts, int *orig, int *z1,
                              int nz1, int *z2, int nz2, unsigned long long *z64, int *z3)
{
    const long long k = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long j = k; j < nz1; j += stride)
        z1[j] = 0;
    for (long long j = k; j < nz2; j += stride)
        z2[j] = 0;
    if (k == 0)
        *z64 = 0;
    if (k < 4)
        z3[k] = 0;
    if (k < ntot) {
        const int a = (int)k;
        const int c = seg_of(g.atom_off, g.nconf, a);
        const int q = g.pt_off[c] + (a - g.atom_off[c]);
        pts[3 * (size_t)q] = wr[3 * (size_t)a];
        pts[3 * (size_t)q + 1] = wr[3 * (size_t)a + 1];
        pts[3 * (size_t)q + 2] = wr[3 * (size_t)a + 2];
        orig[q] = a;
    }
    if (k < nflags && flags[k]) {
        const int c = seg_of(g.flag_off, g.nconf, k);
        const int a0 = g.atom_off[c], n = g.atom_off[c + 1] - a0;
        const long long kk = k - g.flag_off[c];
        const int q = (int)(kk / n), i = (int)(kk % n);
        const double *t = g.cand + 3 * (size_t)(g.cand_off[c] + q);
        const double *w = wr + 3 * (size_t)(a0 + i);
        const size_t o = (size_t)g.pt_off[c] + n + (scan[k] - scan[g.flag_off[c]]);
        pts[3 * o] = w[0] + t[0];
        pts[3 * o + 1] = w[1] + t[1];
        pts[3 * o + 2] = w[2] + t[2];
        orig[o] = a0 + i;
    }
}

// Box index (neighborhoods_base.h:179-224): ceil(tp * (bl - 2) / xd), originals
// clamped into [1, bl-2], images into [0, bl-1]; boxes numbered globally.
__global__ void box_index_kernel(Seg g, const double *pts, int *box, int *box_count)
{
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= g.pt_off[g.nconf])
        return;
    const int c = seg_of(g.pt_off, g.nconf, p);
    const int n = g.atom_off[c + 1] - g.atom_off[c];
    const bool original = p - g.pt_off[c] < n;
    const SegGeom &b = g.geo[c];
    int ix[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const double tp = pts[3 * (size_t)p + d] - b.lo[d];
        int v = (int)ceil(tp * (b.bl[d] - 2) / b.xd[d]);
        if (original) {
            if (v == 0)
                v = 1;
            if (v == b.bl[d] - 1)
                --v;
        } else {
            if (v < 0)
                v = 0;
            if (v >= b.bl[d])
                v = b.bl[d] - 1;
        }
        ix[d] = v;
    }
    const int gb = g.box_off[c] + (ix[0] * b.bl[1] + ix[1]) * b.bl[2] + ix[2];
    box[p] = gb;
    atomicAdd(&box_count[gb], 1);
}

// interior box w of structure c (walk order i, j, k from 1)
__device__ __forceinline__ int interior_box(const SegGeom &b, int w)
{
    const int nj = b.bl[1] - 2, nk = b.bl[2] - 2;
    const int i = w / (nj * nk) + 1, j = (w / nk) % nj + 1, k = w % nk + 1;
    return (i * b.bl[1] + j) * b.bl[2] + k;
}

// Originals in interior box w (walk order over the chunk), and its box
// within the structure (bl) and over the chunk (gb).
__device__ __forceinline__ int interior_originals(const Seg &g, const int *box_start,
                                                  const int *items, int w, int &c, int &bl,
                                                  int &gb)
{
    c = seg_of(g.int_off, g.nconf, w);
    bl = interior_box(g.geo[c], w - g.int_off[c]);
    gb = g.box_off[c] + bl;
    const int lim = g.pt_off[c] + (g.atom_off[c + 1] - g.atom_off[c]);
    int k = 0;
    for (int q = box_start[gb]; q < box_start[gb + 1]; ++q)
        k += items[q] < lim;
    return k;
}

// The originals of interior box w take the processing ranks prefix,
// prefix + 1, ... in box order.
__device__ __forceinline__ void rank_interior(const Seg &g, const int *box_start,
                                              const int *items, int c, int bl, int gb, int r,
                                              int *rank, int *centre_box)
{
    const int p0 = g.pt_off[c], lim = p0 + (g.atom_off[c + 1] - g.atom_off[c]);
    for (int q = box_start[gb]; q < box_start[gb + 1]; ++q) {
        const int p = items[q];
        if (p < lim) {
            const int a = g.atom_off[c] + (p - p0);
            rank[a] = r++;
            centre_box[a] = bl;
        }
    }
}

// Originals per interior box, in the lexicographic walk order of construct().
__global__ void interior_count_kernel(Seg g, const int *box_start, const int *items,
                                            int nint, int *count)
{
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= nint)
        return;
    int c, bl, gb;
    count[w] = interior_originals(g, box_start, items, w, c, bl, gb);
}

// Processing rank of every original: prefix over interior boxes + slot.
__global__ void centre_rank_kernel(Seg g, const int *box_start, const int *items,
                                         const int *prefix, int nint, int *rank, int *centre_box)
{
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= nint)
        return;
    int c, bl, gb;
    (void)interior_originals(g, box_start, items, w, c, bl, gb);
    rank_interior(g, box_start, items, c, bl, gb, prefix[w], rank, centre_box);
}

struct Construct {
    const double *pts;
    const int *orig, *box_start, *items, *types, *rank, *centre_box;
    int ntot;
    double cutoffsq;
    int cap;        // MODE 2: staged entries per list (list a at a cap)
    int *overflow;  // MODE 2: set when a list outgrows its bin
    int *mate;      // MODE 1, 2: staged index of each staged entry's mirror
};

// construct() (neighborhood.cpp:89-141) for one centre per wave.  MODE 0
// counts the entries of every list, MODE 1 writes them with their keys at
// the cursors (the counts' exclusive scan), MODE 2 counts and writes them in
// one pass into bins of cb.cap entries per list (cursors from zero; an entry
// past its bin is dropped and sets *cb.overflow, and the build is redone
// with MODE 0 and 1).
// The candidates of the 27 neighbour boxes, taken in the reference's
// traversal order (l1, l2, l3 from -1, then each box's points in order),
// are numbered 0 .. total-1 and the lanes test 64 consecutive numbers at a
// time; a lane finds its box by a branch-free binary search over the
// boxes' running sizes (held by lanes 0..26).  An accepted candidate's
// event number (its rank among the centre's accepted candidates in that
// order) is the count so far plus the accepted lanes below it, so the
// keys, and the lists they order, are those of the serial traversal.
// Ranks are global over a chunk, which keeps each structure's order.
// Wave-scope order of LDS accesses (a wave's LDS operations complete in
// issue order; this keeps the compiler from moving them across).
__device__ __forceinline__ void wave_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kAcceptBuf = 256;  // accepted candidates a wave buffers

template <int MODE>
__global__ __launch_bounds__(256) void construct_kernel(Seg g, Construct cb, int *cnt,
                                                        int *cursor, uint64_t *key, int *st_nbr,
                                                        int *st_ctr)
{
    const int lane = threadIdx.x & 63;
    const int a = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (a >= cb.ntot)
        return;  // uniform over the wave
    const int c = seg_of(g.atom_off, g.nconf, a);
    const SegGeom &geo = g.geo[c];
    const int bl1 = geo.bl[1], bl2 = geo.bl[2], box0 = g.box_off[c];
    const int indi = g.pt_off[c] + (a - g.atom_off[c]);  // the centre's point
    const int b = cb.centre_box[a];
    const int bi = b / (bl1 * bl2), bj = (b / bl2) % bl1, bk = b % bl2;
    const double pi0 = cb.pts[3 * (size_t)indi], pi1 = cb.pts[3 * (size_t)indi + 1],
                 pi2 = cb.pts[3 * (size_t)indi + 2];
    const uint64_t krank = (uint64_t)(unsigned)cb.rank[a] << 32;
    const uint64_t below = (1ull << lane) - 1;

    // lane k < 27: the first point of box k and the running size of boxes 0..k.
    // A box holds its points in ascending index: originals by atom, then
    // images.  The points up to the centre's own are originals of atoms up to
    // the centre, which never pass a <= oj (or indi != indj), so the box is
    // taken from the first point past the centre's; the accepted candidates,
    // their order and their event numbers are unchanged.
    int first = 0, size = 0;
    if (lane < 27) {
        const int nb = box0 + ((bi + lane / 9 - 1) * bl1 + (bj + (lane / 3) % 3 - 1)) * bl2 +
                       (bk + lane % 3 - 1);
        first = cb.box_start[nb];
        size = cb.box_start[nb + 1] - first;
        int lo = 0, hi = size;  // first item > indi
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (cb.items[first + mid] <= indi)
                lo = mid + 1;
            else
                hi = mid;
        }
        first += lo;
        size -= lo;
    }
    int incl = size;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o)
            incl += v;
    }
    const int excl = incl - size;
    const int total = __shfl(incl, 26);

    // MODE 1, 2: the accepted candidates (their points) wait in the wave's
    // LDS buffer and are written together, one lane per entry, so the
    // writes of a centre take about one pass instead of one per batch
    __shared__ int accepted[4][kAcceptBuf];
    int *abuf = accepted[threadIdx.x / 64];
    int nacc = 0;     // buffered (uniform)
    unsigned ev = 0;  // events before the buffer's first (uniform)
    auto flush = [&]() {
        wave_barrier();
        int own0 = 0;
        if (lane == 0)
            own0 = atomicAdd(&cursor[a], nacc);
        own0 = __shfl(own0, 0);
        for (int e = lane; e < nacc; e += 64) {
            const int indj = abuf[e];
            const int oj = cb.orig[indj];
            const uint64_t kv = krank | (ev + (unsigned)e);
            int64_t q = own0 + e;
            bool put = true;
            if (MODE == 2) {
                put = q < cb.cap;
                q += (int64_t)a * cb.cap;
            }
            const int64_t q1 = q;
            const bool put1 = put;
            if (put) {
                key[q] = kv;
                st_nbr[q] = indj;
                st_ctr[q] = indi;
            } else {
                *cb.overflow = 1;
            }
            if (a != oj) {
                q = atomicAdd(&cursor[oj], 1);
                if (MODE == 2) {
                    put = q < cb.cap;
                    q += (int64_t)oj * cb.cap;
                }
                if (put) {
                    key[q] = kv;
                    st_nbr[q] = indi;
                    st_ctr[q] = indj;
                    cb.mate[q] = (int)q1;
                } else {
                    *cb.overflow = 1;
                }
                if (put1)
                    cb.mate[q1] = (int)q;
            } else if (put1) {
                // an image of the centre is its own mirror: the reaction it
                // takes back from its own atom cancels the force it gave
                // (the opposite image is another entry of the same list)
                cb.mate[q1] = (int)q1;
            }
        }
        ev += (unsigned)nacc;
        nacc = 0;
        wave_barrier();
    };
    int own = 0;
    for (int tb = 0; tb < total; tb += 64) {
        const int f = tb + lane;
        // box of candidate number f: the number of boxes whose running size is <= f
        int k = 0;
#pragma unroll
        for (int step = 16; step >= 1; step >>= 1) {
            const int probe = k + step - 1;
            const int v = __shfl(incl, probe < 27 ? probe : 26);
            if (probe < 27 && v <= f)
                k += step;
        }
        const int kk = k < 27 ? k : 26;
        const int t = __shfl(first, kk) + (f - __shfl(excl, kk));
        bool ok = false;
        int oj = 0, indj = 0;
        if (f < total) {
            indj = cb.items[t];
            const double r0 = cb.pts[3 * (size_t)indj] - pi0;
            const double r1 = cb.pts[3 * (size_t)indj + 1] - pi1;
            const double r2 = cb.pts[3 * (size_t)indj + 2] - pi2;
            const double dijsq = r0 * r0 + r1 * r1 + r2 * r2;
            oj = cb.orig[indj];
            ok = dijsq < cb.cutoffsq && indi != indj && a <= oj;
        }
        const uint64_t acc = __ballot(ok);
        const int nok = __popcll(acc);
        if (MODE == 0) {
            if (ok && a != oj)
                atomicAdd(&cnt[oj], 1);
            own += nok;
        } else if (nok) {
            if (nacc + nok > kAcceptBuf)
                flush();
            if (ok)
                abuf[nacc + __popcll(acc & below)] = indj;
            nacc += nok;
        }
    }
    if (MODE == 0 && lane == 0)
        atomicAdd(&cnt[a], own);
    if (MODE != 0 && nacc)
        flush();
}


// Clears the list counters [n], the 64-bit entry total and the longest
// list before a counted build that follows a one-pass build.
__global__ void zero_counts_kernel(int *cnt, int n, unsigned long long *z64, int *largest)
{
    const int stride = gridDim.x * blockDim.x;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < n; k += stride)
        cnt[k] = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *z64 = 0;
        *largest = 0;
    }
}

// Budgets of one chunk: its atoms (set before the build), its image flags,
// boxes and interior boxes (the chunk ends early at the structure that would
// pass them), so every point, box and flag index fits in int32.
constexpr int kChunkAtoms = 1 << 21;
// Point buffers sized by the bound ntot + nflags up to this many points
// (24 MB of positions) without reading the image total back.
constexpr long long kPointBound = 1 << 20;
constexpr long long kChunkFlags = INT_MAX / 4;
constexpr long long kChunkBoxes = INT_MAX / 4;

template <class T>
const T *at(const DBuf &b, size_t off)
{
    return reinterpret_cast<const T *>(static_cast<const unsigned char *>(b.p) + off);
}

// Sizes the store for n atoms; clear zeroes the offsets (a builder that
// writes every offset passes false).
hipError_t init_store(NeighborStore &st, int n, hipStream_t s, bool clear = true)
{
    st.n = n;
    st.P = 0;
    st.has_mirror = false;
    hipError_t e = st.offsets.ensure(sizeof(int) * ((size_t)n + 1));
    if (e == hipSuccess)
        e = st.center_type.ensure(sizeof(int) * std::max(n, 1));
    if (e == hipSuccess && clear)
        e = hipMemsetAsync(st.offsets.p, 0, sizeof(int) * ((size_t)n + 1), s);
    return e;
}

// Host tables and arrays sent up in one copy through pinned memory: each
// part at a 16-byte aligned offset.  The parts are copied into the pinned
// buffer when sent, so the caller's arrays may change afterwards.
struct Upload {
    struct Part {
        const void *src;
        size_t off, bytes;
    };
    std::vector<Part> parts;
    size_t size = 0;
    template <class T>
    size_t add(const T *v, size_t n)
    {
        const size_t off = (size + 15) & ~size_t(15);
        parts.push_back({v, off, sizeof(T) * n});
        size = off + sizeof(T) * n;
        return off;
    }
    template <class T>
    size_t add(const std::vector<T> &v) { return add(v.data(), v.size()); }
    hipError_t send(HBuf &h, DBuf &d, hipStream_t s) const
    {
        const size_t n = std::max<size_t>(size, 16);
        hipError_t e = h.ensure(n);
        if (e == hipSuccess)
            e = d.ensure(n);
        if (e != hipSuccess)
            return e;
        for (const Part &q : parts)
            if (q.bytes)
                std::memcpy(h.as<unsigned char>() + q.off, q.src, q.bytes);
        return hipMemcpyAsync(d.p, h.p, n, hipMemcpyHostToDevice, s);
    }
};

// Entries that the bins of a one-pass build may hold (6.4 GB of staging).
constexpr long long kBinEntries = 1LL << 27;

// Atoms per chunk: kChunkAtoms, or less when MTPX_NEIGHBOR_CHUNK_ATOMS asks
// for it (a smaller peak of builder scratch for very large batches).
int chunk_atoms()
{
    const char *v = std::getenv("MTPX_NEIGHBOR_CHUNK_ATOMS");
    const long k = v ? std::strtol(v, nullptr, 10) : 0;
    return k > 0 && k < kChunkAtoms ? (int)k : kChunkAtoms;
}

// Structures [c0, c1) -- fewer when a budget ends the chunk; *done says how
// many -- into `out`, atoms numbered from the chunk's first atom.  Errors
// name the structure when `named`.
int build_chunk(int c0, int c1, const int *atom_offsets, const double *cells, const int *pbc,
                const double *pos, const int *types, double cutoff, hipStream_t s,
                NeighborStore &out, NeighborScratch &w, int *done, bool named, std::string &err)
{
    int nconf = c1 - c0;
    const int base = atom_offsets[c0];
    int ntot = atom_offsets[c1] - base;
    *done = nconf;
    DTRY(init_store(out, ntot, s, ntot == 0));
    if (ntot == 0) {
        DTRY(hipStreamSynchronize(s));
        return MTPX_OK;
    }
    auto fail_at = [&](int c, const std::string &what, int code) {
        err = named ? "structure " + std::to_string(c0 + c) + ": " + what : what;
        return code;
    };
    cells += 9 * (size_t)c0;
    pbc += 3 * (size_t)c0;
    pos += 3 * (size_t)base;
    types += base;
    // host tables: offsets, cells
    std::vector<int> atom_off((size_t)nconf + 1), wrapf((size_t)nconf);
    for (int c = 0; c <= nconf; ++c)
        atom_off[c] = atom_offsets[c0 + c] - base;
    std::vector<Cell> cl((size_t)nconf);
    for (int c = 0; c < nconf; ++c) {
        const int *pb = pbc + 3 * (size_t)c;
        wrapf[c] = pb[0] && pb[1] && pb[2];
        std::copy(cells + 9 * (size_t)c, cells + 9 * (size_t)c + 9, cl[c].m);
        if (wrapf[c] && atom_off[c + 1] > atom_off[c] && !cell_inverse(cl[c].m, cl[c].inv))
            return fail_at(c, "singular cell", MTPX_E_INVALID);
    }
    // scalars: [0] scan totals, [8..9] the 64-bit entry total, [10] bin
    // overflow, [11] longest list, [12] entry total of a one-pass build
    DTRY(w.scalars.ensure(sizeof(int) * 16));
    int *scal = w.scalars.as<int>();
    // the structure tables: one copy; the positions and species are staged
    // in pinned memory, which the wrap kernel reads in place (it copies the
    // species to the centre types, which the later kernels read)
    Upload head;
    const size_t o_atoms = head.add(atom_off), o_wrap = head.add(wrapf), o_cell = head.add(cl);
    DTRY(head.send(w.up_head, w.seg_head, s));
    const size_t pos_bytes = sizeof(double) * 3 * (size_t)ntot;
    DTRY(w.up_pos.ensure(pos_bytes + sizeof(int) * (size_t)ntot));
    std::memcpy(w.up_pos.p, pos, pos_bytes);
    std::memcpy(w.up_pos.as<unsigned char>() + pos_bytes, types, sizeof(int) * (size_t)ntot);
    void *hpos = nullptr;
    DTRY(hipHostGetDevicePointer(&hpos, w.up_pos.p, 0));
    const double *dpos = static_cast<const double *>(hpos);
    const int *dtypes_host = reinterpret_cast<const int *>(static_cast<unsigned char *>(hpos) +
                                                           pos_bytes);
    const int *dtypes = out.center_type.as<int>();  // device copy, written by the wrap kernel
    Seg g{};
    g.nconf = nconf;
    g.atom_off = at<int>(w.seg_head, o_atoms);
    g.wrap = at<int>(w.seg_head, o_wrap);
    g.cell = at<Cell>(w.seg_head, o_cell);
    DTRY(w.wrapped.ensure(sizeof(double) * 3 * (size_t)ntot));
    double *wr = w.wrapped.as<double>();
    // workgroups per structure: about 2048 atoms each, at most 64
    int nmax = 0;
    for (int c = 0; c < nconf; ++c)
        nmax = std::max(nmax, atom_off[c + 1] - atom_off[c]);
    const int B = std::min(64, std::max(1, (nmax + 2047) / 2048));
    const size_t npart = 6 * (size_t)nconf * B;
    DTRY(w.minmax.ensure(sizeof(double) * npart));
    DTRY(w.down.ensure(sizeof(double) * npart));
    hipLaunchKernelGGL(wrap_minmax_kernel, dim3((unsigned)((size_t)nconf * B)), dim3(256), 0, s, g,
                       dpos, dtypes_host, B, wr, w.minmax.as<double>(), out.center_type.as<int>());
    DTRY(hipMemcpyAsync(w.down.p, w.minmax.p, sizeof(double) * npart, hipMemcpyDeviceToHost, s));
    DTRY(hipStreamSynchronize(s));
    const double *part = w.down.as<double>();
    std::vector<double> mm(6 * (size_t)nconf);
    for (int c = 0; c < nconf; ++c)
        for (int d = 0; d < 3; ++d) {
            double l = part[6 * (size_t)c * B + d], h = part[6 * (size_t)c * B + 3 + d];
            for (int k = 1; k < B; ++k) {
                const double pl = part[6 * ((size_t)c * B + k) + d];
                const double ph = part[6 * ((size_t)c * B + k) + 3 + d];
                l = pl < l ? pl : l;
                h = ph > h ? ph : h;
            }
            mm[6 * (size_t)c + d] = l;
            mm[6 * (size_t)c + 3 + d] = h;
        }

    // per structure: AABB with the extent fix, image candidates, boxes
    std::vector<SegGeom> geo((size_t)nconf);
    std::vector<double> cand, cc;
    std::vector<int> cand_off(1, 0), box_off(1, 0), int_off(1, 0);
    std::vector<long long> flag_off(1, 0);
    for (int c = 0; c < nconf; ++c) {
        const int n = atom_off[c + 1] - atom_off[c];
        SegGeom &gc = geo[c];
        gc = SegGeom{};
        gc.cutoff = cutoff;
        long long nflag = 0;
        long long nbox = 0, nint = 0;
        if (n > 0) {
            for (int d = 0; d < 3; ++d) {
                gc.lo[d] = mm[6 * (size_t)c + d];
                gc.hi[d] = mm[6 * (size_t)c + 3 + d];
                if (gc.hi[d] - gc.lo[d] < cutoff)  // extent_impl, :140-143
                    gc.hi[d] = gc.lo[d] + cutoff;
            }
            int rc = image_candidates(cells + 9 * (size_t)c, pbc + 3 * (size_t)c, gc.lo, gc.hi,
                                      cutoff, cc, err);
            if (rc != MTPX_OK)
                return fail_at(c, err, rc);
            const long long ncand = (long long)cc.size() / 3;
            if (ncand * n > INT_MAX)
                return fail_at(c, "too many periodic image candidates", MTPX_E_CAPACITY);
            nflag = ncand * n;
            for (int d = 0; d < 3; ++d) {
                gc.xd[d] = gc.hi[d] - gc.lo[d];
                const double count = std::floor((gc.hi[d] - gc.lo[d]) / cutoff) + 2;
                if (!std::isfinite(count) || count >= 2e9)
                    return fail_at(c, "Neighbor spatial box count exceeds integer range",
                                   MTPX_E_RANGE);
                gc.bl[d] = (int)count;
                if (gc.bl[d] == 2)
                    gc.bl[d] = 3;
            }
            nbox = (long long)gc.bl[0] * gc.bl[1] * gc.bl[2];
            if (nbox > INT_MAX / 2)
                return fail_at(c, "Neighbor spatial box count exceeds integer range",
                               MTPX_E_RANGE);
            nint = (long long)(gc.bl[0] - 2) * (gc.bl[1] - 2) * (gc.bl[2] - 2);
            nbox += 1;  // the structure's closing counter
        }
        if (flag_off.back() + nflag > kChunkFlags || box_off.back() + nbox > kChunkBoxes ||
            int_off.back() + nint > kChunkBoxes) {
            if (c == 0)
                return fail_at(c, "too many periodic images or boxes for the neighbour builder",
                               MTPX_E_CAPACITY);
            nconf = c;  // the chunk ends before this structure
            break;
        }
        if (n > 0)
            cand.insert(cand.end(), cc.begin(), cc.end());
        cand_off.push_back((int)(cand.size() / 3));
        flag_off.push_back(flag_off.back() + nflag);
        box_off.push_back(box_off.back() + (int)nbox);
        int_off.push_back(int_off.back() + (int)nint);
    }
    if (nconf < c1 - c0) {
        *done = nconf;
        ntot = atom_off[nconf];
        out.n = ntot;
        g.nconf = nconf;
    }
    const long long nflags = flag_off.back();
    const int nboxes = box_off.back(), nint = int_off.back();
    Upload tabs;
    const size_t o_cand_off = tabs.add(cand_off), o_box_off = tabs.add(box_off),
                 o_int_off = tabs.add(int_off), o_flag_off = tabs.add(flag_off),
                 o_geo = tabs.add(geo.data(), (size_t)nconf), o_cand = tabs.add(cand);
    DTRY(tabs.send(w.up_tabs, w.seg_tabs, s));
    g.cand_off = at<int>(w.seg_tabs, o_cand_off);
    g.box_off = at<int>(w.seg_tabs, o_box_off);
    g.int_off = at<int>(w.seg_tabs, o_int_off);
    g.flag_off = at<long long>(w.seg_tabs, o_flag_off);
    g.geo = at<SegGeom>(w.seg_tabs, o_geo);
    g.cand = at<double>(w.seg_tabs, o_cand);

    // image flags, their scan, and the point offsets on the device.  The
    // point buffers and grids take the bound ntot + nflags when it is small
    // or already allocated (no host synchronisation for the image counts;
    // threads past the device total exit), else the total read back.
    long long npts_max = (long long)ntot + nflags;  // < 2^30 by the chunk budgets
    const bool bound = npts_max <= kPointBound || w.pts.bytes >= sizeof(double) * 3 * npts_max;
    DTRY(w.flags.ensure(sizeof(int) * (size_t)std::max<long long>(nflags, 1)));
    if (nflags > kScanLdsMax) {
        // flags with the scan's tile sums, then the two scan passes
        const long long ntiles = (nflags + kScanTile - 1) / kScanTile;
        DTRY(w.scan.ensure(sizeof(int) * (size_t)nflags));
        DTRY(w.box_cur.ensure(sizeof(int) * (size_t)ntiles));
        int *sums = w.box_cur.as<int>();
        hipLaunchKernelGGL(image_flag_tiles_kernel, dim3((unsigned)ntiles), dim3(kScanBlock), 0,
                           s, g, wr, nflags, w.flags.as<int>(), sums);
        hipLaunchKernelGGL(scan_sums, dim3(1), dim3(1024), 0, s, sums, (int)ntiles, scal);
        hipLaunchKernelGGL(scan_tiles, dim3((unsigned)ntiles), dim3(kScanBlock), 0, s,
                           w.flags.as<int>(), (int64_t)nflags, INT_MAX, sums, w.scan.as<int>(),
                           nullptr);
    } else if (nflags > 0) {
        DTRY(w.scan.ensure(sizeof(int) * (size_t)nflags));
        hipLaunchKernelGGL(image_flag_kernel, dim3(blocks(nflags, 256)), dim3(256), 0, s, g,
                           wr, nflags, w.flags.as<int>());
        DTRY(scan_exclusive(w.flags.as<int>(), nflags, w.scan.as<int>(), w.box_cur, scal, s));
    }
    DTRY(w.seg_imgs.ensure(sizeof(int) * ((size_t)nconf + 1)));
    DTRY(w.seg_pts.ensure(sizeof(int) * ((size_t)nconf + 1)));
    if (nconf + 1 <= kScan1Threads * kOffsetsPerThread) {
        hipLaunchKernelGGL(point_offsets_kernel, dim3(1), dim3(kScan1Threads), 0, s, g,
                           w.flags.as<int>(), w.scan.as<int>(), w.seg_pts.as<int>());
    } else {
        hipLaunchKernelGGL(point_count_kernel, dim3(blocks(nconf + 1, 256)), dim3(256), 0, s, g,
                           w.flags.as<int>(), w.scan.as<int>(), w.seg_imgs.as<int>());
        DTRY(scan_exclusive(w.seg_imgs.as<int>(), (int64_t)nconf + 1, w.seg_pts.as<int>(),
                            w.tmp, scal, s));
    }
    g.pt_off = w.seg_pts.as<int>();
    const int *npts = g.pt_off + nconf;  // device
    if (!bound) {
        DTRY(hipMemcpyAsync(w.down.p, npts, sizeof(int), hipMemcpyDeviceToHost, s));
        DTRY(hipStreamSynchronize(s));
        npts_max = *w.down.as<int>();
    }
    DTRY(w.pts.ensure(sizeof(double) * 3 * (size_t)npts_max));
    DTRY(w.orig.ensure(sizeof(int) * (size_t)npts_max));
    DTRY(w.cnt.ensure(sizeof(int) * ((size_t)nboxes + 1)));
    DTRY(w.cursor.ensure(sizeof(int) * ((size_t)ntot + 1)));
    int *box_count = w.cnt.as<int>();
    int *cnt = w.cursor.as<int>();
    unsigned long long *total64 = reinterpret_cast<unsigned long long *>(scal + 8);
    hipLaunchKernelGGL(points_kernel, dim3(blocks(std::max<long long>(ntot, nflags), 256)),
                       dim3(256), 0, s, g, wr, ntot, nflags, w.flags.as<int>(), w.scan.as<int>(),
                       w.pts.as<double>(), w.orig.as<int>(), box_count, nboxes + 1, cnt, ntot + 1,
                       total64, scal + 10);

    // boxes: counts, starts, stable placement
    DTRY(w.box.ensure(sizeof(int) * (size_t)npts_max));
    DTRY(w.box_start.ensure(sizeof(int) * ((size_t)nboxes + 1)));
    DTRY(w.box_cur.ensure(sizeof(int) * ((size_t)nboxes + 1)));
    DTRY(w.box_items.ensure(sizeof(int) * (size_t)npts_max));
    hipLaunchKernelGGL(box_index_kernel, dim3(blocks(npts_max, 256)), dim3(256), 0, s, g,
                       w.pts.as<double>(), w.box.as<int>(), box_count);
    DTRY(scan_exclusive(box_count, (int64_t)nboxes + 1, w.box_start.as<int>(), w.tmp,
                        w.scalars.as<int>(), s, w.box_cur.as<int>()));
    // the image flags are dead after points_kernel: their buffer takes
    // the unsorted placement (growing it waits for the queued work)
    DTRY(w.flags.ensure(sizeof(int) * (size_t)std::max<long long>(npts_max, 1)));
    int *unsorted = w.flags.as<int>();
    hipLaunchKernelGGL(box_place_kernel, dim3(blocks(npts_max, 256)), dim3(256), 0, s,
                       w.box.as<int>(), npts, w.box_cur.as<int>(), unsorted);
    hipLaunchKernelGGL(box_rank_kernel, dim3(blocks(npts_max, 256)), dim3(256), 0, s,
                       w.box.as<int>(), w.box_start.as<int>(), npts, unsorted,
                       w.box_items.as<int>());

    // processing ranks of the centres
    DTRY(w.rank.ensure(sizeof(int) * (2 * (size_t)ntot + 2 * ((size_t)nint + 1))));
    int *rank = w.rank.as<int>();
    int *centre_box = rank + ntot;
    int *icount = centre_box + ntot;
    int *iprefix = icount + (nint + 1);
    if (nint > 0) {
        hipLaunchKernelGGL(interior_count_kernel, dim3(blocks(nint, 256)), dim3(256), 0, s,
                           g, w.box_start.as<int>(), w.box_items.as<int>(), nint, icount);
        DTRY(scan_exclusive(icount, nint, iprefix, w.tmp, scal, s));
        hipLaunchKernelGGL(centre_rank_kernel, dim3(blocks(nint, 256)), dim3(256), 0, s, g,
                           w.box_start.as<int>(), w.box_items.as<int>(), iprefix, nint, rank,
                           centre_box);
    }

    // construct: count, offsets, fill, rank within lists
    Construct cb;
    cb.pts = w.pts.as<double>();
    cb.orig = w.orig.as<int>();
    cb.box_start = w.box_start.as<int>();
    cb.items = w.box_items.as<int>();
    cb.types = dtypes;
    cb.rank = rank;
    cb.centre_box = centre_box;
    cb.ntot = ntot;
    cb.cutoffsq = cutoff * cutoff;
    cb.cap = 0;
    cb.overflow = scal + 10;
    cb.mate = nullptr;  // set once the staging is sized
    DTRY(w.down.ensure(sizeof(int) * 16));
    int *down = w.down.as<int>();
    auto ensure_entries = [&](size_t n) -> hipError_t {
        const size_t nz = std::max<size_t>(n, 1);
        for (DBuf *b : {&out.idx, &out.type, &out.mirror, &w.st_nbr, &w.st_ctr, &w.st_mate,
                        &w.st_final})
            if (hipError_t e = b->ensure(sizeof(int) * nz))
                return e;
        for (DBuf *b : {&out.x, &out.y, &out.z, &out.d})
            if (hipError_t e = b->ensure(sizeof(double) * nz))
                return e;
        return w.key.ensure(sizeof(uint64_t) * nz);
    };
    auto rank_lists = [&](int cap, const int *overflow) {
        hipLaunchKernelGGL(list_rank_kernel, dim3((ntot + 3) / 4), dim3(256), 0, s,
                           out.offsets.as<int>(), ntot, cap, overflow, w.key.as<uint64_t>(),
                           w.st_nbr.as<int>(), w.st_ctr.as<int>(), w.pts.as<double>(),
                           w.orig.as<int>(), dtypes, out.idx.as<int>(), out.type.as<int>(),
                           out.x.as<double>(), out.y.as<double>(), out.z.as<double>(),
                           out.d.as<double>(), w.st_final.as<int>());
        hipLaunchKernelGGL(mirror_kernel, dim3((ntot + 3) / 4), dim3(256), 0, s,
                           out.offsets.as<int>(), ntot, cap, overflow, w.st_mate.as<int>(),
                           w.st_final.as<int>(), out.mirror.as<int>());
    };

    // One pass into bins sized from the previous counted build: the entry
    // total comes back with the final synchronisation.  A list that outgrows
    // its bin sends the chunk through the counted build below.
    const long long cap = w.bin_cap;
    if (cap > 0 && (long long)ntot * cap <= kBinEntries) {
        cb.cap = (int)cap;
        DTRY(ensure_entries((size_t)ntot * cap));
        cb.mate = w.st_mate.as<int>();
        hipLaunchKernelGGL(construct_kernel<2>, dim3((ntot + 3) / 4), dim3(256), 0, s, g, cb,
                           nullptr, cnt, w.key.as<uint64_t>(), w.st_nbr.as<int>(),
                           w.st_ctr.as<int>());
        DTRY(scan_exclusive(cnt, (int64_t)ntot + 1, out.offsets.as<int>(), w.tmp, scal + 12, s,
                            nullptr, (int)cap));
        rank_lists((int)cap, scal + 10);
        DTRY(hipMemcpyAsync(down, scal + 10, sizeof(int) * 3, hipMemcpyDeviceToHost, s));
        DTRY(hipGetLastError());
        DTRY(hipStreamSynchronize(s));
        if (down[0] == 0) {
            out.P = down[2];
            out.has_mirror = true;
            return MTPX_OK;
        }
        cb.cap = 0;
        hipLaunchKernelGGL(zero_counts_kernel, dim3(blocks(ntot + 1, 256)), dim3(256), 0, s, cnt,
                           ntot + 1, total64, scal + 11);
    }

    // counted build: count, offsets, fill at the cursors, rank within lists
    hipLaunchKernelGGL(construct_kernel<0>, dim3((ntot + 3) / 4), dim3(256), 0, s, g, cb,
                       cnt, nullptr, nullptr, nullptr, nullptr);
    hipLaunchKernelGGL(sum64_kernel, dim3(std::min<unsigned>(blocks(ntot, 256), 1024)), dim3(256),
                       0, s, cnt, (int64_t)ntot, total64, scal + 11);
    // the offsets, and the same values over the counts as the fill cursors
    DTRY(scan_exclusive(cnt, (int64_t)ntot + 1, out.offsets.as<int>(), w.tmp, scal, s, cnt));
    DTRY(hipMemcpyAsync(down, scal + 8, sizeof(int) * 4, hipMemcpyDeviceToHost, s));
    DTRY(hipStreamSynchronize(s));
    unsigned long long P64 = 0;
    std::memcpy(&P64, down, sizeof P64);
    const int longest = down[3];
    if (P64 > (unsigned long long)INT32_MAX) {
        err = named ? "batch has more than 2^31 - 1 neighbour entries"
                    : "structure has more than 2^31 - 1 neighbour entries";
        return MTPX_E_CAPACITY;
    }
    // bins for the next build of this size: the longest list and a margin
    w.bin_cap = (long long)longest + longest / 4 + 8;
    const int64_t P = (int64_t)P64;
    out.P = P;
    DTRY(ensure_entries((size_t)P));
    out.has_mirror = true;
    if (P == 0)
        return MTPX_OK;
    cb.mate = w.st_mate.as<int>();
    hipLaunchKernelGGL(construct_kernel<1>, dim3((ntot + 3) / 4), dim3(256), 0, s, g, cb,
                       nullptr, cnt, w.key.as<uint64_t>(), w.st_nbr.as<int>(),
                       w.st_ctr.as<int>());
    rank_lists(0, nullptr);
    DTRY(hipGetLastError());
    DTRY(hipStreamSynchronize(s));
    return MTPX_OK;
}

// Appends a chunk's lists (atoms from a0, entries from p0) to `out`.
int append_store(NeighborStore &out, const NeighborStore &ch, int a0, int64_t p0, hipStream_t s,
                 std::string &err)
{
    const int nc = ch.n;
    const int64_t Pc = ch.P;
    const size_t keep = (size_t)p0, need = (size_t)std::max<int64_t>(p0 + Pc, 1);
    DTRY(grow_keep(out.idx, sizeof(int) * need, sizeof(int) * keep, s));
    DTRY(grow_keep(out.type, sizeof(int) * need, sizeof(int) * keep, s));
    DTRY(grow_keep(out.x, sizeof(double) * need, sizeof(double) * keep, s));
    DTRY(grow_keep(out.y, sizeof(double) * need, sizeof(double) * keep, s));
    DTRY(grow_keep(out.z, sizeof(double) * need, sizeof(double) * keep, s));
    DTRY(grow_keep(out.d, sizeof(double) * need, sizeof(double) * keep, s));
    DTRY(grow_keep(out.mirror, sizeof(int) * need, sizeof(int) * keep, s));
    if (nc > 0)
        DTRY(hipMemcpyAsync(out.center_type.as<int>() + a0, ch.center_type.p, sizeof(int) * nc,
                            hipMemcpyDeviceToDevice, s));
    if (Pc > 0) {
        DTRY(hipMemcpyAsync(out.type.as<int>() + p0, ch.type.p, sizeof(int) * Pc,
                            hipMemcpyDeviceToDevice, s));
        DTRY(hipMemcpyAsync(out.x.as<double>() + p0, ch.x.p, sizeof(double) * Pc,
                            hipMemcpyDeviceToDevice, s));
        DTRY(hipMemcpyAsync(out.y.as<double>() + p0, ch.y.p, sizeof(double) * Pc,
                            hipMemcpyDeviceToDevice, s));
        DTRY(hipMemcpyAsync(out.z.as<double>() + p0, ch.z.p, sizeof(double) * Pc,
                            hipMemcpyDeviceToDevice, s));
        DTRY(hipMemcpyAsync(out.d.as<double>() + p0, ch.d.p, sizeof(double) * Pc,
                            hipMemcpyDeviceToDevice, s));
    }
    const int64_t work = std::max<int64_t>(Pc, (int64_t)nc + 1);
    hipLaunchKernelGGL(append_lists_kernel, dim3(blocks(work, 256)), dim3(256), 0, s,
                       ch.offsets.as<int>(), ch.idx.as<int>(), ch.mirror.as<int>(), nc, Pc, a0,
                       p0, out.offsets.as<int>(), out.idx.as<int>(), out.mirror.as<int>());
    DTRY(hipGetLastError());
    DTRY(hipStreamSynchronize(s));
    return MTPX_OK;
}

}  // namespace

int build_neighbors_gpu(const double cell[9], const int pbc[3], int n, const double *pos,
                        const int *types, double cutoff, hipStream_t s, NeighborStore &out,
                        NeighborScratch &w, std::string &err)
{
    const int off[2] = {0, n};
    int done = 0;
    return build_chunk(0, 1, off, cell, pbc, pos, types, cutoff, s, out, w, &done, false, err);
}

// A batch goes through build_chunk in one piece when it fits the budgets
// (the usual case: then the chunk is the batch's store), else chunk by chunk
// into `tmp`, appended in order.
int build_neighbors_batch_gpu(int nconf, const int *atom_offsets, const double *cells,
                              const int *pbc, const double *pos, const int *types, double cutoff,
                              hipStream_t s, NeighborStore &out, NeighborStore &tmp,
                              NeighborScratch &w, std::string &err)
{
    const int ntot = atom_offsets[nconf];
    int64_t P = 0;
    bool in_out = false;  // out holds the first chunk itself
    const int limit = chunk_atoms();
    for (int c0 = 0; c0 < nconf || (nconf == 0 && c0 == 0);) {
        int c1 = std::min(c0 + 1, nconf);
        while (c1 < nconf && atom_offsets[c1 + 1] - atom_offsets[c0] <= limit)
            ++c1;
        const bool whole = c0 == 0 && c1 == nconf;
        NeighborStore &dst = whole ? out : tmp;
        int done = 0;
        int rc = build_chunk(c0, c1, atom_offsets, cells, pbc, pos, types, cutoff, s, dst, w,
                             &done, true, err);
        if (rc != MTPX_OK)
            return rc;
        if (whole && done == c1 - c0)
            return MTPX_OK;
        if (whole) {  // a budget ended the first chunk: it moves to tmp
            std::swap(out, tmp);
            in_out = false;
        }
        if (c0 == 0 && !in_out) {
            DTRY(init_store(out, ntot, s));
            in_out = true;
        }
        if ((int64_t)P + tmp.P > INT32_MAX) {
            err = "batch has more than 2^31 - 1 neighbour entries";
            return MTPX_E_CAPACITY;
        }
        rc = append_store(out, tmp, atom_offsets[c0], P, s, err);
        if (rc != MTPX_OK)
            return rc;
        P += tmp.P;
        out.P = P;
        c0 += done;
    }
    out.has_mirror = true;  // every chunk's entries came with their mirrors
    return MTPX_OK;
}

}  // namespace mtpx
