// Device neighbour-list builder reproducing the reference BOXED builder
// (base/neighborhoods_base.h:31-266, base/neighborhood.cpp:77-146) bit for
// bit.  Compiled with -ffp-contract=off; every floating-point expression
// keeps the reference's operation order, and fp64 division and sqrt are
// IEEE correctly rounded on gfx950.
//
// Pipeline (all on one stream):
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
#include <thread>
#include <cmath>

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

// load_positions (neighborhoods_base.h:113-127)
__global__ void wrap_kernel(const double *pos, int n, Cell c, int wrap, double *pts)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    double p[3] = {pos[3 * i], pos[3 * i + 1], pos[3 * i + 2]};
    if (wrap) {
        double f[3];
        dev_row_times(p, c.inv, f);
        f[0] -= floor(f[0]);
        f[1] -= floor(f[1]);
        f[2] -= floor(f[2]);
        dev_row_times(f, c.m, p);
    }
    pts[3 * i] = p[0];
    pts[3 * i + 1] = p[1];
    pts[3 * i + 2] = p[2];
}

// Component-wise min/max over the originals; one workgroup, ordered.
__global__ __launch_bounds__(256) void minmax_kernel(const double *pts, int n, double *out6)
{
    __shared__ double lo[256][3], hi[256][3];
    const int t = threadIdx.x;
    double l[3] = {pts[0], pts[1], pts[2]}, h[3] = {pts[0], pts[1], pts[2]};
    for (int i = t; i < n; i += 256)
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            const double v = pts[3 * i + d];
            l[d] = v < l[d] ? v : l[d];
            h[d] = v > h[d] ? v : h[d];
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
        out6[t] = lo[0][t];
        out6[3 + t] = hi[0][t];
    }
}

struct Bounds {
    double lo[3], hi[3], cutoff;
};

// flag[c*n + i] = image c of atom i lies in [lo - rc, hi + rc] (append_images, :72-80)
__global__ void image_flag_kernel(const double *pts, int n, const double *cand, int ncand,
                                  Bounds b, int *flags)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= (int64_t)n * ncand)
        return;
    const int c = (int)(k / n), i = (int)(k % n);
    const double p0 = pts[3 * i] + cand[3 * c], p1 = pts[3 * i + 1] + cand[3 * c + 1],
                 p2 = pts[3 * i + 2] + cand[3 * c + 2];
    const bool out = p0 < b.lo[0] - b.cutoff || p1 < b.lo[1] - b.cutoff ||
                     p2 < b.lo[2] - b.cutoff || p0 > b.hi[0] + b.cutoff ||
                     p1 > b.hi[1] + b.cutoff || p2 > b.hi[2] + b.cutoff;
    flags[k] = out ? 0 : 1;
}

__global__ void image_write_kernel(const double *cand, int n, int64_t total, const int *flags,
                                   const int *scan, double *pts, int *orig)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= total || !flags[k])
        return;
    const int c = (int)(k / n), i = (int)(k % n);
    const int64_t q = n + scan[k];
    pts[3 * q] = pts[3 * i] + cand[3 * c];
    pts[3 * q + 1] = pts[3 * i + 1] + cand[3 * c + 1];
    pts[3 * q + 2] = pts[3 * i + 2] + cand[3 * c + 2];
    orig[q] = i;
}

__global__ void orig_identity_kernel(int *orig, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        orig[i] = i;
}

struct BoxGeom {
    double lo[3], xd[3];
    int bl[3];
};

// Box index (neighborhoods_base.h:179-224): ceil(tp * (bl - 2) / xd), originals
// clamped into [1, bl-2], images into [0, bl-1].
__global__ void box_index_kernel(const double *pts, int n, int npts, BoxGeom g, int *box,
                                 int *box_count)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npts)
        return;
    int ix[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const double tp = pts[3 * i + d] - g.lo[d];
        int v = (int)ceil(tp * (g.bl[d] - 2) / g.xd[d]);
        if (i < n) {
            if (v == 0)
                v = 1;
            if (v == g.bl[d] - 1)
                --v;
        } else {
            if (v < 0)
                v = 0;
            if (v >= g.bl[d])
                v = g.bl[d] - 1;
        }
        ix[d] = v;
    }
    const int b = (ix[0] * g.bl[1] + ix[1]) * g.bl[2] + ix[2];
    box[i] = b;
    atomicAdd(&box_count[b], 1);
}

// Place each point at box_start[b] + (number of points of box b with a smaller
// index): the first pass drops points in any order, the second ranks them.
__global__ void box_place_kernel(const int *box, int npts, int *box_cur, int *items)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npts)
        return;
    const int q = atomicAdd(&box_cur[box[i]], 1);
    items[q] = i;
}

// One thread per point: its slot in its box is the number of the box's
// points with a smaller index (a box of a small cell can hold every point).
__global__ void box_rank_kernel(const int *box, const int *box_start, int npts,
                                const int *unsorted, int *items)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npts)
        return;
    const int b = box[i];
    const int s = box_start[b], e = box_start[b + 1];
    int r = 0;
    for (int u = s; u < e; ++u)
        r += unsorted[u] < i;
    items[s + r] = i;
}

// Originals per interior box, in the lexicographic walk order of construct().
__global__ void interior_count_kernel(const int *box_start, const int *items, BoxGeom g, int n,
                                      int *count)
{
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    const int ni = (g.bl[0] - 2), nj = (g.bl[1] - 2), nk = (g.bl[2] - 2);
    if (w >= ni * nj * nk)
        return;
    const int i = w / (nj * nk) + 1, j = (w / nk) % nj + 1, k = w % nk + 1;
    const int b = (i * g.bl[1] + j) * g.bl[2] + k;
    int c = 0;
    for (int q = box_start[b]; q < box_start[b + 1]; ++q)
        c += items[q] < n;
    count[w] = c;
}

// Processing rank of every original: prefix over interior boxes + slot.
__global__ void centre_rank_kernel(const int *box_start, const int *items, const int *prefix,
                                   BoxGeom g, int n, int *rank, int *centre_box)
{
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    const int ni = (g.bl[0] - 2), nj = (g.bl[1] - 2), nk = (g.bl[2] - 2);
    if (w >= ni * nj * nk)
        return;
    const int i = w / (nj * nk) + 1, j = (w / nk) % nj + 1, k = w % nk + 1;
    const int b = (i * g.bl[1] + j) * g.bl[2] + k;
    int r = prefix[w];
    for (int q = box_start[b]; q < box_start[b + 1]; ++q) {
        const int p = items[q];
        if (p < n) {
            rank[p] = r++;
            centre_box[p] = b;
        }
    }
}

struct Construct {
    const double *pts;
    const int *orig, *box_start, *items, *types, *rank, *centre_box;
    int n;
    int bl1, bl2;
    double cutoffsq;
};

// construct() (neighborhood.cpp:89-141) for one centre per wave.  MODE 0
// counts the entries of every list, MODE 1 writes them with their keys.
// The lanes test 64 candidates of a box at a time; an accepted candidate's
// event number (its rank among the centre's accepted candidates in the
// reference's traversal order) is the count so far plus the accepted lanes
// below it, so the keys, and the lists they order, are those of the serial
// traversal.
template <int MODE>
__global__ __launch_bounds__(256) void construct_kernel(Construct c, int *cnt, int *cursor,
                                                        uint64_t *key, int *st_idx, int *st_type,
                                                        double *st_vec, double *st_d)
{
    const int lane = threadIdx.x & 63;
    const int indi = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (indi >= c.n)
        return;  // uniform over the wave
    const int b = c.centre_box[indi];
    const int bi = b / (c.bl1 * c.bl2), bj = (b / c.bl2) % c.bl1, bk = b % c.bl2;
    const double pi0 = c.pts[3 * indi], pi1 = c.pts[3 * indi + 1], pi2 = c.pts[3 * indi + 2];
    const uint64_t krank = (uint64_t)(unsigned)c.rank[indi] << 32;
    const uint64_t below = (1ull << lane) - 1;
    unsigned ev = 0;
    int own = 0;
    for (int l1 = -1; l1 <= 1; l1++)
        for (int l2 = -1; l2 <= 1; l2++)
            for (int l3 = -1; l3 <= 1; l3++) {
                const int nb = ((bi + l1) * c.bl1 + (bj + l2)) * c.bl2 + (bk + l3);
                const int t0 = c.box_start[nb], t1 = c.box_start[nb + 1];
                for (int tb = t0; tb < t1; tb += 64) {
                    const int t = tb + lane;
                    bool ok = false;
                    double r0 = 0.0, r1 = 0.0, r2 = 0.0, dijsq = 0.0;
                    int oj = 0;
                    if (t < t1) {
                        const int indj = c.items[t];
                        r0 = c.pts[3 * indj] - pi0;
                        r1 = c.pts[3 * indj + 1] - pi1;
                        r2 = c.pts[3 * indj + 2] - pi2;
                        dijsq = r0 * r0 + r1 * r1 + r2 * r2;
                        oj = c.orig[indj];
                        ok = dijsq < c.cutoffsq && indi != indj && indi <= oj;
                    }
                    const uint64_t acc = __ballot(ok);
                    if (ok) {
                        if (MODE == 0) {
                            if (indi != oj)
                                atomicAdd(&cnt[oj], 1);
                        } else {
                            const double dij = sqrt(dijsq);
                            const uint64_t k = krank | (ev + (unsigned)__popcll(acc & below));
                            int q = atomicAdd(&cursor[indi], 1);
                            key[q] = k;
                            st_idx[q] = oj;
                            st_type[q] = c.types[oj];
                            st_vec[3 * (int64_t)q] = r0;
                            st_vec[3 * (int64_t)q + 1] = r1;
                            st_vec[3 * (int64_t)q + 2] = r2;
                            st_d[q] = dij;
                            if (indi != oj) {
                                q = atomicAdd(&cursor[oj], 1);
                                key[q] = k;
                                st_idx[q] = indi;
                                st_type[q] = c.types[indi];
                                st_vec[3 * (int64_t)q] = -r0;
                                st_vec[3 * (int64_t)q + 1] = -r1;
                                st_vec[3 * (int64_t)q + 2] = -r2;
                                st_d[q] = dij;
                            }
                        }
                    }
                    ev += (unsigned)__popcll(acc);
                    own += __popcll(acc);
                }
            }
    if (MODE == 0 && lane == 0)
        atomicAdd(&cnt[indi], own);
}

// Rank every staged entry within its list by key and write it to its final
// slot (SoA).  One thread per entry.
__global__ void list_rank_kernel(const int *offsets, const int *entry_list, int64_t P,
                                 const uint64_t *key, const int *st_idx, const int *st_type,
                                 const double *st_vec, const double *st_d, int *idx, int *type,
                                 double *x, double *y, double *z, double *d)
{
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= P)
        return;
    const int l = entry_list[q];
    const int s = offsets[l], e = offsets[l + 1];
    const uint64_t k = key[q];
    int r = 0;
    for (int u = s; u < e; ++u)
        r += key[u] < k;
    const int64_t o = s + r;
    idx[o] = st_idx[q];
    type[o] = st_type[q];
    x[o] = st_vec[3 * q];
    y[o] = st_vec[3 * q + 1];
    z[o] = st_vec[3 * q + 2];
    d[o] = st_d[q];
}

__global__ void entry_list_kernel(const int *offsets, int n, int *entry_list)
{
    const int i = blockIdx.x;
    for (int q = offsets[i] + threadIdx.x; q < offsets[i + 1]; q += blockDim.x)
        entry_list[q] = i;
}

__global__ void gather_types_kernel(const int *types, int n, int *center_type)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        center_type[i] = types[i];
}

// ---- exclusive scan of int32 (three passes) ---------------------------
constexpr int kScanBlock = 256, kScanItems = 8, kScanTile = kScanBlock * kScanItems;

__global__ __launch_bounds__(kScanBlock) void scan_tile_sums(const int *in, int64_t n, int *sums)
{
    __shared__ int buf[kScanBlock];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int s = 0;
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + (int64_t)k * kScanBlock + threadIdx.x;
        if (i < n)
            s += in[i];
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

__global__ __launch_bounds__(kScanBlock) void scan_tiles(const int *in, int64_t n,
                                                          const int *sums, int *out)
{
    __shared__ int buf[kScanBlock];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int v[kScanItems];
    int s = 0;
    for (int k = 0; k < kScanItems; ++k) {
        v[k] = base + k < n ? in[base + k] : 0;
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
        if (base + k < n)
            out[base + k] = run;
        run += v[k];
    }
}

// 64-bit sum of n non-negative ints into *total (zeroed by the caller): the
// list-length total, checked against the int32 entry indices before any
// offset is trusted.
__global__ __launch_bounds__(256) void sum64_kernel(const int *in, int64_t n,
                                                    unsigned long long *total)
{
    __shared__ unsigned long long buf[256];
    unsigned long long s = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        s += (unsigned)in[i];
    buf[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w)
            buf[threadIdx.x] += buf[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        atomicAdd(total, buf[0]);
}

// Exclusive scan; *total receives the sum (device), returns the error.
hipError_t scan_exclusive(const int *in, int64_t n, int *out, DBuf &tmp, int *total,
                          hipStream_t s)
{
    const int64_t ntiles = std::max<int64_t>(1, (n + kScanTile - 1) / kScanTile);
    hipError_t e = tmp.ensure(sizeof(int) * (size_t)ntiles);
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(scan_tile_sums, dim3((unsigned)ntiles), dim3(kScanBlock), 0, s, in, n,
                       tmp.as<int>());
    hipLaunchKernelGGL(scan_sums, dim3(1), dim3(1024), 0, s, tmp.as<int>(), (int)ntiles, total);
    hipLaunchKernelGGL(scan_tiles, dim3((unsigned)ntiles), dim3(kScanBlock), 0, s, in, n,
                       tmp.as<int>(), out);
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

int build_neighbors_gpu(const double cell[9], const int pbc[3], int n, const double *pos,
                        const int *types, double cutoff, hipStream_t s, NeighborStore &out,
                        NeighborScratch &w, std::string &err)
{
    out.n = n;
    out.P = 0;
    DTRY(out.offsets.ensure(sizeof(int) * ((size_t)n + 1)));
    DTRY(hipMemsetAsync(out.offsets.p, 0, sizeof(int) * ((size_t)n + 1), s));
    DTRY(out.center_type.ensure(sizeof(int) * std::max(n, 1)));
    if (n == 0) {
        DTRY(hipStreamSynchronize(s));
        return MTPX_OK;
    }
    const bool fully = pbc[0] && pbc[1] && pbc[2];
    Cell c;
    std::copy(cell, cell + 9, c.m);
    if (fully && !cell_inverse(cell, c.inv)) {
        err = "singular cell";
        return MTPX_E_INVALID;
    }
    DTRY(w.pos.ensure(sizeof(double) * 3 * n));
    DTRY(w.types.ensure(sizeof(int) * n));
    DTRY(w.minmax.ensure(sizeof(double) * 8));
    DTRY(w.scalars.ensure(sizeof(int) * 16));
    DTRY(hipMemcpyAsync(w.pos.p, pos, sizeof(double) * 3 * n, hipMemcpyHostToDevice, s));
    DTRY(hipMemcpyAsync(w.types.p, types, sizeof(int) * n, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(gather_types_kernel, dim3(blocks(n, 256)), dim3(256), 0, s,
                       w.types.as<int>(), n, out.center_type.as<int>());
    // the points buffer is sized after the image count is known; wrap into scratch first
    DTRY(w.tmp.ensure(sizeof(double) * 3 * n));
    double *wrapped = w.tmp.as<double>();
    hipLaunchKernelGGL(wrap_kernel, dim3(blocks(n, 256)), dim3(256), 0, s, w.pos.as<double>(), n,
                       c, fully ? 1 : 0, wrapped);
    hipLaunchKernelGGL(minmax_kernel, dim3(1), dim3(256), 0, s, wrapped, n, w.minmax.as<double>());
    double mm[6];
    DTRY(hipMemcpyAsync(mm, w.minmax.p, sizeof mm, hipMemcpyDeviceToHost, s));
    DTRY(hipStreamSynchronize(s));
    Bounds bd;
    for (int d = 0; d < 3; ++d) {
        bd.lo[d] = mm[d];
        bd.hi[d] = mm[3 + d];
        if (bd.hi[d] - bd.lo[d] < cutoff)  // extent_impl, :140-143
            bd.hi[d] = bd.lo[d] + cutoff;
    }
    bd.cutoff = cutoff;

    std::vector<double> cand;
    int rc = image_candidates(cell, pbc, bd.lo, bd.hi, cutoff, cand, err);
    if (rc != MTPX_OK)
        return rc;
    const int ncand = (int)cand.size() / 3;
    int nimg = 0;
    const int64_t total = (int64_t)ncand * n;
    if (total > INT_MAX) {
        err = "too many periodic image candidates";
        return MTPX_E_CAPACITY;
    }
    if (ncand > 0) {
        DTRY(w.cand.ensure(sizeof(double) * cand.size()));
        DTRY(hipMemcpyAsync(w.cand.p, cand.data(), sizeof(double) * cand.size(),
                            hipMemcpyHostToDevice, s));
        DTRY(w.flags.ensure(sizeof(int) * total));
        DTRY(w.scan.ensure(sizeof(int) * total));
        hipLaunchKernelGGL(image_flag_kernel, dim3(blocks(total, 256)), dim3(256), 0, s, wrapped,
                           n, w.cand.as<double>(), ncand, bd, w.flags.as<int>());
        DTRY(scan_exclusive(w.flags.as<int>(), total, w.scan.as<int>(), w.box_cur,
                            w.scalars.as<int>(), s));
        DTRY(hipMemcpyAsync(&nimg, w.scalars.p, sizeof(int), hipMemcpyDeviceToHost, s));
        DTRY(hipStreamSynchronize(s));
    }
    const int npts = n + nimg;
    DTRY(w.pts.ensure(sizeof(double) * 3 * npts));
    DTRY(w.orig.ensure(sizeof(int) * npts));
    DTRY(hipMemcpyAsync(w.pts.p, wrapped, sizeof(double) * 3 * n, hipMemcpyDeviceToDevice, s));
    hipLaunchKernelGGL(orig_identity_kernel, dim3(blocks(n, 256)), dim3(256), 0, s,
                       w.orig.as<int>(), n);
    if (nimg > 0)
        hipLaunchKernelGGL(image_write_kernel, dim3(blocks(total, 256)), dim3(256), 0, s,
                           w.cand.as<double>(), n, total, w.flags.as<int>(), w.scan.as<int>(),
                           w.pts.as<double>(), w.orig.as<int>());

    // boxes (extent_impl, :145-225)
    BoxGeom g;
    for (int d = 0; d < 3; ++d) {
        g.lo[d] = bd.lo[d];
        g.xd[d] = bd.hi[d] - bd.lo[d];
        const double count = std::floor((bd.hi[d] - bd.lo[d]) / cutoff) + 2;
        if (!std::isfinite(count) || count >= 2e9) {
            err = "Neighbor spatial box count exceeds integer range";
            return MTPX_E_RANGE;
        }
        g.bl[d] = (int)count;
        if (g.bl[d] == 2)
            g.bl[d] = 3;
    }
    const int64_t nbox = (int64_t)g.bl[0] * g.bl[1] * g.bl[2];
    if (nbox > INT_MAX / 2) {
        err = "Neighbor spatial box count exceeds integer range";
        return MTPX_E_RANGE;
    }
    DTRY(w.box.ensure(sizeof(int) * npts));
    DTRY(w.box_start.ensure(sizeof(int) * (nbox + 1)));
    DTRY(w.box_cur.ensure(sizeof(int) * (nbox + 1)));
    DTRY(w.box_items.ensure(sizeof(int) * npts));
    DTRY(w.flags.ensure(sizeof(int) * std::max<int64_t>(npts, nbox + 1)));
    int *box_count = w.cnt.ensure(sizeof(int) * (nbox + 1)) == hipSuccess ? w.cnt.as<int>() : nullptr;
    if (!box_count) {
        err = "neighbour build: out of memory";
        return MTPX_E_ALLOC;
    }
    DTRY(hipMemsetAsync(box_count, 0, sizeof(int) * (nbox + 1), s));
    hipLaunchKernelGGL(box_index_kernel, dim3(blocks(npts, 256)), dim3(256), 0, s,
                       w.pts.as<double>(), n, npts, g, w.box.as<int>(), box_count);
    DTRY(scan_exclusive(box_count, nbox + 1, w.box_start.as<int>(), w.tmp, w.scalars.as<int>(), s));
    DTRY(hipMemcpyAsync(w.box_cur.p, w.box_start.p, sizeof(int) * (nbox + 1),
                        hipMemcpyDeviceToDevice, s));
    int *unsorted = w.flags.as<int>();
    hipLaunchKernelGGL(box_place_kernel, dim3(blocks(npts, 256)), dim3(256), 0, s,
                       w.box.as<int>(), npts, w.box_cur.as<int>(), unsorted);
    hipLaunchKernelGGL(box_rank_kernel, dim3(blocks(npts, 256)), dim3(256), 0, s,
                       w.box.as<int>(), w.box_start.as<int>(), (int)npts, unsorted,
                       w.box_items.as<int>());

    // processing ranks of the centres
    const int64_t ninterior = (int64_t)(g.bl[0] - 2) * (g.bl[1] - 2) * (g.bl[2] - 2);
    DTRY(w.rank.ensure(sizeof(int) * (2 * (size_t)n + 2 * (ninterior + 1))));
    int *rank = w.rank.as<int>();
    int *centre_box = rank + n;
    int *icount = centre_box + n;
    int *iprefix = icount + (ninterior + 1);
    hipLaunchKernelGGL(interior_count_kernel, dim3(blocks(ninterior, 256)), dim3(256), 0, s,
                       w.box_start.as<int>(), w.box_items.as<int>(), g, n, icount);
    DTRY(scan_exclusive(icount, ninterior, iprefix, w.tmp, w.scalars.as<int>(), s));
    hipLaunchKernelGGL(centre_rank_kernel, dim3(blocks(ninterior, 256)), dim3(256), 0, s,
                       w.box_start.as<int>(), w.box_items.as<int>(), iprefix, g, n, rank,
                       centre_box);

    // construct: count, offsets, fill, rank within lists
    Construct cs;
    cs.pts = w.pts.as<double>();
    cs.orig = w.orig.as<int>();
    cs.box_start = w.box_start.as<int>();
    cs.items = w.box_items.as<int>();
    cs.types = w.types.as<int>();
    cs.rank = rank;
    cs.centre_box = centre_box;
    cs.n = n;
    cs.bl1 = g.bl[1];
    cs.bl2 = g.bl[2];
    cs.cutoffsq = cutoff * cutoff;
    DTRY(w.cursor.ensure(sizeof(int) * ((size_t)n + 1)));
    int *cnt = w.cursor.as<int>();
    DTRY(hipMemsetAsync(cnt, 0, sizeof(int) * ((size_t)n + 1), s));
    // one wave per centre, four per workgroup
    hipLaunchKernelGGL(construct_kernel<0>, dim3((n + 3) / 4), dim3(256), 0, s, cs, cnt,
                       nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
    // the entry total in 64 bits: offsets and entry indices are int32
    unsigned long long *total64 = reinterpret_cast<unsigned long long *>(w.scalars.as<int>() + 8);
    DTRY(hipMemsetAsync(total64, 0, sizeof *total64, s));
    hipLaunchKernelGGL(sum64_kernel, dim3(std::min<unsigned>(blocks(n, 256), 1024)), dim3(256), 0,
                       s, cnt, (int64_t)n, total64);
    DTRY(scan_exclusive(cnt, (int64_t)n + 1, out.offsets.as<int>(), w.tmp, w.scalars.as<int>(), s));
    unsigned long long P64 = 0;
    DTRY(hipMemcpyAsync(&P64, total64, sizeof P64, hipMemcpyDeviceToHost, s));
    DTRY(hipStreamSynchronize(s));
    if (P64 > (unsigned long long)INT32_MAX) {
        err = "structure has more than 2^31 - 1 neighbour entries";
        return MTPX_E_CAPACITY;
    }
    const int64_t P = (int64_t)P64;
    out.P = P;
    const size_t Pz = (size_t)std::max<int64_t>(P, 1);
    DTRY(out.idx.ensure(sizeof(int) * Pz));
    DTRY(out.type.ensure(sizeof(int) * Pz));
    DTRY(out.x.ensure(sizeof(double) * Pz));
    DTRY(out.y.ensure(sizeof(double) * Pz));
    DTRY(out.z.ensure(sizeof(double) * Pz));
    DTRY(out.d.ensure(sizeof(double) * Pz));
    if (P == 0)
        return MTPX_OK;
    DTRY(w.key.ensure(sizeof(uint64_t) * Pz));
    DTRY(w.st_idx.ensure(sizeof(int) * Pz));
    DTRY(w.st_type.ensure(sizeof(int) * Pz));
    DTRY(w.st_vec.ensure(sizeof(double) * 3 * Pz));
    DTRY(w.st_d.ensure(sizeof(double) * Pz));
    DTRY(hipMemcpyAsync(cnt, out.offsets.p, sizeof(int) * n, hipMemcpyDeviceToDevice, s));
    hipLaunchKernelGGL(construct_kernel<1>, dim3((n + 3) / 4), dim3(256), 0, s, cs, nullptr, cnt,
                       w.key.as<uint64_t>(), w.st_idx.as<int>(), w.st_type.as<int>(),
                       w.st_vec.as<double>(), w.st_d.as<double>());
    DTRY(w.flags.ensure(sizeof(int) * Pz));
    int *entry_list = w.flags.as<int>();
    hipLaunchKernelGGL(entry_list_kernel, dim3(n), dim3(64), 0, s, out.offsets.as<int>(), n,
                       entry_list);
    hipLaunchKernelGGL(list_rank_kernel, dim3(blocks(P, 256)), dim3(256), 0, s,
                       out.offsets.as<int>(), entry_list, P, w.key.as<uint64_t>(),
                       w.st_idx.as<int>(), w.st_type.as<int>(), w.st_vec.as<double>(),
                       w.st_d.as<double>(), out.idx.as<int>(), out.type.as<int>(),
                       out.x.as<double>(), out.y.as<double>(), out.z.as<double>(),
                       out.d.as<double>());
    DTRY(hipGetLastError());
    DTRY(hipStreamSynchronize(s));
    return MTPX_OK;
}

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
__global__ void append_lists_kernel(const int *offsets, const int *idx, int n, int64_t P, int a0,
                                    int64_t p0, int *out_offsets, int *out_idx)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k <= n)
        out_offsets[a0 + k] = (int)(p0 + offsets[k]);
    if (k < P)
        out_idx[p0 + k] = a0 + idx[k];
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

namespace {

// The structures [0, nconf) one after the other on stream s, concatenated
// into `out` (atom and entry indices relative to the block's first atom).
int build_block(int nconf, const int *atom_offsets, const double *cells, const int *pbc,
                const double *pos, const int *types, double cutoff, hipStream_t s,
                NeighborStore &out, NeighborStore &tmp, NeighborScratch &w, int first,
                std::string &err)
{
    const int ntot = atom_offsets[nconf] - atom_offsets[0];
    out.n = ntot;
    out.P = 0;
    DTRY(out.offsets.ensure(sizeof(int) * ((size_t)ntot + 1)));
    DTRY(out.center_type.ensure(sizeof(int) * std::max(ntot, 1)));
    DTRY(hipMemsetAsync(out.offsets.p, 0, sizeof(int) * ((size_t)ntot + 1), s));
    int64_t P = 0;
    for (int c = 0; c < nconf; ++c) {
        const int a0 = atom_offsets[c] - atom_offsets[0], nc = atom_offsets[c + 1] - atom_offsets[c];
        int rc = build_neighbors_gpu(cells + 9 * (size_t)c, pbc + 3 * (size_t)c, nc,
                                     pos + 3 * (size_t)a0, types + a0, cutoff, s, tmp, w, err);
        if (rc != MTPX_OK) {
            err = "structure " + std::to_string(first + c) + ": " + err;
            return rc;
        }
        const int64_t Pc = tmp.P, Pn = P + Pc;
        if (Pn > INT32_MAX) {
            err = "batch has more than 2^31 - 1 neighbour entries";
            return MTPX_E_CAPACITY;
        }
        const size_t keep = (size_t)P, need = (size_t)std::max<int64_t>(Pn, 1);
        DTRY(grow_keep(out.idx, sizeof(int) * need, sizeof(int) * keep, s));
        DTRY(grow_keep(out.type, sizeof(int) * need, sizeof(int) * keep, s));
        DTRY(grow_keep(out.x, sizeof(double) * need, sizeof(double) * keep, s));
        DTRY(grow_keep(out.y, sizeof(double) * need, sizeof(double) * keep, s));
        DTRY(grow_keep(out.z, sizeof(double) * need, sizeof(double) * keep, s));
        DTRY(grow_keep(out.d, sizeof(double) * need, sizeof(double) * keep, s));
        if (nc > 0)
            DTRY(hipMemcpyAsync(out.center_type.as<int>() + a0, tmp.center_type.p,
                                sizeof(int) * nc, hipMemcpyDeviceToDevice, s));
        if (Pc > 0) {
            DTRY(hipMemcpyAsync(out.type.as<int>() + P, tmp.type.p, sizeof(int) * Pc,
                                hipMemcpyDeviceToDevice, s));
            DTRY(hipMemcpyAsync(out.x.as<double>() + P, tmp.x.p, sizeof(double) * Pc,
                                hipMemcpyDeviceToDevice, s));
            DTRY(hipMemcpyAsync(out.y.as<double>() + P, tmp.y.p, sizeof(double) * Pc,
                                hipMemcpyDeviceToDevice, s));
            DTRY(hipMemcpyAsync(out.z.as<double>() + P, tmp.z.p, sizeof(double) * Pc,
                                hipMemcpyDeviceToDevice, s));
            DTRY(hipMemcpyAsync(out.d.as<double>() + P, tmp.d.p, sizeof(double) * Pc,
                                hipMemcpyDeviceToDevice, s));
        }
        const int64_t work = std::max<int64_t>(Pc, (int64_t)nc + 1);
        hipLaunchKernelGGL(append_lists_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256),
                           0, s, tmp.offsets.as<int>(), tmp.idx.as<int>(), nc, Pc, a0, P,
                           out.offsets.as<int>(), out.idx.as<int>());
        DTRY(hipGetLastError());
        P = Pn;
    }
    DTRY(hipStreamSynchronize(s));
    out.P = P;
    return MTPX_OK;
}

void release_store(NeighborStore &st)
{
    for (DBuf *b : {&st.offsets, &st.idx, &st.type, &st.x, &st.y, &st.z, &st.d, &st.center_type})
        b->release();
}

}  // namespace

// Every structure's build is a short chain of small launches with a few
// host synchronisations, so a large batch is split into contiguous blocks
// of structures (balanced by atom count) built by host threads, each on a
// stream, scratch and lists of its own; the blocks are then appended in
// order on the caller's stream.  The lists are those of the one-by-one
// build, entry for entry.
int build_neighbors_batch_gpu(int nconf, const int *atom_offsets, const double *cells,
                              const int *pbc, const double *pos, const int *types, double cutoff,
                              hipStream_t s, NeighborStore &out, NeighborStore &tmp,
                              NeighborScratch &w, std::string &err)
{
    const int ntot = atom_offsets[nconf];
    constexpr int kWorkers = 4;  // the hardware queues a process gets (8 measured 6-8 % faster)
    if (nconf < 4 * kWorkers)
        return build_block(nconf, atom_offsets, cells, pbc, pos, types, cutoff, s, out, tmp, w, 0,
                           err);
    // contiguous blocks of about equal atom counts (at least one structure each)
    int cut[kWorkers + 1];
    cut[0] = 0;
    for (int k = 1; k < kWorkers; ++k) {
        const int64_t want = (int64_t)ntot * k / kWorkers;
        int c = cut[k - 1] + 1;
        while (c < nconf - (kWorkers - k) && atom_offsets[c] < want)
            ++c;
        cut[k] = c;
    }
    cut[kWorkers] = nconf;
    int device = 0;
    DTRY(hipGetDevice(&device));
    struct Part {
        hipStream_t s = nullptr;
        NeighborStore lists, one;
        NeighborScratch w;
        std::string err;
        int rc = MTPX_OK;
    };
    std::vector<Part> parts(kWorkers);
    for (Part &q : parts)
        if (hipStreamCreate(&q.s) != hipSuccess) {
            for (Part &r : parts)
                if (r.s)
                    (void)hipStreamDestroy(r.s);
            err = "neighbour build: cannot create a stream";
            return MTPX_E_DEVICE;
        }
    std::vector<std::thread> threads;
    bool spawned = true;
    for (int k = 0; k < kWorkers && spawned; ++k)
        try {
            threads.emplace_back([&, k] {
            Part &q = parts[k];
            if (hipSetDevice(device) != hipSuccess) {
                q.rc = MTPX_E_DEVICE;
                q.err = "neighbour build: cannot select the device";
                return;
            }
            const int c0 = cut[k], a0 = atom_offsets[c0];
            q.rc = build_block(cut[k + 1] - c0, atom_offsets + c0, cells + 9 * (size_t)c0,
                               pbc + 3 * (size_t)c0, pos + 3 * (size_t)a0, types + a0, cutoff, q.s,
                               q.lists, q.one, q.w, c0, q.err);
            });
        } catch (...) {  // no thread: the remaining blocks run on this one
            spawned = false;
        }
    for (std::thread &t : threads)
        t.join();
    for (int k = (int)threads.size(); k < kWorkers; ++k) {
        Part &q = parts[k];
        const int c0 = cut[k], a0 = atom_offsets[c0];
        q.rc = build_block(cut[k + 1] - c0, atom_offsets + c0, cells + 9 * (size_t)c0,
                           pbc + 3 * (size_t)c0, pos + 3 * (size_t)a0, types + a0, cutoff, q.s,
                           q.lists, q.one, q.w, c0, q.err);
    }
    int rc = MTPX_OK;
    int64_t P = 0;
    for (Part &q : parts) {
        if (rc == MTPX_OK && q.rc != MTPX_OK) {
            rc = q.rc;
            err = q.err;
        }
        P += q.lists.P;
    }
    if (rc == MTPX_OK && P > INT32_MAX) {
        rc = MTPX_E_CAPACITY;
        err = "batch has more than 2^31 - 1 neighbour entries";
    }
    hipError_t e = hipSuccess;
    if (rc == MTPX_OK) {
        const size_t Pz = (size_t)std::max<int64_t>(P, 1);
        out.n = ntot;
        out.P = P;
        for (DBuf *b : {&out.idx, &out.type})
            if (e == hipSuccess)
                e = b->ensure(sizeof(int) * Pz);
        for (DBuf *b : {&out.x, &out.y, &out.z, &out.d})
            if (e == hipSuccess)
                e = b->ensure(sizeof(double) * Pz);
        if (e == hipSuccess)
            e = out.offsets.ensure(sizeof(int) * ((size_t)ntot + 1));
        if (e == hipSuccess)
            e = out.center_type.ensure(sizeof(int) * std::max(ntot, 1));
        int64_t p0 = 0;
        for (int k = 0; k < kWorkers && e == hipSuccess; ++k) {
            const Part &q = parts[k];
            const int a0 = atom_offsets[cut[k]], nk = atom_offsets[cut[k + 1]] - a0;
            const int64_t Pk = q.lists.P;
            auto copy = [&](const DBuf &from, const DBuf &to, size_t at, size_t bytes) {
                if (e == hipSuccess && bytes)
                    e = hipMemcpyAsync(static_cast<char *>(to.p) + at, from.p, bytes,
                                       hipMemcpyDeviceToDevice, s);
            };
            if (e == hipSuccess)
                e = hipStreamSynchronize(q.s);
            copy(q.lists.center_type, out.center_type, sizeof(int) * a0, sizeof(int) * nk);
            copy(q.lists.type, out.type, sizeof(int) * p0, sizeof(int) * Pk);
            copy(q.lists.x, out.x, sizeof(double) * p0, sizeof(double) * Pk);
            copy(q.lists.y, out.y, sizeof(double) * p0, sizeof(double) * Pk);
            copy(q.lists.z, out.z, sizeof(double) * p0, sizeof(double) * Pk);
            copy(q.lists.d, out.d, sizeof(double) * p0, sizeof(double) * Pk);
            if (e == hipSuccess) {
                const int64_t work = std::max<int64_t>(Pk, (int64_t)nk + 1);
                hipLaunchKernelGGL(append_lists_kernel, dim3((unsigned)((work + 255) / 256)),
                                   dim3(256), 0, s, q.lists.offsets.as<int>(),
                                   q.lists.idx.as<int>(), nk, Pk, a0, p0, out.offsets.as<int>(),
                                   out.idx.as<int>());
                e = hipGetLastError();
            }
            p0 += Pk;
        }
        if (e == hipSuccess)
            e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            rc = e == hipErrorOutOfMemory ? MTPX_E_ALLOC : MTPX_E_DEVICE;
            err = std::string("neighbour build: ") + hipGetErrorString(e);
        }
    }
    for (Part &q : parts) {
        (void)hipStreamSynchronize(q.s);
        (void)hipStreamDestroy(q.s);
        release_store(q.lists);
        release_store(q.one);
        q.w.release_all();
    }
    return rc;
}

}  // namespace mtpx
