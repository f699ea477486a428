// The normal equations of the linear fit on the fp64 matrix cores
// (Trainer_MTP::TrainLinearFast, train/train_mtp.cpp:2383-2427): the Gram
// [A y]^T [A y] of the weighted design rows, without forming A.
//
//   gram_kernel          upper 16x16 tiles of the Gram of a row range
//                        (v_mfma_f64_16x16x4f64), one partial per range
//   chunk_reduce_kernel  first stage of the fixed-order sum of the partials
#include "mtpx_internal.hpp"

#include <algorithm>

namespace mtpx {

namespace {

typedef double d4v __attribute__((ext_vector_type(4)));

// Gram of the extended rows e_r = [sw_r comp[src_r + q] (q < p), y_r, 0...]
// (length pp, a multiple of 16) on the matrix cores.  The Gram is
// symmetric, so only its upper 16x16 tiles (I <= J, nt(nt+1)/2 of them,
// row-major) are summed; each is written with its transpose.  Workgroup
// (x, y) sums e_r e_r^T over row range x for tile group y and writes the
// tiles into partial x (pp x pp); the groups of one row range cover
// disjoint tiles.  Each wave holds a contiguous run of the group's tiles
// (at most kGramTiles), so consecutive tiles share their row block I and
// each step loads the I operand once.
//
// The rows reach LDS through a three-stage pipeline with one barrier per
// block of `rows` rows: while the matrix cores work on block b, the values
// of block b+1 are loaded (their offsets and weights already sit in an LDS
// table) and the offsets and weights of block b+2 are loaded into that
// table.  The row data thus never waits on a dependent offset load.
//
// v_mfma_f64_16x16x4f64: A operand 16x4 (lane l holds A[l%16][l/16]), B
// operand 4x16 (lane l holds B[l/16][l%16]), result 16x16 with lane l
// holding D[l/16 + 4v][l%16], v = 0..3.  For the tile (I, J) of the Gram,
// A[i][k] = e_{r+k}[16I+i] and B[k][j] = e_{r+k}[16J+j]: both operands read
// lane l's value e_{r+l/16}[16c + l%16] of a column block c.
constexpr int kGramPad = 2;      // LDS row padding (doubles)
constexpr int kGramTiles = 4;    // tiles per wave
constexpr int kGramWaves = 8;    // waves per workgroup
constexpr int kGramThreads = 64 * kGramWaves;
constexpr int kGramStage = 4096; // doubles per LDS buffer (rows * pp at most)
constexpr int kGramPer = kGramStage / kGramThreads;  // staged values per thread
constexpr int kGramMaxRows = 32;

// Rows per LDS buffer: a multiple of 4 with rows * (pp + pad) <= kGramStage.
int gram_rows(int pp)
{
    int r = kGramMaxRows;
    while (r > 4 && r * (pp + kGramPad) > kGramStage)
        r /= 2;
    return r;
}

struct GramMeta {
    int64_t src[3][kGramMaxRows];  // row offset into comp, -1 past the range
    double sw[3][kGramMaxRows], y[3][kGramMaxRows];
};

__global__ __launch_bounds__(kGramThreads, 4) void gram_kernel(
    const double *comp, const int64_t *src, const double *sw, const double *yw, int64_t R, int p,
    int pp, int rows, int64_t rows_per_block, int tiles_per_group, double *partial)
{
    extern __shared__ double stage[];  // [2][rows][pp + kGramPad]
    __shared__ GramMeta meta;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ld = pp + kGramPad;
    const int nt = pp / 16;
    const int ntri = nt * (nt + 1) / 2;
    // this wave's run of tiles [t0, t0 + cnt) of the group's [g0, g1)
    const int g0 = blockIdx.y * tiles_per_group;
    const int g1 = min(ntri, g0 + tiles_per_group);
    const int per = (g1 - g0 + kGramWaves - 1) / kGramWaves;
    const int t0 = g0 + wave * per;
    const int cnt = max(0, min(per, g1 - t0));
    int TI[kGramTiles], TJ[kGramTiles];
    {
        int t = min(t0, ntri - 1), I = 0;
        while (t >= nt - I) {
            t -= nt - I;
            ++I;
        }
        int J = I + t;
#pragma unroll
        for (int k = 0; k < kGramTiles; ++k) {
            TI[k] = I;
            TJ[k] = J;
            if (++J == nt) {
                ++I;
                J = min(I, nt - 1);
                I = min(I, nt - 1);
            }
        }
    }
    d4v acc[kGramTiles];
#pragma unroll
    for (int k = 0; k < kGramTiles; ++k)
        acc[k] = d4v{0.0, 0.0, 0.0, 0.0};
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = min(R, r0 + rows_per_block);
    const int nb = r1 > r0 ? (int)((r1 - r0 + rows - 1) / rows) : 0;
    // offsets and weights of block j into table slot j % 3 (thread tid < rows)
    int64_t msrc = -1;
    double msw = 0.0, my = 0.0;
    auto meta_load = [&](int j) {
        const int64_t r = r0 + (int64_t)j * rows + tid;
        msrc = -1;
        msw = my = 0.0;
        if (r < r1) {
            msrc = src[r];
            msw = sw[r];
            my = yw[r];
        }
    };
    auto meta_store = [&](int j) {
        meta.src[j % 3][tid] = msrc;
        meta.sw[j % 3][tid] = msw;
        meta.y[j % 3][tid] = my;
    };
    // staged value i of this thread: element e = tid + i * kGramThreads of
    // the block, row e / pp and column e % pp
    const int nstage = rows * pp;
    const int step_r = kGramThreads / pp, step_q = kGramThreads % pp;
    double v[kGramPer];
    auto fetch = [&](int j) {
        const int slot = j % 3;
        int rr = tid / pp, q = tid % pp;
#pragma unroll
        for (int i = 0; i < kGramPer; ++i) {
            double x = 0.0;
            if (tid + i * kGramThreads < nstage) {
                const int64_t o = meta.src[slot][rr];
                if (o >= 0) {
                    if (q < p)
                        x = meta.sw[slot][rr] * comp[o + q];
                    else if (q == p)
                        x = meta.y[slot][rr];
                }
            }
            v[i] = x;
            rr += step_r;
            q += step_q;
            if (q >= pp) {
                q -= pp;
                ++rr;
            }
        }
    };
    auto store = [&](double *buf) {
        int rr = tid / pp, q = tid % pp;
#pragma unroll
        for (int i = 0; i < kGramPer; ++i) {
            if (tid + i * kGramThreads < nstage)
                buf[rr * ld + q] = v[i];
            rr += step_r;
            q += step_q;
            if (q >= pp) {
                q -= pp;
                ++rr;
            }
        }
    };
    // prologue: tables of blocks 0 and 1, values of block 0
    if (tid < rows) {
        meta_load(0);
        meta_store(0);
        meta_load(1);
        meta_store(1);
    }
    __syncthreads();
    if (nb > 0) {
        fetch(0);
        store(stage);
    }
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const bool more1 = b + 1 < nb, more2 = b + 2 < nb;
        if (more2 && tid < rows)
            meta_load(b + 2);
        if (more1)
            fetch(b + 1);
        const double *buf = stage + (b & 1) * rows * ld;
        for (int k4 = 0; k4 < rows; k4 += 4) {
            const double *row = buf + (k4 + lane / 16) * ld + lane % 16;
            double a = 0.0;
#pragma unroll
            for (int k = 0; k < kGramTiles; ++k) {
                if (k < cnt) {
                    if (k == 0 || TI[k] != TI[k - 1])
                        a = row[16 * TI[k]];
                    const double bv = TJ[k] == TI[k] ? a : row[16 * TJ[k]];
                    acc[k] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, bv, acc[k], 0, 0, 0);
                }
            }
        }
        if (more1)
            store(stage + ((b + 1) & 1) * rows * ld);
        if (more2 && tid < rows)
            meta_store(b + 2);
        __syncthreads();
    }
    double *out = partial + (size_t)blockIdx.x * pp * pp;
#pragma unroll
    for (int k = 0; k < kGramTiles; ++k) {
        if (k < cnt) {
            const int I = TI[k], J = TJ[k];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const int i = 16 * I + lane / 16 + 4 * w, j = 16 * J + lane % 16;
                out[(size_t)i * pp + j] = acc[k][w];
                if (I != J)
                    out[(size_t)j * pp + i] = acc[k][w];
            }
        }
    }
}

// Ordered sums of consecutive runs of `chunk` rows of a [nrows][cols]
// array: out[g][k] = sum of rows g*chunk .. (g+1)*chunk-1 in row order.
__global__ __launch_bounds__(256) void chunk_reduce_kernel(const double *rows, int nrows, int cols,
                                                           int chunk, double *out)
{
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= cols)
        return;
    const int g = blockIdx.y;
    const int a = g * chunk, e = min(nrows, a + chunk);
    double s = 0.0;
    int r = a;
    for (; r + 8 <= e; r += 8) {
        double x[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            x[q] = rows[(size_t)(r + q) * cols + k];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            s += x[q];
    }
    for (; r < e; ++r)
        s += rows[(size_t)r * cols + k];
    out[(size_t)g * cols + k] = s;
}

}  // namespace

int gram_padded(int p) { return (p + 1 + 15) / 16 * 16; }

// Row ranges of the Gram: two workgroups per CU, fewer when the partials
// (nblocks x pp x pp) would pass 256 MiB or a range would hold under one
// LDS block of rows.
int gram_blocks(int64_t R, int p, int num_cus)
{
    const int pp = gram_padded(p);
    const int64_t cap = std::max<int64_t>(1, (int64_t(256) << 20) / (8LL * pp * pp));
    const int64_t by_rows = std::max<int64_t>(1, (R + gram_rows(pp) - 1) / gram_rows(pp));
    return (int)std::max<int64_t>(1, std::min<int64_t>({2LL * num_cus, cap, by_rows}));
}

// Partials need (nblocks + kGramChunks) x pp x pp doubles: the row-range
// partials, then the chunk sums; the result goes to out (pp x pp).
constexpr int kGramChunkRows = 32;
size_t gram_partial_doubles(int p, int nblocks)
{
    const size_t pp = gram_padded(p);
    return ((size_t)nblocks + (nblocks + kGramChunkRows - 1) / kGramChunkRows) * pp * pp;
}

bool gram_fits(int p)
{
    const int pp = gram_padded(p);
    return gram_rows(pp) * (pp + kGramPad) <= kGramStage;
}

hipError_t launch_gram(const double *comp, const int64_t *src, const double *sw, const double *yw,
                       int64_t R, int p, int nblocks, double *partial, double *out, hipStream_t s)
{
    const int pp = gram_padded(p);
    const int rows = gram_rows(pp);
    if (!gram_fits(p))
        return hipErrorInvalidValue;
    const int64_t per = ((R + nblocks - 1) / nblocks + rows - 1) / rows * rows;
    const size_t lds = sizeof(double) * 2 * rows * (pp + kGramPad);
    const int nt = pp / 16;
    const int ntri = nt * (nt + 1) / 2;
    const int cap = kGramWaves * kGramTiles;
    const int groups = (ntri + cap - 1) / cap;
    const int tiles_per_group = (ntri + groups - 1) / groups;
    hipLaunchKernelGGL(gram_kernel, dim3(nblocks, groups), dim3(kGramThreads), lds, s, comp,
                       src, sw, yw, R, p, pp, rows, std::max<int64_t>(per, rows), tiles_per_group,
                       partial);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    // fixed-order two-stage sum of the partials
    const int cols = pp * pp;
    const int nch = (nblocks + kGramChunkRows - 1) / kGramChunkRows;
    double *mid = partial + (size_t)nblocks * cols;
    hipLaunchKernelGGL(chunk_reduce_kernel, dim3((cols + 255) / 256, nch), dim3(256), 0, s,
                       partial, nblocks, cols, kGramChunkRows, mid);
    e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    return launch_rows_reduce(mid, nch, cols, out, false, s);
}

}  // namespace mtpx
