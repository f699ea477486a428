// Linear-fit kernels for gfx950 (fp64).
//
//   lin_site_kernel   E/F/S components of every linear coefficient
//                     (PotMTP::CalcEFSCmpt_R, potentials/potential_mtp.cpp:
//                     2675-2707, over CalcSiteBasisDers, :3163-3280): for a
//                     species column, the atom count; for a moment column
//                     s, sum_i m_map(s), dm/dr_j scattered into the force
//                     rows of i and of its neighbours, and -sum dm/dr_j r_j
//                     into the stress rows.
//   rows_kernel       AddLinearFast rows (train/train_mtp.cpp:1289-1395):
//                     component rows scaled by sqrt(w), targets sqrt(w) y
//   gram_kernel       [A y]^T [A y] on the fp64 matrix cores
//                     (v_mfma_f64_16x16x4f64), partial per workgroup
//
// lin_site_kernel runs one wave per site.  The reference propagates the
// Jacobian of every moment w.r.t. all 3 n_i coordinates through the rules.
// Here the scalar moments are differentiated through the sparse site
// Jacobian L[s][b] = dm_map(s)/dm_b instead: L is computed once per site by
// a step table (the rule-table machinery), then lanes take neighbours and
// accumulate dm_s/dr_j = sum_b L[s][b] grad_r(f_b Y_b)(r_j) for a chunk of
// scalars at a time.
#include "mtp_device.hpp"

namespace mtpx {

namespace {

typedef double d4v __attribute__((ext_vector_type(4)));

// Walk of the slots (nu, mu, alpha) with the chunk's entries: for a slot
// that has entries, grad_r(f Y) = (f' - nu f/d) Y u + (f/d) grad_u Y is
// formed once and added, times L, to each of the slot's scalars.
// Walk of the slots (nu, mu, alpha) for one chunk of scalars: where the
// chunk's mask of the slot is set, grad_r(f Y) = (f' - nu f/d) Y u +
// (f/d) grad_u Y is formed once and added, times L, to those scalars'
// derivatives (registers; the mask and its bits are wave-uniform).
template <int NU, class P>
__device__ __forceinline__ void lin_shells(const DevModel &m, const DevLin &L, const Nbr<P::M> &q,
                                           const double *prev, int &slot, const int *mask,
                                           const int *lidx, const double *ws,
                                           double (&acc)[3 * kLinChunk])
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
            const double h = q.fd[mu] - NU * q.f[mu] * q.invd;
            const double fdi = q.f[mu] * q.invd;
#pragma unroll
            for (int a = NU; a >= 0; --a)
#pragma unroll
                for (int b = NU - a; b >= 0; --b) {
                    const int i = shell_index(NU, a, b);
                    const int sl = slot + i;
                    const int mk = mask[sl];
                    if (mk) {
                        const double hy = h * cur[i];
                        double gx = hy * q.ux, gy = hy * q.uy, gz = hy * q.uz;
                        if constexpr (NU > 0) {
                            if (a > 0)
                                gx += (a * fdi) * prev[shell_index(NU - 1, a - 1, b)];
                            if (b > 0)
                                gy += (b * fdi) * prev[shell_index(NU - 1, a, b - 1)];
                            if (NU - a - b > 0)
                                gz += ((NU - a - b) * fdi) * prev[shell_index(NU - 1, a, b)];
                        }
                        const int *li = lidx + (size_t)sl * kLinChunk;
#pragma unroll
                        for (int k = 0; k < kLinChunk; ++k)
                            if (mk & (1 << k)) {
                                const double lv = ws[li[k]];
                                acc[3 * k] += lv * gx;
                                acc[3 * k + 1] += lv * gy;
                                acc[3 * k + 2] += lv * gz;
                            }
                    }
                }
            slot += shell_size(NU);
        }
    }
    if constexpr (NU < P::NUMAX) {
        if (P::deeper(m, NU))
            lin_shells<NU + 1, P>(m, L, q, cur, slot, mask, lidx, ws, acc);
    }
}

template <class Tgt>
__device__ __forceinline__ void reduce_rows_lin(const double *red, int nrows, int row0, int lane,
                                                Tgt tgt)
{
    wave_sync();
    const double acc = chunk_row_sum(red, lane);
    if (lane < nrows)
        tgt(row0 + lane, acc);
    wave_sync();
}

template <class P, int kMaxWaves>
__global__ __launch_bounds__(kWave *kMaxWaves) void lin_site_kernel(DevModel m, DevLin L,
                                                                    DevNeighbors nb, LinOut out)
{
    extern __shared__ double lds[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nwaves = blockDim.x / kWave;
    const Shared Ls = shared_layout(m, lds);
    double *ws = lds + shared_doubles(m, false) + (size_t)wave * L.priv;
    double *mom = ws, *red = ws + m.red0;
    const int p = m.Z + m.S;

    stage_shared(m, Ls, false, tid, blockDim.x);
    for (int k = m.dummy + lane; k < m.red0; k += kWave)
        ws[k] = 0.0;
    for (int k = L.one + lane; k < L.L0; k += kWave)
        ws[k] = k == L.one ? 1.0 : 0.0;
    for (int k = L.part0 + lane; k < L.acc; k += kWave)
        ws[k] = 0.0;
    __syncthreads();

    for (int i = blockIdx.x * nwaves + wave; i < nb.n; i += gridDim.x * nwaves) {
        const int ti = nb.center_type[i];
        const int beg = nb.offsets[i];
        const int n = nb.offsets[i + 1] - beg;
        const int c = out.center_structure[i];
        for (int k = lane; k < m.K; k += kWave)
            mom[k] = 0.0;
        wave_sync();

        // ---- moments (as the E/F/S kernel) --------------------------------
        for (int base = 0; base < n; base += kWave) {
            FwdCtx cx{red, mom, Ls.slot_basic, lane, 0};
            Nbr<P::M> q;
            load_neighbor<P>(m, nb, Ls.coef, ti, beg + base + lane, lane < n - base, q);
            fwd_shells<0, P>(m, cx, q, nullptr);
            const int rest = cx.slot % kChunk;
            if (rest)
                reduce_chunk(red, rest, cx.slot - rest, Ls.slot_basic, mom, lane);
        }
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                mom[m.dup[2 * k]] = mom[m.dup[2 * k + 1]];
        wave_sync();
        run_rules<false, false>(m.fwd_steps, m.fwd_level_step, m.fwd_level_comb, m.fwd_comb, m.nfwd, ws,
                         lane, 0);

        // ---- energy components -------------------------------------------
        for (int s = lane; s < m.S; s += kWave)
            atomicAdd(&out.ec[(size_t)c * p + m.Z + s], mom[Ls.map[s]]);
        if (lane == 0)
            atomicAdd(&out.ec[(size_t)c * p + ti], 1.0);

        // ---- site Jacobian of the scalars w.r.t. the basics ----------------
        for (int k = L.L0 + lane; k < L.L0 + L.nL; k += kWave)
            ws[k] = 0.0;
        wave_sync();
        run_rules<false, false>(L.steps, L.level_step, L.level_comb, L.comb, L.nlev, ws, lane, 0);

        // ---- force and stress components, CH scalars at a time ------------
        for (int ch = 0; ch < L.nchunks; ++ch) {
            const int s0 = ch * L.CH, nch = min(L.CH, m.S - s0);
            const int *mask = L.slot_mask + (size_t)ch * m.nslots;
            const int *lidx = L.slot_L + (size_t)ch * m.nslots * kLinChunk;
            for (int base = 0; base < n; base += kWave) {
                double acc[3 * kLinChunk];
#pragma unroll
                for (int r = 0; r < 3 * kLinChunk; ++r)
                    acc[r] = 0.0;
                const bool valid = lane < n - base;
                const int64_t pe = beg + base + lane;
                Nbr<P::M> q;
                load_neighbor<P>(m, nb, Ls.coef, ti, pe, valid, q);
                int slot = 0;
                lin_shells<0, P>(m, L, q, nullptr, slot, mask, lidx, ws, acc);
                // the site's own rows: + sum_j dm/dr_j
                int row = 0;
                auto flush_self = [&](int nrows) {
                    reduce_rows_lin(red, nrows, row - nrows, lane, [&](int r, double v) {
                        atomicAdd(&out.fc[((size_t)i * 3 + r % 3) * p + m.Z + s0 + r / 3], v);
                    });
                };
#pragma unroll
                for (int r = 0; r < 3 * kLinChunk; ++r)
                    if (r < 3 * nch) {
                        red[(row % kChunk) * kRedStride + lane] = acc[r];
                        ++row;
                        if (row % kChunk == 0)
                            flush_self(kChunk);
                    }
                if (row % kChunk)
                    flush_self(row % kChunk);
                // the neighbours' rows: - dm/dr_j
                if (valid) {
                    const int j = nb.idx[pe];
#pragma unroll
                    for (int r = 0; r < 3 * kLinChunk; ++r)
                        if (r < 3 * nch)
                            atomicAdd(&out.fc[((size_t)j * 3 + r % 3) * p + m.Z + s0 + r / 3],
                                      -acc[r]);
                }
                // stress rows: - sum_j (dm/dr_j)_a r_jb
                const double rv[3] = {q.x, q.y, q.z};
                row = 0;
                auto flush = [&](int nrows) {
                    reduce_rows_lin(red, nrows, row - nrows, lane, [&](int r, double v) {
                        atomicAdd(&out.sc[((size_t)c * 9 + r % 9) * p + m.Z + s0 + r / 9], v);
                    });
                };
#pragma unroll
                for (int sl = 0; sl < kLinChunk; ++sl)
                    if (sl < nch)
#pragma unroll
                        for (int a = 0; a < 3; ++a)
#pragma unroll
                            for (int b = 0; b < 3; ++b) {
                                red[(row % kChunk) * kRedStride + lane] = -acc[3 * sl + a] * rv[b];
                                ++row;
                                if (row % kChunk == 0)
                                    flush(kChunk);
                            }
                if (row % kChunk)
                    flush(row % kChunk);
            }
        }
        wave_sync();
    }
}

// AddLinearFast rows: A[r][q] = sw_r comp[src_r + q], y[r] = y_r.
__global__ __launch_bounds__(256) void rows_kernel(const double *comp, const int64_t *src,
                                                   const double *sw, const double *yw, int64_t R,
                                                   int p, double *A, double *y)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= R * p)
        return;
    const int64_t r = t / p;
    const int q = (int)(t % p);
    A[t] = sw[r] * comp[src[r] + q];
    if (q == 0)
        y[r] = yw[r];
}

// Gram of the extended rows e_r = [sw_r comp[src_r + q] (q < p), y_r, 0...]
// (length pp, a multiple of 16).  Workgroup (x, y) sums e_r e_r^T over row
// range x for the 16 output tiles of group y (4 per wave) on the matrix cores
// and writes them into partial x (pp x pp).
//
// v_mfma_f64_16x16x4f64: A operand 16x4 (lane l holds A[l%16][l/16]), B
// operand 4x16 (lane l holds B[l/16][l%16]), result 16x16 with lane l
// holding D[l/16 + 4v][l%16], v = 0..3.  For the tile (I, J) of the Gram,
// A[i][k] = e_{r+k}[16I+i] and B[k][j] = e_{r+k}[16J+j].
constexpr int kGramRows = 32;   // rows staged per step
constexpr int kGramPad = 2;     // LDS row padding (doubles)
constexpr int kTilesPerWave = 4;

__global__ __launch_bounds__(256) void gram_kernel(const double *comp, const int64_t *src,
                                                   const double *sw, const double *yw, int64_t R,
                                                   int p, int pp, int64_t rows_per_block,
                                                   double *partial)
{
    extern __shared__ double tile[];  // [kGramRows][pp + kGramPad]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ld = pp + kGramPad;
    const int nt = pp / 16;
    const int ntiles = nt * nt;
    const int tile0 = blockIdx.y * 4 * kTilesPerWave + wave * kTilesPerWave;
    d4v accv[kTilesPerWave];
#pragma unroll
    for (int k = 0; k < kTilesPerWave; ++k)
        accv[k] = d4v{0.0, 0.0, 0.0, 0.0};
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = min(R, r0 + rows_per_block);
    for (int64_t rb = r0; rb < r1; rb += kGramRows) {
        __syncthreads();
        for (int t = tid; t < kGramRows * pp; t += blockDim.x) {
            const int rr = t / pp, q = t % pp;
            const int64_t r = rb + rr;
            double v = 0.0;
            if (r < r1) {
                if (q < p)
                    v = sw[r] * comp[src[r] + q];
                else if (q == p)
                    v = yw[r];
            }
            tile[rr * ld + q] = v;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kTilesPerWave; ++k) {
            const int t = tile0 + k;
            if (t < ntiles) {
                const int I = t / nt, J = t % nt;
                d4v cacc = accv[k];
#pragma unroll
                for (int k4 = 0; k4 < kGramRows; k4 += 4) {
                    const double a = tile[(k4 + lane / 16) * ld + 16 * I + lane % 16];
                    const double b = tile[(k4 + lane / 16) * ld + 16 * J + lane % 16];
                    cacc = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, cacc, 0, 0, 0);
                }
                accv[k] = cacc;
            }
        }
    }
    double *out = partial + (size_t)blockIdx.x * pp * pp;
#pragma unroll
    for (int k = 0; k < kTilesPerWave; ++k) {
        const int t = tile0 + k;
        if (t < ntiles) {
            const int I = t / nt, J = t % nt;
#pragma unroll
            for (int v = 0; v < 4; ++v)
                out[(size_t)(16 * I + lane / 16 + 4 * v) * pp + 16 * J + lane % 16] = accv[k][v];
        }
    }
}

// Waves per workgroup: the level-10 kernel fits 256 registers (eight waves);
// the others use up to 512 (one wave per SIMD).
template <class P>
struct LinWaves {
    static constexpr int value = 4;
};
template <>
struct LinWaves<ProfLevel10> {
    static constexpr int value = 8;
};

template <class P>
void launch_lin_variant(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                        const LinOut &out, const EfsLaunch &cfg, hipStream_t s)
{
    constexpr int W = LinWaves<P>::value;
    hipLaunchKernelGGL((lin_site_kernel<P, W>), dim3(cfg.grid), dim3(kWave * cfg.waves),
                       cfg.lds_bytes, s, m, L, nb, out);
}

}  // namespace

bool lin_configure(const DevModel &m, const DevLin &L, int n, int num_cus, size_t lds_limit,
                   EfsLaunch &cfg)
{
    const size_t sh = shared_doubles(m, false) * sizeof(double);
    const size_t priv = (size_t)L.priv * sizeof(double);
    if (sh + priv > lds_limit)
        return false;
    cfg.lds_tables = false;
    const int wcap = efs_variant(m, m.R) == 2 ? 8 : 4;
    cfg.waves = (int)std::min<size_t>(wcap, (lds_limit - sh) / priv);
    cfg.lds_bytes = sh + cfg.waves * priv;
    const int per_cu = std::max<int>(1, (int)(lds_limit / cfg.lds_bytes));
    const int need = (std::max(n, 1) + cfg.waves - 1) / cfg.waves;
    cfg.grid = std::max(1, std::min(need, num_cus * per_cu));
    cfg.rows = cfg.grid * cfg.waves;
    return true;
}

hipError_t launch_lin_site(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                           const LinOut &out, const EfsLaunch &cfg, hipStream_t s)
{
    switch (efs_variant(m, m.R)) {
    case 0: launch_lin_variant<ProfLevel16>(m, L, nb, out, cfg, s); break;
    case 1: launch_lin_variant<ProfLevel20>(m, L, nb, out, cfg, s); break;
    case 2: launch_lin_variant<ProfLevel10>(m, L, nb, out, cfg, s); break;
    case 3: launch_lin_variant<ProfSmall>(m, L, nb, out, cfg, s); break;
    default: launch_lin_variant<ProfGeneric>(m, L, nb, out, cfg, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_lin_rows(const double *comp, const int64_t *src, const double *sw,
                           const double *yw, int64_t R, int p, double *A, double *y, hipStream_t s)
{
    const int64_t work = R * p;
    if (work > 0)
        hipLaunchKernelGGL(rows_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, s,
                           comp, src, sw, yw, R, p, A, y);
    return hipGetLastError();
}

int gram_padded(int p) { return (p + 1 + 15) / 16 * 16; }

hipError_t launch_gram(const double *comp, const int64_t *src, const double *sw, const double *yw,
                       int64_t R, int p, int nblocks, double *partial, hipStream_t s)
{
    const int pp = gram_padded(p);
    const int64_t per = ((R + nblocks - 1) / nblocks + kGramRows - 1) / kGramRows * kGramRows;
    const size_t lds = sizeof(double) * kGramRows * (pp + kGramPad);
    const int nt = pp / 16;
    const int groups = (nt * nt + 4 * kTilesPerWave - 1) / (4 * kTilesPerWave);
    hipLaunchKernelGGL(gram_kernel, dim3(nblocks, groups), dim3(256), lds, s, comp, src, sw, yw, R,
                       p, pp, std::max<int64_t>(per, kGramRows), partial);
    return hipGetLastError();
}

}  // namespace mtpx
