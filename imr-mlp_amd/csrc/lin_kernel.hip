// Linear-fit kernels for gfx950 (fp64).
//
//   lin_jac_kernel    one wave per site: the scalar moments (the site's
//                     energy components) and the sparse site Jacobian
//                     L[s][b] = dm_s/dm_b, exported in walk order
//                     (PotMTP::CalcEFSCmpt_R, potentials/potential_mtp.cpp:
//                     2675-2707, over CalcSiteBasisDers, :3163-3280)
//   lin_tile_kernel   one wave per (structure, chunk of scalars): force rows
//                     sum_{e in list(i)} D_e - sum_{e: idx[e] = i} D_e with
//                     D_e = dm_s/dr_e = sum_b L[s][b] grad_r(f_b Y_b)(r_e),
//                     accumulated in an LDS tile in site order, and the
//                     stress components -sum_e D_e r_e
//   lin_reduce_kernel energy components and species counts per structure,
//                     ordered
//   rows_kernel       AddLinearFast rows (train/train_mtp.cpp:1289-1395):
//                     component rows scaled by sqrt(w), targets sqrt(w) y
//
// The reference propagates the Jacobian of every moment w.r.t. all 3 n_i
// coordinates through the rules.  Here the scalar moments are
// differentiated through L instead: L comes from a step table (the
// rule-table machinery) once per site, then lanes take neighbour entries and
// form D_e for a chunk of scalars at a time.  The chunks group scalars that
// share basic moments (build_lin_plan).
//
// The file is compiled twice (two objects, so the two halves of the longest
// compile run in parallel): MTPX_LIN_PART 2 holds the tile kernels of the
// compiled level-16 walk and of level 20 (launch_lin_tile_part2); the
// default part holds everything else.
#include "mtp_device.hpp"

#include <type_traits>

#ifndef MTPX_LIN_PART
#define MTPX_LIN_PART 1
#endif

namespace mtpx {
namespace {
#include "lin_plan_level16.inc"
}  // namespace
}  // namespace mtpx

namespace mtpx {

namespace {

// Read-only model table in the constant address space: wave-uniform
// indices compile to scalar loads (SGPRs, no VALU work).
typedef const int __attribute__((address_space(4))) const_int;

// The tables of one chunk for a walk.  Compile-time walks (exact
// profiles) read the chunk's slot masks (4 per word) with scalar loads and
// hold its L values in walk order in two lane registers, read with
// readlane: no dependent vector load in the walk.  Runtime walks read the
// per-slot mask and L-index tables.
struct LinWalk {
    const int *mask;      // [nslots]
    const int *lidx;      // [nslots][kLinChunk]
    const const_int *mw;  // [kLinMaskWords] slot masks of the chunk, 4 per word
    double lc0, lc1;      // lane l: L values of entries l and 64 + l
    int pos;              // next entry (uniform)
    const double *lch;    // runtime walks of the tile kernel: L values in walk order
};

__device__ __forceinline__ double readlane_d(double v, int l)
{
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, l);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Compile-time loop: f(integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f)
{
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Inverse of shell_index: the (a, b) of the i-th monomial of shell nu.
constexpr int shell_a(int nu, int i)
{
    int a = nu;
    while (i > nu - a) {
        i -= nu - a + 1;
        --a;
    }
    return a;
}
constexpr int shell_b(int nu, int i)
{
    int a = nu;
    while (i > nu - a) {
        i -= nu - a + 1;
        --a;
    }
    return nu - a - i;
}
constexpr bool shell_inverse_ok()
{
    for (int nu = 0; nu <= kMaxNu; ++nu)
        for (int i = 0; i < shell_size(nu); ++i)
            if (shell_index(nu, shell_a(nu, i), shell_b(nu, i)) != i || shell_b(nu, i) < 0)
                return false;
    return true;
}
static_assert(shell_inverse_ok(), "shell_a/shell_b must invert shell_index");

// The entries of one slot of the chunk: each scalar k whose bit is set in
// the slot's mask gets L[k][slot] * grad_r(f Y) added to its derivative
// (registers; the mask and its bits are wave-uniform).
template <class P>
__device__ __forceinline__ void lin_apply(int mk, int sl, double gx, double gy, double gz,
                                          LinWalk &w, const double *ws,
                                          double (&acc)[kLinAcc])
{
    static_for<0, kLinChunk>([&](auto K) __attribute__((always_inline)) {
        constexpr int k = decltype(K)::value;
        if (mk & (1 << k)) {
            double lv;
            if constexpr (P::exact) {
                const int e = w.pos++;
                lv = readlane_d(e < 64 ? w.lc0 : w.lc1, e & 63);
            } else {
                lv = w.lch ? w.lch[w.pos++] : ws[w.lidx[(size_t)sl * kLinChunk + k]];
            }
            acc[3 * k] += lv * gx;
            acc[3 * k + 1] += lv * gy;
            acc[3 * k + 2] += lv * gz;
        }
    });
}

// Walk of the slots (nu, mu, alpha) in slot order for one chunk.  Where the
// chunk's mask of a slot is set, grad_r(f Y) = (f' - nu f/d) Y u + (f/d)
// grad_u Y is formed once and applied to the slot's entries.  The exact
// profiles walk at compile time (constant slot and monomial indices, masks
// read from lane registers); the runtime profiles loop and read the mask
// table.
template <int NU, class P>
__device__ __forceinline__ void lin_shells(const DevModel &m, const Nbr<P::M> &q,
                                           const double *prev, int &slot, LinWalk &w,
                                           const double *ws, double (&acc)[kLinAcc])
{
    double cur[shell_size(NU)];
    if constexpr (NU == 0)
        cur[0] = 1.0;
    else
        next_shell<NU, P::M>(prev, cur, q);
    if constexpr (P::exact) {
        static_for<0, P::M>([&](auto MU) __attribute__((always_inline)) {
            constexpr int mu = decltype(MU)::value;
            if (P::active(m, mu, NU)) {
                __builtin_amdgcn_sched_barrier(0);
                const double h = q.fd[mu] - NU * q.f[mu] * q.invd;
                const double fdi = q.f[mu] * q.invd;
                static_for<0, shell_size(NU)>([&](auto I) __attribute__((always_inline)) {
                    constexpr int i = decltype(I)::value;
                    constexpr int a = shell_a(NU, i), b = shell_b(NU, i), c = NU - a - b;
                    const int sl = slot + i;
                    const int word = w.mw[sl / 4];
                    const int mk = (word >> (8 * (sl % 4))) & 0xff;
                    if (mk) {
                        const double hy = h * cur[i];
                        double gx = hy * q.ux, gy = hy * q.uy, gz = hy * q.uz;
                        if constexpr (a > 0) {
                            constexpr int ix = shell_index(NU - 1, a - 1, b);
                            gx += (a * fdi) * prev[ix];
                        }
                        if constexpr (b > 0) {
                            constexpr int iy = shell_index(NU - 1, a, b - 1);
                            gy += (b * fdi) * prev[iy];
                        }
                        if constexpr (c > 0) {
                            constexpr int iz = shell_index(NU - 1, a, b);
                            gz += (c * fdi) * prev[iz];
                        }
                        lin_apply<P>(mk, sl, gx, gy, gz, w, ws, acc);
                    }
                });
                slot += shell_size(NU);
            }
        });
    } else {
#pragma unroll
        for (int mu = 0; mu < P::M; ++mu) {
            if (P::active(m, mu, NU)) {
                const double h = q.fd[mu] - NU * q.f[mu] * q.invd;
                const double fdi = q.f[mu] * q.invd;
                for (int a = NU; a >= 0; --a)
                    for (int b = NU - a; b >= 0; --b) {
                        const int i = shell_index(NU, a, b), sl = slot + i;
                        const int mk = w.mask[sl];
                        if (!mk)
                            continue;
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
                        lin_apply<P>(mk, sl, gx, gy, gz, w, ws, acc);
                    }
                slot += shell_size(NU);
            }
        }
    }
    if constexpr (NU < P::NUMAX) {
        if (P::deeper(m, NU))
            lin_shells<NU + 1, P>(m, q, cur, slot, w, ws, acc);
    }
}

// ---- walk of a compiled plan ---------------------------------------------
// For a model whose plan equals a generated table (lin_plan_*.inc) every
// mask, walk position and L index is a compile-time constant: the walk is
// straight-line code over the chunk's used slots only, with each L value an
// LDS broadcast read at a constant offset (no mask tests, no readlane).

constexpr int popc(int x)
{
    int n = 0;
    for (; x; x &= x - 1)
        ++n;
    return n;
}

// First slot of the (nu, mu) block of an exact profile: degree ascending,
// then mu ascending over the functions that reach the degree.
template <class P>
constexpr int exact_slot_base(int nu, int mu)
{
    int s = 0;
    for (int v = 0; v < nu; ++v)
        for (int u = 0; u < P::M; ++u)
            if (P::nm[u] >= v)
                s += shell_size(v);
    for (int u = 0; u < mu; ++u)
        if (P::nm[u] >= nu)
            s += shell_size(nu);
    return s;
}

template <class P>
constexpr int exact_slot_count()
{
    return exact_slot_base<P>(P::NUMAX + 1, 0);
}

// Walk position of the first entry of slot `sl` in chunk `c`.
template <class CP>
constexpr int walk_pos(int c, int sl)
{
    int e = 0;
    for (int s = 0; s < sl; ++s)
        e += popc(CP::mask[c][s]);
    return e;
}

// The L values of the chunk's walk come in walk order in two lane
// registers (lane l holds entries l and 64 + l), read with readlane at
// constant lanes.
template <class CP, int C, int NU, class P>
__device__ __forceinline__ void lin_shells_cp(const Nbr<P::M> &q, const double *prev,
                                              double (&acc)[kLinAcc], double lc0, double lc1)
{
    double cur[shell_size(NU)];
    if constexpr (NU == 0)
        cur[0] = 1.0;
    else
        next_shell<NU, P::M>(prev, cur, q);
    static_for<0, P::M>([&](auto MU) __attribute__((always_inline)) {
        constexpr int mu = decltype(MU)::value;
        if constexpr (P::nm[mu] >= NU) {
            const double h = q.fd[mu] - NU * q.f[mu] * q.invd;
            const double fdi = q.f[mu] * q.invd;
            static_for<0, shell_size(NU)>([&](auto I) __attribute__((always_inline)) {
                constexpr int i = decltype(I)::value;
                constexpr int sl = exact_slot_base<P>(NU, mu) + i;
                constexpr int mk = CP::mask[C][sl];
                if constexpr (mk != 0) {
                    constexpr int a = shell_a(NU, i), b = shell_b(NU, i), c = NU - a - b;
                    const double hy = h * cur[i];
                    double gx = hy * q.ux, gy = hy * q.uy, gz = hy * q.uz;
                    if constexpr (a > 0)
                        gx += (a * fdi) * prev[shell_index(NU - 1, a - 1, b)];
                    if constexpr (b > 0)
                        gy += (b * fdi) * prev[shell_index(NU - 1, a, b - 1)];
                    if constexpr (c > 0)
                        gz += (c * fdi) * prev[shell_index(NU - 1, a, b)];
                    constexpr int e0 = walk_pos<CP>(C, sl);
                    static_for<0, kLinChunk>([&](auto K) __attribute__((always_inline)) {
                        constexpr int k = decltype(K)::value;
                        if constexpr ((mk >> k) & 1) {
                            constexpr int e = e0 + popc(mk & ((1 << k) - 1));
                            const double lv = readlane_d(e < kWave ? lc0 : lc1, e % kWave);
                            acc[3 * k] += lv * gx;
                            acc[3 * k + 1] += lv * gy;
                            acc[3 * k + 2] += lv * gz;
                        }
                    });
                }
            });
        }
    });
    if constexpr (NU < P::NUMAX)
        lin_shells_cp<CP, C, NU + 1, P>(q, cur, acc, lc0, lc1);
}

// The compiled walk of chunk `ch` (a chain of uniform compares).
template <class CP, int C, class P>
__device__ __forceinline__ void lin_chunk_cp(int ch, const Nbr<P::M> &q, double (&acc)[kLinAcc],
                                             double lc0, double lc1)
{
    if (ch == C) {
        lin_shells_cp<CP, C, 0, P>(q, nullptr, acc, lc0, lc1);
        return;
    }
    if constexpr (C + 1 < CP::nchunks)
        lin_chunk_cp<CP, C + 1, P>(ch, q, acc, lc0, lc1);
}

// ---- tile path --------------------------------------------------------------
// lin_jac_kernel, one wave per site: the scalar moments (energy components)
// and the site Jacobian L, whose values the walks read, exported in walk
// order (chunk after chunk) to lw[site][nwalk].
template <class P, int kMaxWaves>
__global__ __launch_bounds__(kWave *kMaxWaves) void lin_jac_kernel(DevModel m, DevLin L,
                                                                   DevNeighbors nb, LinGroup g)
{
    extern __shared__ double lds[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nwaves = blockDim.x / kWave;
    const Shared Ls = shared_layout(m, lds, false);  // no adjoint seeds
    double *ws = lds + shared_doubles(m, false, false) + (size_t)wave * L.priv;
    double *mom = ws, *red = ws + L.red0;

    stage_shared(m, Ls, false, tid, blockDim.x);
    for (int k = L.dummy + lane; k < L.red0; k += kWave)
        ws[k] = 0.0;
    // the walk order's work-space indices, the same for every site: held in
    // lane registers where they fit (entry lane + 64 k in register k)
    constexpr int kWalkRegs = 16;
    const bool walk_regs = L.nwalk <= kWalkRegs * kWave;
    int widx[kWalkRegs];
#pragma unroll
    for (int k = 0; k < kWalkRegs; ++k) {
        const int e = lane + kWave * k;
        widx[k] = walk_regs && e < L.nwalk ? L.walk[e] : 0;
    }
    __syncthreads();

    for (int i = g.a0 + blockIdx.x * nwaves + wave; i < g.a1; i += gridDim.x * nwaves) {
        const int ti = nb.center_type[i];
        const int beg = nb.offsets[i];
        const int n = nb.offsets[i + 1] - beg;
        for (int k = lane; k < m.K; k += kWave)
            mom[k] = 0.0;
        wave_sync();
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
        run_rules<false, false>(L.fwd_steps, L.fwd_level_step, L.fwd_level_comb, L.fwd_comb,
                                L.nfwd, ws, lane);
        double *srow = g.site + (size_t)(i - g.a0) * m.S;
        for (int s = lane; s < m.S; s += kWave)
            srow[s] = mom[Ls.map[s]];
        for (int k = L.one + lane; k < L.L0 + L.nL; k += kWave)
            ws[k] = k == L.one ? 1.0 : 0.0;
        wave_sync();
        run_rules<false, false>(L.steps, L.level_step, L.level_comb, L.comb, L.nlev, ws, lane);
        double *lw = g.lw + (size_t)(i - g.a0) * L.nwalk;
        if (walk_regs) {
#pragma unroll
            for (int k = 0; k < kWalkRegs; ++k)
                if (lane + kWave * k < L.nwalk)
                    lw[lane + kWave * k] = ws[widx[k]];
        } else {
            for (int e = lane; e < L.nwalk; e += kWave)
                lw[e] = ws[L.walk[e]];
        }
        wave_sync();
    }
}

// One (structure, chunk) per wave: the force rows of the structure's atoms
// for the chunk's scalars,
//   fc[i][a][Z+s] = sum_{e in list(i)} D_e[a][s] - sum_{e: idx[e] = i} D_e[a][s],
// accumulated over the structure's sites in the wave's own tile (in LDS, or
// for a structure larger than a tile in the rows of fc itself), in site
// order: one wave is the only writer of its rows, so the sums are
// repeatable.  The structure's stress components -sum_e D_e[a][s] r_e[b]
// (a <= b; the tensor is symmetric) are summed per lane in registers and
// over the wave at the end.  The site's walk-order L values come in lane
// registers (compiled and exact walks) or through a stage in LDS (run-time
// walks).
template <class P, class CP>
__global__ __launch_bounds__(kWave) void lin_tile_kernel(DevModel m, DevLin L, DevNeighbors nb,
                                                         LinTile t)
{
    const bool lds_tile = t.rows_cap > 0;
    extern __shared__ double lds[];
    const int lane = threadIdx.x;
    // chunk-major: the waves that run at the same time mostly walk the same
    // chunk, whose code then stays in the instruction cache
    const int item = blockIdx.x;
    if (item >= t.count * t.nchunks)
        return;
    const int c = t.structs[item % t.count], ch = item / t.count;
    const int i0 = t.soff[c], i1 = t.soff[c + 1], N = i1 - i0;
    // the chunk's scalars: its output columns are Z + cols[k]
    const int q0 = L.chunk_s0[ch], w = L.chunk_s0[ch + 1] - q0;
    const int *cols = L.chunk_scalar + q0;
    const int wb = L.walk_off[ch], ne = L.walk_off[ch + 1] - wb;
    // tile row: [3][kLinChunk] and one pad double, so that rows are an odd
    // number of doubles apart and the lanes' atomics on different rows fall
    // in different banks
    constexpr int kRow = 3 * kLinChunk + 1;

    // compiled and exact walks read a site's L values from lane registers;
    // the run-time walks from a stage in LDS
    constexpr bool kLaneL = !std::is_void_v<CP> || P::exact;
    double *coef = lds;
    const int ncr = m.Z * m.Z * m.M * m.R;
    double *lch = lds + ((ncr + 3) & ~3);
    double *tile = lch + (kLaneL ? 0 : ((L.max_walk + 3) & ~3));
    for (int k = lane; k < ncr; k += kWave)
        coef[k] = m.radial[k];
    if (lds_tile)
        for (int k = lane; k < N * kRow; k += kWave)
            tile[k] = 0.0;
    // The stress of a scalar, sum over sites of the site virial of a
    // rotation-invariant function of the site's neighbour vectors, is
    // symmetric: the upper triangle is summed (component u is (kSymA[u],
    // kSymB[u])) and mirrored.
    constexpr int kSymA[6] = {0, 0, 0, 1, 1, 2}, kSymB[6] = {0, 1, 2, 1, 2, 2};
    double st[6 * kLinChunk];
#pragma unroll
    for (int k = 0; k < 6 * kLinChunk; ++k)
        st[k] = 0.0;
    // fc rows of the structure: fc[(i0 + j) 3p + a p + Z + cols[k]]
    double *frow = t.fc + (size_t)i0 * 3 * t.p + t.Z;
    int col[kLinChunk];  // uniform
#pragma unroll
    for (int k = 0; k < kLinChunk; ++k)
        col[k] = k < w ? cols[k] : 0;
    wave_sync();

    // The next site's first 128 L values and first batch of entries are
    // fetched one site ahead (a wave per SIMD: their latency would otherwise
    // stall it); the rest of a long walk and further batches load in place.
    auto fetch_l = [&](int i, double &l0, double &l1) {
        const double *src = t.lw + (size_t)(i - t.a0) * L.nwalk + wb;
        l0 = lane < ne ? src[lane] : 0.0;
        l1 = kWave + lane < ne ? src[kWave + lane] : 0.0;
    };
    // List bounds and species are read two sites ahead with vector loads
    // (lane-dependent addresses; lanes 0 and 1 hold begin and end) and taken
    // into scalars at the top of the next site, so that the next site's
    // entries can be fetched a whole site ahead: scalar loads would share
    // the LDS wait counter and make every LDS wait wait for them too.
    int zero = 0;
    asm volatile("" : "+v"(zero));  // a lane value the compiler cannot fold
    int vb = 0, vt = 0;
    auto fetch_bounds = [&](int i) {
        vb = nb.offsets[i + (lane & 1)];
        vt = nb.center_type[i + zero];
    };
    int nbeg = 0, nend = 0, nti = 0;  // the next site's bounds and species
    auto take_bounds = [&]() {
        nbeg = __builtin_amdgcn_readlane(vb, 0);
        nend = __builtin_amdgcn_readlane(vb, 1);
        nti = __builtin_amdgcn_readfirstlane(vt);
    };
    double nl0 = 0.0, nl1 = 0.0;
    EntryRaw nx{0.0, 0.0, 0.0, 0.0, 0, -1};
    int cbeg = 0, cend = 0, cti = 0;  // this site's
    if (i0 < i1) {
        fetch_bounds(i0);
        take_bounds();
        cbeg = nbeg;
        cend = nend;
        cti = nti;
        fetch_l(i0, nl0, nl1);
        nx = fetch_entry(nb, cbeg + lane, lane < cend - cbeg);
        if (i0 + 1 < i1)
            fetch_bounds(i0 + 1);
    }
    for (int i = i0; i < i1; ++i) {
        const double cl0 = nl0, cl1 = nl1;
        if (i + 1 < i1)
            take_bounds();  // the next site's, loaded at the end of the last walk
        if constexpr (!kLaneL) {
            if (lane < ne)
                lch[lane] = nl0;
            if (kWave + lane < ne)
                lch[kWave + lane] = nl1;
            if (ne > 2 * kWave) {
                const double *src = t.lw + (size_t)(i - t.a0) * L.nwalk + wb;
                for (int e = 2 * kWave + lane; e < ne; e += kWave)
                    lch[e] = src[e];
            }
        }
        const EntryRaw first = nx;
        const int ti = cti, beg = cbeg, n = cend - cbeg;
        if constexpr (!kLaneL)
            wave_sync();
        // at least one pass, for the next site's loads below, also for a
        // site without neighbours (its pass adds zeros)
        for (int base = 0; base < max(n, 1); base += kWave) {
            const bool valid = lane < n - base;
            const int64_t pe = beg + base + lane;
            const EntryRaw en = base == 0 ? first : fetch_entry(nb, pe, valid);
            Nbr<P::M> q;
            neighbor_from<P>(m, coef, ti, en, valid, q);
            // The next site's loads are issued once this batch's entry is in
            // registers: loads still in flight at the top of this loop would
            // make its wait for the entry wait for them too.
            if (base == 0 && i + 1 < i1) {
                fetch_l(i + 1, nl0, nl1);
                nx = fetch_entry(nb, nbeg + lane, lane < nend - nbeg);
                cbeg = nbeg;
                cend = nend;
                cti = nti;
            }
            double acc[kLinAcc];
#pragma unroll
            for (int r = 0; r < kLinAcc; ++r)
                acc[r] = 0.0;
            if constexpr (!std::is_void_v<CP>) {
                lin_chunk_cp<CP, 0, P>(ch, q, acc, cl0, cl1);
            } else {
                LinWalk wk;
                wk.pos = 0;
                wk.lch = nullptr;
                if constexpr (P::exact) {
                    wk.mw = (const const_int *)(L.maskw + (size_t)ch * kLinMaskWords);
                    wk.lc0 = cl0;
                    wk.lc1 = cl1;
                } else {
                    wk.mask = L.slot_mask + (size_t)ch * m.nslots;
                    wk.lch = lch;
                }
                int slot = 0;
                lin_shells<0, P>(m, q, nullptr, slot, wk, lch, acc);
            }
            // the bounds of the site after next: loaded after the walk (a
            // value loaded before it could be moved between registers inside
            // the walk, which then waits for every load in flight), taken at
            // the top of the next site
            if (base == 0 && i + 2 < i1)
                fetch_bounds(i + 2);
            // the neighbour's row: minus this entry's derivatives
            const int jl = valid ? en.j - i0 : -1;
            if ((unsigned)jl < (unsigned)N) {
                if (lds_tile) {
                    double *row = tile + (size_t)jl * kRow;
#pragma unroll
                    for (int k = 0; k < kLinChunk; ++k)
                        if (k < w)
#pragma unroll
                            for (int a = 0; a < 3; ++a)
                                atomicAdd(row + a * kLinChunk + k, -acc[3 * k + a]);
                } else {
                    double *row = frow + (size_t)jl * 3 * t.p;
#pragma unroll
                    for (int k = 0; k < kLinChunk; ++k)
                        if (k < w)
#pragma unroll
                            for (int a = 0; a < 3; ++a)
                                atomicAdd(row + (size_t)a * t.p + col[k], -acc[3 * k + a]);
                }
            }
            // stress: -D_a r_b for a <= b
            const double r3[3] = {q.x, q.y, q.z};
#pragma unroll
            for (int k = 0; k < kLinChunk; ++k)
#pragma unroll
                for (int u = 0; u < 6; ++u)
                    st[u * kLinChunk + k] -= acc[3 * k + kSymA[u]] * r3[kSymB[u]];
            // the centre's row: the sum of this batch's derivatives
            int vi;
            const double v = wave_reduce_scatter<kLinAcc>(acc, lane, vi);
            if (vi >= 0 && vi / 3 < w) {
                const int k = vi / 3, a = vi % 3;
                if (lds_tile)
                    atomicAdd(tile + (size_t)(i - i0) * kRow + a * kLinChunk + k, v);
                else
                    atomicAdd(frow + (size_t)(i - i0) * 3 * t.p + (size_t)a * t.p + cols[k], v);
            }
        }
        if constexpr (!kLaneL)
            wave_sync();  // the next site's values overwrite the stage
    }
    if (lds_tile) {
        wave_sync();
        for (int k = lane; k < N * 3 * w; k += kWave) {
            const int j = k / (3 * w), r = k % (3 * w), a = r / w, kk = r % w;
            frow[(size_t)j * 3 * t.p + (size_t)a * t.p + cols[kk]] =
                tile[(size_t)j * kRow + a * kLinChunk + kk];
        }
    }
#pragma unroll
    for (int u = 0; u < 6; ++u)
#pragma unroll
        for (int k = 0; k < kLinChunk; ++k)
            if (k < w) {
                const double v = wave_sum(st[u * kLinChunk + k]);
                if (lane == 0) {
                    const int a = kSymA[u], b = kSymB[u];
                    t.sc[((size_t)c * 9 + 3 * a + b) * t.p + t.Z + col[k]] = v;
                    if (a != b)
                        t.sc[((size_t)c * 9 + 3 * b + a) * t.p + t.Z + col[k]] = v;
                }
            }
}

#if MTPX_LIN_PART == 1
// Energy components of a group's structures: ordered sums of the sites'
// scalar moments over each structure's atoms, and the species counts.
// Threads [0, nc S) take the sums, one per (structure, scalar), and the
// next nc Z the counts, so no wave runs both loops.
__global__ __launch_bounds__(256) void lin_reduce_kernel(int S, int Z, int p, const int *soff,
                                                         const int *center_type, LinGroup g,
                                                         double *ec)
{
    const int64_t nc = g.c1 - g.c0;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nc * (S + Z))
        return;
    const bool sum = t < nc * S;
    const int64_t u = sum ? t : t - nc * S;
    const int c = g.c0 + (int)(sum ? u / S : u / Z);
    const int r = sum ? (int)(u % S) : S + (int)(u % Z);
    const int i0 = soff[c], i1 = soff[c + 1];
    if (sum) {
        // loads of several atoms in flight; the sum stays in atom order
        const double *src = g.site + (size_t)(i0 - g.a0) * S + r;
        const size_t st = (size_t)S;
        double acc = 0.0;
        int i = i0;
        for (; i + 8 <= i1; i += 8, src += 8 * st) {
            double v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = src[k * st];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                acc += v[k];
        }
        for (; i < i1; ++i, src += st)
            acc += *src;
        ec[(size_t)c * p + Z + r] = acc;
    } else {
        const int sp = r - S;
        int cnt = 0, i = i0;
        for (; i + 8 <= i1; i += 8) {  // eight loads in flight
            int v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = center_type[i + k];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                cnt += v[k] == sp;
        }
        for (; i < i1; ++i)
            cnt += center_type[i] == sp;
        ec[(size_t)c * p + sp] = (double)cnt;
    }
}

// Clears what the linear-fit kernels leave unwritten: the species columns
// of the force rows and the stress rows (whole).
__global__ __launch_bounds__(256) void lin_clear_kernel(double *comp, int64_t frows, int64_t srows,
                                                        int p, int Z)
{
    const int64_t nf = frows * Z, total = nf + srows * p;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        if (t < nf)
            comp[(t / Z) * p + t % Z] = 0.0;
        else
            comp[frows * p + (t - nf)] = 0.0;
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

// Waves per workgroup: the level-10 kernel fits 256 registers (eight waves);
// the others use up to 512 (one wave per SIMD).
#endif  // MTPX_LIN_PART == 1

template <class P>
constexpr int lin_waves()
{
    return std::is_same_v<P, ProfLevel10> ? 8 : 4;
}

template <class P>
void launch_jac_variant(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                        const LinGroup &g, const EfsLaunch &cfg, hipStream_t s)
{
    constexpr int W = lin_waves<P>();
    hipLaunchKernelGGL((lin_jac_kernel<P, W>), dim3(cfg.grid), dim3(kWave * cfg.waves),
                       cfg.lds_bytes, s, m, L, nb, g);
}

template <class P, class CP = void>
void launch_tile_variant(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                         const LinTile &t, size_t lds_bytes, hipStream_t s)
{
    const int items = t.count * t.nchunks;
    const unsigned grid = (unsigned)((items + 7) / 8 * 8);
    hipLaunchKernelGGL((lin_tile_kernel<P, CP>), dim3(grid), dim3(kWave), lds_bytes, s, m, L, nb,
                       t);
}

static_assert(exact_slot_count<ProfLevel16>() == LinPlanLevel16::nslots,
              "the compiled level-16 walk must cover the level-16 profile's slots");

}  // namespace

#if MTPX_LIN_PART == 2
// tile kernels of variant 5 (level 16, compiled walk) and 1 (level 20)
void launch_lin_tile_part2(int variant, const DevModel &m, const DevLin &L,
                           const DevNeighbors &nb, const LinTile &t, size_t lds_bytes,
                           hipStream_t s)
{
    if (variant == 5)
        launch_tile_variant<ProfLevel16, LinPlanLevel16>(m, L, nb, t, lds_bytes, s);
    else
        launch_tile_variant<ProfLevel20>(m, L, nb, t, lds_bytes, s);
}
#else
// in the other object of this file
void launch_lin_tile_part2(int variant, const DevModel &m, const DevLin &L,
                           const DevNeighbors &nb, const LinTile &t, size_t lds_bytes,
                           hipStream_t s);

// The E/F/S variant, or the generic one where the compile-time walk's
// tables do not hold the plan; 5: the level-16 profile with the compiled
// level-16 walk.
int lin_variant(const DevModel &m, const DevLin &L)
{
    const int v = efs_variant(m, m.R);
    if (v == 0 && L.compiled_walk)
        return 5;
    return v <= 2 && !L.lane_walk ? 4 : v;
}

// True when the plan equals the compiled level-16 walk (same chunks and
// scalars, masks and L indices), so that walk computes exactly what the run-time walk would.
bool lin_walk_compiled(const LinPlan &lp, int nslots)
{
    using CP = LinPlanLevel16;
    if (!lp.lane_walk || lp.nchunks != CP::nchunks || nslots != CP::nslots)
        return false;
    for (int c = 0; c <= CP::nchunks; ++c)
        if (lp.chunk_s0[c] != CP::chunk_s0[c])
            return false;
    for (int q = 0; q < CP::S; ++q)
        if ((int)lp.chunk_scalar.size() != CP::S || lp.chunk_scalar[q] != CP::scalar[q])
            return false;
    for (int c = 0; c < CP::nchunks; ++c) {
        for (int s = 0; s < CP::nslots; ++s)
            if (lp.slot_mask[(size_t)c * nslots + s] != CP::mask[c][s])
                return false;
        for (int e = 0; e < kLinEntries; ++e)
            if (lp.clist[(size_t)c * kLinEntries + e] != CP::clist[c][e])
                return false;
    }
    return true;
}

bool lin_configure(const DevModel &m, const DevLin &L, int n, int num_cus, size_t lds_limit,
                   EfsLaunch &cfg)
{
    const size_t sh = shared_doubles(m, false, false) * sizeof(double);
    const size_t priv = (size_t)L.priv * sizeof(double);
    if (sh + priv > lds_limit)
        return false;
    cfg.lds_tables = false;
    const int wcap = lin_variant(m, L) == 2 ? 8 : 4;
    cfg.waves = (int)std::min<size_t>(wcap, (lds_limit - sh) / priv);
    cfg.lds_bytes = sh + cfg.waves * priv;
    const int per_cu = std::max<int>(1, (int)(lds_limit / cfg.lds_bytes));
    const int need = (std::max(n, 1) + cfg.waves - 1) / cfg.waves;
    cfg.grid = std::max(1, std::min(need, num_cus * per_cu));
    cfg.rows = cfg.grid * cfg.waves;
    return true;
}

size_t lin_tile_lds(const DevModel &m, const DevLin &L, int rows)
{
    const size_t ncr = ((size_t)m.Z * m.Z * m.M * m.R + 3) & ~size_t(3);
    // the L-value stage of the run-time walks (the small and generic profiles)
    const int v = lin_variant(m, L);
    const size_t stage = v == 3 || v == 4 ? ((size_t)L.max_walk + 3) & ~size_t(3) : 0;
    return sizeof(double) * (ncr + stage + (size_t)rows * (3 * kLinChunk + 1));
}

hipError_t launch_lin_jac(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                          const LinGroup &g, const EfsLaunch &cfg, hipStream_t s)
{
    if (g.a1 <= g.a0)
        return hipSuccess;
    switch (lin_variant(m, L)) {
    case 0:
    case 5: launch_jac_variant<ProfLevel16>(m, L, nb, g, cfg, s); break;
    case 1: launch_jac_variant<ProfLevel20>(m, L, nb, g, cfg, s); break;
    case 2: launch_jac_variant<ProfLevel10>(m, L, nb, g, cfg, s); break;
    case 3: launch_jac_variant<ProfSmall>(m, L, nb, g, cfg, s); break;
    default: launch_jac_variant<ProfGeneric>(m, L, nb, g, cfg, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_lin_tile(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                           const LinTile &t, hipStream_t s)
{
    if (t.count <= 0 || t.nchunks <= 0)
        return hipSuccess;
    const size_t lds = lin_tile_lds(m, L, t.rows_cap);
    switch (const int v = lin_variant(m, L)) {
    case 0: launch_tile_variant<ProfLevel16>(m, L, nb, t, lds, s); break;
    case 1:
    case 5: launch_lin_tile_part2(v, m, L, nb, t, lds, s); break;
    case 2: launch_tile_variant<ProfLevel10>(m, L, nb, t, lds, s); break;
    case 3: launch_tile_variant<ProfSmall>(m, L, nb, t, lds, s); break;
    default: launch_tile_variant<ProfGeneric>(m, L, nb, t, lds, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_lin_clear(double *comp, int64_t frows, int64_t srows, int p, int Z,
                            hipStream_t s)
{
    const int64_t total = frows * Z + srows * p;
    if (total > 0)
        hipLaunchKernelGGL(lin_clear_kernel,
                           dim3((unsigned)std::min<int64_t>((total + 255) / 256, 4096)), dim3(256),
                           0, s, comp, frows, srows, p, Z);
    return hipGetLastError();
}

hipError_t launch_lin_reduce(const DevModel &m, const int *soff, const int *center_type,
                             const LinGroup &g, double *ec, hipStream_t s)
{
    const int64_t work = (int64_t)(g.c1 - g.c0) * (m.S + m.Z);
    if (work > 0)
        hipLaunchKernelGGL(lin_reduce_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                           s, m.S, m.Z, m.Z + m.S, soff, center_type, g, ec);
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

#endif  // MTPX_LIN_PART
}  // namespace mtpx
