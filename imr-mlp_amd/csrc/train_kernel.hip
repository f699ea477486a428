// Training kernels for gfx950 (fp64).
//
//   structure_reduce_kernel  per-structure energy and virial from site values
//                            (the virial when per-atom virials are given)
//   loss_kernel              weighted E/F/S loss, its adjoints dL/dE, dL/dF,
//                            dL/dS and the seven metrics, one wave per
//                            structure (Trainer_MTP::AddLossGard,
//                            train/train_mtp.cpp:3839-3996)
//   grad_kernel              coefficient gradient of
//                              G = sum_i [dLdE_c E_i + sum_j W_ij . dE_i/dr_ij]
//                              W_ij = dLdF_i - dLdF_idx(j) - dLdS_c r_ij
//                            (AccumulateEFSCombinationGard,
//                            potentials/potential_mtp.cpp:6896-6923, over
//                            accumulate_site_parameter_gradient, :3348-3550)
//   rows_reduce_kernel       ordered sum of the per-wave gradient rows
//
// The gradient kernel runs one wave per atom, like the E/F/S kernel, in
// directional form instead of forming the reference's per-pair Jacobians:
//   1. lanes over neighbours: basic moments m_b = sum_j f Y and their
//      tangents along W, q_b = sum_j W_j . grad_r(f Y), reduced together
//      through the transpose buffer;
//   2. the product rules carry (m, Q) forward: Q_o += c (Q_l m_r + m_l Q_r);
//      then dG/dxi_s = dLdE m_map(s) + Q_map(s);
//   3. reverse rules carry (A, Gb) with seeds (xi, dLdE xi):
//      A_x += c A_o m_r,  Gb_x += c (Gb_o m_r + A_o Q_r), so at a basic
//      Gb_b = dG/dm_b and A_b = dG/dq_b;
//   4. lanes over neighbours again: with U = sum A Y, V = sum nu A Y,
//      H = sum Gb Y and Wg = sum A W.grad_u(Y) over the basics of radial
//      function mu,
//        dG/dc[ti,tj,mu,k] += alpha Q_k + beta Q'_k,
//        alpha = H - (w_u/d) V + Wg/d,  beta = w_u U,  w_u = W . u,
//      summed over the neighbours of species tj by a typed transpose
//      reduction into the wave's gradient accumulator.
// Each wave accumulates over its atoms in LDS and writes one gradient row;
// the rows are summed in a fixed order, so the gradient is repeatable bit
// for bit for a given launch shape.
#include "mtp_device.hpp"

namespace mtpx {

namespace {

__global__ __launch_bounds__(kWave) void structure_reduce_kernel(const int *soff, int nconf,
                                                                 const double *site_energy,
                                                                 const double *site_virial,
                                                                 double *energy, double *stress)
{
    const int c = blockIdx.x, lane = threadIdx.x;
    if (c >= nconf)
        return;
    double e = 0.0, v[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = soff[c] + lane; i < soff[c + 1]; i += kWave) {
        e += site_energy[i];
        if (site_virial)
#pragma unroll
            for (int k = 0; k < 9; ++k)
                v[k] += site_virial[9 * (size_t)i + k];
    }
    e = wave_sum(e);
#pragma unroll
    for (int k = 0; k < 9; ++k)
        v[k] = wave_sum(v[k]);
    if (lane == 0) {
        energy[c] = e;
        if (stress)
#pragma unroll
            for (int k = 0; k < 9; ++k)
                stress[9 * (size_t)c + k] = v[k];
    }
}

__global__ __launch_bounds__(kWave) void loss_kernel(LossArgs a)
{
    const int c = blockIdx.x, lane = threadIdx.x;
    if (c >= a.nconf)
        return;
    const int a0 = a.soff[c], a1 = a.soff[c + 1], N = a1 - a0;
    const int *act = a.active + 3 * c;  // energy, forces, stress terms in the loss
    double lf = 0.0, sqf = 0.0;
    for (int i = a0 + lane; i < a1; i += kWave) {
        double g0 = 0.0, g1 = 0.0, g2 = 0.0;
        if (act[1]) {
            const double w = a.wF[i];
            const double d0 = a.F[3 * (size_t)i] - a.tF[3 * (size_t)i];
            const double d1 = a.F[3 * (size_t)i + 1] - a.tF[3 * (size_t)i + 1];
            const double d2 = a.F[3 * (size_t)i + 2] - a.tF[3 * (size_t)i + 2];
            const double ff = (d0 * d0 + d1 * d1) + d2 * d2;
            lf += w * ff;
            sqf += ff;
            g0 = 2.0 * w * d0;
            g1 = 2.0 * w * d1;
            g2 = 2.0 * w * d2;
        }
        a.dLdF[3 * (size_t)i] = g0;
        a.dLdF[3 * (size_t)i + 1] = g1;
        a.dLdF[3 * (size_t)i + 2] = g2;
    }
    lf = wave_sum(lf);
    sqf = wave_sum(sqf);
    if (lane != 0)
        return;
    double ls = 0.0, sqs = 0.0, le = 0.0, sqe = 0.0, dE = 0.0;
    double dS[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (N > 0 && act[2]) {
        const double w = a.wS[c];
        for (int q = 0; q < 9; ++q) {
            const double d = a.S[9 * (size_t)c + q] - a.tS[9 * (size_t)c + q];
            sqs += d * d;
            dS[q] = 2.0 * w * d;
        }
        ls = w * sqs;
    }
    if (N > 0 && act[0]) {
        const double w = a.wE[c];
        const double d = a.E[c] - a.tE[c];
        const double ff = d * d;
        le = w * ff;
        sqe = ff / N / N;
        dE = 2.0 * w * d;
    }
    a.dLdE[c] = dE;
    for (int q = 0; q < 9; ++q)
        a.dLdS[9 * (size_t)c + q] = dS[q];
    double *row = a.metric_rows + 7 * (size_t)c;
    row[0] = (lf + ls) + le;
    row[1] = le;
    row[2] = lf;
    row[3] = ls;
    row[4] = sqe;
    row[5] = sqf;
    row[6] = sqs;
}

// Ordered column sums of a [rows][cols] array (metrics, gradient rows).  A
// workgroup takes kRowCols columns; its kRowGroups row groups each sum a
// contiguous run of rows in row order (eight loads in flight), and the
// group sums are added in group order, so the result is the same bits on
// every run.
constexpr int kRowCols = 16, kRowGroups = 16;
__global__ __launch_bounds__(256) void rows_reduce_kernel(const double *rows, int nrows, int cols,
                                                          double *out, int accumulate)
{
    __shared__ double part[kRowGroups][kRowCols];
    const int c = threadIdx.x % kRowCols, g = threadIdx.x / kRowCols;
    const int k = blockIdx.x * kRowCols + c;
    const int per = (nrows + kRowGroups - 1) / kRowGroups;
    const int r1 = min(nrows, (g + 1) * per);
    double s = 0.0;
    if (k < cols) {
        int r = g * per;
        for (; r + 8 <= r1; r += 8) {
            double v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                v[q] = rows[(size_t)(r + q) * cols + k];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                s += v[q];
        }
        for (; r < r1; ++r)
            s += rows[(size_t)r * cols + k];
    }
    part[g][c] = s;
    __syncthreads();
    if (g == 0 && k < cols) {
        double t = part[0][c];
        for (int q = 1; q < kRowGroups; ++q)
            t += part[q][c];
        out[k] = accumulate ? out[k] + t : t;
    }
}

// ---- gradient kernel ---------------------------------------------------

// First slot of the (nu, mu) block in the canonical slot order.
template <class P>
__device__ __forceinline__ int slot_base(const DevModel &m, int nu, int mu)
{
    if constexpr (P::exact) {
        int s = 0;
        for (int n = 0; n < nu; ++n)
            for (int q = 0; q < P::M; ++q)
                if (P::nm[q] >= n)
                    s += shell_size(n);
        for (int q = 0; q < mu; ++q)
            if (P::nm[q] >= nu)
                s += shell_size(nu);
        return s;
    } else {
        return m.slot_base[nu * kMaxMu + mu];
    }
}

// Transpose-buffer reduction of `nrows` rows; tgt(row, sum) for each row.
template <class Tgt>
__device__ __forceinline__ void reduce_rows(const double *red, int nrows, int row0, int lane,
                                            Tgt tgt)
{
    wave_sync();
    const double acc = chunk_row_sum(red, lane);
    if (lane < nrows)
        tgt(row0 + lane, acc);
    wave_sync();
}

// As reduce_rows, with one sum per neighbour species: column j counts for
// species ctype[j] (-1: no neighbour).
template <class Tgt>
__device__ __forceinline__ void reduce_rows_typed(const double *red, int nrows, int row0,
                                                  int lane, const int *ctype, int Z, Tgt tgt)
{
    wave_sync();
    const double2 *row = reinterpret_cast<const double2 *>(red + (lane & (kChunk - 1)) * kRedStride +
                                                           (lane >> 4) * 16);
    const int4 *ty = reinterpret_cast<const int4 *>(ctype + (lane >> 4) * 16);
    double v[16];
    int t[16];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        const double2 x = row[jj];
        v[2 * jj] = x.x;
        v[2 * jj + 1] = x.y;
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int4 x = ty[jj];
        t[4 * jj] = x.x;
        t[4 * jj + 1] = x.y;
        t[4 * jj + 2] = x.z;
        t[4 * jj + 3] = x.w;
    }
    for (int tj = 0; tj < Z; ++tj) {
        double a0 = 0.0, a1 = 0.0;
#pragma unroll
        for (int jj = 0; jj < 16; jj += 2) {
            a0 += t[jj] == tj ? v[jj] : 0.0;
            a1 += t[jj + 1] == tj ? v[jj + 1] : 0.0;
        }
        const double acc = xor16_sum(xor32_sum(a0 + a1));
        if (lane < nrows)
            tgt(row0 + lane, tj, acc);
    }
    wave_sync();
}

struct GradNbr {
    double wx, wy, wz, wu;  // W_ij and W_ij . u
};

// W_ij = dLdF_i - dLdF_idx(j) - dLdS r_ij (zero for lanes without an entry)
template <class P>
__device__ __forceinline__ GradNbr pair_weight(const DevNeighbors &nb, const TrainArgs &t,
                                               const double fi[3], const double S[9],
                                               int64_t p, bool valid, const Nbr<P::M> &q)
{
    GradNbr g{0, 0, 0, 0};
    if (valid) {
        const int j = nb.idx[p];
        double w[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            w[a] = fi[a] - t.dLdF[3 * (size_t)j + a];
            w[a] -= S[3 * a] * q.x;
            w[a] -= S[3 * a + 1] * q.y;
            w[a] -= S[3 * a + 2] * q.z;
        }
        g.wx = w[0];
        g.wy = w[1];
        g.wz = w[2];
        g.wu = (g.wx * q.ux + g.wy * q.uy) + g.wz * q.uz;
    }
    return g;
}

// Rows of the first pass alternate m and q of one slot; the sums go to the
// pair of the slot's basic moment (m at 2b, q at 2b + 1).
struct DualCtx {
    double *red, *ws;
    const int *slot_basic;
    int lane, row;
};

// Powers u_x^k, u_y^k, u_z^k for k = 0 .. N: every monomial of every shell
// is a product of three of them, so the passes below hold 3 (N + 1) values
// per lane instead of two whole shells (at level 20, 27 doubles against 81),
// which lets the kernel run two waves per SIMD.
template <int N, int MMAX>
__device__ __forceinline__ void unit_powers(const Nbr<MMAX> &q, double *px, double *py, double *pz)
{
    px[0] = py[0] = pz[0] = 1.0;
#pragma unroll
    for (int k = 1; k <= N; ++k) {
        px[k] = px[k - 1] * q.ux;
        py[k] = py[k - 1] * q.uy;
        pz[k] = pz[k - 1] * q.uz;
    }
}

// W . grad_u Y_abc = a W_x Y_(a-1)bc + b W_y Y_a(b-1)c + c W_z Y_ab(c-1),
// with the weights (wx, wy, wz) as given
template <int NU>
__device__ __forceinline__ double grad_u_dot(int a, int b, const double *px, const double *py,
                                             const double *pz, double wx, double wy, double wz)
{
    const int c = NU - a - b;
    double gy = 0.0;
    if (a > 0)
        gy = fma(a * wx, px[a - 1] * (py[b] * pz[c]), gy);
    if (b > 0)
        gy = fma(b * wy, px[a] * (py[b - 1] * pz[c]), gy);
    if (c > 0)
        gy = fma(c * wz, px[a] * (py[b] * pz[c - 1]), gy);
    return gy;
}

// Step 1: per (nu, mu) block, rows m = f Y and q = W . grad_r(f Y)
//   = Y (f' - nu f/d) w_u + (f/d) W . grad_u Y.
template <int NU, class P>
__device__ __forceinline__ void fwd_dual_shells(const DevModel &m, DualCtx &cx,
                                                const Nbr<P::M> &q, const GradNbr &g,
                                                const double *px, const double *py,
                                                const double *pz)
{
    auto flush = [&]() {
        reduce_rows(cx.red, kChunk, cx.row - kChunk, cx.lane, [&](int r, double acc) {
            const int b = cx.slot_basic[r >> 1];
            if (b >= 0)
                cx.ws[2 * b + (r & 1)] += acc;
        });
    };
#pragma unroll
    for (int mu = 0; mu < P::M; ++mu) {
        if (P::active(m, mu, NU)) {
            __builtin_amdgcn_sched_barrier(0);
            const double hw = (q.fd[mu] - NU * q.f[mu] * q.invd) * g.wu;
            const double fd = q.f[mu] * q.invd;
#pragma unroll
            for (int a = NU; a >= 0; --a)
#pragma unroll
                for (int b = NU - a; b >= 0; --b) {
                    const double y = px[a] * (py[b] * pz[NU - a - b]);
                    const double gy = grad_u_dot<NU>(a, b, px, py, pz, g.wx, g.wy, g.wz);
                    cx.red[(cx.row % kChunk) * kRedStride + cx.lane] = q.f[mu] * y;
                    ++cx.row;
                    cx.red[(cx.row % kChunk) * kRedStride + cx.lane] = hw * y + fd * gy;
                    ++cx.row;
                    if (cx.row % kChunk == 0)
                        flush();
                }
        }
    }
    if constexpr (NU < P::NUMAX) {
        if (P::deeper(m, NU))
            fwd_dual_shells<NU + 1, P>(m, cx, q, g, px, py, pz);
    }
}

// Step 4, all radial functions at once, monomial by monomial with the
// radial functions innermost: per mu, alpha_mu (without its beta-like
// term) and U_mu,
//   alpha += G Y + A (W/d . grad_u Y - nu (w_u/d) Y),  U += A Y.
template <int NU, class P>
__device__ __forceinline__ void rad_shells(const DevModel &m, const double2 *AG,
                                           const double *px, const double *py, const double *pz,
                                           const GradNbr &g, double invd, double *alpha,
                                           double *U)
{
    const double ncw = -NU * g.wu * invd;
    const double wxd = g.wx * invd, wyd = g.wy * invd, wzd = g.wz * invd;
#pragma unroll
    for (int a = NU; a >= 0; --a)
#pragma unroll
        for (int b = NU - a; b >= 0; --b) {
            const int i = shell_index(NU, a, b);
            const double y = px[a] * (py[b] * pz[NU - a - b]);
            const double t = fma(ncw, y, grad_u_dot<NU>(a, b, px, py, pz, wxd, wyd, wzd));
#pragma unroll
            for (int mu = 0; mu < P::M; ++mu)
                if (P::active(m, mu, NU)) {
                    const double2 w = AG[slot_base<P>(m, NU, mu) + i];  // {A, G}, LDS broadcast
                    U[mu] = fma(w.x, y, U[mu]);
                    alpha[mu] = fma(w.y, y, fma(w.x, t, alpha[mu]));
                }
        }
    if constexpr (NU < P::NUMAX) {
        if (P::deeper(m, NU))
            rad_shells<NU + 1, P>(m, AG, px, py, pz, g, invd, alpha, U);
    }
}

template <class P, bool kTabLds, int kMaxWaves>
__global__ __launch_bounds__(kWave *kMaxWaves) void grad_kernel(DevModel m, DevNeighbors nb,
                                                                TrainArgs t)
{
    extern __shared__ double lds[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nwaves = blockDim.x / kWave;
    const Shared L = shared_layout(m, lds, false);  // seeds are read from global memory
    double *ws = lds + shared_doubles(m, kTabLds, false) + (size_t)wave * m.tr_priv;
    // {value, dual} pairs: {m, Q} for the moments, {A, G} for the adjoints
    double2 *wp = reinterpret_cast<double2 *>(ws);
    double *red1 = ws + m.tr_red1, *red4 = ws + m.tr_red4;
    double2 *AG = reinterpret_cast<double2 *>(ws + m.tr_stage);
    double *grad = ws + m.tr_grad;  // radial part of the gradient
    const int rowid = blockIdx.x * nwaves + wave;
    // species and moment part: accumulated in the wave's own gradient row
    double *grow = t.grad_rows + (size_t)rowid * m.ncoef;
    int *ctype = reinterpret_cast<int *>(ws + m.tr_ctype);

    stage_shared(m, L, kTabLds, tid, blockDim.x);
    for (int k = m.dummy + lane; k < m.red0; k += kWave)
        wp[k] = double2{0.0, 0.0};
    for (int k = lane; k < m.nradial; k += kWave)
        grad[k] = 0.0;
    for (int k = m.nradial + lane; k < m.ncoef; k += kWave)
        grow[k] = 0.0;
    __syncthreads();
    const int2 *fwd_tab = kTabLds ? L.fwd_steps : m.fwd_steps;
    const int2 *bwd_tab = kTabLds ? L.bwd_steps : m.bwd_steps;
    const int MR = P::exact ? P::M * P::RMAX : m.M * m.R;

    for (int i = rowid; i < nb.n; i += gridDim.x * nwaves) {
        const int ti = nb.center_type[i];
        const int beg = nb.offsets[i];
        const int n = nb.offsets[i + 1] - beg;
        const int c = t.center_structure[i];
        const double se = t.dLdE[c];
        double S[9], fi[3];
#pragma unroll
        for (int k = 0; k < 9; ++k)
            S[k] = t.dLdS[9 * (size_t)c + k];
#pragma unroll
        for (int a = 0; a < 3; ++a)
            fi[a] = t.dLdF[3 * (size_t)i + a];
        for (int k = lane; k < m.K; k += kWave)
            wp[k] = double2{0.0, 0.0};
        wave_sync();

        // ---- 1. basic moments and their tangents ----------------------------
        for (int base = 0; base < n; base += kWave) {
            DualCtx cx{red1, ws, L.slot_basic, lane, 0};
            Nbr<P::M> q;
            const bool valid = lane < n - base;
            const int64_t p = beg + base + lane;
            load_neighbor<P>(m, nb, L.coef, ti, p, valid, q);
            const GradNbr g = pair_weight<P>(nb, t, fi, S, p, valid, q);
            double px[P::NUMAX + 1], py[P::NUMAX + 1], pz[P::NUMAX + 1];
            unit_powers<P::NUMAX>(q, px, py, pz);
            fwd_dual_shells<0, P>(m, cx, q, g, px, py, pz);
            const int rest = cx.row % kChunk;
            if (rest)
                reduce_rows(red1, rest, cx.row - rest, lane, [&](int r, double acc) {
                    const int b = L.slot_basic[r >> 1];
                    if (b >= 0)
                        ws[2 * b + (r & 1)] += acc;
                });
        }
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k)
                wp[m.dup[2 * k]] = wp[m.dup[2 * k + 1]];
        // the zero slots and partial sums may lie under a transpose buffer
        for (int k = m.dummy + lane; k < m.red0; k += kWave)
            wp[k] = double2{0.0, 0.0};
        wave_sync();

        // ---- 2. rules forward with tangents; moment and species gradient ----
        run_rules<true, false>(fwd_tab, m.fwd_level_step, m.fwd_level_comb, m.fwd_comb, m.nfwd, ws,
                               lane);
        for (int s = lane; s < m.S; s += kWave) {
            const double2 x = wp[L.map[s]];
            grow[m.nradial + m.Z + s] += se * x.x + x.y;
        }
        if (lane == 0)
            grow[m.nradial + ti] += se;

        // ---- 3. reverse rules: A with seeds xi, G with seeds dLdE xi --------
        for (int k = lane; k < m.K; k += kWave) {
            const double sd = m.seed[k];
            wp[m.K4 + k] = double2{sd, se * sd};
        }
        wave_sync();
        run_rules<true, true>(bwd_tab, m.bwd_level_step, m.bwd_level_comb, m.bwd_comb, m.nbwd, ws,
                              lane);
        if (lane == 0)
            for (int k = 0; k < m.ndup; ++k) {
                const double2 v = wp[m.K4 + m.dup[2 * k]];
                double2 &t = wp[m.K4 + m.dup[2 * k + 1]];
                t = double2{t.x + v.x, t.y + v.y};
            }
        wave_sync();
        // slot-ordered {A, G} (the stage may lie over the moment pairs, which
        // are no longer read; the adjoint pairs are not under it)
        for (int s = lane; s < m.nslots; s += kWave) {
            const int b = L.slot_basic[s];
            AG[s] = b >= 0 ? wp[m.K4 + b] : double2{0.0, 0.0};
        }
        wave_sync();

        // ---- 4. radial coefficient gradient ---------------------------------
        const int gbase = ti * m.Z * MR;
        for (int base = 0; base < n; base += kWave) {
            Nbr<P::M> q;
            int tj;
            const bool valid = lane < n - base;
            const int64_t p = beg + base + lane;
            const double win = load_geometry<P::M, !P::exact>(m, nb, p, valid, q, tj, ti);
            const GradNbr g = pair_weight<P>(nb, t, fi, S, p, valid, q);
            ctype[lane] = win != 0.0 ? tj : -1;
            double alpha[P::M], U[P::M];
#pragma unroll
            for (int mu = 0; mu < P::M; ++mu)
                alpha[mu] = U[mu] = 0.0;
            double px[P::NUMAX + 1], py[P::NUMAX + 1], pz[P::NUMAX + 1];
            unit_powers<P::NUMAX>(q, px, py, pz);
            rad_shells<0, P>(m, AG, px, py, pz, g, q.invd, alpha, U);
            double Q[P::RMAX], dQ[P::RMAX];
            radial_basis<P>(m, ti, tj, q.d, Q, dQ);
            int row = 0;
            auto flush = [&](int nrows) {
                reduce_rows_typed(red4, nrows, row - nrows, lane, ctype, m.Z,
                                  [&](int r, int tj2, double acc) {
                                      grad[gbase + tj2 * MR + r] += acc;
                                  });
            };
#pragma unroll
            for (int mu = 0; mu < P::M; ++mu) {
                if (P::exact || mu < m.M) {
                    const double al = alpha[mu] * win, be = g.wu * U[mu] * win;
#pragma unroll
                    for (int k = 0; k < P::RMAX; ++k)
                        if (P::exact || k < m.R) {
                            red4[(row % kChunk) * kRedStride + lane] = al * Q[k] + be * dQ[k];
                            ++row;
                            if (row % kChunk == 0)
                                flush(kChunk);
                        }
                }
            }
            if (row % kChunk)
                flush(row % kChunk);
        }
        wave_sync();
    }
    // the radial part of this wave's gradient row
    for (int k = lane; k < m.nradial; k += kWave)
        grow[k] = grad[k];
}

template <class P>
struct GradWaves {
    static constexpr int value = 4;
};

template <class P>
void launch_grad_variant(const DevModel &m, const DevNeighbors &nb, const TrainArgs &t,
                         const EfsLaunch &cfg, hipStream_t s)
{
    constexpr int W = GradWaves<P>::value;
    if (cfg.lds_tables)
        hipLaunchKernelGGL((grad_kernel<P, true, W>), dim3(cfg.grid), dim3(kWave * cfg.waves),
                           cfg.lds_bytes, s, m, nb, t);
    else
        hipLaunchKernelGGL((grad_kernel<P, false, W>), dim3(cfg.grid), dim3(kWave * cfg.waves),
                           cfg.lds_bytes, s, m, nb, t);
}

}  // namespace

bool grad_configure(const DevModel &m, int n, int num_cus, size_t lds_limit, EfsLaunch &cfg)
{
    return configure_launch(m, n, num_cus, 4, lds_limit, m.tr_priv, cfg, -1, false);
}

hipError_t launch_structure_reduce(const int *soff, int nconf, const double *site_energy,
                                   const double *site_virial, double *energy, double *stress,
                                   hipStream_t s)
{
    if (nconf > 0)
        hipLaunchKernelGGL(structure_reduce_kernel, dim3(nconf), dim3(kWave), 0, s, soff, nconf,
                           site_energy, site_virial, energy, stress);
    return hipGetLastError();
}

hipError_t launch_loss(const LossArgs &a, hipStream_t s)
{
    if (a.nconf > 0)
        hipLaunchKernelGGL(loss_kernel, dim3(a.nconf), dim3(kWave), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_rows_reduce(const double *rows, int nrows, int cols, double *out, bool accumulate,
                              hipStream_t s)
{
    if (cols > 0)
        hipLaunchKernelGGL(rows_reduce_kernel, dim3((cols + kRowCols - 1) / kRowCols), dim3(256),
                           0, s, rows, nrows, cols, out, accumulate ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_grad(const DevModel &m, const DevNeighbors &nb, const TrainArgs &t,
                       const EfsLaunch &cfg, hipStream_t s)
{
    switch (efs_variant(m, m.R)) {
    case 0: launch_grad_variant<ProfLevel16>(m, nb, t, cfg, s); break;
    case 1: launch_grad_variant<ProfLevel20>(m, nb, t, cfg, s); break;
    case 2: launch_grad_variant<ProfLevel10>(m, nb, t, cfg, s); break;
    case 3: launch_grad_variant<ProfSmall>(m, nb, t, cfg, s); break;
    default: launch_grad_variant<ProfGeneric>(m, nb, t, cfg, s); break;
    }
    return hipGetLastError();
}

}  // namespace mtpx
