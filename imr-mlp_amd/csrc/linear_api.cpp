// C ABI, linear-fit part (include/mtpx.h): E/F/S components of the linear
// coefficients, the weighted design rows and the normal equations of the
// linear fit, and the orthogonalisation of the radial functions.  Host
// code; no exceptions escape.
#include "context.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace {

struct CompLayout {
    int p;
    size_t fc, sc, ec, total;  // offsets in doubles
};

CompLayout comp_layout(const mtpx_context *ctx)
{
    CompLayout l;
    l.p = ctx->model.Z + ctx->model.S;
    l.fc = 0;
    l.sc = (size_t)ctx->n * 3 * l.p;
    l.ec = l.sc + (size_t)ctx->nconf * 9 * l.p;
    l.total = l.ec + (size_t)ctx->nconf * l.p;
    return l;
}

// Budget of one group's per-site Jacobian values (MTPX_LIN_GROUP_MB, tuning;
// 8 GiB by default); a structure larger than the budget forms a group of
// its own.
size_t group_budget()
{
    const char *e = getenv("MTPX_LIN_GROUP_MB");
    const long v = e ? atol(e) : 0;
    return (v > 0 ? (size_t)v : (size_t)8192) << 20;
}

// Components of every structure of the resident topology into ctx->comp,
// group by group:
//   lin_jac_kernel    per site: the scalar moments and the walk-order values
//                     of the site Jacobian;
//   lin_reduce_kernel energy components and species counts per structure;
//   lin_tile_kernel   one wave per (structure, chunk of scalars): force and
//                     stress components, each row written once.
// The tile kernel's launches go by structure size: the LDS tile of a launch
// holds the force rows of its largest structure, so structures of similar
// size share a launch; larger structures than one LDS tile holds accumulate
// in their rows of the output instead.  Every sum has a fixed order.
int run_lin(mtpx_context *ctx)
{
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no neighbour lists");
    if (int rc = check_species(ctx))
        return rc;
    if (!ctx->has_lin)
        return set_error(ctx, MTPX_E_MODEL, "linear fit unavailable: " + ctx->lin_err);
    const CompLayout cl = comp_layout(ctx);
    hipStream_t s = ctx->stream;
    HIP_TRY(ctx->comp.ensure(sizeof(double) * std::max<size_t>(cl.total, 1)),
            "allocate components");
    if (ctx->n == 0) {
        if (cl.total)
            HIP_TRY(launch_fill_zero(ctx->comp.as<double>(), cl.total, s), "clear components");
        return MTPX_OK;
    }
    const DevModel &m = ctx->dm;
    const DevLin &L = ctx->dl;
    const size_t per_atom = sizeof(double) * ((size_t)L.nwalk + m.S);
    const size_t budget = group_budget();
    const std::vector<int> &so = ctx->soff_host;

    // groups of whole structures
    struct Range {
        int c0, c1;
    };
    std::vector<Range> groups;
    size_t max_atoms = 1;
    for (int c0 = 0; c0 < ctx->nconf;) {
        int c1 = c0 + 1;
        while (c1 < ctx->nconf && (size_t)(so[c1 + 1] - so[c0]) * per_atom <= budget)
            ++c1;
        groups.push_back({c0, c1});
        max_atoms = std::max(max_atoms, (size_t)(so[c1] - so[c0]));
        c0 = c1;
    }
    HIP_TRY(ctx->lin_lw.ensure(sizeof(double) * (size_t)L.nwalk * max_atoms),
            "allocate site Jacobians");
    HIP_TRY(ctx->lin_site.ensure(sizeof(double) * (size_t)m.S * max_atoms),
            "allocate site rows");

    // Size classes of the tile launches: a class holds the structures of at
    // most `cap` atoms not held by a smaller class; the last class (cap 0)
    // takes the structures too large for an LDS tile.
    const size_t row_bytes = sizeof(double) * (3 * kLinChunk + 1);  // the tile's row stride
    const size_t base = lin_tile_lds(m, L, 0);
    int max_rows = ctx->lds_limit > base ? (int)((ctx->lds_limit - base) / row_bytes) : 0;
    // MTPX_LIN_TILE_ROWS (tests, tuning): a smaller LDS tile; 0 takes every
    // structure through its output rows
    if (const char *e = getenv("MTPX_LIN_TILE_ROWS"))
        max_rows = std::min(max_rows, std::max(0, atoi(e)));
    // The tile kernel runs one wave per SIMD (its registers allow no more),
    // so every structure whose tile fits a quarter of the LDS shares the
    // first class: one launch, largest structures first, the small ones
    // filling its tail.
    std::vector<int> caps;
    const size_t quarter_bytes = ctx->lds_limit / 4;
    const int quarter = quarter_bytes > base ? (int)((quarter_bytes - base) / row_bytes) : 0;
    if (quarter > 0 && quarter < max_rows)
        caps.push_back(quarter);
    for (int c : {384, 512, 768})
        if (c > quarter && c < max_rows)
            caps.push_back(c);
    if (max_rows > 0)
        caps.push_back(max_rows);
    const int ncls = (int)caps.size() + 1;
    // structure lists of every (group, class), one upload
    std::vector<int> lists;
    std::vector<std::vector<int>> cls_off(groups.size(), std::vector<int>(ncls + 1, 0));
    for (size_t gi = 0; gi < groups.size(); ++gi) {
        std::vector<std::vector<int>> by((size_t)ncls);
        for (int c = groups[gi].c0; c < groups[gi].c1; ++c) {
            const int N = so[c + 1] - so[c];
            if (N == 0)
                continue;
            int k = 0;
            while (k < (int)caps.size() && N > caps[k])
                ++k;
            by[k].push_back(c);
        }
        for (int k = 0; k < ncls; ++k) {
            // largest structures first: the longest waves start first
            std::stable_sort(by[k].begin(), by[k].end(), [&](int x, int y) {
                return so[x + 1] - so[x] > so[y + 1] - so[y];
            });
            cls_off[gi][k] = (int)lists.size();
            lists.insert(lists.end(), by[k].begin(), by[k].end());
        }
        cls_off[gi][ncls] = (int)lists.size();
    }
    HIP_TRY(upload(ctx->lin_tiles, lists, s), "upload structure lists");
    // The kernels write every component but the species columns of the
    // force and stress rows (and the stress rows of empty structures), so
    // only those are cleared, unless a structure adds into its force rows
    // directly (the class past the largest LDS tile): then all are.
    bool direct = false;
    for (size_t gi = 0; gi < groups.size(); ++gi)
        direct = direct || cls_off[gi][ncls] > cls_off[gi][ncls - 1];
    if (direct)
        HIP_TRY(launch_fill_zero(ctx->comp.as<double>(), cl.total, s), "clear components");
    else
        HIP_TRY(launch_lin_clear(ctx->comp.as<double>(), (int64_t)ctx->n * 3,
                                 (int64_t)ctx->nconf * 9, cl.p, m.Z, s),
                "clear components");

    double *comp = ctx->comp.as<double>();
    const DevNeighbors nb = dev_neighbors(ctx);
    for (size_t gi = 0; gi < groups.size(); ++gi) {
        const Range &r = groups[gi];
        LinGroup g;
        g.c0 = r.c0;
        g.c1 = r.c1;
        g.a0 = so[r.c0];
        g.a1 = so[r.c1];
        g.site = ctx->lin_site.as<double>();
        g.lw = ctx->lin_lw.as<double>();
        if (g.a1 > g.a0) {
            EfsLaunch cfg;
            if (!lin_configure(m, L, g.a1 - g.a0, ctx->num_cus, ctx->lds_limit, cfg))
                return set_error(ctx, MTPX_E_CAPACITY,
                                 "model needs more LDS than a CU provides for the linear fit");
            HIP_TRY(launch_lin_jac(m, L, nb, g, cfg, s), "launch linear-fit site kernel");
        }
        HIP_TRY(launch_lin_reduce(m, ctx->soff.as<int>(), ctx->center_type.as<int>(), g,
                                  comp + cl.ec, s),
                "launch linear-fit reduction");
        for (int k = ncls - 1; k >= 0; --k) {  // the classes of larger structures first
            LinTile t;
            t.structs = ctx->lin_tiles.as<int>() + cls_off[gi][k];
            t.count = cls_off[gi][k + 1] - cls_off[gi][k];
            t.nchunks = L.nchunks;
            const bool lds_tile = k < (int)caps.size();
            t.rows_cap = lds_tile ? caps[k] : 0;
            t.soff = ctx->soff.as<int>();
            t.lw = g.lw;
            t.a0 = g.a0;
            t.p = cl.p;
            t.Z = m.Z;
            t.fc = comp + cl.fc;
            t.sc = comp + cl.sc;
            HIP_TRY(launch_lin_tile(m, L, nb, t, s), "launch linear-fit tile kernel");
        }
    }
    return MTPX_OK;
}

// AddLinearFast (train/train_mtp.cpp:1289-1395) row order per structure:
// force rows of the atoms with a positive weight (x, y, z), the 9 stress
// rows, the energy row; each scaled by sqrt(w), targets likewise.
int build_rows(mtpx_context *ctx, int64_t &R)
{
    if (!ctx->has_labels)
        return set_error(ctx, MTPX_E_INVALID, "no labels");
    const CompLayout cl = comp_layout(ctx);
    const Model &M = ctx->model;
    const bool fix = ctx->fix_species;
    std::vector<double> csp;
    if (fix)
        csp.assign(M.coef.begin() + M.nradial(), M.coef.begin() + M.nradial() + M.Z);
    if (ctx->rows_gen == ctx->label_gen && ctx->rows_p == cl.p && ctx->rows_fix == fix &&
        (!fix || ctx->rows_species == csp)) {
        R = ctx->rows_R;  // descriptors of these labels are resident
        return MTPX_OK;
    }
    // fix_species_coeffs (train/train_mtp.cpp:1300-1302, 1381-1392): rows
    // start at the moment columns; energy targets less sum_s n_s c_s
    const size_t off = fix ? (size_t)M.Z : 0;
    std::vector<double> esub((size_t)ctx->nconf, 0.0);
    if (fix && ctx->n > 0) {
        std::vector<int> ct((size_t)ctx->n);
        HIP_TRY(hipMemcpyAsync(ct.data(), ctx->center_type.p, sizeof(int) * ct.size(),
                               hipMemcpyDeviceToHost, ctx->stream),
                "copy species");
        HIP_TRY(hipStreamSynchronize(ctx->stream), "copy species");
        for (int c = 0; c < ctx->nconf; ++c) {
            std::vector<double> cnt((size_t)M.Z, 0.0);
            for (int i = ctx->soff_host[c]; i < ctx->soff_host[c + 1]; ++i)
                cnt[(size_t)ct[i]] += 1.0;
            for (int t = 0; t < M.Z; ++t)
                esub[c] += cnt[t] * csp[t];
        }
    }
    std::vector<int64_t> src;
    std::vector<double> sw, yw;
    for (int c = 0; c < ctx->nconf; ++c) {
        const int a0 = ctx->soff_host[c], a1 = ctx->soff_host[c + 1];
        const int *act = &ctx->active_h[3 * (size_t)c];
        if (act[1])
            for (int i = a0; i < a1; ++i) {
                if (!(ctx->wF_h[i] > 0))
                    continue;
                const double w = std::sqrt(ctx->wF_h[i]);
                for (int a = 0; a < 3; ++a) {
                    src.push_back((int64_t)(cl.fc + ((size_t)i * 3 + a) * cl.p + off));
                    sw.push_back(w);
                    yw.push_back(w * ctx->tF_h[3 * (size_t)i + a]);
                }
            }
        if (act[2]) {
            const double w = std::sqrt(ctx->wS_h[c]);
            for (int q = 0; q < 9; ++q) {
                src.push_back((int64_t)(cl.sc + ((size_t)c * 9 + q) * cl.p + off));
                sw.push_back(w);
                yw.push_back(w * ctx->tS_h[9 * (size_t)c + q]);
            }
        }
        if (act[0]) {
            const double w = std::sqrt(ctx->wE_h[c]);
            src.push_back((int64_t)(cl.ec + (size_t)c * cl.p + off));
            sw.push_back(w);
            yw.push_back(w * (ctx->tE_h[c] - esub[c]));
        }
    }
    R = (int64_t)src.size();
    HIP_TRY(upload(ctx->row_src, src, ctx->stream), "upload rows");
    HIP_TRY(upload(ctx->row_sw, sw, ctx->stream), "upload rows");
    HIP_TRY(upload(ctx->row_y, yw, ctx->stream), "upload rows");
    ctx->rows_gen = ctx->label_gen;
    ctx->rows_p = cl.p;
    ctx->rows_R = R;
    ctx->rows_fix = fix;
    ctx->rows_species = csp;
    return MTPX_OK;
}

// Columns of a linear-fit row: Z + S, or S with the species coefficients fixed.
int row_width(const mtpx_context *ctx)
{
    return ctx->model.S + (ctx->fix_species ? 0 : ctx->model.Z);
}

}  // namespace

extern "C" {

int mtpx_efs_components(mtpx_context *ctx, double *energy_cmpts, double *force_cmpts,
                        double *stress_cmpts)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (need_linear(ctx, "mtpx_efs_components") != MTPX_OK)
        return MTPX_E_MODEL;
    (void)hipSetDevice(ctx->device);
    int rc = run_lin(ctx);
    if (rc != MTPX_OK)
        return rc;
    const CompLayout cl = comp_layout(ctx);
    const double *comp = ctx->comp.as<double>();
    HIP_TRY(hipStreamSynchronize(ctx->stream), "components");
    if (force_cmpts && cl.sc > cl.fc)
        HIP_TRY(hipMemcpy(force_cmpts, comp + cl.fc, sizeof(double) * (cl.sc - cl.fc),
                          hipMemcpyDeviceToHost),
                "copy force components");
    if (stress_cmpts && cl.ec > cl.sc)
        HIP_TRY(hipMemcpy(stress_cmpts, comp + cl.sc, sizeof(double) * (cl.ec - cl.sc),
                          hipMemcpyDeviceToHost),
                "copy stress components");
    if (energy_cmpts && cl.total > cl.ec)
        HIP_TRY(hipMemcpy(energy_cmpts, comp + cl.ec, sizeof(double) * (cl.total - cl.ec),
                          hipMemcpyDeviceToHost),
                "copy energy components");
    return MTPX_OK;
}

int mtpx_linear_rows(mtpx_context *ctx, int64_t *nrows, double *A, double *y)
{
    if (!ctx || !nrows)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no structures");
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (need_linear(ctx, "mtpx_linear_rows") != MTPX_OK)
        return MTPX_E_MODEL;
    (void)hipSetDevice(ctx->device);
    int64_t R = 0;
    int rc = build_rows(ctx, R);
    if (rc != MTPX_OK)
        return rc;
    if (!A && !y) {
        *nrows = R;
        return MTPX_OK;
    }
    if (!A || !y)
        return set_error(ctx, MTPX_E_INVALID, "A and y are both needed");
    if (*nrows < R)
        return set_error(ctx, MTPX_E_RANGE, "row buffer too small");
    rc = run_lin(ctx);
    if (rc != MTPX_OK)
        return rc;
    const int p = row_width(ctx);
    HIP_TRY(ctx->rowsA.ensure(sizeof(double) * std::max<int64_t>(R * p, 1)), "allocate rows");
    HIP_TRY(ctx->rowsY.ensure(sizeof(double) * std::max<int64_t>(R, 1)), "allocate rows");
    HIP_TRY(launch_lin_rows(ctx->comp.as<double>(), ctx->row_src.as<int64_t>(),
                            ctx->row_sw.as<double>(), ctx->row_y.as<double>(), R, p,
                            ctx->rowsA.as<double>(), ctx->rowsY.as<double>(), ctx->stream),
            "launch rows");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "rows");
    if (R > 0) {
        HIP_TRY(hipMemcpy(A, ctx->rowsA.p, sizeof(double) * R * p, hipMemcpyDeviceToHost),
                "copy rows");
        HIP_TRY(hipMemcpy(y, ctx->rowsY.p, sizeof(double) * R, hipMemcpyDeviceToHost),
                "copy targets");
    }
    *nrows = R;
    return MTPX_OK;
}

int mtpx_linear_system(mtpx_context *ctx, double *G, double *b)
{
    if (!ctx || !G || !b)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no structures");
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (need_linear(ctx, "mtpx_linear_system") != MTPX_OK)
        return MTPX_E_MODEL;
    if (!gram_fits(row_width(ctx)))
        return set_error(ctx, MTPX_E_CAPACITY, "linear system of more than 1007 coefficients");
    (void)hipSetDevice(ctx->device);
    int64_t R = 0;
    int rc = build_rows(ctx, R);
    if (rc != MTPX_OK)
        return rc;
    hipStream_t s = ctx->stream;
    for (auto &e : ctx->tev)
        if (!e)
            HIP_TRY(hipEventCreate(&e), "create events");
    HIP_TRY(hipEventRecord(ctx->tev[0], s), "record event");
    rc = run_lin(ctx);
    if (rc != MTPX_OK)
        return rc;
    HIP_TRY(hipEventRecord(ctx->tev[1], s), "record event");
    const int p = row_width(ctx);
    const int pp = gram_padded(p);
    HIP_TRY(ctx->gram_out.ensure(sizeof(double) * pp * pp), "allocate Gram");
    if (R == 0) {
        HIP_TRY(hipMemsetAsync(ctx->gram_out.p, 0, sizeof(double) * pp * pp, s), "clear Gram");
    } else {
        const int nblocks = gram_blocks(R, p, ctx->num_cus);
        HIP_TRY(ctx->gram_part.ensure(sizeof(double) * gram_partial_doubles(p, nblocks)),
                "allocate Gram partials");
        HIP_TRY(launch_gram(ctx->comp.as<double>(), ctx->row_src.as<int64_t>(),
                            ctx->row_sw.as<double>(), ctx->row_y.as<double>(), R, p, nblocks,
                            ctx->gram_part.as<double>(), ctx->gram_out.as<double>(), s),
                "launch Gram");
        HIP_TRY(hipEventRecord(ctx->tev[2], s), "record event");
    }
    std::vector<double> g((size_t)pp * pp);
    HIP_TRY(hipMemcpyAsync(g.data(), ctx->gram_out.p, sizeof(double) * pp * pp,
                           hipMemcpyDeviceToHost, s),
            "copy Gram");
    HIP_TRY(hipEventRecord(ctx->tev[3], s), "record event");
    HIP_TRY(hipStreamSynchronize(s), "Gram");
    float t03 = 0, t01 = 0, t12 = 0;
    (void)hipEventElapsedTime(&t03, ctx->tev[0], ctx->tev[3]);
    (void)hipEventElapsedTime(&t01, ctx->tev[0], ctx->tev[1]);
    if (R > 0)
        (void)hipEventElapsedTime(&t12, ctx->tev[1], ctx->tev[2]);
    ctx->lin_timings[0] = t03;
    ctx->lin_timings[1] = t01;
    ctx->lin_timings[2] = t12;
    ctx->lin_timings[3] = (double)R;
    for (int i = 0; i < p; ++i) {
        for (int j = 0; j < p; ++j)
            G[(size_t)i * p + j] = g[(size_t)i * pp + j];
        b[i] = g[(size_t)i * pp + p];
    }
    return MTPX_OK;
}

// PotMTP::Orthogonalize (potentials/potential_mtp.cpp:3849-3930): for each
// radial function k, subtract from c_k its projection on every earlier c_k2
// -- divided by |c_k|^2, the reference's choice, not |c_k2|^2 -- then
// normalise with sqrt(sum (c^2 + 1e-10)).  Vectors run over (ti, tj, k).
int mtpx_set_fix_species_coeffs(mtpx_context *ctx, int fix)
{
    if (!ctx)
        return MTPX_E_INVALID;
    ctx->fix_species = fix != 0;
    return MTPX_OK;
}

int mtpx_orthogonalize(mtpx_context *ctx)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    Model &m = ctx->model;
    const int Z = m.Z, M = m.M, R = m.R;
    std::vector<double> x(m.coef);
    double *c = x.data();
    auto at = [&](int pair, int mu, int k) { return (size_t)pair * M * R + (size_t)mu * R + k; };
    for (int k = 0; k < M; ++k) {
        for (int k2 = 0; k2 < k; ++k2) {
            double norm = 0.0, scal = 0.0;
            for (int pr = 0; pr < Z * Z; ++pr)
                for (int l = 0; l < R; ++l)
                    norm += c[at(pr, k, l)] * c[at(pr, k, l)];
            for (int pr = 0; pr < Z * Z; ++pr)
                for (int l = 0; l < R; ++l)
                    scal += c[at(pr, k, l)] * c[at(pr, k2, l)];
            for (int pr = 0; pr < Z * Z; ++pr)
                for (int l = 0; l < R; ++l)
                    c[at(pr, k, l)] -= c[at(pr, k2, l)] * scal / norm;
        }
        double norm = 0.0;
        for (int pr = 0; pr < Z * Z; ++pr)
            for (int l = 0; l < R; ++l)
                norm += c[at(pr, k, l)] * c[at(pr, k, l)] + 1e-10;
        norm = std::sqrt(norm);
        for (int pr = 0; pr < Z * Z; ++pr)
            for (int l = 0; l < R; ++l)
                c[at(pr, k, l)] /= norm;
    }
    return mtpx_set_coeffs(ctx, x.data());
}

int mtpx_last_linear_timings(const mtpx_context *ctx, double out[4])
{
    if (!ctx || !out)
        return MTPX_E_INVALID;
    std::memcpy(out, ctx->lin_timings, sizeof ctx->lin_timings);
    return MTPX_OK;
}

}  // extern "C"
