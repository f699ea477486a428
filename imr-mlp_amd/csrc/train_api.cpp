// C ABI, training part (include/mtpx.h): batches of structures, labels, the
// loss and its adjoints, the coefficient gradient and the penalty.  Host
// code; no exceptions escape.
#include "context.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace {

// Uploads n values, or zeros when the host array is absent.
template <class T>
hipError_t upload_or_zero(DBuf &b, const T *host, size_t n, hipStream_t s)
{
    hipError_t e = b.ensure(sizeof(T) * std::max<size_t>(n, 1));
    if (e != hipSuccess || n == 0)
        return e;
    if (host)
        return hipMemcpyAsync(b.p, host, sizeof(T) * n, hipMemcpyHostToDevice, s);
    return hipMemsetAsync(b.p, 0, sizeof(T) * n, s);
}

// PotMTP::AddPenaltyGard with radial_mode 0 (potentials/potential_mtp.cpp:
// 6568-6742).  Radial coefficients c[ti][tj][mu][k]; for each radial
// function mu its coefficient vector v_mu runs over (ti, tj, k).
//   w (|v_mu|^2 - 1)^2 for every mu, w (v_mu . v_nu)^2 for mu < nu,
//   l2 x^2 + l1 |x| for every moment coefficient x (species excluded);
// the L1 term's derivative is taken as +l1 for x > 0 and -l1 otherwise, as
// the reference does.
void penalty(const Model &m, double w, double l2, double l1, double &loss, double *grad)
{
    const int Z = m.Z, M = m.M, R = m.R;
    const double *c = m.coef.data();
    auto at = [&](int pair, int mu, int k) { return (size_t)pair * M * R + (size_t)mu * R + k; };
    for (int mu = 0; mu < M; ++mu) {
        double sq = 0.0;
        for (int pair = 0; pair < Z * Z; ++pair)
            for (int k = 0; k < R; ++k)
                sq += c[at(pair, mu, k)] * c[at(pair, mu, k)];
        loss += w * (sq - 1) * (sq - 1);
        const double f = w * 4 * (sq - 1);
        for (int pair = 0; pair < Z * Z; ++pair)
            for (int k = 0; k < R; ++k)
                grad[at(pair, mu, k)] += f * c[at(pair, mu, k)];
    }
    for (int mu = 0; mu < M; ++mu)
        for (int nu = mu + 1; nu < M; ++nu) {
            double dot = 0.0;
            for (int pair = 0; pair < Z * Z; ++pair)
                for (int k = 0; k < R; ++k)
                    dot += c[at(pair, mu, k)] * c[at(pair, nu, k)];
            loss += w * dot * dot;
            const double f = w * 2 * dot;
            for (int pair = 0; pair < Z * Z; ++pair)
                for (int k = 0; k < R; ++k) {
                    grad[at(pair, mu, k)] += f * c[at(pair, nu, k)];
                    grad[at(pair, nu, k)] += f * c[at(pair, mu, k)];
                }
        }
    const size_t first = (size_t)m.nradial() + Z;
    for (int s = 0; s < m.S; ++s) {
        const double x = c[first + s];
        loss += x * x * l2;
        loss += std::fabs(x) * l1;
    }
    for (int s = 0; s < m.S; ++s) {
        const double x = c[first + s];
        grad[first + s] += 2 * x * l2;
        grad[first + s] += x > 0 ? l1 : -l1;
    }
}

int need_topology(mtpx_context *ctx)
{
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no neighbour lists");
    return check_species(ctx);
}

// E/F/S of the batch and the per-structure energy and virial.
int batch_forward(mtpx_context *ctx, bool deterministic)
{
    int rc = run_efs(ctx, deterministic, true);
    if (rc != MTPX_OK)
        return rc;
    const int nc = std::max(ctx->nconf, 1);
    HIP_TRY(ctx->benergy.ensure(sizeof(double) * nc), "allocate batch outputs");
    HIP_TRY(ctx->bstress.ensure(sizeof(double) * 9 * nc), "allocate batch outputs");
    if (ctx->n == 0 && ctx->nconf > 0) {
        HIP_TRY(hipMemsetAsync(ctx->benergy.p, 0, sizeof(double) * nc, ctx->stream), "clear");
        HIP_TRY(hipMemsetAsync(ctx->bstress.p, 0, sizeof(double) * 9 * nc, ctx->stream), "clear");
    } else {
        HIP_TRY(launch_structure_reduce(ctx->soff.as<int>(), ctx->nconf,
                                        ctx->site_energy.as<double>(),
                                        ctx->site_virial.as<double>(), ctx->benergy.as<double>(),
                                        ctx->bstress.as<double>(), ctx->stream),
                "launch structure reduction");
    }
    ctx->has_batch_out = true;
    return MTPX_OK;
}

int loss_forward(mtpx_context *ctx)
{
    const int nc = ctx->nconf, n = ctx->n;
    HIP_TRY(ctx->dLdE.ensure(sizeof(double) * std::max(nc, 1)), "allocate adjoints");
    HIP_TRY(ctx->dLdF.ensure(sizeof(double) * 3 * std::max(n, 1)), "allocate adjoints");
    HIP_TRY(ctx->dLdS.ensure(sizeof(double) * 9 * std::max(nc, 1)), "allocate adjoints");
    HIP_TRY(ctx->metric_rows.ensure(sizeof(double) * 7 * std::max(nc, 1)), "allocate metrics");
    HIP_TRY(ctx->metrics.ensure(sizeof(double) * 7), "allocate metrics");
    LossArgs a;
    a.soff = ctx->soff.as<int>();
    a.nconf = nc;
    a.active = ctx->active.as<int>();
    a.E = ctx->benergy.as<double>();
    a.F = ctx->forces.as<double>();
    a.S = ctx->bstress.as<double>();
    a.tE = ctx->tE.as<double>();
    a.wE = ctx->wE.as<double>();
    a.tF = ctx->tF.as<double>();
    a.wF = ctx->wF.as<double>();
    a.tS = ctx->tS.as<double>();
    a.wS = ctx->wS.as<double>();
    a.dLdE = ctx->dLdE.as<double>();
    a.dLdF = ctx->dLdF.as<double>();
    a.dLdS = ctx->dLdS.as<double>();
    a.metric_rows = ctx->metric_rows.as<double>();
    HIP_TRY(launch_loss(a, ctx->stream), "launch loss");
    if (nc > 0)
        HIP_TRY(launch_rows_reduce(a.metric_rows, nc, 7, ctx->metrics.as<double>(), false,
                                   ctx->stream),
                "launch metric reduction");
    else
        HIP_TRY(hipMemsetAsync(ctx->metrics.p, 0, sizeof(double) * 7, ctx->stream), "clear");
    ctx->has_adjoints = true;
    return MTPX_OK;
}

// Gradient of the resident adjoints into ctx->grad (device, [ncoef]).
int grad_forward(mtpx_context *ctx)
{
    const DevModel &m = ctx->dm;
    EfsLaunch cfg;
    if (!grad_configure(m, ctx->n, ctx->num_cus, ctx->lds_limit, cfg))
        return set_error(ctx, MTPX_E_CAPACITY,
                         "model needs more LDS than a CU provides for the gradient");
    HIP_TRY(ctx->grad_rows.ensure(sizeof(double) * (size_t)cfg.rows * m.ncoef),
            "allocate gradient rows");
    HIP_TRY(ctx->grad.ensure(sizeof(double) * m.ncoef), "allocate gradient");
    if (ctx->n == 0) {
        HIP_TRY(hipMemsetAsync(ctx->grad.p, 0, sizeof(double) * m.ncoef, ctx->stream),
                "clear gradient");
        return MTPX_OK;
    }
    TrainArgs t;
    t.center_structure = ctx->center_structure.as<int>();
    t.dLdE = ctx->dLdE.as<double>();
    t.dLdF = ctx->dLdF.as<double>();
    t.dLdS = ctx->dLdS.as<double>();
    t.grad_rows = ctx->grad_rows.as<double>();
    HIP_TRY(launch_grad(m, dev_neighbors(ctx), t, cfg, ctx->stream), "launch gradient kernel");
    HIP_TRY(launch_rows_reduce(t.grad_rows, cfg.rows, m.ncoef, ctx->grad.as<double>(), false,
                               ctx->stream),
            "launch gradient reduction");
    return MTPX_OK;
}

}  // namespace

extern "C" {

int mtpx_set_structures(mtpx_context *ctx, int nconf, const int *atom_offsets,
                        const double *cells, const int *pbc, const double *pos, const int *types,
                        double cutoff)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (nconf < 0 || !atom_offsets || (nconf > 0 && (!cells || !pbc)) || !(cutoff > 0) ||
        !std::isfinite(cutoff))
        return set_error(ctx, MTPX_E_INVALID, "invalid batch arguments");
    if (atom_offsets[0] != 0)
        return set_error(ctx, MTPX_E_INVALID, "atom offsets must start at 0");
    for (int c = 0; c < nconf; ++c)
        if (atom_offsets[c + 1] < atom_offsets[c])
            return set_error(ctx, MTPX_E_INVALID, "atom offsets must be non-decreasing");
    const int N = atom_offsets[nconf];
    if (N > 0 && (!pos || !types))
        return set_error(ctx, MTPX_E_INVALID, "invalid batch arguments");
    if (!all_finite(cells, 9 * (size_t)nconf))
        return set_error(ctx, MTPX_E_INVALID, "non-finite cell");
    if (!all_finite(pos, 3 * (size_t)N))
        return set_error(ctx, MTPX_E_INVALID, "non-finite position");
    std::vector<int> tbuf;
    if (int rc = map_species(ctx, types, (size_t)N, false, tbuf, types))
        return rc;
    const int Z = ctx->has_model ? ctx->model.Z : 1 << 30;
    int maxs = -1;
    if (!species_in_range(types, (size_t)N, Z, maxs))
        return set_error(ctx, MTPX_E_INVALID, "species out of range");
    (void)hipSetDevice(ctx->device);
    ctx->has_nbh = false;
    ctx->rev_ready = false;
    ctx->has_batch_out = ctx->has_adjoints = ctx->has_labels = false;
    std::string err;
    int rc = build_neighbors_batch_gpu(nconf, atom_offsets, cells, pbc, pos, types, cutoff,
                                       ctx->stream, ctx->nbh, ctx->nbh_tmp, ctx->scratch, err);
    if (rc != MTPX_OK)
        return set_error(ctx, rc, err);
    ctx->nconf = nconf;
    ctx->single_n = -1;
    ctx->max_species = maxs;
    ctx->soff_host.assign(atom_offsets, atom_offsets + nconf + 1);
    std::vector<int> cs((size_t)N);
    for (int c = 0; c < nconf; ++c)
        for (int i = atom_offsets[c]; i < atom_offsets[c + 1]; ++i)
            cs[i] = c;
    HIP_TRY(upload(ctx->soff, ctx->soff_host, ctx->stream), "upload structure offsets");
    HIP_TRY(upload(ctx->center_structure, cs, ctx->stream), "upload structure index");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "upload structure index");
    ctx->has_nbh = true;
    return MTPX_OK;
}

int mtpx_structure_count(const mtpx_context *ctx, int *nconf)
{
    if (!ctx || !nconf)
        return MTPX_E_INVALID;
    if (!ctx->has_nbh)
        return MTPX_E_NO_TOPOLOGY;
    *nconf = ctx->nconf;
    return MTPX_OK;
}

int mtpx_compute_batch(mtpx_context *ctx, int deterministic, double *energy, double *forces,
                       double *stress, double *site_energies)
{
    if (!ctx)
        return MTPX_E_INVALID;
    (void)hipSetDevice(ctx->device);
    int rc = need_topology(ctx);
    if (rc == MTPX_OK)
        rc = batch_forward(ctx, deterministic != 0);
    if (rc != MTPX_OK)
        return rc;
    const size_t nc = (size_t)ctx->nconf, n = (size_t)ctx->n;
    const bool add = ctx->add_efs;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "compute batch");
    if (energy)
        rc = copy_out(ctx, energy, ctx->benergy.p, nc, add, "copy energies");
    if (rc == MTPX_OK && stress)
        rc = copy_out(ctx, stress, ctx->bstress.p, 9 * nc, add, "copy stresses");
    if (rc == MTPX_OK && forces)
        rc = copy_out(ctx, forces, ctx->forces.p, 3 * n, add, "copy forces");
    if (rc == MTPX_OK && site_energies)
        rc = copy_out(ctx, site_energies, ctx->site_energy.p, n, add, "copy site energies");
    return rc;
}

int mtpx_loss_weights(const mtpx_loss_settings *s, int nconf, const int *atom_offsets,
                      const int *has, const double *target_forces, const double *fitness,
                      const double *atomic_fitness, int *active, double *energy_weight,
                      double *force_weight, double *stress_weight)
{
    if (!s || nconf < 0 || !atom_offsets || (nconf > 0 && (!has || !active)))
        return MTPX_E_INVALID;
    for (int c = 0; c < nconf; ++c) {
        const int a0 = atom_offsets[c], N = atom_offsets[c + 1] - a0;
        if (N < 0)
            return MTPX_E_INVALID;
        const int *h = has + 3 * c;
        int *act = active + 3 * c;
        act[0] = N > 0 && s->weight_energy > 0 && h[0];
        act[1] = N > 0 && s->weight_forces > 0 && h[1];
        act[2] = N > 0 && s->weight_stress > 0 && h[2];
        // force normalisation from the labels (train_mtp.cpp:3872-3881)
        double cc = 1.0;
        if (N > 0 && s->force_norm_f > 0 && h[1]) {
            if (!target_forces)
                return MTPX_E_INVALID;
            double avef = 0.0;
            for (int i = a0; i < a0 + N; ++i) {
                const double *f = target_forces + 3 * (size_t)i;
                avef += (f[0] * f[0] + f[1] * f[1]) + f[2] * f[2];
            }
            avef /= N;
            cc = s->force_norm_d / (s->force_norm_d + std::pow(s->force_norm_f * avef,
                                                               s->force_norm_p));
        }
        if (energy_weight)
            energy_weight[c] = act[0] ? s->weight_energy / std::pow((double)N, s->energy_pow) *
                                            (fitness ? fitness[c] : 1.0) * cc
                                      : 0.0;
        if (stress_weight)
            stress_weight[c] =
                act[2] ? s->weight_stress / std::pow((double)N, s->stress_pow) * cc : 0.0;
        if (force_weight) {
            const double wf =
                act[1] ? s->weight_forces / std::pow((double)N, s->force_pow) * cc : 0.0;
            for (int i = a0; i < a0 + N; ++i)
                force_weight[i] = atomic_fitness ? wf * atomic_fitness[i] : wf;
        }
    }
    return MTPX_OK;
}

int mtpx_set_labels(mtpx_context *ctx, const int *active, const double *target_energy,
                    const double *energy_weight, const double *target_forces,
                    const double *force_weight, const double *target_stress,
                    const double *stress_weight)
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_nbh)
        return set_error(ctx, MTPX_E_NO_TOPOLOGY, "no structures");
    const int nc = ctx->nconf, n = ctx->n;
    if (nc > 0 && !active)
        return set_error(ctx, MTPX_E_INVALID, "null active flags");
    bool any[3] = {false, false, false};
    for (int c = 0; c < nc; ++c)
        for (int k = 0; k < 3; ++k)
            any[k] = any[k] || active[3 * c + k];
    if ((any[0] && (!target_energy || !energy_weight)) ||
        (any[1] && (!target_forces || !force_weight)) ||
        (any[2] && (!target_stress || !stress_weight)))
        return set_error(ctx, MTPX_E_INVALID, "labels missing for an active loss term");
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->stream;
    HIP_TRY(upload_or_zero(ctx->active, active, 3 * (size_t)nc, s), "upload labels");
    HIP_TRY(upload_or_zero(ctx->tE, any[0] ? target_energy : nullptr, nc, s), "upload labels");
    HIP_TRY(upload_or_zero(ctx->wE, any[0] ? energy_weight : nullptr, nc, s), "upload labels");
    HIP_TRY(upload_or_zero(ctx->tF, any[1] ? target_forces : nullptr, 3 * (size_t)n, s),
            "upload labels");
    HIP_TRY(upload_or_zero(ctx->wF, any[1] ? force_weight : nullptr, n, s), "upload labels");
    HIP_TRY(upload_or_zero(ctx->tS, any[2] ? target_stress : nullptr, 9 * (size_t)nc, s),
            "upload labels");
    HIP_TRY(upload_or_zero(ctx->wS, any[2] ? stress_weight : nullptr, nc, s), "upload labels");
    HIP_TRY(hipStreamSynchronize(s), "upload labels");
    auto keep = [](std::vector<double> &dst, const double *src, size_t len) {
        if (src)
            dst.assign(src, src + len);
        else
            dst.assign(len, 0.0);
    };
    ctx->active_h.assign(active ? active : nullptr, active ? active + 3 * (size_t)nc : nullptr);
    keep(ctx->tE_h, any[0] ? target_energy : nullptr, nc);
    keep(ctx->wE_h, any[0] ? energy_weight : nullptr, nc);
    keep(ctx->tF_h, any[1] ? target_forces : nullptr, 3 * (size_t)n);
    keep(ctx->wF_h, any[1] ? force_weight : nullptr, n);
    keep(ctx->tS_h, any[2] ? target_stress : nullptr, 9 * (size_t)nc);
    keep(ctx->wS_h, any[2] ? stress_weight : nullptr, nc);
    ctx->has_labels = true;
    ++ctx->label_gen;
    ctx->has_adjoints = false;
    return MTPX_OK;
}

int mtpx_prepare_loss(mtpx_context *ctx, double metrics[7])
{
    if (!ctx)
        return MTPX_E_INVALID;
    if (!ctx->has_batch_out)
        return set_error(ctx, MTPX_E_INVALID, "mtpx_compute_batch has not run on this batch");
    if (!ctx->has_labels)
        return set_error(ctx, MTPX_E_INVALID, "no labels");
    (void)hipSetDevice(ctx->device);
    int rc = loss_forward(ctx);
    if (rc != MTPX_OK)
        return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "loss");
    if (metrics)
        HIP_TRY(hipMemcpy(metrics, ctx->metrics.p, sizeof(double) * 7, hipMemcpyDeviceToHost),
                "copy metrics");
    return MTPX_OK;
}

int mtpx_accumulate_gradient(mtpx_context *ctx, const double *dLdE, const double *dLdF,
                             const double *dLdS, int accumulate, double *gradient)
{
    if (!ctx || !gradient)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    int rc = need_topology(ctx);
    if (rc == MTPX_OK)
        rc = need_linear(ctx, "mtpx_accumulate_gradient");
    if (rc != MTPX_OK)
        return rc;
    (void)hipSetDevice(ctx->device);
    const int nc = ctx->nconf, n = ctx->n;
    hipStream_t s = ctx->stream;
    if (dLdE || dLdF || dLdS) {
        HIP_TRY(upload_or_zero(ctx->dLdE, dLdE, nc, s), "upload adjoints");
        HIP_TRY(upload_or_zero(ctx->dLdF, dLdF, 3 * (size_t)n, s), "upload adjoints");
        HIP_TRY(upload_or_zero(ctx->dLdS, dLdS, 9 * (size_t)nc, s), "upload adjoints");
        ctx->has_adjoints = false;  // no longer those of mtpx_prepare_loss
    } else if (!ctx->has_adjoints) {
        return set_error(ctx, MTPX_E_INVALID, "no adjoints: run mtpx_prepare_loss first");
    }
    rc = grad_forward(ctx);
    if (rc != MTPX_OK)
        return rc;
    const int nco = ctx->dm.ncoef;
    std::vector<double> g((size_t)nco);
    HIP_TRY(hipMemcpyAsync(g.data(), ctx->grad.p, sizeof(double) * nco, hipMemcpyDeviceToHost, s),
            "copy gradient");
    HIP_TRY(hipStreamSynchronize(s), "gradient");
    for (int k = 0; k < nco; ++k)
        gradient[k] = accumulate ? gradient[k] + g[k] : g[k];
    return MTPX_OK;
}

int mtpx_penalty(const mtpx_context *ctx, double weight, double reg_l2, double reg_l1,
                 double *loss, double *grad)
{
    if (!ctx || !loss || !grad)
        return MTPX_E_INVALID;
    if (!ctx->has_model)
        return MTPX_E_NO_MODEL;
    if (!ctx->model.linear())
        return MTPX_E_MODEL;  // the trainer's penalty of the linear MTP
    penalty(ctx->model, weight, reg_l2, reg_l1, *loss, grad);
    return MTPX_OK;
}

int mtpx_loss_grad(mtpx_context *ctx, int deterministic, double penalty_weight, double reg_l2,
                   double reg_l1, double *loss, double *grad, double metrics[7])
{
    if (!ctx || !loss || !grad)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    int rc = need_topology(ctx);
    if (rc == MTPX_OK)
        rc = need_linear(ctx, "mtpx_loss_grad");
    if (rc != MTPX_OK)
        return rc;
    if (!ctx->has_labels)
        return set_error(ctx, MTPX_E_INVALID, "no labels");
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->stream;
    for (auto &e : ctx->tev)
        if (!e)
            HIP_TRY(hipEventCreate(&e), "create events");
    HIP_TRY(hipEventRecord(ctx->tev[0], s), "record event");
    rc = batch_forward(ctx, deterministic != 0);
    if (rc != MTPX_OK)
        return rc;
    HIP_TRY(hipEventRecord(ctx->tev[1], s), "record event");
    rc = loss_forward(ctx);
    if (rc != MTPX_OK)
        return rc;
    HIP_TRY(hipEventRecord(ctx->tev[2], s), "record event");
    rc = grad_forward(ctx);
    if (rc != MTPX_OK)
        return rc;
    HIP_TRY(hipEventRecord(ctx->tev[3], s), "record event");
    const int nco = ctx->dm.ncoef;
    std::vector<double> g((size_t)nco);
    double met[7];
    HIP_TRY(hipMemcpyAsync(g.data(), ctx->grad.p, sizeof(double) * nco, hipMemcpyDeviceToHost, s),
            "copy gradient");
    HIP_TRY(hipMemcpyAsync(met, ctx->metrics.p, sizeof met, hipMemcpyDeviceToHost, s),
            "copy metrics");
    HIP_TRY(hipStreamSynchronize(s), "loss and gradient");
    float t[3] = {0, 0, 0}, tt = 0;
    (void)hipEventElapsedTime(&tt, ctx->tev[0], ctx->tev[3]);
    for (int k = 0; k < 3; ++k)
        (void)hipEventElapsedTime(&t[k], ctx->tev[k], ctx->tev[k + 1]);
    ctx->train_timings[0] = tt;
    for (int k = 0; k < 3; ++k)
        ctx->train_timings[k + 1] = t[k];
    // Trainer_MTP::AccumulateGard: mean over structures, then the penalty
    double f = ctx->nconf > 0 ? met[0] / ctx->nconf : 0.0;
    for (int k = 0; k < nco; ++k)
        grad[k] = ctx->nconf > 0 ? g[k] / ctx->nconf : 0.0;
    penalty(ctx->model, penalty_weight, reg_l2, reg_l1, f, grad);
    *loss = f;
    if (metrics)
        std::memcpy(metrics, met, sizeof met);
    return MTPX_OK;
}

int mtpx_last_train_timings(const mtpx_context *ctx, double out_ms[4])
{
    if (!ctx || !out_ms)
        return MTPX_E_INVALID;
    std::memcpy(out_ms, ctx->train_timings, sizeof ctx->train_timings);
    return MTPX_OK;
}

}  // extern "C"
