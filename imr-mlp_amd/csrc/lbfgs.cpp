// C ABI, the trainer's L-BFGS loop (include/mtpx.h: mtpx_lbfgs_minimize,
// mtpx_train_lbfgs).  Host code; no exceptions escape.
//
// Trainer_MTP::TrainNonLinearLBFGS (train/train_mtp.cpp:4300-4339) drives the
// vendored LBFGSpp solver -- LBFGSSolver::minimize (deplibs/LBFGSpp/include/
// LBFGS.h) with the Lewis-Overton line search, the library's default
// (LBFGSpp/LineSearchLewisOverton.h, Param.h:224-243) -- over
// Trainer_MTP::operator() (:4256-4295): coefficients x = x_s / scaling, the
// loss and gradient of the whole training set (AccumulateGard: the mean over
// structures plus the penalty), the gradient multiplied by scaling.  This
// file restates that iteration in its own code, with the loss and gradient
// of every evaluation computed on the device by mtpx_loss_grad:
//   * the two-loop recursion of the limited-memory inverse Hessian with m
//     corrections and theta = y'y / s'y (BFGSMat::apply_Hv), a correction
//     kept when s'y > 1e-12 |s| |y|;
//   * directions that are not finite or not descending restart from -g;
//   * first step 1 / |d|, later steps 1 (unless set), capped so that no
//     coefficient moves more than max_step_move;
//   * the line search doubles the step until the sufficient-decrease test
//     fails, then bisects [mu, nu]; it accepts a step that satisfies both
//     Wolfe tests or reaches the step cap;
//   * stop when |g| <= epsilon, |g| <= epsilon_rel |x|, max |g_i| <= epsgmax,
//     the relative decrease over `past` iterations is below delta, or after
//     max_iterations.
// The objective may overwrite the iterate it is given: Trainer_MTP::operator()
// receives the solver's own iterate (minimize(*this, x_in, ...) with x_in the
// trainer's member, which operator() then divides by scaling in place), so in
// the reference every evaluation leaves the solver at x / scaling.
// mtpx_train_lbfgs keeps that behaviour unless unscale_iterate is 0.
#include "context.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

double dot(const std::vector<double> &a, const std::vector<double> &b)
{
    double s = 0;
    for (size_t k = 0; k < a.size(); ++k)
        s += a[k] * b[k];
    return s;
}
double norm(const std::vector<double> &a) { return std::sqrt(dot(a, a)); }
double maxabs(const std::vector<double> &a)
{
    double m = 0;
    for (double v : a)
        m = std::max(m, std::fabs(v));
    return m;
}
bool finite(const std::vector<double> &a)
{
    for (double v : a)
        if (!std::isfinite(v))
            return false;
    return true;
}

// Limited-memory inverse Hessian: m (s, y) pairs in a ring.
struct Memory {
    int m = 6, ncorr = 0, ptr = 6;
    double theta = 1;
    std::vector<std::vector<double>> s, y;
    std::vector<double> ys, alpha;
    void reset(int n, int mm)
    {
        m = mm;
        theta = 1;
        s.assign(m, std::vector<double>(n));
        y.assign(m, std::vector<double>(n));
        ys.assign(m, 0);
        alpha.assign(m, 0);
        ncorr = 0;
        ptr = m;
    }
    void add(const std::vector<double> &ds, const std::vector<double> &dy)
    {
        const int loc = ptr % m;
        s[loc] = ds;
        y[loc] = dy;
        ys[loc] = dot(s[loc], y[loc]);
        theta = dot(y[loc], y[loc]) / ys[loc];
        if (ncorr < m)
            ++ncorr;
        ptr = loc + 1;
    }
    // res = a H v
    void apply(const std::vector<double> &v, double a, std::vector<double> &res)
    {
        const size_t n = v.size();
        res.resize(n);
        for (size_t k = 0; k < n; ++k)
            res[k] = a * v[k];
        int j = ptr % m;
        for (int i = 0; i < ncorr; ++i) {
            j = (j + m - 1) % m;
            alpha[j] = dot(s[j], res) / ys[j];
            for (size_t k = 0; k < n; ++k)
                res[k] -= alpha[j] * y[j][k];
        }
        for (size_t k = 0; k < n; ++k)
            res[k] /= theta;
        for (int i = 0; i < ncorr; ++i) {
            const double beta = dot(y[j], res) / ys[j];
            for (size_t k = 0; k < n; ++k)
                res[k] += (alpha[j] - beta) * s[j][k];
            j = (j + 1) % m;
        }
    }
};

// A line-search failure (the solver's exceptions): the message and status.
struct Stop {
    int code;
    std::string msg;
};

}  // namespace

extern "C" {

void mtpx_lbfgs_default_params(mtpx_lbfgs_params *p)
{
    if (!p)
        return;
    p->m = 6;
    p->epsilon = 1e-5;
    p->epsilon_rel = 1e-5;
    p->epsgmax = 0;
    p->past = 0;
    p->delta = 0;
    p->max_iterations = 0;
    p->max_linesearch = 20;
    p->min_step = 1e-20;
    p->max_step = 1e20;
    p->f_dec_coeff = 1e-4;
    p->s_curv_coeff = 0.9;
    p->max_step_move = 1e20;
    p->machine_prec = 1e-16;
    p->initial_step = -1;
    p->first_initial_step = -1;
    p->unscale_iterate = 1;
}

}  // extern "C"

namespace {

// LBFGSParam::check_param (Param.h:250-285), the conditions on the fields
// the solver and the Lewis-Overton search read.
const char *check_params(const mtpx_lbfgs_params &P)
{
    if (P.m <= 0)
        return "'m' must be positive";
    if (P.epsilon < 0)
        return "'epsilon' must be non-negative";
    if (P.epsilon_rel < 0)
        return "'epsilon_rel' must be non-negative";
    if (P.past < 0)
        return "'past' must be non-negative";
    if (P.delta < 0)
        return "'delta' must be non-negative";
    if (P.max_iterations < 0)
        return "'max_iterations' must be non-negative";
    if (P.max_linesearch <= 0)
        return "'max_linesearch' must be positive";
    if (P.min_step < 0)
        return "'min_step' must be positive";
    if (P.max_step < P.min_step)
        return "'max_step' must be greater than 'min_step'";
    if (!(P.f_dec_coeff > 0 && P.f_dec_coeff < 1))
        return "'f_dec_coeff' must satisfy 0 < f_dec_coeff <1";
    if (!(P.s_curv_coeff > P.f_dec_coeff && P.s_curv_coeff < 1))
        return "'s_curv_coeff must satisfy f_dec_coeff < s_curv_coeff < 1";
    return nullptr;
}

using Objective = double (*)(void *user, double *x, double *grad, int n);

// LBFGSSolver::minimize with LineSearchLewisOverton.  Throws Stop.
int minimize(const mtpx_lbfgs_params &P, int n, std::vector<double> &x, Objective fg, void *user,
             double &fx, int &nevals)
{
    std::vector<double> grad((size_t)n), gradp((size_t)n), xp((size_t)n), drt((size_t)n);
    std::vector<double> dx((size_t)n), dgr((size_t)n);
    std::vector<double> fpast((size_t)std::max(P.past, 1));
    Memory H;
    H.reset(n, P.m);
    auto f = [&](std::vector<double> &at, std::vector<double> &g) {
        ++nevals;
        return fg(user, at.data(), g.data(), n);
    };
    auto converged = [&] {
        const double gn = norm(grad);
        return gn <= P.epsilon || gn <= P.epsilon_rel * norm(x) || maxabs(grad) <= P.epsgmax;
    };
    fx = f(x, grad);
    if (P.past > 0)
        fpast[0] = fx;
    if (converged())
        return 1;
    for (int i = 0; i < n; ++i)
        drt[i] = -grad[i];
    double step = P.first_initial_step < 0 ? 1.0 / norm(drt) : P.first_initial_step;
    for (int k = 1;; ++k) {
        xp = x;
        gradp = grad;
        if (!finite(drt) || dot(grad, drt) >= 0) {
            H.reset(n, P.m);
            for (int i = 0; i < n; ++i)
                drt[i] = -grad[i];
        }
        const double step_max = std::min(P.max_step, P.max_step_move / maxabs(drt));
        step = std::min(step, step_max);
        // ---- line search: doubling, then bisection of [mu, nu] -------------
        if (step <= 0)
            throw Stop{MTPX_E_SOLVER, "'step' must be positive"};
        const double fx_init = fx, dg_init = dot(grad, drt);
        if (dg_init > 0)
            throw Stop{MTPX_E_SOLVER, "the moving direction increases the objective function value"};
        const double dgtest = P.f_dec_coeff * dg_init, dstest = P.s_curv_coeff * dg_init;
        const double drmax = maxabs(drt);
        double cap = step_max;
        if (cap * drmax > P.max_step_move)
            cap = P.max_step_move / drmax;
        step = std::min(step, cap);
        double mu = 0.0, nu = cap;
        bool bracketed = false;
        for (int count = 1;; ++count) {
            for (int i = 0; i < n; ++i)
                x[i] = xp[i] + step * drt[i];
            fx = f(x, grad);
            if (!std::isfinite(fx))
                throw Stop{MTPX_E_SOLVER, "inf or nan"};
            if (fx > fx_init + step * dgtest) {
                nu = step;
                bracketed = true;
            } else {
                // a decreasing step at the cap is accepted without curvature
                if (step >= cap || !(dot(grad, drt) < dstest))
                    break;
                mu = step;
            }
            if (count >= P.max_linesearch)
                throw Stop{MTPX_E_SOLVER, "exceed max linesearch"};
            if (bracketed && (nu - mu) < P.machine_prec * nu)
                throw Stop{MTPX_E_SOLVER, "width too small"};
            step = bracketed ? 0.5 * (mu + nu) : step * 2.0;
            if (step < P.min_step)
                throw Stop{MTPX_E_SOLVER, "linesearch step below minimum allowed value"};
            step = std::min(step, cap);
        }
        // ---- convergence tests ---------------------------------------------
        if (converged())
            return k;
        if (P.past > 0) {
            const double fxd = fpast[k % P.past];
            if (k >= P.past &&
                std::fabs(fxd - fx) <= P.delta * std::max(std::max(std::fabs(fx), std::fabs(fxd)), 1.0))
                return k;
            fpast[k % P.past] = fx;
        }
        if (P.max_iterations != 0 && k >= P.max_iterations)
            return k;
        for (int i = 0; i < n; ++i) {
            dx[i] = x[i] - xp[i];
            dgr[i] = grad[i] - gradp[i];
        }
        if (finite(dx) && finite(dgr) && dot(dx, dgr) > 1e-12 * norm(dx) * norm(dgr))
            H.add(dx, dgr);
        H.apply(grad, -1.0, drt);
        step = P.initial_step < 0 ? 1.0 : P.initial_step;
    }
}

// Trainer_MTP::operator() over a context: coefficients x / scaling, the
// device loss and gradient, the gradient times scaling.
struct TrainObjective {
    mtpx_context *ctx;
    const std::vector<double> *sc;
    std::vector<double> coef, graw;
    int deterministic, unscale;
    double penalty_weight, reg_l2, reg_l1;
    double *history;
    int history_cap, nhist = 0;

    static double call(void *user, double *x, double *g, int n)
    {
        auto &o = *static_cast<TrainObjective *>(user);
        const std::vector<double> &sc = *o.sc;
        for (int k = 0; k < n; ++k)
            o.coef[k] = x[k] / sc[k];
        int rc = mtpx_set_coeffs(o.ctx, o.coef.data());
        double fx = 0;
        if (rc == MTPX_OK)
            rc = mtpx_loss_grad(o.ctx, o.deterministic, o.penalty_weight, o.reg_l2, o.reg_l1, &fx,
                                o.graw.data(), nullptr);
        if (rc != MTPX_OK)
            throw Stop{rc, o.ctx->err};
        for (int k = 0; k < n; ++k)
            g[k] = o.graw[k] * sc[k];
        if (o.unscale)
            for (int k = 0; k < n; ++k)
                x[k] = o.coef[k];
        if (o.history && o.nhist < o.history_cap)
            o.history[o.nhist++] = fx;
        return fx;
    }
};

// The callback of mtpx_lbfgs_minimize; a nonzero status stops the solver.
struct UserObjective {
    mtpx_lbfgs_objective fn;
    void *user;
    static double call(void *self, double *x, double *g, int n)
    {
        auto &o = *static_cast<UserObjective *>(self);
        double fx = 0;
        const int rc = o.fn(o.user, x, g, n, &fx);
        if (rc != 0)
            throw Stop{MTPX_E_INVALID, "objective returned status " + std::to_string(rc)};
        return fx;
    }
};

}  // namespace

extern "C" {

int mtpx_lbfgs_minimize(const mtpx_lbfgs_params *params, int n, double *x,
                        mtpx_lbfgs_objective objective, void *user, int *iterations, double *fx,
                        int *evaluations, char *message, int message_cap)
{
    auto say = [&](const std::string &m) {
        if (message && message_cap > 0) {
            const size_t len = std::min(m.size(), (size_t)message_cap - 1);
            std::memcpy(message, m.data(), len);
            message[len] = 0;
        }
    };
    say("");
    if (!params || !x || !objective || n <= 0) {
        say("null argument");
        return MTPX_E_INVALID;
    }
    if (const char *bad = check_params(*params)) {
        say(bad);
        return MTPX_E_INVALID;
    }
    std::vector<double> xv(x, x + n);
    UserObjective o{objective, user};
    int k = 0, nevals = 0, rc = MTPX_OK;
    double f = 0;
    try {
        k = minimize(*params, n, xv, &UserObjective::call, &o, f, nevals);
    } catch (const Stop &s) {
        rc = s.code;
        say(s.msg);
    } catch (const std::exception &e) {
        rc = MTPX_E_ALLOC;
        say(e.what());
    }
    std::memcpy(x, xv.data(), sizeof(double) * n);
    if (iterations)
        *iterations = k;
    if (fx)
        *fx = f;
    if (evaluations)
        *evaluations = nevals;
    return rc;
}

int mtpx_train_lbfgs(mtpx_context *ctx, const mtpx_lbfgs_params *params, const double *scaling,
                     double *x, int deterministic, double penalty_weight, double reg_l2,
                     double reg_l1, int *iterations, double *loss, double *history,
                     int history_cap, int *evaluations)
{
    if (!ctx || !params)
        return set_error(ctx, MTPX_E_INVALID, "null argument");
    if (!ctx->has_model)
        return set_error(ctx, MTPX_E_NO_MODEL, "no model loaded");
    if (need_linear(ctx, "mtpx_train_lbfgs") != MTPX_OK)
        return MTPX_E_MODEL;
    if (const char *bad = check_params(*params))
        return set_error(ctx, MTPX_E_INVALID, bad);
    const int n = ctx->model.ncoef();
    std::vector<double> sc((size_t)n, 1.0);
    if (scaling)
        for (int k = 0; k < n; ++k) {
            if (!(scaling[k] != 0) || !std::isfinite(scaling[k]))
                return set_error(ctx, MTPX_E_INVALID, "scaling must be finite and nonzero");
            sc[k] = scaling[k];
        }
    std::vector<double> xv((size_t)n);
    for (int k = 0; k < n; ++k)
        xv[k] = x ? x[k] : ctx->model.coef[k] * sc[k];
    TrainObjective o;
    o.ctx = ctx;
    o.sc = &sc;
    o.coef.assign((size_t)n, 0.0);
    o.graw.assign((size_t)n, 0.0);
    o.deterministic = deterministic;
    o.unscale = params->unscale_iterate;
    o.penalty_weight = penalty_weight;
    o.reg_l2 = reg_l2;
    o.reg_l1 = reg_l1;
    o.history = history;
    o.history_cap = history ? history_cap : 0;
    int k = 0, nevals = 0, rc = MTPX_OK;
    double f = 0;
    try {
        k = minimize(*params, n, xv, &TrainObjective::call, &o, f, nevals);
    } catch (const Stop &s) {
        rc = set_error(ctx, s.code, s.msg);
    } catch (const std::exception &e) {
        rc = set_error(ctx, MTPX_E_ALLOC, e.what());
    }
    if (x)
        std::memcpy(x, xv.data(), sizeof(double) * n);
    if (iterations)
        *iterations = k;
    if (loss)
        *loss = f;
    if (evaluations)
        *evaluations = nevals;
    return rc;
}

}  // extern "C"
