// Driver for the reference's vendored L-BFGS solver (deplibs/LBFGSpp:
// LBFGSSolver<double, LineSearchLewisOverton>, header-only, with the Eigen
// headers the reference vendors), compiled by oracle/Makefile into
// oracle/_ref/liblbfgs_ref.so.  Test infrastructure only.
//
// ref_lbfgs_minimize runs LBFGSSolver::minimize over a C callback.  As in
// Trainer_MTP::TrainNonLinearLBFGS (train/train_mtp.cpp:4336), the solver is
// handed the caller's vector itself and the objective receives that same
// vector, so a callback that overwrites x -- as Trainer_MTP::operator() does
// when it divides by the scaling -- changes the solver's iterate exactly as
// it does in the trainer.
#include <Eigen/Core>
#include <LBFGS.h>

#include <cstring>
#include <exception>
#include <string>

typedef int (*ref_objective)(void *user, double *x, double *grad, int n, double *f);

struct RefParams {
    int m;
    double epsilon, epsilon_rel, epsgmax;
    int past;
    double delta;
    int max_iterations, max_linesearch;
    double min_step, max_step, f_dec_coeff, s_curv_coeff, max_step_move, machine_prec;
    double initial_step, first_initial_step;
    int unscale_iterate;  // not read here: the callback decides
};

namespace {

struct Functor {
    ref_objective fn;
    void *user;
    double operator()(const Eigen::VectorXd &x, Eigen::VectorXd &g)
    {
        double f = 0;
        // x is the solver's iterate; the trainer's objective writes through
        // its alias, which the const_cast reproduces.
        double *xp = const_cast<double *>(x.data());
        if (fn(user, xp, g.data(), (int)x.size(), &f) != 0)
            throw std::runtime_error("objective returned nonzero");
        return f;
    }
};

}  // namespace

extern "C" int ref_lbfgs_minimize(const RefParams *p, int n, double *x, ref_objective fn,
                                  void *user, int *iterations, double *fx, char *msg, int msgcap)
{
    LBFGSpp::LBFGSParam<double> param;
    param.m = p->m;
    param.epsilon = p->epsilon;
    param.epsilon_rel = p->epsilon_rel;
    param.epsgmax = p->epsgmax;
    param.past = p->past;
    param.delta = p->delta;
    param.max_iterations = p->max_iterations;
    param.linesearch = LBFGSpp::LBFGS_LINESEARCH_LEWIS_OVERTON;
    param.max_linesearch = p->max_linesearch;
    param.min_step = p->min_step;
    param.max_step = p->max_step;
    param.f_dec_coeff = p->f_dec_coeff;
    param.s_curv_coeff = p->s_curv_coeff;
    param.max_step_move = p->max_step_move;
    param.machine_prec = p->machine_prec;
    param.initial_step = p->initial_step;
    param.first_initial_step = p->first_initial_step;
    Eigen::VectorXd xv = Eigen::Map<Eigen::VectorXd>(x, n);
    Functor f{fn, user};
    double fv = 0;
    int rc = 0, it = 0;
    if (msg && msgcap > 0)
        msg[0] = 0;
    try {
        LBFGSpp::LBFGSSolver<double, LBFGSpp::LineSearchLewisOverton> solver(param);
        it = solver.minimize(f, xv, fv);
    } catch (const std::exception &e) {
        rc = 1;
        if (msg && msgcap > 0) {
            std::strncpy(msg, e.what(), (size_t)msgcap - 1);
            msg[msgcap - 1] = 0;
        }
    }
    std::memcpy(x, xv.data(), sizeof(double) * n);
    if (iterations)
        *iterations = it;
    if (fx)
        *fx = fv;
    return rc;
}
