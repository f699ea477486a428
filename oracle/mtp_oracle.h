/*
 * mtp_oracle.h -- CPU restatement of IMR-MLP's MTP energy/force/stress and
 * training loss-gradient path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: it may be loaded by
 * tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of bench.py,
 * and by nothing else.  The product (imr-mlp_amd/) never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the IMR-MLP source tree.
 */
#ifndef MTP_ORACLE_H
#define MTP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One radial basis (basis/basis.h:104-278): RBChebyshev (0), RBChebyCos (1),
 * RBChebyshevPoly4 (2), RBChebyshevPoly5 (3), RBChebyshevConfigurable (4;
 * basis/basis.cpp:866-1031 with basis/cutoff.cpp and basis/xtrans.cpp). */
typedef struct orc_basis {
    int type;
    double rmin, rmax, scaling;   /* min_val, max_val, scaling */
    double b;                     /* rb_b of the Poly4/Poly5 bases */
    /* RBChebyshevConfigurable: cutoff type (Cutoff::CutoffType order),
     * shift type (XTransForm::ShiftType order), basis_function_type
     * one_minus_chebyshev, and their parameters */
    int cut, shift, one_minus;
    double cut_b, cut_r1, cut_r2, lambda, scale_lambda;
} orc_basis;

/* Linear MTP (potentials/potential_mtp.h:93, coefficient layout
 * potentials/potential_mtp.h:170-176); one shared radial basis, or one per
 * ordered species pair when split (potential_mtp.cpp:188-265). */
typedef struct orc_model {
    int Z, M, R;                  /* species_count, radial_funcs_count, rb_size */
    double rmin, rmax, scaling;   /* the first basis; rmax is replaced by the cutoff below */
    double cutoff;                /* max over the pair bases of max_dist */
    int split;                    /* radial_basis_split */
    orc_basis *bases;             /* [1] or [Z*Z] (pair ti * Z + tj) */
    char *tag;                    /* potential_tag text after '=', trimmed ("" if none) */
    int K, B, T, S;               /* alpha_moments_count, basic, times, scalar moments */
    int *basic;                   /* [B][4] {mu, a, b, c} */
    int *times;                   /* [T][4] {l, r, c, out} */
    int *map;                     /* [S] alpha_moment_mapping */
    int *nu;                      /* [B] a+b+c (nu_arr_list) */
    int max_nu1;                  /* max_alpha_index_basic = max nu + 1 */
    int max_mu;                   /* max mu + 1 */
    int nradial, ncoef;           /* Z*Z*M*R, nradial + Z + S (linear MTP) */
    double *coef;                 /* [radial | species | moments] */
    /* MTP-M site-energy head (potentials/potential_mtp_m.h:3383-3456; the
     * heads of runtime/mtp/cpu/mtp_cpu.cpp:291-368): 0 linear MTP, 1
     * mtp_m_li, 2 mtp_m_q2, 3 mtp_m_fs, 4 mtp_m_n1, 5 mtp_m_n2.  With a head
     * the coefficients are [radial | species Z | descriptor species P*Z |
     * moments P*S | head Mc] and E_i = species[t] + head(Q),
     * Q_p = dspecies[p*Z + t] + sum_s moments[p*S + s] m_map(s). */
    int head, P, h1, h2, act;     /* act: 0 tanh, 1 relu, 2 sigmoid, 3 linear */
    int Mc;
} orc_model;

/* Directed neighbour lists in CSR form (base/anyneighborhoods.h:26-67). */
typedef struct orc_nbh {
    int n;                        /* centres (atoms) */
    int64_t P;                    /* directed entries */
    int *offsets;                 /* [n+1] */
    int *idx;                     /* [P] original index of the neighbour */
    int *types;                   /* [P] species of the neighbour */
    double *vec;                  /* [P][3] r_j - r_i */
    double *dist;                 /* [P] |r_j - r_i| */
    int *pt;                      /* [P] extended point index (originals, then images) */
    int *center_types;            /* [n] */
    int npts;                     /* originals + periodic images */
    double *pts;                  /* [npts][3] re-wrapped originals, then images */
    int *orig;                    /* [npts] */
    int boxle[3];
} orc_nbh;

typedef struct orc_loss_settings {
    double weight_eng, weight_force, weight_stress;          /* 1, 0.01, 1e-4 */
    double eng_pow, force_pow, stress_pow;                   /* 1, 0, 1 */
    double force_norm_d, force_norm_f, force_norm_p;         /* 0.1, 0, 1 */
} orc_loss_settings;

/* One training configuration's labels. */
typedef struct orc_config {
    int n;
    int has_energy, has_forces, has_stress;
    double energy;                /* target E */
    const double *forces;         /* [n][3] target F */
    const double *stress;         /* [3][3] target S */
    double fitness;               /* Atoms::fitness (1 by default) */
    const double *atomic_fitness; /* [n] or NULL */
} orc_config;

/* ---- model ---------------------------------------------------------- */
orc_model *orc_model_load_text(const char *text, char *err, int errlen);
void orc_model_free(orc_model *m);
int orc_model_info(const orc_model *m, int *out11);   /* Z M R K B T S max_nu1 max_mu nradial ncoef */
int orc_model_head(const orc_model *m, int *out6);    /* head P h1 h2 act Mc; returns head */
void orc_model_get_coeffs(const orc_model *m, double *x);
void orc_model_set_coeffs(orc_model *m, const double *x);
void orc_model_tables(const orc_model *m, int *basic, int *times, int *map, double *rb3);
int orc_model_save_text(const orc_model *m, char *buf, int buflen);
void orc_orthogonalize(orc_model *m);

/* ---- radial basis --------------------------------------------------- */
void orc_rb_calc_der(const orc_model *m, double r, double *val, double *der);
void orc_rb_calc_der_pair(const orc_model *m, int ti, int tj, double r, double *val,
                          double *der);

/* ---- structures and neighbours -------------------------------------- */
void orc_wrap(const double *cell, const int *pbc, int n, double *pos);
void orc_cell_inverse(const double *cell, double *inv);
orc_nbh *orc_build_neighbors(const double *cell, const int *pbc, int n, const double *pos,
                             const int *types, double cutoff, char *err, int errlen);
orc_nbh *orc_nbh_from_csr(int n, const int *offsets, const int *idx, const int *types,
                          const double *vec, const double *dist, const int *center_types);
void orc_nbh_free(orc_nbh *h);
int64_t orc_nbh_size(const orc_nbh *h, int *n, int *npts, int *boxle);
void orc_nbh_export(const orc_nbh *h, int *offsets, int *idx, int *types, double *vec,
                    double *dist, int *pt, int *center_types);
void orc_nbh_export_points(const orc_nbh *h, double *pts, int *orig);

/* ---- inference ------------------------------------------------------ */
void orc_site_efs(const orc_model *m, const orc_nbh *h, int i, double *site_energy,
                  double *ders /* [n_i][3] */);
void orc_efs(const orc_model *m, const orc_nbh *h, double *energy, double *forces,
             double *stress, double *site_energies);
void orc_efs_omp(const orc_model *m, const orc_nbh *h, int nthreads, double *energy,
                 double *forces, double *stress, double *site_energies);
void orc_energy(const orc_model *m, const orc_nbh *h, double *energy, double *site_energies);
void orc_site_moments(const orc_model *m, const orc_nbh *h, int i, double *moments);

/* ---- training ------------------------------------------------------- */
void orc_accumulate_fp_grad(const orc_model *m, const orc_nbh *h, int i, double se_weight,
                            const double *f_weight, double *grad);
void orc_accumulate_efs_combination_grad(const orc_model *m, const orc_nbh *h, double dLdE,
                                         const double *dLdF, const double *dLdS, double *grad);
int orc_add_loss_grad(const orc_model *m, const orc_nbh *h, const orc_loss_settings *s,
                      const orc_config *c, double *loss, double *grad, double *metrics);
void orc_add_penalty_grad(const orc_model *m, double weight, double reg_l2, double reg_l1,
                          double *loss, double *grad);
int orc_loss_grad_batch(const orc_model *m, int nconf, orc_nbh *const *hs,
                        const orc_config *cs, const orc_loss_settings *s, double penalty_weight,
                        double reg_l2, double reg_l1, int nthreads, double *f, double *g);

/* ---- linear fit ----------------------------------------------------- */
void orc_efs_components(const orc_model *m, const orc_nbh *h, double *energy_cmpts,
                        double *force_cmpts /* [n][3][p] */, double *stress_cmpts /* [3][3][p] */);
int64_t orc_linear_rows(const orc_model *m, const orc_nbh *h, const orc_loss_settings *s,
                        const orc_config *c, double *A, double *y);
/* orc_linear_rows with Trainer_MTP::fix_species_coeffs: rows of S values
 * (the species columns dropped), energy targets less the species part. */
int64_t orc_linear_rows_ex(const orc_model *m, const orc_nbh *h, const orc_loss_settings *s,
                           const orc_config *c, int fix_species, double *A, double *y);
int64_t orc_linear_row_count(const orc_loss_settings *s, const orc_config *c);
void orc_gram(int64_t rows, int p, const double *A, const double *y, double *G, double *b);
int orc_linear_system_batch(const orc_model *m, int nconf, orc_nbh *const *hs,
                            const orc_config *cs, const orc_loss_settings *s, int nthreads,
                            double *G, double *b);
int orc_linear_system_batch_ex(const orc_model *m, int nconf, orc_nbh *const *hs,
                               const orc_config *cs, const orc_loss_settings *s, int fix_species,
                               int nthreads, double *G, double *b);

/* ---- flop convention shared with the benchmark ---------------------- */
double orc_efs_flops(const orc_model *m, const orc_nbh *h);

#ifdef __cplusplus
}
#endif
#endif
