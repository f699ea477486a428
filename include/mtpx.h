/*
 * mtpx.h -- C ABI of the MI355X-native MTP energy/force/stress and training
 * loss-gradient path.
 *
 * Plain C: pointers, sizes and int status codes; no exceptions cross this
 * boundary and no torch or C++ types appear in it.  One context per host
 * thread and device; a context is not thread-safe (as one PotMTP object is
 * not, apps/calc_efs.cpp:335-338).  Every entry point returns MTPX_OK or a
 * negative MTPX_E* code and records a message readable with
 * mtpx_last_error().
 *
 * Each declaration names the reference interface it replaces (paths are
 * relative to the IMR-MLP source tree).
 */
#ifndef MTPX_H
#define MTPX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTPX_OK 0
#define MTPX_E_INVALID -1     /* bad argument or inconsistent sizes */
#define MTPX_E_MODEL -2       /* malformed or unsupported .mtp model */
#define MTPX_E_NO_MODEL -3    /* operation needs a loaded model */
#define MTPX_E_NO_TOPOLOGY -4 /* operation needs neighbour lists */
#define MTPX_E_DEVICE -5      /* HIP runtime failure */
#define MTPX_E_ALLOC -6       /* device or host allocation failed */
#define MTPX_E_CAPACITY -7    /* size beyond a documented limit */
#define MTPX_E_RANGE -8       /* neighbour image/box range not representable */
#define MTPX_E_SOLVER -9      /* the L-BFGS solver stopped on an error (its text) */

typedef struct mtpx_context mtpx_context;

/* Radial basis kinds, cutoffs and coordinate transforms of a model view, with
 * the values of the reference's RadialBasis, RadialCutoff and RadialTransform
 * (runtime/mtp/gpu-direct/mtp_gpu_direct.h:152-190). */
#define MTPX_RB_CHEBYSHEV 0
#define MTPX_RB_CHEBYCOS 1
#define MTPX_RB_CHEBYSHEV_POLY5 2
#define MTPX_RB_CHEBYSHEV_CONFIGURABLE 3
#define MTPX_RB_CHEBYSHEV_POLY4 4
#define MTPX_RB_POLYB 5          /* refused: MTPX_E_MODEL */
#define MTPX_RB_POLYBCOS 6       /* refused: MTPX_E_MODEL */
#define MTPX_CUT_QUADRATIC 0
#define MTPX_CUT_COSINE 1
#define MTPX_CUT_POLY5 2
#define MTPX_CUT_NORMALIZED_QUADRATIC 3
#define MTPX_CUT_COSINE_LEFT 4
#define MTPX_CUT_COSINE_UNSCALED 5
#define MTPX_CUT_COSINE_SQUARED 6
#define MTPX_CUT_SINE_SQUARED 7
#define MTPX_CUT_POLY3 8
#define MTPX_CUT_POLY4 9
#define MTPX_CUT_SMOOTHSTEP5 10
#define MTPX_CUT_SMOOTHSTEP7 11
#define MTPX_SHIFT_LINEAR 0
#define MTPX_SHIFT_EXPONENTIAL 1
#define MTPX_SHIFT_EXPONENTIAL_LEFT 2
#define MTPX_SHIFT_I2 3
#define MTPX_SHIFT_EXPONENTIAL_TANH 4
/* Site-energy models and activations, the values of MTPGpuModel and
 * MTPGpuActivation (mtp_gpu_direct.h:196-213): the linear MTP and the MTP-M
 * heads mtp_m_q2, mtp_m_fs, mtp_m_n1, mtp_m_n2 and mtp_m_li. */
#define MTPX_MODEL_LINEAR 0
#define MTPX_MODEL_MTPM_QUADRATIC 1
#define MTPX_MODEL_MTPM_ASINH 2
#define MTPX_MODEL_MTPM_NN1 3
#define MTPX_MODEL_MTPM_NN2 4
#define MTPX_MODEL_MTPM_LINEAR 5
#define MTPX_ACT_TANH 0
#define MTPX_ACT_RELU 1
#define MTPX_ACT_SIGMOID 2
#define MTPX_ACT_LINEAR 3

/* One radial basis: MTPGpuRadialBasisView (mtp_gpu_direct.h:215-236), as
 * MTPGpuEvaluator's radial_basis_for fills it
 * (potentials/mtp_gpu_adapter.cpp:110-212). */
typedef struct mtpx_radial_basis_view {
    int radial_basis;            /* MTPX_RB_* */
    double min_dist, max_dist, scaling;
    /* RBChebyshevConfigurable: */
    int cutoff;                  /* MTPX_CUT_* */
    int transform;               /* MTPX_SHIFT_* */
    double cutoff_parameter;     /* RBChebyshevPoly4/5 rb_b, or the configurable cutoff_b */
    double transform_parameter;  /* shift_lambda */
    int one_minus_chebyshev;     /* basis_function_type one_minus_chebyshev */
    double cutoff_r1, cutoff_r2; /* smoothstep7 interval */
    double transform_scale_parameter; /* shift_scale_lambda */
    /* PolyB / PolyBCos orthogonalisation tables (those kinds are refused) */
    const double *polynomial_matrix;
    const double *polynomial_normalizations;
} mtpx_radial_basis_view;

/* Flat model view: MTPGpuPotentialView (mtp_gpu_direct.h:239-289), field for
 * field, as MTPGpuEvaluator::initialize fills it
 * (potentials/mtp_gpu_adapter.cpp:427-441) and make_lammps_pair_view does
 * for the LAMMPS pair styles.  Arrays are borrowed for the call and copied.
 *
 * - spmap [max_type] maps the caller's atom types to species in
 *   [-1, species_count); -1 drops the atom from site requests.  Every type
 *   the context is later given (neighbour builds, batches, CSR lists, site
 *   requests) goes through it and must lie in [0, max_type).
 * - With pair_radial_basis_count == 0 the one basis is {radial_basis,
 *   min_dist, max_dist, scaling}, of kind MTPX_RB_CHEBYSHEV or
 *   MTPX_RB_CHEBYCOS.  Otherwise pair_radial_bases holds species_count^2
 *   bases in (centre, neighbour) species order: a split model, or one basis
 *   repeated (a non-split Poly4/Poly5/configurable model, as the adapter
 *   passes it).
 * - cutoff is the list cutoff, PotMTP::cutoff: the largest max_dist of the
 *   bases (0 takes that value).
 * - model selects the site-energy head.  MTPX_MODEL_LINEAR reads
 *   species_coeffs [species_count] and moment_coeffs [alpha_scalar_moments];
 *   an MTP-M head reads species_coeffs [species_count],
 *   descriptor_species_coeffs [descriptor_count][species_count],
 *   descriptor_moment_coeffs [descriptor_count][alpha_scalar_moments] and
 *   model_coeffs [model_coeffs_count], with moment_coeffs NULL.
 * - max_mu, max_alpha_index_basic and nu_arr_list are recomputed from
 *   alpha_index_basic and not read.
 * Refused with MTPX_E_MODEL: PolyB / PolyBCos bases, a RBChebyshevPoly5 or
 * configurable basis without pair descriptors, and the legacy NN scalar
 * gather (scalar_gather != 0). */
typedef struct mtpx_model_view {
    int species_count;          /* Z */
    int max_type;               /* entries of spmap */
    const int *spmap;           /* [max_type] */

    int alpha_moments_count;    /* K */
    int alpha_index_basic_count;/* B */
    int alpha_index_times_count;/* T */
    int alpha_scalar_moments;   /* S */

    int radial_func_count;      /* M */
    int rb_size;                /* R */
    int max_mu;
    int max_alpha_index_basic;

    double min_dist, max_dist;  /* the shared basis's interval */
    double cutoff;              /* list cutoff (0: the largest max_dist) */
    double scaling;             /* the shared basis's scaling */
    int radial_basis;           /* MTPX_RB_* of the shared basis */

    const mtpx_radial_basis_view *pair_radial_bases; /* [Z*Z] or NULL */
    int pair_radial_basis_count;                     /* 0 or Z*Z */

    const double *radial_coeffs;    /* [Z][Z][M][R] */
    int radial_coeffs_count;        /* Z*Z*M*R, or 0 for that */
    const double *species_coeffs;   /* [Z] */
    const double *moment_coeffs;    /* [S] (linear MTP only) */

    int model;                      /* MTPX_MODEL_* */
    int descriptor_count;           /* q (0 for the linear MTP) */
    int scalar_gather;              /* legacy NN inference: refused */
    const double *input_mean, *input_inverse_std, *input_species;
    const double *descriptor_species_coeffs; /* [q][Z] */
    const double *descriptor_moment_coeffs;  /* [q][S] */
    const double *model_coeffs;              /* [model_coeffs_count] */
    int model_coeffs_count;
    int model_activation;           /* MTPX_ACT_* */
    int model_hidden1;
    int model_hidden2;

    const int *alpha_index_basic;   /* [B][4] {mu, a, b, c} */
    const int *alpha_index_times;   /* [T][4] {l, r, c, out} */
    const int *alpha_moment_mapping;/* [S] */
    const int *nu_arr_list;         /* not read */
} mtpx_model_view;

/* ---- context ---------------------------------------------------------
 * MTPGpuDirect construction / destruction
 * (runtime/mtp/gpu-direct/mtp_gpu_direct.h:789-796). */
int mtpx_create(int device, mtpx_context **out);
void mtpx_destroy(mtpx_context *ctx);
/* MTPGpuDirect's `std::string* error` out-parameters (mtp_gpu_direct.h:800-920). */
const char *mtpx_last_error(const mtpx_context *ctx);
/* Library build string (kernel variants, target). */
const char *mtpx_version(void);

/* ---- model -----------------------------------------------------------
 * MTPGpuDirect::initialize(const MTPGpuPotentialView&)
 * (mtp_gpu_direct.h:800-806), with the checks of validate_potential_view
 * (runtime/mtp/gpu-direct/mtp_gpu_direct.cu:419-660): MTPX_E_INVALID for an
 * inconsistent view (the reference's texts), MTPX_E_MODEL for a kind this
 * library does not evaluate.  The species map stays with the model. */
int mtpx_load_model(mtpx_context *ctx, const mtpx_model_view *view);
/* Host-only: the .mtp text (PotMTP::Save layout, as mtpx_save_model_text) of
 * the model a view describes, after the same checks; buf / cap / len as
 * mtpx_save_model_text, the first error into err.  No device needed. */
int mtpx_format_model_view(const mtpx_model_view *view, char *buf, size_t cap, size_t *len,
                           char *err, int errlen);
/* The species map of the LAMMPS pair styles (make_lammps_pair_view,
 * mtp_gpu_direct.h:291-330) for the loaded model: spmap [max_type] in
 * [-1, Z), applied as mtpx_load_model's; NULL restores the identity map
 * over [0, Z) that a text or GPM load sets. */
int mtpx_set_species_map(mtpx_context *ctx, int max_type, const int *spmap);
/* PotMTP::Load (potentials/potential_mtp.cpp:119-571): .mtp text with a
 * shared radial basis or one per ordered species pair (radial_basis_split),
 * of the kinds RBChebyshev, RBChebyCos, RBChebyshevPoly4, RBChebyshevPoly5
 * and RBChebyshevConfigurable with any of its cutoffs and shifts
 * (basis/basis.h:19-29, basis/cutoff.h, basis/xtrans.h); scaling defaults
 * to 0.01; the
 * potential_tag is read as the reference's metadata (a structured tag
 * declares a linear MTP or a short-range MTP-M potential).  An MTP-M
 * potential (PotMTP_M::Load, potentials/potential_mtp_m.h:1950-2240, with
 * the head metadata of read_mtp_gpu_metadata, runtime/mtp/mlip.cpp:70-296:
 * a structured tag and / or "# mtp_*" lines) carries a site-energy head --
 * mtp_m_li, mtp_m_q2, mtp_m_fs, mtp_m_n1 or mtp_m_n2 -- over q descriptors;
 * its E/F/S, energies, sites and batch losses run on the device, its
 * training and linear-fit entry points return MTPX_E_MODEL. */
int mtpx_load_model_text(mtpx_context *ctx, const char *text);
/* Host-only parse of .mtp text (no device needed): sizes Z M R K B T S ncoef
 * into out8, the flat coefficients into coeffs (may be NULL), the first
 * error into err.  Same grammar and defaults as mtpx_load_model_text. */
int mtpx_parse_model_text(const char *text, int out8[8], double *coeffs, char *err, int errlen);
/* PotMTP::Save (potentials/potential_mtp.cpp:647-785, 1052-1061) of the
 * loaded model with its current coefficients: the .mtp text, numbers in
 * "%.17e", the potential_tag as the reference's metadata JSON.  buf may be
 * NULL (only *len, the text length without the terminating 0, is set);
 * otherwise cap must exceed that length (MTPX_E_CAPACITY if not). */
int mtpx_save_model_text(const mtpx_context *ctx, char *buf, size_t cap, size_t *len);
/* Host-only PotMTP::Load then PotMTP::Save of .mtp text (no device needed);
 * buf / cap / len as mtpx_save_model_text, the parse error into err. */
int mtpx_format_model_text(const char *text, char *buf, size_t cap, size_t *len, char *err,
                           int errlen);
/* GPM v2 model bundles (tools/gpm_container.h; the MTP node of
 * potentials/gpm_codec.cpp:190-382).  Loading: ModelBundle::load /
 * MLIPCore::read_model_text's GPM branch (runtime/mtp/mlip.cpp:354-383) for
 * a root model of type "mtp" or "mtp_m", blocks stored raw or zstd (the
 * system's libzstd.so.1, opened at run time); each radial basis keeps its
 * own scaling.  Saving: ModelBundle::save_potential (inference profile,
 * potentials/model_bundle.cpp:131-155) with blocks raw, or zstd at
 * zstd_level > 0; buf / cap / len as mtpx_save_model_text, without a
 * terminating 0 (cap must be at least *len).  The host-only forms need no
 * device: mtpx_gpm_to_text is GPM::mtp_text (tools/gpm_mtp.h:160-289),
 * mtpx_gpm_from_text the bundle of .mtp text, mtpx_parse_model_gpm the
 * sizes and coefficients of a bundle as mtpx_parse_model_text. */
int mtpx_load_model_gpm(mtpx_context *ctx, const void *bytes, size_t n);
int mtpx_save_model_gpm(const mtpx_context *ctx, int zstd_level, void *buf, size_t cap,
                        size_t *len);
int mtpx_gpm_to_text(const void *bytes, size_t n, char *buf, size_t cap, size_t *len, char *err,
                     int errlen);
int mtpx_gpm_from_text(const char *text, int zstd_level, void *buf, size_t cap, size_t *len,
                       char *err, int errlen);
int mtpx_parse_model_gpm(const void *bytes, size_t n, int out8[8], double *coeffs, char *err,
                         int errlen);
/* Sizes: Z M R K B T S ncoef (ncoef = Z*Z*M*R + Z + S for the linear MTP,
 * Z*Z*M*R + Z*(q+1) + q*S + model_coeffs_count with an MTP-M head). */
int mtpx_model_info(const mtpx_context *ctx, int out8[8]);
/* The site-energy head of the loaded potential (PotMTP_M::model_metadata,
 * potentials/potential_mtp_m.h:1564-1589; mlip::site_model_type,
 * runtime/mtp/mlip.h:54): out6 = {head, q, hidden1, hidden2, activation,
 * model_coeffs_count} with head 0 for the linear MTP (q 1), 1 mtp_m_li,
 * 2 mtp_m_q2, 3 mtp_m_fs, 4 mtp_m_n1, 5 mtp_m_n2 and activation 0 TANH,
 * 1 RELU, 2 SIGMOID, 3 LINEAR.  With a head the coefficients are ordered
 * [radial | species Z | descriptor species q*Z | moment q*S | head]. */
int mtpx_model_head(const mtpx_context *ctx, int out6[6]);
/* Host-only: the head of .mtp text, as mtpx_model_head (no device needed). */
int mtpx_parse_model_head(const char *text, int out6[6], char *err, int errlen);
/* PotMTP::cutoff (potentials/potential_mtp.cpp:300-310): the largest
 * max_dist of the radial bases, the list cutoff of the model. */
int mtpx_model_cutoff(const mtpx_context *ctx, double *cutoff);
/* PotMTP::get_coeffs / set_coeffs (potential_mtp.cpp:4160-4245) in the flat
 * order [radial | species | moment] (with a head, mtpx_model_head's order);
 * MTPGpuDirect::update_coefficients
 * (mtp_gpu_direct.h:813-818). */
int mtpx_get_coeffs(const mtpx_context *ctx, double *coeffs);
int mtpx_set_coeffs(mtpx_context *ctx, const double *coeffs);

/* ---- structures and neighbour lists ----------------------------------
 * Atoms::wrap (base/structures.cpp:1282-1305) on host arrays: cell rows are
 * lattice vectors, pos is [n][3] Cartesian, wrapped in place. */
int mtpx_wrap(const double cell[9], const int pbc[3], int n, double *pos);

/* Neighborhoods(atom, cutoff) with BOXED_NEBH
 * (base/neighborhood.cpp:77-146, base/neighborhoods_base.h:31-266), built
 * on the device.  The lists are bit-identical to the reference builder's:
 * same (centre, neighbour, image) entries in the same order, displacements
 * and distances equal bit for bit.  pos are the caller's (already wrapped)
 * positions; types are species indices.  The lists stay resident. */
int mtpx_build_neighbors(mtpx_context *ctx, const double cell[9], const int pbc[3], int n,
                         const double *pos, const int *types, double cutoff);
/* Number of directed entries of the resident lists. */
int mtpx_neighbor_count(const mtpx_context *ctx, int64_t *entries, int *centers);
/* Copy the resident lists to the host in the reference's Neighborhood layout
 * (base/anyneighborhoods.h:26-36): offsets [n+1], indices_, chemmap_, pos_
 * ([P][3]), distances_, centertype. */
int mtpx_get_neighbors(const mtpx_context *ctx, int *offsets, int *indices, int *types,
                       double *vecs, double *dists, int *center_types);
/* Upload host CSR lists, the layout MTPGpuBatch::build packs
 * (potentials/mtp_gpu_adapter.cpp:1011-1200). */
int mtpx_set_neighbors(mtpx_context *ctx, int n, const int *offsets, const int *indices,
                       const int *types, const double *vecs, const double *dists,
                       const int *center_types);

/* ---- energy, forces, stress ------------------------------------------
 * PotMTP::getEFS(Atoms&, AnyNeighborhoods&) (potential_mtp.cpp:1899-1933) and
 * MTPGpuDirect::compute_batch (mtp_gpu_direct.h:892).  Outputs: total energy,
 * forces [n][3], stress [3][3] (extensive virial, eV, S_ab = -sum D_a r_b),
 * site energies [n].  Any output pointer may be NULL.  deterministic != 0
 * orders every reduction (no floating-point atomics): byte-repeatable.
 * Lists built by mtpx_build_neighbors or mtpx_set_structures are always
 * assembled that way (each entry's reaction is gathered through the entry
 * of the other list that points back); lists from mtpx_set_neighbors use
 * floating-point atomics unless deterministic is set. */
int mtpx_efs(mtpx_context *ctx, int deterministic, double *energy, double *forces,
             double *stress, double *site_energies);
/* PotMTP::getE (potentials/potential_mtp.cpp:2604-2621, over
 * CalcSiteBasisImpl :3024-3122): energies only, no gradient.  energies
 * [nconf] (one per structure of the resident topology), site_energies [N];
 * either may be NULL. */
int mtpx_energy(mtpx_context *ctx, double *energies, double *site_energies);
/* Same computation, outputs left on the device (benchmarking). */
int mtpx_efs_device(mtpx_context *ctx, int deterministic);
/* Device-side timing of the last mtpx_efs_device / mtpx_efs call, measured
 * with HIP events on the library's stream, in milliseconds:
 * {E/F/S kernel + reductions, E/F/S kernel alone, reductions, 0}. */
int mtpx_last_timings(const mtpx_context *ctx, double out_ms[4]);
/* No counterpart in the reference (its evaluations have no device timers):
 * enabled != 0 (the default) records those HIP events on every E/F/S call;
 * 0 skips them (about 7 us per call on a 32,000-atom cell: three event
 * records and their read-back), and mtpx_last_timings then reports zeros. */
int mtpx_set_timings(mtpx_context *ctx, int enabled);

/* No counterpart in the reference: an allocation-free mtpx_efs for callers
 * that cannot allocate device memory (serving loops, harnesses that
 * forbid hipMalloc).  It launches on the context's own stream and
 * synchronises it before returning, so it cannot be recorded into a HIP
 * graph.  The fast (non-deterministic) E/F/S of
 * the resident model and lists, written to the caller's device buffers on
 * the context's device: forces [n][3] (overwritten), site_energies [n],
 * energy_stress [10] (energy, then the 3x3 stress row-major).  The per-wave
 * partial sums live in one static device array of 65,536 doubles (512 KiB)
 * per GPU, held until the process ends; a launch whose partial rows would
 * exceed it runs fewer workgroups instead, and a model whose single
 * workgroup would exceed it is refused with MTPX_E_CAPACITY.  Calls on one
 * GPU share that array: calls that overlap in time on one GPU (from several
 * contexts or threads) race.  Allocates nothing; returns after the results
 * are in the caller's buffers. */
int mtpx_efs_noalloc(mtpx_context *ctx, double *forces, double *site_energies,
                     double *energy_stress);

/* PotMTP's add_efs member (potentials/potential.h:188; getEFS
 * potentials/potential_mtp.cpp:1904-1907): 0 (the default) makes mtpx_efs
 * and mtpx_compute_batch overwrite energy, forces, stress and site energies;
 * 1 adds the results onto what the caller's arrays hold. */
int mtpx_set_add_efs(mtpx_context *ctx, int add_efs);

/* ---- CSR site requests with ghost atoms ------------------------------
 * MTPGpuBatchRequest / MTPGpuComputeRequest
 * (runtime/mtp/gpu-direct/mtp_gpu_direct.h:359-440, :455-517) as driven by
 * the LAMMPS pair style mlip/gpudirect
 * (LAMMPS/USER-MLIP/pair_MLIP_gpu_direct.cpp:577-603) and computed on the
 * CPU by MLIPCore::compute (runtime/mtp/mlip.cpp:907-1191).  Atoms 0 ..
 * ntotal-1 are owned (< nlocal) or ghosts; centre c is atom centers[c]
 * (< nlocal) with neighbours neighbors[offsets[c] .. offsets[c+1]-1] & mask,
 * atom indices < ntotal (ghosts allowed).  Per entry r = x[j] - x[i] (or the
 * given neighbor_vectors); entries with r.r == 0, r.r >= cutoff^2 or a
 * neighbour of species -1 are skipped, and so are centres of species -1
 * (the reference's species map returning -1; under the identity map, any
 * negative type).
 *
 * Outputs (each may be NULL):
 *   force [ntotal][3]: f_i += sum_j D_j, f_j -= D_j; added onto the array
 *     when accumulate_force (the reference default and LAMMPS semantics),
 *     overwritten otherwise;
 *   total_energy; global_virial [6] xx yy zz xy xz yz (symmetric part of
 *     -sum D r^T); both overwritten;
 *   site_energy [nlocal]: E_i of each centre at its atom index, 0 for owned
 *     atoms that are not centres; overwritten;
 *   site_virial [ntotal][6]: per entry -1/2 D r^T (symmetrised for the
 *     off-diagonal terms) to the centre and half to the neighbour (ghosts
 *     included), the LAMMPS per-atom virial of mlip.cpp:1164-1190;
 *     overwritten.
 * reuse_topology keeps the centres, offsets and neighbour indices of the
 * previous request (the counts must match) and refreshes types and
 * positions; when the kept centres change (a centre's species turns -1 or
 * back) the caller's offsets and neighbours are read and checked again.  deterministic orders every sum (no floating-point atomics).
 * Independent of the resident lists of mtpx_build_neighbors /
 * mtpx_set_structures, which stay as they are. */
typedef struct mtpx_site_request {
    int center_count;              /* centres (LAMMPS inum) */
    int nlocal;                    /* owned atoms */
    int ntotal;                    /* owned + ghost atoms */
    const int *centers;            /* [center_count] atom of each centre; NULL: 0 .. center_count-1 */
    const int *offsets;            /* [center_count + 1] */
    const int *neighbors;          /* [offsets[center_count]] atom indices (before the mask) */
    int neighbor_index_mask;       /* LAMMPS NEIGHMASK; -1 keeps every bit */
    const double *neighbor_vectors;/* [P][3] r_j - r_i, or NULL to take x[j] - x[i] */
    const int *type;               /* [ntotal] atom types through the species map
                                      (identity over 0 .. Z-1 unless a view or
                                      mtpx_set_species_map gave one); an atom
                                      whose species is -1 is skipped, and so is
                                      a negative type under the identity map */
    const double *x;               /* [ntotal][3]; may be NULL with neighbor_vectors */
    double *force;                 /* [ntotal][3] */
    double *total_energy;
    double *global_virial;         /* [6] */
    double *site_energy;           /* [nlocal] */
    double *site_virial;           /* [ntotal][6] */
    int accumulate_force;
    int reuse_topology;
    int deterministic;
} mtpx_site_request;
int mtpx_compute_sites(mtpx_context *ctx, const mtpx_site_request *req);

/* ---- training batches -------------------------------------------------
 * A batch is nconf structures stored one after the other: structure c owns
 * atoms atom_offsets[c] .. atom_offsets[c+1]-1 of pos [N][3] and types [N],
 * its cell is cells[9c .. 9c+8] and its periodicity pbc[3c .. 3c+2].  The
 * lists of every structure are built on the device as by
 * mtpx_build_neighbors and concatenated into one CSR with global atom
 * indices: the flattened topology of MTPGpuBatchRequest
 * (mtp_gpu_direct.h:452-517) and MTPGpuBatch::build
 * (potentials/mtp_gpu_adapter.cpp:1011-1200).  All structures are built in
 * the same kernel launches; batches above 2^21 atoms (or the environment
 * variable MTPX_NEIGHBOR_CHUNK_ATOMS, when smaller) are built in chunks of
 * whole structures.  Replaces the resident lists; mtpx_build_neighbors /
 * mtpx_set_neighbors make a batch of one. */
int mtpx_set_structures(mtpx_context *ctx, int nconf, const int *atom_offsets,
                        const double *cells, const int *pbc, const double *pos, const int *types,
                        double cutoff);
/* Number of structures of the resident topology. */
int mtpx_structure_count(const mtpx_context *ctx, int *nconf);
/* MTPGpuDirect::compute_batch (mtp_gpu_direct.h:892) over the batch: per
 * structure energy [nconf] and stress [nconf][9] (as mtpx_efs), forces
 * [N][3] and site energies [N].  Any output may be NULL; the outputs stay
 * resident for mtpx_prepare_loss. */
int mtpx_compute_batch(mtpx_context *ctx, int deterministic, double *energy, double *forces,
                       double *stress, double *site_energies);

/* Loss settings of Trainer_MTP (train/train_mtp.cpp:2552-2568; the
 * defaults 1, 0.01, 1e-4, 1, 0, 1, 0.1, 0, 1 are the reference's). */
typedef struct mtpx_loss_settings {
    double weight_energy, weight_forces, weight_stress;
    double energy_pow, force_pow, stress_pow;   /* weights divided by N^pow */
    double force_norm_d, force_norm_f, force_norm_p;
} mtpx_loss_settings;
/* Host-only: the per-structure weights Trainer_MTP::AddLossGard applies
 * (train/train_mtp.cpp:3839-3996).  has [nconf][3] flags labels present
 * (energy, forces, stress); target_forces [N][3] (used by the force
 * normalisation), fitness [nconf] and atomic_fitness [N] may be NULL
 * (weight 1).  Out: active [nconf][3] (the term is part of the loss),
 * energy_weight [nconf], force_weight [N], stress_weight [nconf]. */
int mtpx_loss_weights(const mtpx_loss_settings *s, int nconf, const int *atom_offsets,
                      const int *has, const double *target_forces, const double *fitness,
                      const double *atomic_fitness, int *active, double *energy_weight,
                      double *force_weight, double *stress_weight);
/* MTPGpuLossRequest labels (mtp_gpu_direct.h:561-579): active [nconf][3],
 * target_energy [nconf], energy_weight [nconf], target_forces [N][3],
 * force_weight [N], target_stress [nconf][9], stress_weight [nconf].  Arrays
 * of inactive terms may be NULL. */
int mtpx_set_labels(mtpx_context *ctx, const int *active, const double *target_energy,
                    const double *energy_weight, const double *target_forces,
                    const double *force_weight, const double *target_stress,
                    const double *stress_weight);
/* MTPGpuDirect::prepare_loss: the weighted loss of the last
 * mtpx_compute_batch outputs against the labels, summed over structures;
 * the adjoints dL/dE, dL/dF, dL/dS stay resident.  metrics [7]: total,
 * energy, force and stress loss, squared per-atom energy error, squared
 * force error, squared stress error (mtp_gpu_direct.h:561-566). */
int mtpx_prepare_loss(mtpx_context *ctx, double metrics[7]);
/* MTPGpuDirect::accumulate_gradient / PotMTP::AccumulateEFSCombinationGard
 * (mtp_gpu_direct.h:523-555; potentials/potential_mtp.cpp:6896-6923): the
 * coefficient gradient [ncoef] of sum_c (dLdE_c E_c + sum_i dLdF_i . F_i +
 * dLdS_c : S_c), in the flat order [radial | species | moment].  dLdE
 * [nconf], dLdF [N][3], dLdS [nconf][9] (row-major 3x3); all three NULL use
 * the adjoints of mtpx_prepare_loss.  accumulate != 0 adds to gradient.
 * The sum is ordered: repeatable bit for bit. */
int mtpx_accumulate_gradient(mtpx_context *ctx, const double *dLdE, const double *dLdF,
                             const double *dLdS, int accumulate, double *gradient);
/* PotMTP::AddPenaltyGard, radial_mode 0 (potentials/potential_mtp.cpp:
 * 6568-6742), on the current coefficients: adds the orthonormality penalty
 * of the radial functions and L2/L1 regularisation of the moment
 * coefficients to *loss and grad [ncoef]. */
int mtpx_penalty(const mtpx_context *ctx, double weight, double reg_l2, double reg_l1,
                 double *loss, double *grad);
/* Trainer_MTP::AccumulateGard / operator() (train/train_mtp.cpp:3039-3094,
 * :4256-4297) over the resident batch and labels: loss = sum_c L_c / nconf
 * + penalty, grad = sum_c g_c / nconf + penalty gradient; metrics [7] as
 * mtpx_prepare_loss (may be NULL). */
int mtpx_loss_grad(mtpx_context *ctx, int deterministic, double penalty_weight, double reg_l2,
                   double reg_l1, double *loss, double *grad, double metrics[7]);
/* LBFGSpp::LBFGSParam of the trainer's L-BFGS (deplibs/LBFGSpp/include/
 * LBFGSpp/Param.h:99-243), the fields the Lewis-Overton line search reads;
 * the trainer's options lbfgspp:* (train/train_mtp.cpp:59,144-163) set them. */
typedef struct mtpx_lbfgs_params {
    int m;                     /* corrections kept (6) */
    double epsilon;            /* stop when |g| <= epsilon (1e-5) */
    double epsilon_rel;        /* ... or |g| <= epsilon_rel |x| (1e-5) */
    double epsgmax;            /* ... or max |g_i| <= epsgmax (0) */
    int past;                  /* relative-decrease test over `past` iterations (0: off) */
    double delta;              /* its tolerance (0) */
    int max_iterations;        /* 0: no limit */
    int max_linesearch;        /* evaluations per line search (20) */
    double min_step, max_step; /* 1e-20, 1e20 */
    double f_dec_coeff;        /* sufficient decrease (1e-4) */
    double s_curv_coeff;       /* curvature (0.9) */
    double max_step_move;      /* largest move of one coordinate (1e20) */
    double machine_prec;       /* bracket width limit (1e-16) */
    double initial_step;       /* step of later iterations; < 0: 1 */
    double first_initial_step; /* first step; < 0: 1 / |g| */
    /* mtpx_train_lbfgs only.  1 (the trainer's behaviour): every evaluation
     * leaves the solver's iterate at the coefficients x / scaling, because
     * Trainer_MTP::operator() divides the vector it is given -- the solver's
     * own iterate -- in place (train_mtp.cpp:4260-4264, 4336).  0: the
     * iterate stays in the scaled coordinates. */
    int unscale_iterate;
} mtpx_lbfgs_params;
/* The LBFGSParam defaults of the reference's vendored LBFGSpp, with the
 * trainer's epsgmax = 0 (train_mtp.cpp:59) and unscale_iterate = 1. */
void mtpx_lbfgs_default_params(mtpx_lbfgs_params *p);
/* The objective of mtpx_lbfgs_minimize: writes f(x) to *f and its gradient to
 * grad[n]; may overwrite x, as the trainer's objective does.  A nonzero
 * return stops the solver with MTPX_E_INVALID. */
typedef int (*mtpx_lbfgs_objective)(void *user, double *x, double *grad, int n, double *f);
/* LBFGSSolver<double, LineSearchLewisOverton>::minimize (deplibs/LBFGSpp/
 * include/LBFGS.h:81-190, LBFGSpp/LineSearchLewisOverton.h:47-133) over a
 * caller's objective; host only.  x [n]: in, the starting point; out, the
 * final iterate.  iterations, fx, evaluations and message may be NULL.  The
 * solver's exceptions (bad parameters, "exceed max linesearch", "width too
 * small", "inf or nan", ...) return MTPX_E_INVALID (parameters, objective
 * status) or MTPX_E_SOLVER with LBFGSpp's text in message[message_cap]. */
int mtpx_lbfgs_minimize(const mtpx_lbfgs_params *params, int n, double *x,
                        mtpx_lbfgs_objective objective, void *user, int *iterations, double *fx,
                        int *evaluations, char *message, int message_cap);
/* Trainer_MTP::TrainNonLinearLBFGS (train/train_mtp.cpp:4300-4339): the
 * solver above over Trainer_MTP::operator() (:4256-4295) -- coefficients
 * x / scaling, the objective and gradient of mtpx_loss_grad on the resident
 * batch and labels, the gradient times scaling.  scaling [ncoef] or NULL for
 * ones.  x [ncoef] (Trainer_MTP::x_in) or NULL: in, the starting point in
 * scaled coordinates (NULL: the context's coefficients times scaling); out,
 * the final iterate.  The context keeps the coefficients of the last
 * evaluation.  iterations, loss (the last objective value), history (the
 * objective of the first history_cap evaluations) and evaluations may be
 * NULL.  A failed line search returns MTPX_E_SOLVER with the solver's text. */
int mtpx_train_lbfgs(mtpx_context *ctx, const mtpx_lbfgs_params *params, const double *scaling,
                     double *x, int deterministic, double penalty_weight, double reg_l2,
                     double reg_l1, int *iterations, double *loss, double *history,
                     int history_cap, int *evaluations);
/* Device-side timing of the last mtpx_loss_grad, milliseconds:
 * {whole call, E/F/S, loss, gradient}. */
int mtpx_last_train_timings(const mtpx_context *ctx, double out_ms[4]);

/* ---- linear fit -------------------------------------------------------
 * PotMTP::CalcEFSCmpt_R (potentials/potential_mtp.cpp:2675-2707, over
 * CalcSiteBasisDers :3163-3280; potential_mtp.h:1609) for every structure of
 * the resident topology: the energy [nconf][p], force [N][3][p] and stress
 * [nconf][9][p] of each linear coefficient (p = Z + S: species, then moment
 * coefficients), so that E = sum_q x_q energy_cmpts[q] etc.  Outputs may be
 * NULL. */
int mtpx_efs_components(mtpx_context *ctx, double *energy_cmpts, double *force_cmpts,
                        double *stress_cmpts);
/* Trainer_MTP::AddLinearFast rows (train/train_mtp.cpp:1289-1395) for the
 * resident batch and labels: per structure the force rows of the atoms with
 * a positive force weight (x, y, z), the 9 stress rows, the energy row, each
 * scaled by sqrt(weight); y the scaled targets.  A [nrows][p], y [nrows];
 * with A and y NULL only *nrows is set, otherwise *nrows is the capacity on
 * entry and the count on return. */
int mtpx_linear_rows(mtpx_context *ctx, int64_t *nrows, double *A, double *y);
/* Trainer_MTP::fix_species_coeffs (train/train_mtp.cpp:1300-1302,
 * 1381-1392): 1 makes mtpx_linear_rows and mtpx_linear_system leave out the
 * Z species columns (rows of S values, p = S) and subtract
 * sum_s n_s species_coeffs[s] (the model's current species coefficients)
 * from each energy target; 0 (the default) keeps p = Z + S. */
int mtpx_set_fix_species_coeffs(mtpx_context *ctx, int fix);
/* Trainer_MTP::TrainLinearFast assembly (train/train_mtp.cpp:2383-2427):
 * G = A^T A [p][p] and b = A^T y [p] over the rows of mtpx_linear_rows,
 * summed on the fp64 matrix cores in a fixed order; p <= 1007
 * (MTPX_E_CAPACITY beyond). */
int mtpx_linear_system(mtpx_context *ctx, double *G, double *b);
/* PotMTP::Orthogonalize (potentials/potential_mtp.cpp:3849-3930) of the
 * radial coefficients; TrainLinearFast calls it before the assembly. */
int mtpx_orthogonalize(mtpx_context *ctx);
/* Device-side timing of the last mtpx_linear_system, milliseconds:
 * {whole call, components kernel, Gram kernel, rows}. */
int mtpx_last_linear_timings(const mtpx_context *ctx, double out[4]);

#ifdef __cplusplus
}
#endif
#endif
