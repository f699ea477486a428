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

typedef struct mtpx_context mtpx_context;

/* Flat model view: the linear-MTP / RBChebyshev subset of
 * MTPGpuPotentialView (runtime/mtp/gpu-direct/mtp_gpu_direct.h:239-289).
 * Arrays are borrowed for the call and copied. */
typedef struct mtpx_model_view {
    int species_count;          /* Z */
    int radial_func_count;      /* M */
    int rb_size;                /* R */
    double min_dist, max_dist;  /* RBChebyshev interval; max_dist is the cutoff */
    double scaling;             /* radial basis scaling */
    int alpha_moments_count;    /* K */
    int alpha_index_basic_count;/* B */
    int alpha_index_times_count;/* T */
    int alpha_scalar_moments;   /* S */
    const int *alpha_index_basic;   /* [B][4] {mu, a, b, c} */
    const int *alpha_index_times;   /* [T][4] {l, r, c, out} */
    const int *alpha_moment_mapping;/* [S] */
    const double *radial_coeffs;    /* [Z][Z][M][R] */
    const double *species_coeffs;   /* [Z] */
    const double *moment_coeffs;    /* [S] */
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
 * (mtp_gpu_direct.h:800-806). */
int mtpx_load_model(mtpx_context *ctx, const mtpx_model_view *view);
/* PotMTP::Load (potentials/potential_mtp.cpp:119-571): .mtp text, non-split
 * RBChebyshev grammar, scaling defaulting to 0.01. */
int mtpx_load_model_text(mtpx_context *ctx, const char *text);
/* Host-only parse of .mtp text (no device needed): sizes Z M R K B T S ncoef
 * into out8, the flat coefficients into coeffs (may be NULL), the first
 * error into err.  Same grammar and defaults as mtpx_load_model_text. */
int mtpx_parse_model_text(const char *text, int out8[8], double *coeffs, char *err, int errlen);
/* Sizes: Z M R K B T S ncoef (ncoef = Z*Z*M*R + Z + S). */
int mtpx_model_info(const mtpx_context *ctx, int out8[8]);
/* PotMTP::get_coeffs / set_coeffs (potential_mtp.cpp:4160-4245) in the flat
 * order [radial | species | moment]; MTPGpuDirect::update_coefficients
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
 * orders every reduction (no floating-point atomics): byte-repeatable. */
int mtpx_efs(mtpx_context *ctx, int deterministic, double *energy, double *forces,
             double *stress, double *site_energies);
/* Same computation, outputs left on the device (benchmarking). */
int mtpx_efs_device(mtpx_context *ctx, int deterministic);
/* Device-side timing of the last mtpx_efs_device / mtpx_efs call, measured
 * with HIP events on the library's stream, in milliseconds:
 * {E/F/S kernel + reductions, E/F/S kernel alone, reductions, 0}. */
int mtpx_last_timings(const mtpx_context *ctx, double out_ms[4]);

#ifdef __cplusplus
}
#endif
#endif
