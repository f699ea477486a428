// The C-ABI context (include/mtpx.h) and helpers shared by the host files.
#pragma once

#include "mtpx.h"
#include "mtpx_internal.hpp"

#include <string>
#include <vector>

using namespace mtpx;

struct mtpx_context {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    int num_cus = 256;
    size_t lds_limit = 160 * 1024;  // LDS one workgroup may allocate

    bool has_model = false;
    Model model;
    // MTPGpuPotentialView::spmap: caller types [0, max_type) -> species
    // [-1, Z); the identity over [0, Z) unless a view or mtpx_set_species_map
    // set one (spmap_set)
    std::vector<int> spmap;
    int max_type = 0;
    bool spmap_set = false;
    Plan plan;
    DevModel dm{};
    // model buffers
    DBuf radial, species, moment, map, seed, slot_basic, slot_abc, dup, fwd_level, fwd_steps,
        fwd_lcomb, fwd_comb, bwd_level, bwd_steps, bwd_lcomb, bwd_comb, rb_table;
    // MTP-M head tables and the DevHead that points at them
    DBuf head_ids, head_proj, head_dsp, head_coef, head_params;

    // neighbour lists
    bool has_nbh = false;
    NeighborStore nbh;
    NeighborScratch scratch;
    int &n = nbh.n;
    int64_t &P = nbh.P;
    DBuf &offsets = nbh.offsets, &idx = nbh.idx, &type = nbh.type, &x = nbh.x, &y = nbh.y,
         &z = nbh.z, &d = nbh.d, &center_type = nbh.center_type;
    DBuf rev_offsets, rev_pairs;
    std::vector<int> offsets_host;  // [n+1], kept with the reverse index
    bool rev_ready = false;
    int max_species = -1;  // largest species index in the lists

    // structures of the resident topology (one unless a batch is set)
    int nconf = 0;
    std::vector<int> soff_host;          // [nconf+1] first atom of each structure
    DBuf soff, center_structure;         // device copies; [N] structure of each atom
    int single_n = -1;  // soff and center_structure describe one structure of this many atoms

    // outputs
    DBuf forces, site_energy, partial, pair_ders, out10;
    DBuf site_virial, benergy, bstress;  // batch: [N][9], [nconf], [nconf][9]
    EfsLaunch launch{};
    bool has_batch_out = false;          // compute_batch outputs match model and topology

    // training: labels, adjoints, gradient rows
    bool has_labels = false, has_adjoints = false;
    DBuf active, tE, wE, tF, wF, tS, wS;
    DBuf dLdE, dLdF, dLdS, metric_rows, metrics, grad_rows, grad;
    NeighborStore nbh_tmp;
    // host copies of the labels (linear-fit rows)
    std::vector<int> active_h;
    std::vector<double> tE_h, wE_h, tF_h, wF_h, tS_h, wS_h;
    long label_gen = 0;  // bumped by every set_labels

    // linear fit: plan, components [fc | sc | ec], row descriptors, Gram
    bool has_lin = false;
    std::string lin_err;
    LinPlan lin;
    DevLin dl{};
    DBuf lin_level, lin_steps, lin_lcomb, lin_comb, lin_ent, lin_estart, lin_chunk, lin_maskw,
        lin_clist, lin_flevel, lin_fsteps, lin_flcomb, lin_fcomb, lin_walk, lin_walk_off, lin_cscal;
    DBuf comp, row_src, row_sw, row_y, rowsA, rowsY, gram_part, gram_out, lin_pair, lin_site;
    // tile path: walk-order Jacobian values per site, structure lists per size class
    DBuf lin_lw, lin_tiles;
    long rows_gen = -1;  // label_gen and p of the uploaded row descriptors
    int rows_p = -1;
    int64_t rows_R = 0;
    // Trainer_MTP::fix_species_coeffs: rows without the species columns,
    // energy targets less the species part (the coefficients the rows
    // were built with are kept to know when to rebuild them)
    bool fix_species = false, rows_fix = false;
    std::vector<double> rows_species;
    double lin_timings[4] = {0, 0, 0, 0};
    double train_timings[4] = {0, 0, 0, 0};
    hipEvent_t tev[4] = {nullptr, nullptr, nullptr, nullptr};

    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    double timings[4] = {0, 0, 0, 0};
    bool timings_on = true;  // mtpx_set_timings

    // PotMTP::add_efs: E/F/S outputs are added onto the caller's arrays
    bool add_efs = false;

    // device address of this GPU's static scratch array (mtpx_efs_noalloc),
    // taken once at mtpx_create with the device current
    double *noalloc_scratch = nullptr;

    // CSR site requests (mtpx_compute_sites): their own topology, kept for
    // reuse_topology; independent of the resident lists above
    struct Sites {
        bool valid = false;
        int center_count = 0, nlocal = 0, ntotal = 0, rows = 0;
        int64_t P_in = 0;            // entries of the request (before dropped centres)
        std::vector<int> row_atom;   // atom of each kept centre row
        std::vector<int> row_src;    // request centre index of each kept row
        NeighborStore nb;            // offsets, idx, type, x, y, z, d, center_type
        DBuf center_atom, atom_type, pos, vec, atom_row, rev_offsets, rev_pairs, forces,
            site_virial6, site_energy, partial, out10, pair_ders;
        void release()
        {
            for (DBuf *b : {&nb.offsets, &nb.idx, &nb.type, &nb.x, &nb.y, &nb.z, &nb.d,
                            &nb.center_type, &center_atom, &atom_type, &pos, &vec, &atom_row,
                            &rev_offsets, &rev_pairs, &forces, &site_virial6, &site_energy,
                            &partial, &out10, &pair_ders})
                b->release();
        }
    } sites;

    ~mtpx_context()
    {
        for (DBuf *b : {&radial, &species, &moment, &map, &seed, &slot_basic, &slot_abc, &dup,
                        &fwd_level, &fwd_steps, &fwd_lcomb, &fwd_comb, &bwd_level, &bwd_steps,
                        &bwd_lcomb, &bwd_comb, &rb_table, &head_ids, &head_proj, &head_dsp,
                        &head_coef, &head_params, &offsets, &idx, &type, &x, &y, &z, &d,
                        &center_type, &rev_offsets, &rev_pairs, &forces, &site_energy, &partial,
                        &pair_ders, &out10, &soff, &center_structure, &site_virial, &benergy,
                        &bstress, &active, &tE, &wE, &tF, &wF, &tS, &wS, &dLdE, &dLdF, &dLdS,
                        &metric_rows, &metrics, &grad_rows, &grad, &nbh_tmp.offsets,
                        &nbh_tmp.idx, &nbh_tmp.type, &nbh_tmp.x, &nbh_tmp.y, &nbh_tmp.z,
                        &nbh_tmp.d, &nbh_tmp.center_type, &nbh.mirror, &nbh_tmp.mirror,
                        &lin_level, &lin_steps, &lin_lcomb,
                        &lin_comb, &lin_ent, &lin_estart, &lin_chunk, &lin_maskw, &lin_clist,
                        &lin_walk, &lin_walk_off, &lin_cscal,
                        &comp, &row_src, &row_sw, &row_y, &rowsA, &rowsY, &gram_part, &gram_out,
                        &lin_pair, &lin_site, &lin_flevel, &lin_fsteps, &lin_flcomb,
                        &lin_fcomb, &lin_lw, &lin_tiles})
            b->release();
        scratch.release_all();
        sites.release();
        for (auto &e : ev)
            if (e)
                (void)hipEventDestroy(e);
        for (auto &e : tev)
            if (e)
                (void)hipEventDestroy(e);
        if (stream)
            (void)hipStreamDestroy(stream);
    }
};

namespace mtpx {


inline int set_error(mtpx_context *ctx, int code, const std::string &msg)
{
    if (ctx)
        ctx->err = msg;
    return code;
}

// The training, gradient and linear-fit paths restate the linear MTP's
// trainer (train/train_mtp.cpp); a potential with an MTP-M head is evaluated
// (E/F/S, energies, sites, batches, losses) but not trained here.
inline int need_linear(mtpx_context *ctx, const char *what)
{
    if (ctx->has_model && !ctx->model.linear())
        return set_error(ctx, MTPX_E_MODEL,
                         std::string(what) + " supports the linear MTP only (the loaded "
                                             "potential has an MTP-M head)");
    return MTPX_OK;
}

// MTPGpuPotentialView -> host model and species map (model_view.cpp), with
// validate_potential_view's checks; on failure code and err are set.
bool model_from_view(const mtpx_model_view &v, Model &m, std::vector<int> &spmap, int &code,
                     std::string &err);

// Every value finite (branch-free, vectorised).
bool all_finite(const double *v, size_t n);
// Every species in [0, Z); maxs receives the largest (-1 for none).
bool species_in_range(const int *t, size_t n, int Z, int &maxs);

// Caller atom types -> species through the loaded model's species map.
// Without an explicit map (text or GPM loads) `out` is `types` itself and
// nothing is checked here.  With one, every type must lie in [0, max_type)
// ("atom type is outside the species-map range", as the reference's
// requests); allow_unmapped keeps species -1 (site requests skip such
// atoms), otherwise a type mapped to -1 is refused.
int map_species(mtpx_context *ctx, const int *types, size_t n, bool allow_unmapped,
                std::vector<int> &buf, const int *&out);

inline int hip_fail(mtpx_context *ctx, hipError_t e, const char *what)
{
    return set_error(ctx, e == hipErrorOutOfMemory ? MTPX_E_ALLOC : MTPX_E_DEVICE,
                     std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                                                                \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess)                                                              \
            return hip_fail(ctx, e_, what);                                                \
    } while (0)

template <class T>
hipError_t upload(DBuf &b, const std::vector<T> &v, hipStream_t s)
{
    hipError_t e = b.ensure(sizeof(T) * std::max<size_t>(v.size(), 1));
    if (e != hipSuccess || v.empty())
        return e;
    return hipMemcpyAsync(b.p, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice, s);
}

// Copies `count` doubles from the device to dst; with add, adds them onto
// what dst holds (PotMTP::add_efs, the reference's accumulate_force).
int copy_out(mtpx_context *ctx, double *dst, const void *src, size_t count, bool add,
             const char *what);

// Runs the E/F/S kernel over the resident topology (capi.cpp); with
// site_virial the per-atom virials are written too; energy_only skips the
// gradient (site energies and the total only).
int run_efs(mtpx_context *ctx, bool deterministic, bool site_virial = false,
            bool energy_only = false);
// Marks the topology as one structure of all atoms.
int set_single_structure(mtpx_context *ctx);
// Reverse index of the resident lists (and their offsets on the host).
int ensure_reverse_index(mtpx_context *ctx);
// MTPX_E_INVALID when the lists hold a species the model does not have.
int check_species(mtpx_context *ctx);
// Device view of the resident lists.
DevNeighbors dev_neighbors(const mtpx_context *ctx);

}  // namespace mtpx
