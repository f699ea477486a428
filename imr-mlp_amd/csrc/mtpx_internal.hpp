// Internal types shared by the host runtime and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace mtpx {

// Compile-time ceilings of the kernel variants; a model is run by the
// smallest variant whose ceilings it fits.
constexpr int kMaxMu = 8;       // radial functions
constexpr int kMaxNu = 8;       // angular degree a+b+c
constexpr int kMaxR = 16;       // radial basis size
constexpr int kWave = 64;       // CDNA wavefront
constexpr int kChunk = 16;      // slots per LDS reduction chunk
constexpr int kRedStride = 66;  // row stride of the reduction buffer (16-byte rows, no bank conflicts)
// Product-rule step tables: the shortest piece a task is split into, and
// the padding steps after the last level (the kernels read the steps in
// groups of four, so a group that starts in a level's last steps reads at
// most three steps past it).
constexpr int kMinPiece = 2;
constexpr int kRulePad = 3;

// Growable device allocation owned by a context.
struct DBuf {
    void *p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need)
    {
        if (need <= bytes && p)
            return hipSuccess;
        if (p) {
            // queued work may still read the old allocation
            (void)hipDeviceSynchronize();
            (void)hipFree(p);
        }
        p = nullptr;
        bytes = 0;
        const size_t want = need < 64 ? 64 : need;
        hipError_t e = hipMalloc(&p, want);
        if (e == hipSuccess)
            bytes = want;
        return e;
    }
    template <class T> T *as() const { return static_cast<T *>(p); }
    void release()
    {
        if (p)
            (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};

// Pinned host memory (hipHostMalloc) for uploads and read-backs that the
// stream runs asynchronously; growing it assumes that no copy from or into
// it is still queued.
struct HBuf {
    void *p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t need)
    {
        if (need <= bytes && p)
            return hipSuccess;
        release();
        const size_t want = need < 4096 ? 4096 : need;
        hipError_t e = hipHostMalloc(&p, want, 0);
        if (e == hipSuccess)
            bytes = want;
        else
            p = nullptr;
        return e;
    }
    template <class T> T *as() const { return static_cast<T *>(p); }
    void release()
    {
        if (p)
            (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
};

// Resident neighbour lists (SoA) and the builder's scratch.
struct NeighborStore {
    int n = 0;
    int64_t P = 0;
    DBuf offsets, idx, type, x, y, z, d, center_type;
    // mirror[p]: the entry of list idx[p] that is entry p seen from the other
    // end (an image of the centre at the opposite offset; p itself for the
    // images of the centre): lists built here have it, lists handed over do
    // not
    DBuf mirror;
    bool has_mirror = false;
};
struct NeighborScratch {
    DBuf pts, orig, flags, scan, tmp, minmax, box, box_start, box_cur, box_items, rank, cnt,
        cursor, key, st_nbr, st_ctr, st_mate, st_final, scalars;
    // per-structure tables of a batch with the positions and species (atom
    // offsets, wrap flags and cells; candidate, box, interior-box and flag
    // offsets, geometry and image candidates; image counts; point offsets)
    // and the wrapped positions
    DBuf seg_head, seg_tabs, seg_imgs, seg_pts, wrapped;
    // pinned staging of the two table uploads and of the read-backs, and
    // the positions and species, which the wrap kernel reads in place
    HBuf up_head, up_tabs, down, up_pos;
    // entries per atom that the staging of a one-pass build reserves (0: none
    // known yet); set from the longest list of the last counted build
    long long bin_cap = 0;
    void release_all()
    {
        for (DBuf *b : {&pts, &orig, &flags, &scan, &tmp, &minmax, &box, &box_start, &box_cur,
                        &box_items, &rank, &cnt, &cursor, &key, &st_nbr, &st_ctr, &st_mate,
                        &st_final, &scalars, &seg_head, &seg_tabs, &seg_imgs, &seg_pts, &wrapped})
            b->release();
        for (HBuf *b : {&up_head, &up_tabs, &down, &up_pos})
            b->release();
        bin_cap = 0;
    }
};
// Builds the lists on the device (neighbors.hip); returns an MTPX_* code.
int build_neighbors_gpu(const double cell[9], const int pbc[3], int n, const double *pos,
                        const int *types, double cutoff, hipStream_t s, NeighborStore &out,
                        NeighborScratch &w, std::string &err);

// Builds the lists of nconf structures (atoms atom_offsets[c] .. [c+1]) in
// the same launches and concatenates them: atom and entry indices are global.
int build_neighbors_batch_gpu(int nconf, const int *atom_offsets, const double *cells,
                              const int *pbc, const double *pos, const int *types, double cutoff,
                              hipStream_t s, NeighborStore &out, NeighborStore &tmp,
                              NeighborScratch &w, std::string &err);

// A JSON value (the potential_tag metadata, metadata.cpp).
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;
};
bool json_parse(const std::string &text, Json &out, std::string &err);
std::string json_serialize(const Json &v);
// potential_tag of an .mtp file: the fields of a structured tag, or the plain
// text of a legacy one (MTPMetadata::Tag, tools/mtp_metadata.h:93-370).
struct MetaTag {
    std::map<std::string, Json> fields;
    std::string legacy;
};
// MTP-M site-energy heads (potentials/potential_mtp_m.h; the kinds of
// mlip::site_model_type, runtime/mtp/mlip.h:54) and the activations of the
// neural ones (mlip::activation_type).
enum HeadKind { kHeadNone = 0, kHeadLi, kHeadQ2, kHeadFs, kHeadNn1, kHeadNn2 };
enum ActKind { kActTanh = 0, kActRelu, kActSigmoid, kActLinear };
// The head of a potential: kind, descriptor count P (q), hidden layer sizes,
// activation and head coefficient count.  kHeadNone is the linear MTP (P 1).
struct Head {
    int kind = kHeadNone, P = 1, h1 = 0, h2 = 0, act = kActTanh, Mc = 0;
};
bool tag_parse(const std::string &raw, int Z, MetaTag &tag, std::string &err);
// The head a potential declares, from its structured tag and its
// "mtp_<key> = value" lines (read_mtp_gpu_metadata, runtime/mtp/mlip.cpp:
// 70-296), which also asks a head for a model_coeffs section and refuses one
// without a head.
bool head_parse(const std::string &text, const MetaTag &tag, Head &head, std::string &err);
std::string tag_output(const MetaTag &tag, const Head &head);

// Radial basis kinds (basis/basis.h:19-29): the Chebyshev polynomials of
// xi = (2r - (min + max)) / (max - min) times an envelope, and the
// configurable basis (Chebyshev polynomials of a shift x(r) times a cutoff
// function, basis/basis.cpp:866-1031, basis/cutoff.cpp, basis/xtrans.cpp).
enum RadialKind {
    kRBChebyshev = 0,
    kRBChebyCos = 1,
    kRBChebyshevPoly4 = 2,
    kRBChebyshevPoly5 = 3,
    kRBChebyshevConfigurable = 4
};
// Cutoff::CutoffType and XTransForm::ShiftType, in their enum order.
enum CutoffKind {
    kCutQuadratic, kCutNormalizedQuadratic, kCutCosine, kCutCosineLeft, kCutCosineUnscaled,
    kCutCosineSquared, kCutSineSquared, kCutPoly3, kCutPoly4, kCutPoly5, kCutSmoothstep5,
    kCutSmoothstep7
};
enum ShiftKind { kShiftLinear, kShiftExponential, kShiftExponentialLeft, kShiftI2, kShiftExponentialTanh };
struct RadialBasis {
    int kind = kRBChebyshev;
    double rmin = 0, rmax = 0, scaling = 0.01;
    double b = 0;  // rb_b of the Poly4 / Poly5 envelopes
    // RBChebyshevConfigurable: cutoff and shift kinds, one_minus_chebyshev,
    // cutoff_b, cutoff_r1, cutoff_r2, shift_lambda, shift_scale_lambda
    int cut = kCutQuadratic, shift = kShiftLinear;
    bool one_minus = false;
    double cut_b = 0, cut_r1 = 0, cut_r2 = 0, lambda = 0, scale_lambda = 0;
};
// Per-pair basis table on the device: kRbStride doubles per ordered species
// pair.  Envelope kinds: {kind, min, max, scaling, mult, su, pu, pi / max,
// b, 1 / su}; the configurable kind: {kind, min, max, scaling, cutoff,
// shift, one_minus, cutoff_b, r1, r2, lambda, scale_lambda, 1 / (max - min),
// expm1(lambda), tanh(scale_lambda), 0}.
constexpr int kRbStride = 16;

// Host-side model: the linear MTP (potentials/potential_mtp.h:93) or an
// MTP-M potential (potentials/potential_mtp_m.h) plus the launch plan derived
// from its contraction graph.
struct Model {
    int Z = 0, M = 0, R = 0, K = 0, B = 0, T = 0, S = 0;
    // rmin / scaling of the first basis, rmax the largest cutoff of any pair
    double rmin = 0, rmax = 0, scaling = 0.01;
    bool split = false;                // radial_basis_split: one basis per ordered pair
    std::vector<RadialBasis> bases;    // [1] or [Z*Z]
    MetaTag tag;
    // true unless every pair uses the one shared RBChebyshev basis
    bool general_basis() const { return split || (!bases.empty() && bases[0].kind != kRBChebyshev); }
    const RadialBasis &pair_basis(int ti, int tj) const { return split ? bases[ti * Z + tj] : bases[0]; }
    std::vector<int> basic;   // [B][4]
    std::vector<int> times;   // [T][4]
    std::vector<int> map;     // [S]
    // linear MTP: [Z*Z*M*R | Z | S]; with a head (PotMTP_M::Load,
    // potential_mtp_m.h:2057-2063): [Z*Z*M*R | Z | P*Z | P*S | Mc] -- species,
    // descriptor species, moment coefficients per descriptor, head
    std::vector<double> coef;
    Head head;
    bool linear() const { return head.kind == kHeadNone; }
    int nradial() const { return Z * Z * M * R; }
    int nspecies() const { return linear() ? Z : Z * (head.P + 1); }
    int nmoment() const { return head.P * S; }
    int ncoef() const { return nradial() + nspecies() + nmoment() + head.Mc; }
};

// Parses .mtp text (PotMTP::Load grammar).
bool parse_mtp(const std::string &text, Model &m, std::string &err);
// .mtp text of a model in PotMTP::Save layout (potentials/potential_mtp.cpp:
// 647-785, 1052-1061).
std::string save_mtp(const Model &m);
// Validates sizes and index ranges of a model view.
bool validate_model(const Model &m, std::string &err);
// The named settings of a radial basis as AnyBasis::SaveToStream writes
// them on a stream of 17 significant digits, in order.
std::vector<std::pair<std::string, std::string>> basis_settings(const RadialBasis &b, int R);
// GPM v2 model bundles (gpm.cpp): the .mtp text of a bundle's root MTP or
// MTP-M model (GPM::mtp_text, tools/gpm_mtp.h:160-289) with each radial
// basis's own scaling, and the bundle of a model (encode_mtp,
// potentials/gpm_codec.cpp:190-312, in ModelBundle::save_potential's
// manifest); zstd_level > 0 compresses the blocks.
bool gpm_is_bundle(const void *bytes, size_t n);
bool gpm_read(const void *bytes, size_t n, std::string &text, std::vector<double> &scalings,
              std::string &err);
bool gpm_write(const Model &m, int zstd_level, std::string &out, std::string &err);

// Launch plan: basic moments in canonical order, the product rules grouped by
// dependency level and output (forward) or destination (reverse).
struct Plan {
    int numax[kMaxMu];        // per mu: max degree present, -1 if absent
    int numax_all = -1;
    int nslots = 0;           // canonical (nu, mu, alpha) slots
    std::vector<int> slot_basic;   // [nslots] basic index or -1 (padding)
    std::vector<int> slot_abc;     // [nslots] a | b << 8 | c << 16
    std::vector<int> dup;          // [ndup][2] {duplicate basic, source basic}
    // Each wave owns a private LDS work space (indices in doubles):
    //   [0, K4) moments | [K4, 2 K4) adjoints | dummy (a zero slot) |
    //   [part0, red0) partial sums | [red0, priv_doubles) transpose buffer.
    int K4 = 0, dummy = 0, part0 = 0, red0 = 0, priv_doubles = 0;
    // Training work space (doubles): [0, tr_grad) the E/F/S work space
    // without its transpose buffer and its dual copy as pairs (element x at
    // 2x, its dual at 2x + 1), the radial gradient accumulator (tr_grad,
    // nradial) and 64 neighbour species (tr_ctype, as ints).  The transpose
    // buffers of the first and the last neighbour pass (tr_red1, tr_red4) and
    // the slot-ordered {A, G} pairs (tr_stage, nslots4) lie over blocks that
    // are dead in their phase, or after the species where they do not fit
    // there.
    int tr_red1 = 0, tr_red4 = 0, tr_stage = 0, tr_grad = 0, tr_ctype = 0, tr_priv = 0;
    // E/F/S kernel: transpose buffer, slot-ordered adjoints, the wave's
    // energy/virial sums and, with an MTP-M head, the head's work space
    // (descriptors, their adjoints, hidden activations and derivatives, the
    // second layer's adjoints: over the dead transpose buffer where it fits)
    // (offsets in doubles).
    int efs_red = 0, efs_stage = 0, efs_acc = 0, efs_head = 0;
    // first slot of each (nu, mu) block, -1 where absent: [nu * kMaxMu + mu]
    int slot_base[(kMaxNu + 1) * kMaxMu];
    // Lane-major step tables, one per direction.  Level L owns steps
    // [level_step[L], level_step[L+1]) and kRulePad padding steps follow
    // the last level; step s of lane q is
    // entry s * 64 + q, an int2 of work-space indices:
    //   x = l | r << 16,  y = w | first << 16 | last << 17 | c << 18  (c signed)
    //   acc += c * ws[l] * ws[r];  if (last) { ws[w] = init + acc; acc = 0; }
    // with init = ws[w] for targets that start from a value (adjoints and
    // their seeds) and 0 otherwise (a task's sum starts from zero; the first
    // flag marks a task's first entry and is not needed by the kernels).
    // Forward entries read two moments and write a rule output; reverse
    // entries read an adjoint and a moment and write an adjoint (whose
    // initial value is its seed).  A task (all rules of one output, or all
    // reverse entries of one destination) longer than the level's fair share
    // (entries / 64) is split into pieces that write zeroed partial sums; the
    // level's combine list {target, first partial, count, 0} then adds them
    // in order to the target and clears them.  Padding steps have c = 0 and
    // read the dummy slot and write nothing.  Tasks and pieces are spread over the
    // lanes by longest-processing-time assignment.
    std::vector<int> fwd_level_step, fwd_steps, fwd_level_comb, fwd_comb;
    std::vector<int> bwd_level_step, bwd_steps, bwd_level_comb, bwd_comb;
    int max_partials = 0;
    int max_level = 0;
};
bool build_plan(const Model &m, Plan &p, std::string &err);

// Linear-fit plan (sparse Jacobian of the scalar moments w.r.t. the basic
// moments, see build_lin_plan).  Work space per wave (doubles): the E/F/S
// block [0, red0), the transpose buffer, `one` (1.0), the Jacobian values
// [L0, L0 + nL), the step partials [part0, acc); priv = acc.
// Scalars per pass: their derivatives live in registers, and a tile row of
// 3 kLinChunk + 1 doubles keeps a 256-atom structure's tile (with the
// radial coefficients) within a quarter of the 160 KB LDS, one wave per SIMD.
constexpr int kLinChunk = 6;
constexpr int kLinAcc = (3 * kLinChunk + 3) & ~3;  // derivative registers, a multiple of 4
constexpr int kLinEntries = 128;   // (slot, scalar) entries per pass: two lane registers
constexpr int kLinMaskWords = 128; // slot masks of a pass, 4 per word: two lane registers
struct LinPlan {
    int dummy = 0, fpart0 = 0, red0 = 0;  // zero slot, forward partials, transpose buffer
    int nL = 0, one = 0, L0 = 0, part0 = 0, acc = 0, priv = 0;
    int CH = kLinChunk, nchunks = 0, max_chunk_entries = 0;
    bool lane_walk = false;  // maskw/clist valid (nslots <= 4 kLinMaskWords)
    std::vector<int> level_step, steps, level_comb, comb;  // L rules, as Plan's rule tables
    std::vector<int> fwd_level_step, fwd_steps, fwd_level_comb, fwd_comb;  // forward rules
    std::vector<int> chunk_s0;   // [nchunks+1] first position of each chunk in chunk_scalar
    std::vector<int> chunk_scalar;  // [S] the scalars of chunk after chunk
    std::vector<int> slot_mask;  // [nchunks][nslots] bit k: scalar k of the chunk uses the slot
    std::vector<int> slot_L;     // [nchunks][nslots][kLinChunk] L index of each bit
    std::vector<int> maskw;      // [nchunks][kLinMaskWords] slot masks, 4 per word
    std::vector<int> clist;      // [nchunks][kLinEntries] L indices in walk order
    // the L indices of every chunk's walk in walk order, chunk c at
    // [walk_off[c], walk_off[c+1]) (any plan; clist holds the same per chunk)
    std::vector<int> walk, walk_off;
};
bool build_lin_plan(const Model &m, const Plan &p, LinPlan &lp, std::string &err);

// An MTP-M head on the device, one struct in device memory that the E/F/S
// kernel's out-of-line head function reads: kind, descriptors P, distinct
// scalar moments NS, hidden sizes, activation, species and moment counts
// and the head tables.
struct DevHead {
    int kind, P, NS, h1, h2, act, Z, K;
    const int *ids;      // [NS] the distinct moments the scalars map to
    const double *proj;  // [P][NS] moment coefficients summed per distinct moment
    const double *dsp;   // [P][Z] descriptor species coefficients
    const double *c;     // [Mc] head coefficients
};

// Device view passed to the kernels by value.
struct DevModel {
    int Z, M, R, K, B, T, S, nslots;
    double rmin, rmax, scaling, mult, su, pu;
    // general radial bases (split, or another kind than RBChebyshev): per
    // ordered pair kRbStride doubles (RadialBasis); 0 and nullptr for the
    // shared RBChebyshev basis of the scalar fields above
    int rb_general;
    const double *rb_table;
    int numax[kMaxMu];
    int numax_all;
    int ndup;
    int nfwd, nbwd;  // levels
    const double *radial;   // [Z*Z*M*R]
    const double *species;  // [Z]
    const double *moment;   // [S]
    const int *map;         // [S]
    const double *seed;     // [K] sum of moment coefficients mapped to each moment
    const int *slot_basic;  // [nslots]
    const int *slot_abc;    // [nslots] a | b << 8 | c << 16
    const int *dup;         // [ndup][2]
    int max_partials;
    int K4, dummy, part0, red0, priv_doubles;  // per-wave work space (Plan)
    int tr_red1, tr_red4, tr_stage, tr_grad, tr_ctype, tr_priv;
    int efs_red, efs_stage, efs_acc;
    // MTP-M head (kHeadNone: the linear MTP of species, moment and seed),
    // the per-wave head work space (offset in doubles) and the head itself
    int head, efs_head;
    const DevHead *hd;
    int nradial, ncoef;
    int slot_base[(kMaxNu + 1) * kMaxMu];
    int fwd_nsteps, bwd_nsteps;  // steps per lane, all levels and the padding
    const int *fwd_level_step;  // [nfwd+1]
    const int2 *fwd_steps;
    const int *fwd_level_comb;  // [nfwd+1]
    const int4 *fwd_comb;
    const int *bwd_level_step;  // [nbwd+1]
    const int2 *bwd_steps;
    const int *bwd_level_comb;  // [nbwd+1]
    const int4 *bwd_comb;
};

// Neighbour lists resident on the device (SoA).
struct DevNeighbors {
    int n;                  // centres
    int64_t P;              // directed entries
    const int *offsets;     // [n+1]
    const int *idx;         // [P]
    const int *type;        // [P]
    const double *x, *y, *z, *d;  // [P]
    const int *center_type; // [n]
    const int *center;      // [n] atom of each centre row; nullptr: row i is atom i
    const int *mirror = nullptr;  // [P] the opposite entry of each entry, or nullptr
};

struct EfsOut {
    double *forces;         // [n][3] (zeroed by the caller)
    double *site_energy;    // [n]
    double *partial;        // [rows][10] per wave: energy, stress[9]
    double *pair_ders;      // [P][3] (deterministic mode) or nullptr
    double *site_virial;    // [n][9] per-atom -sum_j D_j r_j^T, or nullptr
    double *site_virial6;   // [atoms][6] LAMMPS per-atom virial (half of each entry's
                            // -D r^T to the centre, half to the neighbour), or nullptr
};

// Launch shape of the E/F/S kernel (efs_kernel.hip).
struct EfsLaunch {
    bool lds_tables;   // product-rule step tables staged in LDS
    int waves;         // waves per workgroup
    int grid;          // workgroups
    int rows;          // per-wave partial rows (grid * waves)
    size_t lds_bytes;  // dynamic LDS per workgroup
};
// Chooses the launch shape; false if one wave's work space does not fit the
// LDS a workgroup may allocate (lds_limit bytes, which one CU also holds).
// max_waves > 0 caps the waves per workgroup.
bool efs_configure(const DevModel &m, int n, int num_cus, int max_waves, size_t lds_limit,
                   EfsLaunch &cfg, int table_pref = -1);
int efs_variant(const DevModel &m, int R);
// launch_efs flags: ordered force assembly (per-entry derivatives, no
// atomics); site energies and energy only; with the ordered assembly, each
// atom's own force stored by the kernel (the gather over the mirror entries
// subtracts the reactions).
constexpr int kEfsDeterministic = 1;
constexpr int kEfsEnergyOnly = 2;
constexpr int kEfsOwnForce = 4;
hipError_t launch_efs(const DevModel &m, const DevNeighbors &nb, const EfsOut &out,
                      const EfsLaunch &cfg, int flags, hipStream_t s);
// Linear fit (lin_kernel.hip).
struct DevLin {
    int dummy, red0, nfwd;
    int nL, one, L0, part0, acc, priv, CH, nchunks, nlev;
    int lane_walk;
    int compiled_walk;  // the plan equals the compiled level-16 walk (lin_walk_compiled)
    const int *fwd_level_step, *fwd_level_comb;  // [nfwd + 1]
    const int2 *fwd_steps;
    const int4 *fwd_comb;
    const int *level_step, *level_comb;  // [nlev + 1]
    const int2 *steps;
    const int4 *comb;
    const int *chunk_s0;    // [nchunks + 1] into chunk_scalar
    const int *chunk_scalar;  // [S] the scalars of chunk after chunk
    const int *slot_mask;   // [nchunks][nslots]
    const int *slot_L;      // [nchunks][nslots][kLinChunk]
    const int *maskw;       // [nchunks][kLinMaskWords]
    const int *clist;       // [nchunks][kLinEntries]
    const int *walk;        // [nwalk] L work-space indices in walk order, chunk after chunk
    const int *walk_off;    // [nchunks + 1]
    int nwalk, max_walk;    // entries of all walks; of the longest chunk's walk
};
// One group of whole structures for the linear-fit kernels: atoms
// [a0, a1), structures [c0, c1); per site the scalar moments site
// [a1 - a0][S] and the walk-order Jacobian values lw [a1 - a0][nwalk].
struct LinGroup {
    int a0, a1, c0, c1;
    double *site;
    double *lw;
};
// One launch of the tile kernel: `count` structures of a group, every chunk
// of each (one wave per structure and chunk), force rows accumulated in LDS
// tiles of rows_cap atoms (rows_cap 0: in the rows of fc, for structures
// larger than a tile).
struct LinTile {
    const int *structs;   // [count] structures of this launch
    int count, nchunks, rows_cap;
    const int *soff;      // [nconf+1] first atom of each structure
    const double *lw;     // [atoms of the group][nwalk]
    int a0;               // first atom of the group
    int p, Z;
    double *fc, *sc;      // force [N][3][p] and stress [nconf][9][p] components
};
bool lin_configure(const DevModel &m, const DevLin &L, int n, int num_cus, size_t lds_limit,
                   EfsLaunch &cfg);
bool lin_walk_compiled(const LinPlan &lp, int nslots);
size_t lin_tile_lds(const DevModel &m, const DevLin &L, int rows);
hipError_t launch_lin_jac(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                          const LinGroup &g, const EfsLaunch &cfg, hipStream_t s);
hipError_t launch_lin_tile(const DevModel &m, const DevLin &L, const DevNeighbors &nb,
                           const LinTile &t, hipStream_t s);
// Zeroes the species columns [0, Z) of the first frows rows (the force
// rows) of comp (rows of p doubles) and the next srows rows (the stress
// rows) whole.
hipError_t launch_lin_clear(double *comp, int64_t frows, int64_t srows, int p, int Z,
                            hipStream_t s);
hipError_t launch_lin_reduce(const DevModel &m, const int *soff, const int *center_type,
                             const LinGroup &g, double *ec, hipStream_t s);
hipError_t launch_lin_rows(const double *comp, const int64_t *src, const double *sw,
                           const double *yw, int64_t R, int p, double *A, double *y, hipStream_t s);
// Gram columns padded to a multiple of 16 (p coefficients plus the target).
int gram_padded(int p);
// Whether the Gram kernel stages rows of p + 1 values (p <= 1007).
bool gram_fits(int p);
// Row ranges of the Gram for R rows, and the partial buffer they need.
int gram_blocks(int64_t R, int p, int num_cus);
size_t gram_partial_doubles(int p, int nblocks);
// [A y]^T [A y] of the R extended rows into out (pp x pp), through the
// partials; the sums run in a fixed order for a given R and nblocks.
hipError_t launch_gram(const double *comp, const int64_t *src, const double *sw, const double *yw,
                       int64_t R, int p, int nblocks, double *partial, double *out, hipStream_t s);

// Training (train_kernel.hip).
struct LossArgs {
    const int *soff;     // [nconf+1] first atom of each structure
    int nconf;
    const int *active;   // [nconf][3] energy, force, stress terms present
    const double *E, *F, *S;      // model: [nconf], [n][3], [nconf][9]
    const double *tE, *wE;        // targets and weights: [nconf]
    const double *tF, *wF;        // [n][3], [n]
    const double *tS, *wS;        // [nconf][9], [nconf]
    double *dLdE, *dLdF, *dLdS;   // adjoints: [nconf], [n][3], [nconf][9]
    double *metric_rows;          // [nconf][7]
};
struct TrainArgs {
    const int *center_structure;  // [n]
    const double *dLdE, *dLdF, *dLdS;
    double *grad_rows;            // [rows][ncoef]
};
bool grad_configure(const DevModel &m, int n, int num_cus, size_t lds_limit, EfsLaunch &cfg);
hipError_t launch_structure_reduce(const int *soff, int nconf, const double *site_energy,
                                   const double *site_virial, double *energy, double *stress,
                                   hipStream_t s);
hipError_t launch_loss(const LossArgs &a, hipStream_t s);
hipError_t launch_rows_reduce(const double *rows, int nrows, int cols, double *out, bool accumulate,
                              hipStream_t s);
hipError_t launch_grad(const DevModel &m, const DevNeighbors &nb, const TrainArgs &t,
                       const EfsLaunch &cfg, hipStream_t s);

// Site requests (mtpx_compute_sites): per-entry geometry from positions or
// given vectors (neighbors.hip), skipped entries get d = +inf and type 0.
hipError_t launch_site_prepare(int nrows, const int *offsets, const int *center_atom,
                               const int *idx, const int *atom_type, const double *pos,
                               const double *vec, double cutoffsq, int *center_type, int *type,
                               double *x, double *y, double *z, double *d, hipStream_t s);
// Ordered assembly over every atom of a site request (efs_kernel.hip): forces
// and, when site_virial6 is set, the LAMMPS per-atom virial; atom_row [ntotal]
// is the centre row of each atom or -1, rev_offsets/rev_pairs the entries
// whose neighbour is the atom, in ascending order.
hipError_t launch_site_gather(const DevNeighbors &nb, int ntotal, const int *atom_row,
                              const double *pair_ders, const int *rev_offsets,
                              const int *rev_pairs, double *forces, double *site_virial6,
                              hipStream_t s);

// Allocation-free E/F/S (mtpx_efs_noalloc): the per-wave partial rows live
// in a file-scope device array of this many doubles (efs_kernel.hip), one
// copy per GPU, shared by every call on that GPU.
constexpr size_t kNoAllocScratchDoubles = size_t(1) << 16;  // 512 KiB
// Device address of that array on the current device (hipGetSymbolAddress).
hipError_t noalloc_scratch_address(double **ptr);
// Zero-fill kernel (used where a caller may capture the launches).
hipError_t launch_fill_zero(double *p, size_t count, hipStream_t s);

// The per-wave partials reduced in order; with deterministic, the forces
// assembled from the per-entry derivatives: by the mirror entries when nb has
// them (the kernel ran with kEfsOwnForce), else by the reverse index.
hipError_t launch_efs_finish(const DevNeighbors &nb, const EfsOut &out, int rows,
                             bool deterministic, const int *rev_offsets, const int *rev_pairs,
                             double *energy_stress10, hipStream_t s);

}  // namespace mtpx
