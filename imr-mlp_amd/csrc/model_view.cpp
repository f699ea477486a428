// C ABI, model views: the MTPGpuPotentialView of the reference's GPU
// runtime (runtime/mtp/gpu-direct/mtp_gpu_direct.h:215-289) turned into the
// library's host model, with the checks of validate_potential_view
// (runtime/mtp/gpu-direct/mtp_gpu_direct.cu:419-660) and their texts, and the
// species map kept beside it.  Host code; no exceptions escape.
#include "context.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>

namespace mtpx {

namespace {

// RadialBasis (mtp_gpu_direct.h:152-161) -> the library's basis kinds; -1 for
// the kinds it does not evaluate (PolyB, PolyBCos).
int basis_kind(int k)
{
    switch (k) {
    case MTPX_RB_CHEBYSHEV: return kRBChebyshev;
    case MTPX_RB_CHEBYCOS: return kRBChebyCos;
    case MTPX_RB_CHEBYSHEV_POLY5: return kRBChebyshevPoly5;
    case MTPX_RB_CHEBYSHEV_CONFIGURABLE: return kRBChebyshevConfigurable;
    case MTPX_RB_CHEBYSHEV_POLY4: return kRBChebyshevPoly4;
    default: return -1;
    }
}

// RadialCutoff (mtp_gpu_direct.h:163-177) -> Cutoff::CutoffType order.
int cutoff_kind(int c)
{
    static const int table[12] = {kCutQuadratic,       kCutCosine,           kCutPoly5,
                                  kCutNormalizedQuadratic, kCutCosineLeft,   kCutCosineUnscaled,
                                  kCutCosineSquared,   kCutSineSquared,      kCutPoly3,
                                  kCutPoly4,           kCutSmoothstep5,      kCutSmoothstep7};
    return c >= 0 && c < 12 ? table[c] : -1;
}

// MTPGpuModel (mtp_gpu_direct.h:196-204) -> the head kinds.
int head_kind(int model)
{
    switch (model) {
    case MTPX_MODEL_LINEAR: return kHeadNone;
    case MTPX_MODEL_MTPM_QUADRATIC: return kHeadQ2;
    case MTPX_MODEL_MTPM_ASINH: return kHeadFs;
    case MTPX_MODEL_MTPM_NN1: return kHeadNn1;
    case MTPX_MODEL_MTPM_NN2: return kHeadNn2;
    case MTPX_MODEL_MTPM_LINEAR: return kHeadLi;
    default: return -1;
    }
}

struct Fail {
    int code;
    std::string msg;
};

bool bad(Fail &f, int code, const std::string &msg)
{
    f.code = code;
    f.msg = msg;
    return false;
}

bool same_basis(const RadialBasis &a, const RadialBasis &b)
{
    return a.kind == b.kind && a.rmin == b.rmin && a.rmax == b.rmax && a.scaling == b.scaling &&
           a.b == b.b && a.cut == b.cut && a.shift == b.shift && a.one_minus == b.one_minus &&
           a.cut_b == b.cut_b && a.cut_r1 == b.cut_r1 && a.cut_r2 == b.cut_r2 &&
           a.lambda == b.lambda && a.scale_lambda == b.scale_lambda;
}

// One pair descriptor (the split-basis checks of validate_potential_view,
// mtp_gpu_direct.cu:603-655) -> RadialBasis.
bool pair_basis(const mtpx_radial_basis_view &v, RadialBasis &b, Fail &f)
{
    const bool finite = std::isfinite(v.min_dist) && std::isfinite(v.max_dist) &&
                        std::isfinite(v.scaling) && std::isfinite(v.cutoff_parameter) &&
                        std::isfinite(v.transform_parameter) &&
                        std::isfinite(v.transform_scale_parameter) &&
                        std::isfinite(v.cutoff_r1) && std::isfinite(v.cutoff_r2);
    if (v.radial_basis < MTPX_RB_CHEBYSHEV || v.radial_basis > MTPX_RB_POLYBCOS ||
        v.cutoff < MTPX_CUT_QUADRATIC || v.cutoff > MTPX_CUT_SMOOTHSTEP7 ||
        v.transform < MTPX_SHIFT_LINEAR || v.transform > MTPX_SHIFT_EXPONENTIAL_TANH || !finite ||
        v.max_dist <= v.min_dist)
        return bad(f, MTPX_E_INVALID, "invalid split radial basis descriptor");
    const int kind = basis_kind(v.radial_basis);
    if (kind < 0)
        return bad(f, MTPX_E_MODEL,
                   "RBPolyB / RBPolyBCos radial bases are not supported by this library");
    const bool conf = kind == kRBChebyshevConfigurable;
    if (conf && v.cutoff == MTPX_CUT_SMOOTHSTEP7 &&
        !(v.min_dist < v.cutoff_r1 && v.cutoff_r1 <= v.cutoff_r2 && v.cutoff_r2 < v.max_dist))
        return bad(f, MTPX_E_INVALID, "invalid smoothstep7 radial interval");
    if (conf &&
        (v.transform == MTPX_SHIFT_EXPONENTIAL || v.transform == MTPX_SHIFT_EXPONENTIAL_LEFT ||
         v.transform == MTPX_SHIFT_EXPONENTIAL_TANH) &&
        v.transform_parameter != 0.0) {
        const double range = v.max_dist - v.min_dist, lambda = v.transform_parameter;
        const double den = std::expm1(lambda), rate = lambda / range;
        const double first = 2.0 * rate / den, second = -rate * first, third = -rate * second;
        if (!std::isfinite(den) || den == 0.0 || !std::isfinite(first) ||
            !std::isfinite(second) || !std::isfinite(third))
            return bad(f, MTPX_E_INVALID,
                       "invalid configurable exponential transform descriptor");
    }
    b = RadialBasis{};
    b.kind = kind;
    b.rmin = v.min_dist;
    b.rmax = v.max_dist;
    b.scaling = v.scaling;
    if (kind == kRBChebyshevPoly4 || kind == kRBChebyshevPoly5)
        b.b = v.cutoff_parameter;
    if (conf) {
        // radial_parameters -> descriptor (potentials/mtp_gpu_adapter.cpp:204-209)
        b.cut = cutoff_kind(v.cutoff);
        b.shift = v.transform;  // RadialTransform and XTransForm::ShiftType share an order
        b.one_minus = v.one_minus_chebyshev != 0;
        b.cut_b = v.cutoff_parameter;
        b.cut_r1 = v.cutoff_r1;
        b.cut_r2 = v.cutoff_r2;
        b.lambda = v.transform_parameter;
        b.scale_lambda = v.transform_scale_parameter;
    }
    return true;
}

// The head dimensions of validate_potential_view (mtp_gpu_direct.cu:476-551).
bool view_head(const mtpx_model_view &v, Head &h, Fail &f)
{
    const int kind = head_kind(v.model);
    if (kind < 0)
        return bad(f, MTPX_E_INVALID, "unsupported site-energy model in MTPGpuPotentialView");
    if (v.scalar_gather)
        return bad(f, MTPX_E_MODEL,
                   "the legacy NN scalar gather (scalar_gather) is not supported by this library");
    h = Head{};
    if (kind == kHeadNone) {
        if (!v.moment_coeffs || v.descriptor_count != 0 || v.descriptor_species_coeffs ||
            v.descriptor_moment_coeffs || v.model_coeffs || v.model_coeffs_count != 0)
            return bad(f, MTPX_E_INVALID, "invalid classic linear coefficient layout");
        return true;
    }
    if (v.descriptor_count <= 0 || !v.descriptor_species_coeffs || !v.descriptor_moment_coeffs ||
        (!v.model_coeffs && v.model_coeffs_count != 0) || v.moment_coeffs)
        return bad(f, MTPX_E_INVALID, "invalid MTP-M descriptor/model coefficient layout");
    long long expected = 0;
    const long long q = v.descriptor_count, h1 = v.model_hidden1, h2 = v.model_hidden2;
    if (kind == kHeadLi) {
        if (q != 1 || h1 != 0 || h2 != 0)
            return bad(f, MTPX_E_INVALID, "invalid linear MTP-M dimensions");
    } else if (kind == kHeadQ2 || kind == kHeadFs) {
        expected = kind == kHeadQ2 ? 5 : 1;
        if (q != 2 || h1 != 0 || h2 != 0)
            return bad(f, MTPX_E_INVALID, "invalid analytic MTP-M model dimensions");
    } else {
        if (v.model_activation < MTPX_ACT_TANH || v.model_activation > MTPX_ACT_LINEAR || h1 <= 0)
            return bad(f, MTPX_E_INVALID, "invalid neural MTP-M activation or hidden size");
        if (kind == kHeadNn1) {
            if (h2 != 0)
                return bad(f, MTPX_E_INVALID, "NN1 MTP-M must not define a second hidden layer");
            expected = q * h1 + 2 * h1;
        } else {
            if (h2 <= 0 || v.model_activation == MTPX_ACT_LINEAR)
                return bad(f, MTPX_E_INVALID,
                           "NN2 MTP-M requires two hidden layers and a supported nonlinear "
                           "activation");
            expected = q * h1 + h1 + h1 * h2 + 2 * h2;
        }
    }
    if (expected > INT_MAX || v.model_coeffs_count != expected)
        return bad(f, MTPX_E_INVALID, "MTP-M model coefficient count does not match its dimensions");
    h.kind = kind;
    h.P = (int)q;
    h.h1 = (kind == kHeadNn1 || kind == kHeadNn2) ? (int)h1 : 0;
    h.h2 = kind == kHeadNn2 ? (int)h2 : 0;
    h.act = (kind == kHeadNn1 || kind == kHeadNn2) ? v.model_activation : kActTanh;
    h.Mc = (int)expected;
    return true;
}

}  // namespace

bool model_from_view(const mtpx_model_view &v, Model &m, std::vector<int> &spmap, int &code,
                     std::string &err)
{
    Fail f{MTPX_OK, ""};
    auto fail = [&](int c, const std::string &msg) {
        code = c;
        err = msg;
        return false;
    };
    // the order of validate_potential_view's checks (mtp_gpu_direct.cu:419-660)
    if (v.species_count <= 0 || v.max_type <= 0 || !v.spmap)
        return fail(MTPX_E_INVALID, "invalid species_count/max_type/spmap in MTPGpuPotentialView");
    if (v.alpha_moments_count <= 0 || v.alpha_index_basic_count <= 0 ||
        v.alpha_index_basic_count > v.alpha_moments_count || v.alpha_scalar_moments <= 0 ||
        v.alpha_index_times_count < 0)
        return fail(MTPX_E_INVALID, "invalid MTP moment counts in MTPGpuPotentialView");
    if (v.radial_func_count <= 0 || v.rb_size <= 0)
        return fail(MTPX_E_INVALID, "invalid radial_func_count/rb_size in MTPGpuPotentialView");
    if (!(v.max_dist > 0.0))
        return fail(MTPX_E_INVALID, "invalid max_dist in MTPGpuPotentialView");
    if (!v.radial_coeffs || !v.species_coeffs)
        return fail(MTPX_E_INVALID, "missing coefficient pointer in MTPGpuPotentialView");
    Head head;
    if (!view_head(v, head, f))
        return fail(f.code, f.msg);
    const long long Z = v.species_count;
    const long long nrad = Z * Z * v.radial_func_count * v.rb_size;
    if (nrad > INT_MAX || (v.radial_coeffs_count > 0 && v.radial_coeffs_count != nrad) ||
        v.radial_coeffs_count < 0)
        return fail(MTPX_E_INVALID, "radial coefficient count does not match the MTP dimensions");
    if (!v.alpha_index_basic || !v.alpha_moment_mapping)
        return fail(MTPX_E_INVALID, "missing alpha-index pointer in MTPGpuPotentialView");
    if (v.alpha_index_times_count > 0 && !v.alpha_index_times)
        return fail(MTPX_E_INVALID,
                    "alpha_index_times_count is nonzero but alpha_index_times is null");
    for (int i = 0; i < v.max_type; ++i)
        if (v.spmap[i] < -1 || v.spmap[i] >= v.species_count)
            return fail(MTPX_E_INVALID, "species mapping is outside [-1, species_count)");
    for (int i = 0; i < v.alpha_scalar_moments; ++i)
        if (v.alpha_moment_mapping[i] < 0 || v.alpha_moment_mapping[i] >= v.alpha_moments_count)
            return fail(MTPX_E_INVALID, "alpha_moment_mapping entry is out of range");
    if (v.radial_basis < MTPX_RB_CHEBYSHEV || v.radial_basis > MTPX_RB_POLYBCOS)
        return fail(MTPX_E_INVALID, "unsupported radial basis in MTPGpuPotentialView");
    if ((v.radial_basis == MTPX_RB_CHEBYSHEV_CONFIGURABLE ||
         v.radial_basis == MTPX_RB_CHEBYSHEV_POLY4 || v.radial_basis == MTPX_RB_POLYB ||
         v.radial_basis == MTPX_RB_POLYBCOS) &&
        v.pair_radial_basis_count == 0)
        return fail(MTPX_E_INVALID, "configurable radial basis requires explicit pair descriptors");

    m = Model{};
    m.Z = (int)Z;
    m.M = v.radial_func_count;
    m.R = v.rb_size;
    m.K = v.alpha_moments_count;
    m.B = v.alpha_index_basic_count;
    m.T = v.alpha_index_times_count;
    m.S = v.alpha_scalar_moments;
    m.head = head;
    if (v.pair_radial_basis_count != 0) {
        if (!v.pair_radial_bases || v.pair_radial_basis_count != Z * Z)
            return fail(MTPX_E_INVALID, "split radial basis count does not match species_count^2");
        std::vector<RadialBasis> pairs((size_t)(Z * Z));
        for (int p = 0; p < v.pair_radial_basis_count; ++p)
            if (!pair_basis(v.pair_radial_bases[p], pairs[p], f))
                return fail(f.code, f.msg);
        // one descriptor repeated is the adapter's form of a shared basis
        // (potentials/mtp_gpu_adapter.cpp:427-434)
        bool shared = true;
        for (const RadialBasis &b : pairs)
            shared = shared && same_basis(b, pairs[0]);
        m.split = !shared;
        if (shared)
            pairs.resize(1);
        m.bases = std::move(pairs);
    } else {
        if (v.pair_radial_bases)
            return fail(MTPX_E_INVALID,
                        "pair_radial_bases is non-null but pair_radial_basis_count is zero");
        // The runtime's bare-view RBChebyshevPoly5 envelope (mtp_gpu_direct.cu:
        // 1198-1204) is not the CPU basis; native models pass pair descriptors.
        if (v.radial_basis == MTPX_RB_CHEBYSHEV_POLY5)
            return fail(MTPX_E_MODEL,
                        "a RBChebyshevPoly5 basis needs its pair descriptors (the bare-view "
                        "envelope is not the CPU basis)");
        if (!std::isfinite(v.min_dist) || !std::isfinite(v.scaling) || !(v.max_dist > v.min_dist))
            return fail(MTPX_E_INVALID, "invalid radial basis interval in MTPGpuPotentialView");
        RadialBasis b;
        b.kind = basis_kind(v.radial_basis);
        b.rmin = v.min_dist;
        b.rmax = v.max_dist;
        b.scaling = v.scaling;
        m.bases.assign(1, b);
    }
    m.rmin = m.bases[0].rmin;
    m.scaling = m.bases[0].scaling;
    m.rmax = 0;
    for (const RadialBasis &b : m.bases)
        m.rmax = std::max(m.rmax, b.rmax);
    // PotMTP::cutoff (potential_mtp.cpp:300-310): the largest max_dist
    if (v.cutoff != 0.0 && v.cutoff != m.rmax)
        return fail(MTPX_E_INVALID,
                    "cutoff differs from the largest max_dist of the radial bases");
    m.basic.assign(v.alpha_index_basic, v.alpha_index_basic + 4 * (size_t)m.B);
    if (m.T > 0)
        m.times.assign(v.alpha_index_times, v.alpha_index_times + 4 * (size_t)m.T);
    m.map.assign(v.alpha_moment_mapping, v.alpha_moment_mapping + m.S);
    // flat coefficients: [radial | species Z | moment S] for the linear MTP,
    // [radial | species Z | descriptor species q*Z | moment q*S | head] with a
    // head (the adapter's pointers, potentials/mtp_gpu_adapter.cpp:330-390)
    m.coef.assign(v.radial_coeffs, v.radial_coeffs + nrad);
    m.coef.insert(m.coef.end(), v.species_coeffs, v.species_coeffs + Z);
    if (head.kind == kHeadNone) {
        m.coef.insert(m.coef.end(), v.moment_coeffs, v.moment_coeffs + m.S);
    } else {
        m.coef.insert(m.coef.end(), v.descriptor_species_coeffs,
                      v.descriptor_species_coeffs + (size_t)head.P * Z);
        m.coef.insert(m.coef.end(), v.descriptor_moment_coeffs,
                      v.descriptor_moment_coeffs + (size_t)head.P * m.S);
        if (head.Mc > 0)
            m.coef.insert(m.coef.end(), v.model_coeffs, v.model_coeffs + head.Mc);
    }
    std::string verr;
    if (!validate_model(m, verr))
        return fail(MTPX_E_MODEL, verr);
    spmap.assign(v.spmap, v.spmap + v.max_type);
    return true;
}

}  // namespace mtpx

extern "C" {

int mtpx_format_model_view(const mtpx_model_view *view, char *buf, size_t cap, size_t *len,
                           char *err, int errlen)
{
    auto put_err = [&](const std::string &e) {
        if (err && errlen > 0) {
            std::strncpy(err, e.c_str(), (size_t)errlen - 1);
            err[errlen - 1] = 0;
        }
    };
    if (!view || !len) {
        put_err("null argument");
        return MTPX_E_INVALID;
    }
    Model m;
    std::vector<int> spmap;
    int code = MTPX_OK;
    std::string e;
    if (!model_from_view(*view, m, spmap, code, e)) {
        put_err(e);
        return code;
    }
    const std::string text = save_mtp(m);
    *len = text.size();
    if (!buf)
        return MTPX_OK;
    if (cap <= text.size()) {
        put_err("buffer too small");
        return MTPX_E_CAPACITY;
    }
    std::memcpy(buf, text.c_str(), text.size() + 1);
    return MTPX_OK;
}

}  // extern "C"
