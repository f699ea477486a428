// Model I/O and the contraction-graph launch plan (host code).
//
// parse_mtp follows the PotMTP::Load grammar (potentials/potential_mtp.cpp:
// 119-571): optional potential_name, optional scaling (default 0.01, :155),
// species_count, optional potential_tag line (metadata.cpp), one radial
// basis block or, split, one per ordered species pair (RBChebyshev,
// RBChebyCos, RBChebyshevPoly4, RBChebyshevPoly5), optional radial_coeffs (default
// 1e-5 with 1e-3 + k on the channel diagonal, :335-351), the alpha_* tables,
// optional species/moment coefficients (default 1e-3, :471-474).
#include "mtpx_internal.hpp"

#include <iterator>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <sstream>

namespace mtpx {

namespace {

// A cursor with std::istream extraction semantics over the model text.
class Cursor {
  public:
    explicit Cursor(const std::string &t) : s_(t) {}
    bool ok() const { return ok_; }
    void clear() { ok_ = true; }
    std::string line()
    {
        size_t e = s_.find('\n', p_);
        std::string l = s_.substr(p_, e == std::string::npos ? std::string::npos : e - p_);
        p_ = e == std::string::npos ? s_.size() : e + 1;
        if (!l.empty() && l.back() == '\r')
            l.pop_back();
        return l;
    }
    std::string word()
    {
        ws();
        size_t b = p_;
        while (p_ < s_.size() && !std::isspace((unsigned char)s_[p_]))
            ++p_;
        if (p_ == b)
            ok_ = false;
        return s_.substr(b, p_ - b);
    }
    void skip(int n) { p_ = std::min(s_.size(), p_ + (size_t)n); }
    void skip_past(char delim, int limit)
    {
        while (limit-- > 0 && p_ < s_.size())
            if (s_[p_++] == delim)
                return;
    }
    double real()
    {
        ws();
        const char *b = s_.c_str() + p_;
        char *e = nullptr;
        double v = std::strtod(b, &e);
        if (e == b)
            ok_ = false;
        p_ += (size_t)(e - b);
        return v;
    }
    int integer()
    {
        ws();
        const char *b = s_.c_str() + p_;
        char *e = nullptr;
        long v = std::strtol(b, &e, 10);
        if (e == b)
            ok_ = false;
        p_ += (size_t)(e - b);
        return (int)v;
    }
    char peek()
    {
        ws();
        return p_ < s_.size() ? s_[p_] : 0;
    }
    char ch()
    {
        ws();
        if (p_ >= s_.size()) {
            ok_ = false;
            return 0;
        }
        return s_[p_++];
    }

  private:
    void ws()
    {
        while (p_ < s_.size() && std::isspace((unsigned char)s_[p_]))
            ++p_;
    }
    const std::string &s_;
    size_t p_ = 0;
    bool ok_ = true;
};

bool fail(std::string &err, const char *msg)
{
    err = msg;
    return false;
}

// ---- lane-major step tables (shared by the rule plans) -------------------
// A step entry before encoding: {l, r, c, w, first}; w >= 0 is the task's
// target, w <= -2 partial -w - 2.
using Ent = std::array<int, 5>;
using Task = std::vector<Ent>;
struct RawTables {
    std::vector<Ent> steps;                 // lane-major
    std::vector<int> level_step;            // per level: first step
    std::vector<std::array<int, 3>> comb;   // {target, first partial, count}
    std::vector<int> level_comb;
    int max_partials = 0;
    RawTables() : level_step{0}, level_comb{0} {}
};

// One dependency level: tasks longer than a cap are split into pieces
// ending in partial sums, the pieces are spread over the 64 lanes by
// longest-processing-time, and the level takes as many steps as its
// longest lane.  The cap is the one, from the fair share (entries / 64, at
// least kMinPiece) up to the longest task, that gives the fewest steps and
// then the fewest partial sums: a split that does not shorten the level
// only adds combine work.
void emit_level(std::vector<Task> &tasks, RawTables &raw)
{
    size_t total = 0, longest = 0;
    for (auto &t : tasks) {
        total += t.size();
        longest = std::max(longest, t.size());
    }
    struct Layout {
        std::vector<Task> pieces;
        std::vector<std::array<int, 3>> comb;  // target, first partial, count
        int npart = 0;
        std::vector<Task> lane;
        size_t nst = 0;
    };
    auto layout = [&](size_t cap) {
        Layout L;
        for (auto &t : tasks) {
            if (t.size() <= cap) {
                L.pieces.push_back(t);
                continue;
            }
            const int target = t[0][3];
            const int first = L.npart;
            for (size_t b0 = 0; b0 < t.size(); b0 += cap) {
                Task piece(t.begin() + b0, t.begin() + std::min(t.size(), b0 + cap));
                for (Ent &e : piece)
                    e[3] = -2 - L.npart;
                piece[0][4] = 1;
                ++L.npart;
                L.pieces.push_back(std::move(piece));
            }
            L.comb.push_back({target, first, L.npart - first});
        }
        std::vector<int> order(L.pieces.size());
        for (size_t i = 0; i < order.size(); ++i)
            order[i] = (int)i;
        std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
            return L.pieces[a].size() > L.pieces[b].size();
        });
        L.lane.assign(kWave, Task());
        std::vector<size_t> load(kWave, 0);
        for (int t : order) {
            int q = (int)(std::min_element(load.begin(), load.end()) - load.begin());
            L.lane[q].insert(L.lane[q].end(), L.pieces[t].begin(), L.pieces[t].end());
            load[q] += L.pieces[t].size();
        }
        L.nst = *std::max_element(load.begin(), load.end());
        return L;
    };
    const size_t cap0 = std::max<size_t>(kMinPiece, (total + kWave - 1) / kWave);
    Layout best = layout(cap0);
    for (size_t cap = cap0 + 1; cap <= longest; ++cap) {
        Layout L = layout(cap);
        if (L.nst < best.nst || (L.nst == best.nst && L.npart < best.npart))
            best = std::move(L);
    }
    for (const auto &c : best.comb)
        raw.comb.push_back(c);
    raw.max_partials = std::max(raw.max_partials, best.npart);
    raw.level_comb.push_back((int)raw.comb.size());
    const size_t nst = best.nst;
    const size_t base = raw.steps.size() / kWave;
    raw.steps.resize((base + nst) * kWave, Ent{-1, -1, 0, -1, 1});  // padding
    for (int q = 0; q < kWave; ++q)
        for (size_t st = 0; st < best.lane[q].size(); ++st)
            raw.steps[(base + st) * kWave + q] = best.lane[q][st];
    raw.level_step.push_back((int)(base + nst));
}

// Encodes raw entries into int2 work-space steps: x = l | r << 16,
// y = w | first << 16 | last << 17 | c << 18.  map_l / map_r / map_w
// translate raw operands and targets to work-space indices; partial p goes
// to part0 + p and padding reads `dummy` and writes nothing.  kRulePad
// padding steps follow the last level.
template <class ML, class MR, class MW>
void encode_tables(const RawTables &raw, int part0, int dummy, ML map_l, MR map_r, MW map_w,
                   std::vector<int> &steps, std::vector<int> &level_step, std::vector<int> &comb,
                   std::vector<int> &level_comb)
{
    auto target = [&](int w) { return w <= -2 ? part0 + (-w - 2) : map_w(w); };
    const size_t nraw = raw.steps.size();
    steps.assign((nraw + (size_t)kRulePad * kWave) * 2, 0);
    const size_t nst = nraw / kWave;
    for (size_t i = 0; i < nraw + (size_t)kRulePad * kWave; ++i) {
        const Ent e = i < nraw ? raw.steps[i] : Ent{-1, -1, 0, -1, 1};
        int l, r, w, last = 0;
        if (e[0] < 0) {
            l = r = w = dummy;
        } else {
            l = map_l(e[0]);
            r = map_r(e[1]);
            w = target(e[3]);
            // last entry of its task or piece: the lane's next step starts
            // another one, is padding, or the level ends
            const size_t st = i / kWave, q = i % kWave;
            const bool level_end =
                std::find(raw.level_step.begin(), raw.level_step.end(), (int)(st + 1)) !=
                raw.level_step.end();
            if (st + 1 >= nst || level_end)
                last = 1;
            else {
                const Ent &nx = raw.steps[(st + 1) * kWave + q];
                last = nx[0] < 0 || nx[4] != 0;
            }
        }
        steps[2 * i] = l | (r << 16);
        steps[2 * i + 1] = w | (e[4] << 16) | (last << 17) | (int)((unsigned)e[2] << 18);
    }
    level_step = raw.level_step;
    level_comb = raw.level_comb;
    comb.clear();
    for (auto &c : raw.comb)
        comb.insert(comb.end(), {target(c[0]), part0 + c[1], c[2], 0});
}

}  // namespace

namespace {

const char *const kCutNames[] = {"quadratic",      "normalized_quadratic", "cosine",
                                 "cosine_left",    "cosine_unscaled",      "cosine_squared",
                                 "sine_squared",   "poly3",                "poly4",
                                 "poly5",          "smoothstep5",          "smoothstep7"};
const char *const kShiftNames[] = {"linear", "exponential", "exponential_left", "i2",
                                   "exponential_tanh"};

// "key = value" and its number (cutoff.cpp / xtrans.cpp read_value,
// read_double: the whole token must parse and be finite).
bool key_value(Cursor &in, const char *key, std::string &v)
{
    if (in.word() != key || in.word() != "=")
        return false;
    v = in.word();
    return in.ok();
}
bool key_double(Cursor &in, const char *key, double &x)
{
    std::string v;
    if (!key_value(in, key, v))
        return false;
    char *e = nullptr;
    x = std::strtod(v.c_str(), &e);
    return e && *e == 0 && e != v.c_str() && std::isfinite(x);
}

}  // namespace

// RBasis_ChebyshevConfigurable::LoadFromStream (basis/basis.cpp:893-911)
// after the common lines: an optional basis_function_type, then
// Cutoff::load_cutoff (cutoff.cpp:441-454) and XTransForm::load_shift
// (xtrans.cpp:360-371), with the checks of their constructors (basis.cpp
// :875-891, cutoff.cpp:187-206, xtrans.cpp FormulaShift / ExponentialShift).
static bool read_configurable(Cursor &in, RadialBasis &b, std::string &err)
{
    const std::string bad = "Error loading configurable radial basis: ";
    std::string v;
    b.one_minus = false;
    if (in.peek() == 'b') {
        if (!key_value(in, "basis_function_type", v))
            return fail(err, (bad + "expected basis_function_type = <value>").c_str());
        if (v == "one_minus_chebyshev")
            b.one_minus = true;
        else if (v != "chebyshev")
            return fail(err, ("Unknown configurable radial basis function type: " + v).c_str());
    }
    if (!key_value(in, "cutoff_type", v))
        return fail(err, (bad + "expected cutoff_type = <value>").c_str());
    b.cut = -1;
    for (int k = 0; k < 12; ++k)
        if (v == kCutNames[k])
            b.cut = k;
    if (b.cut < 0)
        return fail(err, ("Unknown configurable radial cutoff type: " + v).c_str());
    if (b.cut == kCutPoly3 || b.cut == kCutPoly4 || b.cut == kCutPoly5)
        if (!key_double(in, "cutoff_b", b.cut_b))
            return fail(err, (bad + "invalid cutoff_b").c_str());
    if (b.cut == kCutSmoothstep7)
        if (!key_double(in, "cutoff_r1", b.cut_r1) || !key_double(in, "cutoff_r2", b.cut_r2))
            return fail(err, (bad + "invalid cutoff_r1 / cutoff_r2").c_str());
    if (!key_value(in, "shift_type", v))
        return fail(err, (bad + "expected shift_type = <value>").c_str());
    b.shift = -1;
    for (int k = 0; k < 5; ++k)
        if (v == kShiftNames[k])
            b.shift = k;
    if (b.shift < 0)
        return fail(err, ("Unknown configurable radial shift type: " + v).c_str());
    const bool expo = b.shift == kShiftExponential || b.shift == kShiftExponentialLeft ||
                      b.shift == kShiftExponentialTanh;
    if (expo && !key_double(in, "shift_lambda", b.lambda))
        return fail(err, (bad + "invalid shift_lambda").c_str());
    if (b.shift == kShiftExponentialTanh && !key_double(in, "shift_scale_lambda", b.scale_lambda))
        return fail(err, (bad + "invalid shift_scale_lambda").c_str());
    if (b.cut == kCutCosineLeft && b.rmax == 0.0)
        return fail(err, "cosine_left cutoff requires nonzero max_dist");
    if (b.cut == kCutSmoothstep7 &&
        !(b.rmin < b.cut_r1 && b.cut_r1 <= b.cut_r2 && b.cut_r2 < b.rmax))
        return fail(err, "smoothstep7 cutoff requires min_dist < cutoff_r1 <= cutoff_r2 < max_dist");
    if (b.shift == kShiftExponentialLeft && b.rmax == 0.0)
        return fail(err, "exponential_left shift requires nonzero max_dist");
    if (expo && b.lambda != 0.0) {
        const double den = std::expm1(b.lambda);
        if (!std::isfinite(den) || den == 0.0)
            return fail(err, "shift_lambda produces a non-finite exponential normalization");
    }
    if (b.shift == kShiftExponentialTanh && b.scale_lambda != 0.0 && std::tanh(b.scale_lambda) == 0.0)
        return fail(err, "shift_scale_lambda produces an invalid normalization");
    return true;
}

bool parse_mtp(const std::string &text, Model &m, std::string &err)
{
    m = Model();
    Cursor in(text);
    if (in.line() != "MTP")
        return fail(err, "Can only read MTP format potentials");
    if (in.line() != "version = 1.1.0")
        return fail(err, "MTP file must have version \"1.1.0\"");
    std::string key = in.word();
    if (key == "potential_name") {
        in.skip(2);
        in.word();
        key = in.word();
    }
    m.scaling = 0.01;
    if (key == "scaling") {
        in.skip(2);
        m.scaling = in.real();
        key = in.word();
    }
    if (key != "species_count")
        return fail(err, "Error reading .mtp file, no species_count tag found");
    in.skip(2);
    m.Z = in.integer();
    if (!in.ok() || m.Z <= 0)
        return fail(err, "Error reading .mtp file, invalid species_count");
    key = in.word();
    if (key == "potential_tag") {  // :171-187
        const std::string rest = in.line();
        const size_t eq = rest.find('=');
        if (eq == std::string::npos)
            return fail(err, "Invalid potential_tag assignment");
        if (!tag_parse(rest.substr(eq + 1), m.Z, m.tag, err))
            return false;
        key = in.word();
    }
    if (key == "radial_split" || key == "radial_basis_split") {  // :190-204
        in.skip(2);
        m.split = in.integer() != 0;
        if (!m.split)
            key = in.word();
    }
    // basis_name_to_code and AnyBasis::LoadFromStream (basis/basis.cpp:10-27,
    // :73-117), with the rb_b line of Poly4 / Poly5 (:543-558, :716-731)
    auto read_basis = [&](RadialBasis &b, int &size, const std::string &first) {
        if (first != "radial_basis_type")
            return fail(err, m.split ? "Error reading .mtp file, incorrect pair setting"
                                     : "Error reading .mtp file");
        in.skip(2);
        const std::string name = in.word();
        if (name == "RBChebyshev")
            b.kind = kRBChebyshev;
        else if (name == "RBChebyCos")
            b.kind = kRBChebyCos;
        else if (name == "RBChebyshevPoly4")
            b.kind = kRBChebyshevPoly4;
        else if (name == "RBChebyshevPoly5")
            b.kind = kRBChebyshevPoly5;
        else if (name == "RBChebyshevConfigurable")
            b.kind = kRBChebyshevConfigurable;
        else
            return fail(err, ("unsupported radial basis type: " + name).c_str());
        b.scaling = m.scaling;
        if (in.word() != "min_dist")
            return fail(err, "Error in loading basis: min_dist");
        in.skip(2);
        b.rmin = in.real();
        if (in.word() != "max_dist")
            return fail(err, "Error in loading basis: max_dist");
        in.skip(2);
        b.rmax = in.real();
        if (in.word() != "radial_basis_size")
            return fail(err, "Error in loading basis: radial_basis_size");
        in.skip(2);
        size = in.integer();
        if (!in.ok() || size <= 0)
            return fail(err, "Error in loading basis: radial_basis_size must be positive");
        if (b.kind == kRBChebyshevPoly4 || b.kind == kRBChebyshevPoly5) {
            if (in.word() != "rb_b")
                return fail(err, "Error in loading basis: rb_b");
            in.skip(2);
            b.b = in.real();
            if (!in.ok())
                return fail(err, "Error in loading basis: rb_b");
        }
        if (!std::isfinite(b.rmin) || !std::isfinite(b.rmax) || !(b.rmin < b.rmax))
            return fail(err, "Error in loading basis: min_dist < max_dist is required");
        if (b.kind == kRBChebyshevConfigurable)
            return read_configurable(in, b, err);
        return true;
    };
    if (m.split) {  // :206-265, one basis per ordered species pair
        m.bases.assign((size_t)m.Z * m.Z, RadialBasis());
        std::vector<char> seen((size_t)m.Z * m.Z, 0);
        int last = 0;
        for (int q = 0; q < m.Z * m.Z; ++q) {
            if (in.word() != "pair")
                return fail(err, "Error reading .mtp file, incorrect pair setting");
            const int ci = in.integer(), cj = in.integer();
            if (!in.ok() || ci < 0 || ci >= m.Z || cj < 0 || cj >= m.Z)
                return fail(err, "Error reading .mtp file, invalid radial basis pair");
            if (seen[ci * m.Z + cj]++)
                return fail(err, "Error reading .mtp file, duplicate radial basis pair");
            int size = 0;
            if (!read_basis(m.bases[ci * m.Z + cj], size, in.word()))
                return false;
            if (last && size != last)
                return fail(err, "Error reading .mtp file, split radial bases must have the same "
                                 "radial_basis_size");
            last = size;
        }
        m.R = last;
    } else {
        m.bases.assign(1, RadialBasis());
        if (!read_basis(m.bases[0], m.R, key))
            return false;
    }
    m.rmin = m.bases[0].rmin;
    m.rmax = 0;
    for (const RadialBasis &b : m.bases)
        m.rmax = std::max(m.rmax, b.rmax);
    if (in.word() != "radial_funcs_count")
        return fail(err, "Error reading .mtp file");
    in.skip(2);
    m.M = in.integer();
    if (!in.ok() || m.M < 0)
        return fail(err, "Error reading .mtp file, invalid radial basis dimensions");

    const int Z = m.Z, M = m.M, R = m.R;
    std::vector<double> radial((size_t)Z * Z * M * R, 0.0);
    key = in.word();
    if (key == "radial_coeffs") {
        for (int p = 0; p < Z * Z; ++p) {
            int a = in.integer();
            in.ch();
            int b = in.integer();
            if (!in.ok() || a < 0 || a >= Z || b < 0 || b >= Z)
                return fail(err, "Error reading .mtp file, invalid radial coefficient pair");
            for (int mu = 0; mu < M; ++mu) {
                in.ch();
                for (int k = 0; k < R; ++k) {
                    double v = in.real();
                    in.ch();
                    if (!in.ok())
                        return fail(err, "Error reading .mtp file, missing radial coefficient");
                    radial[((size_t)(a * Z + b) * M + mu) * R + k] = v;
                }
            }
        }
        key = in.word();
    } else {
        for (int p = 0; p < Z * Z; ++p)
            for (int mu = 0; mu < M; ++mu) {
                for (int k = 0; k < R; ++k)
                    radial[((size_t)p * M + mu) * R + k] = 1e-5;
                radial[((size_t)p * M + mu) * R + std::min(mu, R - 1)] = 1e-3 + mu;
            }
    }
    if (key != "alpha_moments_count")
        return fail(err, "Error reading .mtp file, except: alpha_moments_count");
    in.skip(2);
    m.K = in.integer();
    if (in.word() != "alpha_index_basic_count")
        return fail(err, "Error reading .mtp file");
    in.skip(2);
    m.B = in.integer();
    if (!in.ok() || in.word() != "alpha_index_basic" || m.B < 0)
        return fail(err, "Error reading .mtp file");
    in.skip(4);
    m.basic.resize((size_t)m.B * 4);
    int mu_max = -1;
    for (int i = 0; i < m.B; ++i) {
        in.skip_past('{', 1000);
        for (int q = 0; q < 4; ++q) {
            m.basic[4 * i + q] = in.integer();
            if (q < 3)
                in.ch();
        }
        if (!in.ok())
            return fail(err, "Error reading .mtp file");
        mu_max = std::max(mu_max, m.basic[4 * i]);
    }
    if (mu_max != M - 1)
        return fail(err, "Wrong number of radial functions specified");
    in.skip_past('\n', 1000);
    if (in.word() != "alpha_index_times_count")
        return fail(err, "Error reading .mtp file");
    in.skip(2);
    m.T = in.integer();
    if (!in.ok() || in.word() != "alpha_index_times" || m.T < 0)
        return fail(err, "Error reading .mtp file");
    in.skip(4);
    m.times.resize((size_t)m.T * 4);
    for (int i = 0; i < m.T; ++i) {
        in.skip_past('{', 1000);
        for (int q = 0; q < 4; ++q) {
            m.times[4 * i + q] = in.integer();
            if (q < 3)
                in.ch();
        }
        if (!in.ok())
            return fail(err, "Error reading .mtp file");
    }
    in.skip_past('\n', 1000);
    if (in.word() != "alpha_scalar_moments")
        return fail(err, "Error reading .mtp file");
    in.skip(2);
    m.S = in.integer();
    if (!in.ok() || in.word() != "alpha_moment_mapping" || m.S < 0)
        return fail(err, "Error reading .mtp file");
    in.skip(4);
    m.map.resize((size_t)m.S);
    for (int i = 0; i < m.S; ++i) {
        m.map[i] = in.integer();
        in.ch();
        if (!in.ok())
            return fail(err, "Error reading .mtp file");
    }
    in.skip_past('\n', 1000);

    // the MTP-M head, if the potential declares one (its coefficient layout,
    // PotMTP_M::Load, potentials/potential_mtp_m.h:2054-2063)
    if (!head_parse(text, m.tag, m.head, err))
        return false;
    const int nsp = m.nspecies(), nmom = m.nmoment();
    m.coef.assign((size_t)m.ncoef(), 1e-3);
    std::copy(radial.begin(), radial.end(), m.coef.begin());
    double *lin = m.coef.data() + m.nradial();
    key = in.word();
    in.clear();
    if (key == "species_coeffs") {
        in.skip(4);
        for (int i = 0; i < nsp; ++i) {
            lin[i] = in.real();
            in.ch();
            if (!in.ok())
                return fail(err, "Error reading .mtp file, missing species coefficient");
        }
        in.skip_past('\n', 1000);
        key = in.word();
        in.clear();
    }
    if (key == "moment_coeffs") {
        in.skip(2);
        in.skip_past('{', 10);
        for (int i = 0; i < nmom; ++i) {
            lin[nsp + i] = in.real();
            in.ch();
            if (!in.ok())
                return fail(err, "Error reading .mtp file, missing moment coefficient");
        }
        in.skip_past('\n', 1000);
        key = in.word();
        in.clear();
    }
    if (!m.linear() && key == "model_coeffs") {  // :2112-2124
        in.skip(2);
        in.skip_past('{', 10);
        for (int i = 0; i < m.head.Mc; ++i) {
            lin[nsp + nmom + i] = in.real();
            in.ch();
            if (!in.ok())
                return fail(err, "Error reading .mtp file, missing model coefficient");
        }
    }
    return validate_model(m, err);
}

// The "key = value" lines of AnyBasis::SaveToStream (basis/basis.h:50-56,
// the rb_b line of Poly4 / Poly5, basis.cpp:560-564, and the configurable
// basis's basis.cpp:913-919) with numbers as a stream set to 17 significant
// digits writes them (printf "%.17g"), in their order.
std::vector<std::pair<std::string, std::string>> basis_settings(const RadialBasis &b, int R)
{
    static const char *kind_names[] = {"RBChebyshev", "RBChebyCos", "RBChebyshevPoly4",
                                       "RBChebyshevPoly5", "RBChebyshevConfigurable"};
    auto g = [](double v) {
        char buf[64];
        std::snprintf(buf, sizeof buf, "%.17g", v);
        return std::string(buf);
    };
    std::vector<std::pair<std::string, std::string>> o = {{"radial_basis_type", kind_names[b.kind]},
                                                          {"min_dist", g(b.rmin)},
                                                          {"max_dist", g(b.rmax)},
                                                          {"radial_basis_size", std::to_string(R)}};
    if (b.kind == kRBChebyshevPoly4 || b.kind == kRBChebyshevPoly5)
        o.push_back({"rb_b", g(b.b)});
    if (b.kind == kRBChebyshevConfigurable) {
        o.push_back({"basis_function_type", b.one_minus ? "one_minus_chebyshev" : "chebyshev"});
        o.push_back({"cutoff_type", kCutNames[b.cut]});
        if (b.cut == kCutPoly3 || b.cut == kCutPoly4 || b.cut == kCutPoly5)
            o.push_back({"cutoff_b", g(b.cut_b)});
        if (b.cut == kCutSmoothstep7) {
            o.push_back({"cutoff_r1", g(b.cut_r1)});
            o.push_back({"cutoff_r2", g(b.cut_r2)});
        }
        o.push_back({"shift_type", kShiftNames[b.shift]});
        if (b.shift == kShiftExponential || b.shift == kShiftExponentialLeft ||
            b.shift == kShiftExponentialTanh)
            o.push_back({"shift_lambda", g(b.lambda)});
        if (b.shift == kShiftExponentialTanh)
            o.push_back({"shift_scale_lambda", g(b.scale_lambda)});
    }
    return o;
}

// PotMTP::Save (potentials/potential_mtp.cpp:1052-1061): write_header
// (:656-671), write_radial_info (:673-690; AnyBasis::SaveToStream,
// basis/basis.h:50-56, and the rb_b line of Poly4 / Poly5, basis.cpp:560-564,
// :733-737), write_radial_coeff (:692-714), write_rules (:716-752) and
// write_linear_coeff (:754-785), on a stream in std::scientific notation
// with max_digits10 (17) digits: printf "%.17e" for every double.
std::string save_mtp(const Model &m)
{
    std::string o;
    char buf[64];
    auto num = [&](double v) {
        std::snprintf(buf, sizeof buf, "%.17e", v);
        o += buf;
    };
    auto integer = [&](long v) { o += std::to_string(v); };
    static const char *kind_names[] = {"RBChebyshev", "RBChebyCos", "RBChebyshevPoly4",
                                       "RBChebyshevPoly5", "RBChebyshevConfigurable"};
    o += "MTP\nversion = 1.1.0\npotential_name = MTP1m\nscaling = ";
    num(m.bases.empty() ? m.scaling : m.bases[0].scaling);
    o += "\nspecies_count = ";
    integer(m.Z);
    o += "\npotential_tag = " + tag_output(m.tag, m.head) + "\n";
    if (m.split)
        o += "radial_basis_split = 1\n";
    for (size_t q = 0; q < m.bases.size(); ++q) {
        const RadialBasis &b = m.bases[q];
        if (m.split) {
            o += "pair ";
            integer((long)q / m.Z);
            o += ' ';
            integer((long)q % m.Z);
            o += '\n';
        }
        o += "radial_basis_type = ";
        o += kind_names[b.kind];
        o += "\n\tmin_dist = ";
        num(b.rmin);
        o += "\n\tmax_dist = ";
        num(b.rmax);
        o += "\n\tradial_basis_size = ";
        integer(m.R);
        o += '\n';
        if (b.kind == kRBChebyshevPoly4 || b.kind == kRBChebyshevPoly5) {
            o += "\trb_b = ";
            num(b.b);
            o += '\n';
        }
        if (b.kind == kRBChebyshevConfigurable) {  // basis.cpp:913-919
            o += b.one_minus ? "\tbasis_function_type = one_minus_chebyshev\n"
                             : "\tbasis_function_type = chebyshev\n";
            o += std::string("\tcutoff_type = ") + kCutNames[b.cut] + "\n";
            auto line = [&](const char *key, double v) {
                o += std::string("\t") + key + " = ";
                num(v);
                o += '\n';
            };
            if (b.cut == kCutPoly3 || b.cut == kCutPoly4 || b.cut == kCutPoly5)
                line("cutoff_b", b.cut_b);
            if (b.cut == kCutSmoothstep7) {
                line("cutoff_r1", b.cut_r1);
                line("cutoff_r2", b.cut_r2);
            }
            o += std::string("\tshift_type = ") + kShiftNames[b.shift] + "\n";
            if (b.shift == kShiftExponential || b.shift == kShiftExponentialLeft ||
                b.shift == kShiftExponentialTanh)
                line("shift_lambda", b.lambda);
            if (b.shift == kShiftExponentialTanh)
                line("shift_scale_lambda", b.scale_lambda);
        }
    }
    o += "radial_funcs_count = ";
    integer(m.M);
    o += "\nradial_coeffs\n";
    size_t q = 0;
    for (int i = 0; i < m.Z; ++i)
        for (int j = 0; j < m.Z; ++j) {
            o += '\t';
            integer(i);
            o += '-';
            integer(j);
            o += '\n';
            for (int k = 0; k < m.M; ++k) {
                o += "\t\t{";
                for (int l = 0; l < m.R; ++l) {
                    num(m.coef[q++]);
                    o += l != m.R - 1 ? ", " : "}\n";
                }
            }
        }
    o += "alpha_moments_count = ";
    integer(m.K);
    o += "\nalpha_index_basic_count = ";
    integer(m.B);
    o += "\nalpha_index_basic = {";
    auto quad = [&](const int *v, bool last) {
        o += '{';
        for (int k = 0; k < 4; ++k) {
            integer(v[k]);
            if (k < 3)
                o += ", ";
        }
        o += last ? "}" : "}, ";
    };
    for (int i = 0; i < m.B; ++i)
        quad(&m.basic[4 * i], i == m.B - 1);
    o += "}\nalpha_index_times_count = ";
    integer(m.T);
    o += "\nalpha_index_times = {";
    for (int i = 0; i < m.T; ++i)
        quad(&m.times[4 * i], i == m.T - 1);
    o += "}\nalpha_scalar_moments = ";
    integer(m.S);
    o += "\nalpha_moment_mapping = {";
    for (int i = 0; i < m.S; ++i) {
        if (i)
            o += ", ";
        integer(m.map[i]);
    }
    auto list = [&](const char *name, int first, int count) {
        o += name;
        o += " = {";
        for (int i = 0; i < count; ++i) {
            if (i)
                o += ", ";
            num(m.coef[first + i]);
        }
        o += "}\n";
    };
    o += "}\n";
    const int sp = m.nradial(), mo = sp + m.nspecies(), hc = mo + m.nmoment();
    list("species_coeffs", sp, m.nspecies());
    list("moment_coeffs", mo, m.nmoment());
    if (!m.linear()) {
        // PotMTP_M::Save (potentials/potential_mtp_m.h:2256-2336): the head's
        // coefficients and the "# mtp_*" lines of a short-range potential
        static const char *heads[] = {"linear", "mtp_m_li", "mtp_m_q2", "mtp_m_fs", "mtp_m_n1",
                                      "mtp_m_n2"};
        static const char *acts[] = {"TANH", "RELU", "SIGMOID", "LINEAR"};
        list("model_coeffs", hc, m.head.Mc);
        o += std::string("# mtp_model = ") + heads[m.head.kind] + "\n";
        o += "# mtp_descriptor_count = " + std::to_string(m.head.P) + "\n";
        o += "# mtp_model_coeffs_count = " + std::to_string(m.head.Mc) + "\n";
        if (m.head.kind == kHeadNn1 || m.head.kind == kHeadNn2) {
            o += std::string("# mtp_activation = ") + acts[m.head.act] + "\n";
            o += "# mtp_hidden1 = " + std::to_string(m.head.h1) + "\n";
            o += "# mtp_hidden2 = " + std::to_string(m.head.h2) + "\n";
        }
    }
    return o;
}

bool validate_model(const Model &m, std::string &err)
{
    if (m.Z <= 0 || m.M < 1 || m.R <= 0 || m.B < 1 || m.K < m.B || m.T < 0 || m.S < 0)
        return fail(err, "invalid model sizes");
    if (m.M > kMaxMu)
        return fail(err, "radial_funcs_count exceeds the supported maximum (8)");
    if (m.R > kMaxR)
        return fail(err, "radial_basis_size exceeds the supported maximum (16)");
    if (m.K > 65535)
        return fail(err, "alpha_moments_count exceeds the supported maximum (65535)");
    if (m.bases.size() != (m.split ? (size_t)m.Z * m.Z : 1))
        return fail(err, "radial basis table does not match species_count");
    for (const RadialBasis &b : m.bases)
        if (!(b.rmax > b.rmin) || !std::isfinite(b.rmin) || !std::isfinite(b.rmax) ||
            !std::isfinite(b.scaling) || !std::isfinite(b.b) || b.kind < kRBChebyshev ||
            b.kind > kRBChebyshevConfigurable || b.cut < kCutQuadratic ||
            b.cut > kCutSmoothstep7 || b.shift < kShiftLinear || b.shift > kShiftExponentialTanh ||
            !std::isfinite(b.cut_b) || !std::isfinite(b.cut_r1) || !std::isfinite(b.cut_r2) ||
            !std::isfinite(b.lambda) || !std::isfinite(b.scale_lambda))
            return fail(err, "invalid radial basis");
    if (!(m.rmax > m.rmin) || !std::isfinite(m.rmin) || !std::isfinite(m.rmax))
        return fail(err, "invalid radial basis interval");
    const Head &h = m.head;
    if (h.kind < kHeadNone || h.kind > kHeadNn2 || h.act < kActTanh || h.act > kActLinear ||
        h.P < 1 || h.h1 < 0 || h.h2 < 0 || h.Mc < 0 || (h.kind == kHeadNone && (h.P != 1 || h.Mc)))
        return fail(err, "invalid MTP-M head");
    if ((long long)h.P * std::max(m.S, m.Z) > (1 << 24) || h.h1 > (1 << 16) || h.h2 > (1 << 16))
        return fail(err, "MTP-M head exceeds the supported size");
    if ((int)m.basic.size() != 4 * m.B || (int)m.times.size() != 4 * m.T ||
        (int)m.map.size() != m.S || (int)m.coef.size() != m.ncoef())
        return fail(err, "inconsistent model array sizes");
    for (int i = 0; i < m.B; ++i) {
        const int *b = &m.basic[4 * i];
        if (b[0] < 0 || b[0] >= m.M || b[1] < 0 || b[2] < 0 || b[3] < 0)
            return fail(err, "basic moment index out of range");
        if (b[1] + b[2] + b[3] > kMaxNu)
            return fail(err, "basic moment degree exceeds the supported maximum (8)");
    }
    for (int t = 0; t < m.T; ++t) {
        const int *r = &m.times[4 * t];
        if (r[0] < 0 || r[0] >= m.K || r[1] < 0 || r[1] >= m.K || r[3] < 0 || r[3] >= m.K)
            return fail(err, "product rule index out of range");
        if (r[3] < m.B)
            return fail(err, "a product rule writes a basic moment");
    }
    for (int s = 0; s < m.S; ++s)
        if (m.map[s] < 0 || m.map[s] >= m.K)
            return fail(err, "scalar moment mapping out of range");
    return true;
}

namespace {

// Forward rule tasks: outputs of each level, an output's rules in file
// order.
void forward_tables(const Model &m, const std::vector<int> &level, int maxl, RawTables &fwd)
{
    std::vector<std::vector<int>> by_out((size_t)m.K);
    for (int t = 0; t < m.T; ++t)
        by_out[m.times[4 * t + 3]].push_back(t);
    for (int L = 1; L <= maxl; ++L) {
        std::vector<Task> tasks;
        for (int o = 0; o < m.K; ++o) {
            if (level[o] != L || by_out[o].empty())
                continue;
            Task task;
            for (int t : by_out[o]) {
                const int *r = &m.times[4 * t];
                task.push_back({r[0], r[1], r[2], o, 0});
            }
            task[0][4] = 1;
            tasks.push_back(std::move(task));
        }
        emit_level(tasks, fwd);
    }
}

}  // namespace

// Canonical slot order shared with the kernels: for nu ascending, for mu
// ascending (mu with numax[mu] >= nu), for alpha in the shell of degree nu
// enumerated a = nu..0, b = nu-a..0, c = nu-a-b.
bool build_plan(const Model &m, Plan &p, std::string &err)
{
    p = Plan();
    for (int mu = 0; mu < kMaxMu; ++mu)
        p.numax[mu] = -1;
    for (int i = 0; i < m.B; ++i) {
        const int *b = &m.basic[4 * i];
        p.numax[b[0]] = std::max(p.numax[b[0]], b[1] + b[2] + b[3]);
    }
    for (int mu = 0; mu < m.M; ++mu)
        p.numax_all = std::max(p.numax_all, p.numax[mu]);
    // (mu, a, b, c) -> first basic index
    const int dim = kMaxNu + 1;
    std::vector<int> first((size_t)kMaxMu * dim * dim * dim, -1);
    auto key = [&](int mu, int a, int b, int c) { return ((mu * dim + a) * dim + b) * dim + c; };
    for (int i = 0; i < m.B; ++i) {
        const int *b = &m.basic[4 * i];
        int &f = first[key(b[0], b[1], b[2], b[3])];
        if (f < 0)
            f = i;
        else {
            p.dup.push_back(i);
            p.dup.push_back(f);
        }
    }
    for (int nu = 0; nu <= p.numax_all; ++nu)
        for (int mu = 0; mu < m.M; ++mu) {
            if (p.numax[mu] < nu)
                continue;
            for (int a = nu; a >= 0; --a)
                for (int b = nu - a; b >= 0; --b) {
                    p.slot_basic.push_back(first[key(mu, a, b, nu - a - b)]);
                    p.slot_abc.push_back(a | (b << 8) | ((nu - a - b) << 16));
                }
        }
    p.nslots = (int)p.slot_basic.size();
    for (int k = 0; k < (kMaxNu + 1) * kMaxMu; ++k)
        p.slot_base[k] = -1;
    {
        int s = 0;
        for (int nu = 0; nu <= p.numax_all; ++nu)
            for (int mu = 0; mu < m.M; ++mu)
                if (p.numax[mu] >= nu) {
                    p.slot_base[nu * kMaxMu + mu] = s;
                    s += (nu + 1) * (nu + 2) / 2;
                }
    }

    // Dependency levels.  The reference applies the rules in file order
    // (potential_mtp.cpp:2918-2924), so every operand must be complete before
    // a rule reads it; a file that violates this is rejected.
    std::vector<int> last_write((size_t)m.K, -1);
    for (int t = 0; t < m.T; ++t)
        last_write[m.times[4 * t + 3]] = t;
    std::vector<int> level((size_t)m.K, 0);
    for (int t = 0; t < m.T; ++t) {
        const int *r = &m.times[4 * t];
        if (last_write[r[0]] >= t || last_write[r[1]] >= t)
            return fail(err, "product rules are not in dependency order");
        level[r[3]] = std::max(level[r[3]], 1 + std::max(level[r[0]], level[r[1]]));
    }
    int maxl = 0;
    for (int x = 0; x < m.K; ++x)
        maxl = std::max(maxl, level[x]);
    p.max_level = maxl;

    // Private LDS layout of one wave (in doubles): moments, adjoints, a zero
    // slot that padding steps read and write, then the partial sums.
    const int K4 = (m.K + 3) & ~3;
    p.K4 = K4;
    p.dummy = 2 * K4;
    p.part0 = 2 * K4 + 4;

    RawTables fwd, bwd;
    forward_tables(m, level, maxl, fwd);

    // Reverse: destinations of each level from the top down; a destination's
    // entries in reverse file order, the right operand's entry of a rule
    // first (backpropagate_moments, potential_mtp.cpp:3292-3305).  Entry
    // {o, other, c}: A_x += c A_o m_other.
    std::vector<Task> ent((size_t)m.K);
    for (int t = m.T - 1; t >= 0; --t) {
        const int *r = &m.times[4 * t];
        ent[r[1]].push_back({r[3], r[0], r[2], r[1], 0});
        ent[r[0]].push_back({r[3], r[1], r[2], r[0], 0});
    }
    for (int L = maxl - 1; L >= 0; --L) {
        std::vector<Task> tasks;
        for (int x = 0; x < m.K; ++x) {
            if (level[x] != L || ent[x].empty())
                continue;
            Task task = ent[x];
            task[0][4] = 1;
            tasks.push_back(std::move(task));
        }
        emit_level(tasks, bwd);
    }

    // Encode against the private layout (indices in doubles).
    p.max_partials = std::max(fwd.max_partials, bwd.max_partials);
    const int P4 = (p.max_partials + 3) & ~3;
    p.red0 = p.part0 + P4;
    const int N4 = (p.nslots + 3) & ~3;
    // The moment reduction's transpose buffer lies over the adjoint block
    // (unused until the seeds are written; the zero slot and the partial sums
    // under it are cleared again after the neighbour pass) and the force
    // pass's slot-ordered adjoints over the moments (not read after the
    // reverse rules), where they fit; then the wave's energy/virial sums.
    const int RB = kChunk * kRedStride;
    int end;
    if (N4 <= p.K4) {
        p.efs_red = p.K4;
        p.efs_stage = 0;
        end = std::max(p.red0, p.K4 + RB);
    } else {
        p.efs_red = p.efs_stage = p.red0;
        end = p.red0 + std::max(RB, N4);
    }
    p.efs_acc = (end + 3) & ~3;
    p.priv_doubles = p.efs_acc + 12;  // energy, virial[9], padding
    if (!m.linear()) {
        // The head's work space lives from the end of the forward rules to
        // the seeds.  Over that span the moment transpose buffer past the
        // partial sums (and the slot-ordered adjoints, written only after
        // the seeds) are dead: the head goes there where it fits, so the
        // launch keeps its waves and its LDS step tables.
        const long long hd = 2LL * m.head.P + 2LL * m.head.h1 + m.head.h2;
        if (hd > 0xffff)
            return fail(err, "MTP-M head too large: its work space exceeds 65535 doubles");
        if (hd <= p.efs_acc - p.red0) {
            p.efs_head = p.red0;
        } else {
            p.efs_head = p.priv_doubles;
            p.priv_doubles += (int)((hd + 3) & ~3LL);
        }
    }
    if (p.priv_doubles > 0xffff)
        return fail(err, "model too large: per-atom work space exceeds 65535 doubles");
    for (int t = 0; t < m.T; ++t)
        if (m.times[4 * t + 2] < -8192 || m.times[4 * t + 2] > 8191)
            return fail(err, "product-rule multiplicity outside [-8192, 8191]");
    auto same = [](int x) { return x; };
    auto adj = [&p](int x) { return p.K4 + x; };
    encode_tables(fwd, p.part0, p.dummy, same, same, same, p.fwd_steps, p.fwd_level_step,
                  p.fwd_comb, p.fwd_level_comb);
    encode_tables(bwd, p.part0, p.dummy, adj, same, adj, p.bwd_steps, p.bwd_level_step,
                  p.bwd_comb, p.bwd_level_comb);

    // Training work space: the E/F/S work space without its transpose
    // buffer with its dual copy (tangents and second adjoints) interleaved,
    // element x's value and dual in doubles 2x and 2x + 1, then the wave's
    // radial gradient accumulator and the species of the neighbours in
    // flight.  Three more buffers lie over blocks that are dead in the phase
    // that uses them, where they fit: the first neighbour pass's transpose
    // buffer over the adjoint pairs (written with the seeds later), the
    // slot-ordered {A, G} stage over the moment pairs (dead after the reverse
    // rules) and the last pass's transpose buffer over the adjoint pairs
    // (dead after the staging).  Otherwise they get room of their own after
    // the gradient accumulator.
    p.tr_grad = 2 * p.red0;
    p.tr_ctype = p.tr_grad + ((m.nradial() + 3) & ~3);
    end = p.tr_ctype + kWave / 2;  // 64 ints: neighbour species of a batch
    int own_red = -1;
    auto red_region = [&] {
        if (own_red < 0) {
            own_red = end;
            end += RB;
        }
        return own_red;
    };
    const bool over_adjoints = 2 * (p.red0 - K4) >= RB;
    p.tr_red1 = over_adjoints ? 2 * K4 : red_region();
    p.tr_red4 = over_adjoints ? 2 * K4 : red_region();
    if (N4 <= K4) {
        p.tr_stage = 0;
    } else {
        p.tr_stage = end;
        end += 2 * N4;
    }
    p.tr_priv = end;
    return true;
}

namespace {

// Groups the scalar moments into the linear-fit walks' chunks: at most W
// scalars and at most E (slot, scalar) entries each (a scalar with more
// entries is a chunk of its own).  A chunk's walk forms grad(f Y) once per
// slot that any of its scalars uses and the monomial shells up to the
// highest degree among them, so scalars that share slots belong together.
// The grouping minimises an instruction estimate of one walk,
//   7 per slot formed + 6 per (slot, scalar) entry + 2 per monomial of the
//   shells formed + 12 per scalar + 420 per chunk (radial functions,
//   centre-row reduction, stress and row updates),
// by simulated annealing (moves and swaps of scalars between chunks,
// geometric cooling, a fixed-seed generator) from the chunks of
// consecutive scalars.  Deterministic: the same moment structure gives the
// same chunks on every host.  Returns the chunks, each in ascending
// scalar order, costliest first.
std::vector<std::vector<int>> group_scalars(const std::vector<std::vector<int>> &slots,
                                            const std::vector<int> &slot_nu, int W, int E)
{
    const int S = (int)slots.size();
    const int nslots = (int)slot_nu.size(), words = (nslots + 63) / 64;
    std::vector<uint64_t> bits((size_t)S * words, 0);
    std::vector<int> nnz((size_t)S), top((size_t)S, 0);
    for (int s = 0; s < S; ++s) {
        for (int sl : slots[s]) {
            bits[(size_t)s * words + sl / 64] |= uint64_t(1) << (sl % 64);
            top[s] = std::max(top[s], slot_nu[sl]);
        }
        nnz[s] = (int)slots[s].size();
    }
    auto shell_cost = [](int nu) {
        int c = 0;
        for (int n = 1; n <= nu; ++n)
            c += (n + 1) * (n + 2) / 2;
        return c;
    };
    std::vector<uint64_t> u((size_t)words);
    auto cost = [&](const std::vector<int> &g) -> long {
        if (g.empty())
            return 0;
        std::fill(u.begin(), u.end(), 0);
        long ent = 0;
        int nu = 0;
        for (int s : g) {
            for (int w = 0; w < words; ++w)
                u[w] |= bits[(size_t)s * words + w];
            ent += nnz[s];
            nu = std::max(nu, top[s]);
        }
        long used = 0;
        for (uint64_t x : u)
            used += __builtin_popcountll(x);
        return 7 * used + 6 * ent + 2 * shell_cost(nu) + 12 * (long)g.size() + 420;
    };
    auto fits = [&](const std::vector<int> &g) {
        if ((int)g.size() > W)
            return false;
        long ent = 0;
        for (int s : g)
            ent += nnz[s];
        return ent <= E || g.size() == 1;
    };
    // start: consecutive scalars, then three empty chunks to move into
    std::vector<std::vector<int>> gs;
    for (int s = 0; s < S; ++s) {
        if (gs.empty() || !fits([&] {
                auto t = gs.back();
                t.push_back(s);
                return t;
            }()))
            gs.emplace_back();
        gs.back().push_back(s);
    }
    for (int k = 0; k < 3; ++k)
        gs.emplace_back();
    std::vector<long> c((size_t)gs.size());
    for (size_t k = 0; k < gs.size(); ++k)
        c[k] = cost(gs[k]);
    uint64_t state = 0x2545F4914F6CDD1DULL;
    auto next = [&](uint64_t n) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        return (state >> 33) % n;
    };
    auto uniform = [&] {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        return (double)(state >> 11) * 0x1.0p-53;
    };
    const int G = (int)gs.size();
    double T = 200.0;
    const int iters = S > 1 ? 200000 : 0;
    std::vector<int> na, nb;
    for (int it = 0; it < iters; ++it, T = std::max(1.0, T * 0.99997)) {
        const int a = (int)next(G), b = (int)next(G);
        if (a == b || gs[a].empty())
            continue;
        const int i = (int)next(gs[a].size());
        na = gs[a];
        na.erase(na.begin() + i);
        nb = gs[b];
        if (next(2) == 0 || gs[b].empty()) {
            nb.push_back(gs[a][i]);
        } else {
            const int j = (int)next(gs[b].size());
            na.push_back(gs[b][j]);
            nb.erase(nb.begin() + j);
            nb.push_back(gs[a][i]);
        }
        if (!fits(na) || !fits(nb))
            continue;
        const long ca = cost(na), cb = cost(nb), d = ca + cb - c[a] - c[b];
        if (d <= 0 || uniform() < std::exp(-(double)d / T)) {
            gs[a].swap(na);
            gs[b].swap(nb);
            c[a] = ca;
            c[b] = cb;
        }
    }
    std::vector<std::pair<long, std::vector<int>>> out;
    for (int k = 0; k < G; ++k)
        if (!gs[k].empty()) {
            std::sort(gs[k].begin(), gs[k].end());
            out.push_back({c[k], gs[k]});
        }
    std::sort(out.begin(), out.end(), [](const auto &x, const auto &y) {
        return x.first != y.first ? x.first > y.first : x.second[0] < y.second[0];
    });
    std::vector<std::vector<int>> res;
    for (auto &o : out)
        res.push_back(std::move(o.second));
    return res;
}

}  // namespace

// Linear-fit plan.  The scalar moments are polynomials in the basic moments,
// so dm_s/dr_j = sum_b L[s][b] grad_r(f_b Y_b)(r_j) with the sparse site
// Jacobian L[x][b] = dm_x/dm_b.  Its support follows the rules:
// supp(o) = union of supp(l), supp(r); its values follow
//   L[o][b] = sum_rules c (m_r L[l][b] + m_l L[r][b]),
// which is a step table of the same form as the rule tables (each entry adds
// c * ws[m index] * ws[L index]).  Duplicated basics count as their first
// occurrence.
bool build_lin_plan(const Model &m, const Plan &p, LinPlan &lp, std::string &err)
{
    lp = LinPlan();
    const int K = m.K, B = m.B;
    std::vector<int> canon((size_t)B);
    for (int b = 0; b < B; ++b)
        canon[b] = b;
    for (size_t k = 0; k + 1 < p.dup.size(); k += 2)
        canon[p.dup[k]] = p.dup[k + 1];
    std::vector<int> slot_of((size_t)B, -1);
    for (int s = 0; s < p.nslots; ++s)
        if (p.slot_basic[s] >= 0)
            slot_of[p.slot_basic[s]] = s;
    std::vector<std::vector<int>> supp((size_t)K);
    for (int b = 0; b < B; ++b)
        supp[b] = {canon[b]};
    std::vector<int> level((size_t)K, 0);
    for (int t = 0; t < m.T; ++t) {
        const int *r = &m.times[4 * t];
        std::vector<int> u;
        std::set_union(supp[r[0]].begin(), supp[r[0]].end(), supp[r[1]].begin(),
                       supp[r[1]].end(), std::back_inserter(u));
        std::vector<int> v;
        std::set_union(supp[r[3]].begin(), supp[r[3]].end(), u.begin(), u.end(),
                       std::back_inserter(v));
        supp[r[3]].swap(v);
        level[r[3]] = std::max(level[r[3]], 1 + std::max(level[r[0]], level[r[1]]));
    }
    // moments the scalars depend on
    std::vector<char> need((size_t)K, 0);
    for (int s = 0; s < m.S; ++s)
        need[m.map[s]] = 1;
    for (int t = m.T - 1; t >= 0; --t) {
        const int *r = &m.times[4 * t];
        if (need[r[3]])
            need[r[0]] = need[r[1]] = 1;
    }
    // Work-space layout (doubles): moments, a zero slot, the forward
    // partials, then the transpose buffer of the moment reduction, with
    // {one, L, L partials} over it (they are set after the moments).  The
    // forward rules are encoded again for this layout (no adjoint block).
    RawTables fwd;
    forward_tables(m, level, p.max_level, fwd);
    lp.dummy = p.K4;
    lp.fpart0 = lp.dummy + 4;
    lp.red0 = lp.fpart0 + ((fwd.max_partials + 3) & ~3);
    lp.one = lp.red0;
    lp.L0 = lp.one + 4;
    std::vector<int> lbase((size_t)K, -1);
    int nL = 0;
    for (int x = B; x < K; ++x)
        if (need[x]) {
            lbase[x] = nL;
            nL += (int)supp[x].size();
        }
    lp.nL = nL;
    auto lws = [&](int x, int b) {  // work-space index of L[x][b], -1 outside the support
        if (x < B)
            return canon[x] == b ? lp.one : -1;
        const auto &sx = supp[x];
        auto it = std::lower_bound(sx.begin(), sx.end(), b);
        if (it == sx.end() || *it != b)
            return -1;
        return lp.L0 + lbase[x] + (int)(it - sx.begin());
    };
    std::vector<std::vector<int>> by_out((size_t)K);
    for (int t = 0; t < m.T; ++t)
        by_out[m.times[4 * t + 3]].push_back(t);
    RawTables raw;
    for (int L = 1; L <= p.max_level; ++L) {
        std::vector<Task> tasks;
        for (int o = B; o < K; ++o) {
            if (level[o] != L || !need[o] || by_out[o].empty())
                continue;
            for (int b : supp[o]) {
                Task task;
                for (int t : by_out[o]) {
                    const int *r = &m.times[4 * t];
                    const int ll = lws(r[0], b), lr = lws(r[1], b);
                    if (ll >= 0)
                        task.push_back({r[1], ll, r[2], lws(o, b), 0});
                    if (lr >= 0)
                        task.push_back({r[0], lr, r[2], lws(o, b), 0});
                }
                if (task.empty())
                    continue;
                task[0][4] = 1;
                tasks.push_back(std::move(task));
            }
        }
        emit_level(tasks, raw);
    }
    lp.part0 = lp.L0 + ((nL + 3) & ~3);
    const int P4 = (raw.max_partials + 3) & ~3;
    lp.acc = lp.part0 + P4;
    lp.CH = kLinChunk;
    lp.priv = std::max(lp.acc, lp.red0 + kChunk * kRedStride);
    if (lp.priv > 0xffff)
        return fail(err, "model too large for the linear-fit work space");
    auto same = [](int x) { return x; };
    encode_tables(fwd, lp.fpart0, lp.dummy, same, same, same, lp.fwd_steps, lp.fwd_level_step,
                  lp.fwd_comb, lp.fwd_level_comb);
    encode_tables(raw, lp.part0, lp.dummy, same, same, same, lp.steps, lp.level_step, lp.comb,
                  lp.level_comb);
    // Chunks of scalars (group_scalars): at most kLinChunk scalars and at
    // most kLinEntries (slot, scalar) entries each.  Per chunk and slot: a
    // mask of the chunk's scalars whose support holds the slot's basic, and
    // their L indices (`one` where the bit is clear); for the compile-time
    // walks also the masks packed four per word and the L indices in walk
    // order (slot ascending, then scalar).
    std::vector<int> slot_nu((size_t)p.nslots);
    for (int s = 0; s < p.nslots; ++s) {
        const int abc = p.slot_abc[s];
        slot_nu[s] = (abc & 0xff) + ((abc >> 8) & 0xff) + ((abc >> 16) & 0xff);
    }
    std::vector<std::vector<int>> scalar_slots((size_t)m.S);
    for (int s = 0; s < m.S; ++s)
        for (int b : supp[m.map[s]]) {
            if (slot_of[b] < 0)
                return fail(err, "internal error: linear-fit support outside the slots");
            scalar_slots[s].push_back(slot_of[b]);
        }
    const auto chunks = group_scalars(scalar_slots, slot_nu, kLinChunk, kLinEntries);
    lp.chunk_s0.assign(1, 0);
    lp.chunk_scalar.clear();
    for (const auto &g : chunks) {
        int ent = 0;
        for (int s : g) {
            lp.chunk_scalar.push_back(s);
            ent += (int)scalar_slots[s].size();
        }
        lp.chunk_s0.push_back((int)lp.chunk_scalar.size());
        lp.max_chunk_entries = std::max(lp.max_chunk_entries, ent);
    }
    lp.nchunks = (int)lp.chunk_s0.size() - 1;
    lp.slot_mask.assign((size_t)lp.nchunks * p.nslots, 0);
    lp.slot_L.assign((size_t)lp.nchunks * p.nslots * kLinChunk, lp.one);
    for (int c = 0; c < lp.nchunks; ++c)
        for (int q = lp.chunk_s0[c]; q < lp.chunk_s0[c + 1]; ++q) {
            const int s = lp.chunk_scalar[q], k = q - lp.chunk_s0[c], x = m.map[s];
            for (int b : supp[x]) {
                const int sl = slot_of[b], li = lws(x, b);
                if (sl < 0 || li < 0)
                    return fail(err, "internal error: linear-fit support outside the slots");
                const size_t at = (size_t)c * p.nslots + sl;
                lp.slot_mask[at] |= 1 << k;
                lp.slot_L[at * kLinChunk + k] = li;
            }
        }
    // every walk's L indices in walk order (slot ascending, then scalar),
    // chunk after chunk: the values the tile kernel reads per site
    lp.walk_off.assign(1, 0);
    lp.walk.clear();
    for (int c = 0; c < lp.nchunks; ++c) {
        for (int sl = 0; sl < p.nslots; ++sl) {
            const size_t at = (size_t)c * p.nslots + sl;
            for (int k = 0; k < kLinChunk; ++k)
                if (lp.slot_mask[at] & (1 << k))
                    lp.walk.push_back(lp.slot_L[at * kLinChunk + k]);
        }
        lp.walk_off.push_back((int)lp.walk.size());
    }
    lp.lane_walk = p.nslots <= 4 * kLinMaskWords && lp.max_chunk_entries <= kLinEntries;
    lp.maskw.assign((size_t)lp.nchunks * kLinMaskWords, 0);
    lp.clist.assign((size_t)lp.nchunks * kLinEntries, lp.one);
    if (lp.lane_walk)
        for (int c = 0; c < lp.nchunks; ++c) {
            int e = 0;
            for (int sl = 0; sl < p.nslots; ++sl) {
                const size_t at = (size_t)c * p.nslots + sl;
                const int mk = lp.slot_mask[at];
                lp.maskw[(size_t)c * kLinMaskWords + sl / 4] |= mk << (8 * (sl % 4));
                for (int k = 0; k < kLinChunk; ++k)
                    if (mk & (1 << k))
                        lp.clist[(size_t)c * kLinEntries + e++] = lp.slot_L[at * kLinChunk + k];
            }
        }
    return true;
}

}  // namespace mtpx
