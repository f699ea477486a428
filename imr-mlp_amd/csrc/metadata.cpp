// The potential_tag metadata of .mtp files (host code).
//
// PotMTP::Load reads the tag with MTPMetadata::Tag::parse and PotMTP::Save
// writes Tag::output(model_metadata()) (potentials/potential_mtp.cpp:171-187,
// :665; tools/mtp_metadata.h:206-370).  A tag is either structured -- a JSON
// object whose "schema" is "gpml.mtp.metadata" -- or kept as plain text that
// the writer emits under "legacy_tag".  The writer's JSON is the compact
// form the reference's vendored JSON library produces: object keys in byte
// order, no blanks, integral numbers below 2^53 without a fraction and other
// numbers with 17 significant digits, and its string escapes.  This file
// reads and writes that form for the short-range models: the linear MTP
// (type "MTP", model "linear") and MTP-M potentials (type "MTP_M" with one
// of the heads mtp_m_li / q2 / fs / n1 / n2), what the standalone runtime
// reader admits (MTPMetadata::require_model with nonlinear models allowed,
// tools/mtp_metadata.h:520-529; runtime/mtp/mlip.cpp:70-296).  Long-range
// terms (type MTP_LES, "long_range") are refused.
#include "mtpx_internal.hpp"

#include <cctype>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>

namespace mtpx {

namespace {

std::string trim(const std::string &s)
{
    const size_t b = s.find_first_not_of(" \t\r\n");
    if (b == std::string::npos)
        return "";
    return s.substr(b, s.find_last_not_of(" \t\r\n") - b + 1);
}

// ---- JSON reader ----------------------------------------------------------
class Reader {
  public:
    Reader(const std::string &t) : s_(t) {}
    bool value(Json &v, int depth)
    {
        if (depth > 64)
            return false;
        ws();
        if (p_ >= s_.size())
            return false;
        const char c = s_[p_];
        if (c == '{')
            return object(v, depth);
        if (c == '[')
            return array(v, depth);
        if (c == '"') {
            v.kind = Json::Str;
            return string(v.str);
        }
        if (word("null")) {
            v.kind = Json::Null;
            return true;
        }
        if (word("true") || word("false")) {
            v.kind = Json::Bool;
            v.b = s_[p_ - 1] == 'e' && s_[p_ - 2] == 'u';
            return true;
        }
        return number(v);
    }
    bool at_end()
    {
        ws();
        return p_ == s_.size();
    }

  private:
    void ws()
    {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\r' ||
                                  s_[p_] == '\n'))
            ++p_;
    }
    bool word(const char *w)
    {
        const size_t n = std::strlen(w);
        if (s_.compare(p_, n, w) != 0)
            return false;
        p_ += n;
        return true;
    }
    bool number(Json &v)
    {
        const size_t b = p_;
        while (p_ < s_.size() && std::strchr("0123456789+-.eE", s_[p_]))
            ++p_;
        if (p_ == b)
            return false;
        const std::string t = s_.substr(b, p_ - b);
        char *e = nullptr;
        v.kind = Json::Num;
        v.num = std::strtod(t.c_str(), &e);
        return e == t.c_str() + t.size();
    }
    static void utf8(unsigned cp, std::string &out)
    {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xc0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += (char)(0xe0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        } else {
            out += (char)(0xf0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3f));
            out += (char)(0x80 | ((cp >> 6) & 0x3f));
            out += (char)(0x80 | (cp & 0x3f));
        }
    }
    bool hex4(unsigned &u)
    {
        if (p_ + 4 > s_.size())
            return false;
        u = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s_[p_++];
            u <<= 4;
            if (c >= '0' && c <= '9')
                u |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f')
                u |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F')
                u |= (unsigned)(c - 'A' + 10);
            else
                return false;
        }
        return true;
    }
    bool string(std::string &out)
    {
        ++p_;  // opening quote
        out.clear();
        while (p_ < s_.size()) {
            const char c = s_[p_++];
            if (c == '"')
                return true;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= s_.size())
                return false;
            const char e = s_[p_++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                unsigned u;
                if (!hex4(u))
                    return false;
                if (u >= 0xd800 && u <= 0xdbff) {  // surrogate pair
                    unsigned lo;
                    if (p_ + 2 > s_.size() || s_[p_] != '\\' || s_[p_ + 1] != 'u')
                        return false;
                    p_ += 2;
                    if (!hex4(lo) || lo < 0xdc00 || lo > 0xdfff)
                        return false;
                    u = 0x10000 + ((u - 0xd800) << 10) + (lo - 0xdc00);
                } else if (u >= 0xdc00 && u <= 0xdfff) {
                    return false;
                }
                utf8(u, out);
                break;
            }
            default: return false;
            }
        }
        return false;
    }
    bool object(Json &v, int depth)
    {
        ++p_;
        v.kind = Json::Obj;
        ws();
        if (p_ < s_.size() && s_[p_] == '}') {
            ++p_;
            return true;
        }
        for (;;) {
            ws();
            if (p_ >= s_.size() || s_[p_] != '"')
                return false;
            std::string key;
            if (!string(key) || v.obj.count(key))  // duplicate keys are refused
                return false;
            ws();
            if (p_ >= s_.size() || s_[p_++] != ':')
                return false;
            if (!value(v.obj[key], depth + 1))
                return false;
            ws();
            if (p_ >= s_.size())
                return false;
            const char c = s_[p_++];
            if (c == '}')
                return true;
            if (c != ',')
                return false;
        }
    }
    bool array(Json &v, int depth)
    {
        ++p_;
        v.kind = Json::Arr;
        ws();
        if (p_ < s_.size() && s_[p_] == ']') {
            ++p_;
            return true;
        }
        for (;;) {
            v.arr.emplace_back();
            if (!value(v.arr.back(), depth + 1))
                return false;
            ws();
            if (p_ >= s_.size())
                return false;
            const char c = s_[p_++];
            if (c == ']')
                return true;
            if (c != ',')
                return false;
        }
    }
    const std::string &s_;
    size_t p_ = 0;
};

// ---- JSON writer ----------------------------------------------------------
void write_string(const std::string &s, std::string &out)
{
    out += '"';
    for (unsigned char c : s) {
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '/': out += "\\/"; break;
        case '\b': out += "\\b"; break;
        case '\f': out += "\\f"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (c < 0x20 || c == 0x7f) {
                char buf[8];
                std::snprintf(buf, sizeof buf, "\\u%04x", c);
                out += buf;
            } else {
                out += (char)c;
            }
        }
    }
    out += '"';
}

void write_value(const Json &v, std::string &out)
{
    switch (v.kind) {
    case Json::Null: out += "null"; break;
    case Json::Bool: out += v.b ? "true" : "false"; break;
    case Json::Num: {
        char buf[64];
        double ip;
        if (std::fabs(v.num) < 9007199254740992.0 && std::modf(v.num, &ip) == 0)
            std::snprintf(buf, sizeof buf, "%.f", v.num);
        else
            std::snprintf(buf, sizeof buf, "%.17g", v.num);
        out += buf;
        break;
    }
    case Json::Str: write_string(v.str, out); break;
    case Json::Arr:
        out += '[';
        for (size_t k = 0; k < v.arr.size(); ++k) {
            if (k)
                out += ',';
            write_value(v.arr[k], out);
        }
        out += ']';
        break;
    case Json::Obj: {
        out += '{';
        bool first = true;
        for (const auto &kv : v.obj) {  // std::map: byte order of the keys
            if (!first)
                out += ',';
            first = false;
            write_string(kv.first, out);
            out += ':';
            write_value(kv.second, out);
        }
        out += '}';
        break;
    }
    }
}

Json text_value(const char *s)
{
    Json v;
    v.kind = Json::Str;
    v.str = s;
    return v;
}

bool is_element(const std::string &s)
{
    static const std::string symbols =
        " H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn Ga Ge "
        "As Se Br Kr Rb Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce Pr Nd Pm Sm "
        "Eu Gd Tb Dy Ho Er Tm Yb Lu Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Po At Rn Fr Ra Ac Th Pa U "
        "Np Pu Am Cm Bk Cf Es Fm Md No Lr Rf Db Sg Bh Hs Mt Ds Rg Cn Nh Fl Mc Lv Ts Og ";
    if (s.empty() || s.size() > 3 || !(s[0] >= 'A' && s[0] <= 'Z'))
        return false;
    for (size_t k = 1; k < s.size(); ++k)
        if (!(s[k] >= 'a' && s[k] <= 'z'))
            return false;
    return symbols.find(' ' + s + ' ') != std::string::npos;
}

bool fail(std::string &err, const std::string &msg)
{
    err = "MTP metadata: " + msg;
    return false;
}

bool nonempty_text(const Json &v) { return v.kind == Json::Str && !v.str.empty(); }

// MTPMetadata::integer (tools/mtp_metadata.h:38-46): an integral number in
// [minimum, INT_MAX].
bool json_int(const Json &v, int minimum, int &out)
{
    if (v.kind != Json::Num || !std::isfinite(v.num) || v.num < minimum ||
        v.num > 2147483647.0 || std::floor(v.num) != v.num)
        return false;
    out = (int)v.num;
    return true;
}

std::string upper(std::string s)
{
    for (char &c : s)
        c = (char)std::toupper((unsigned char)c);
    return s;
}

// canonical_model (tools/mtp_metadata.h:66-71)
std::string canonical_model(const std::string &name)
{
    return name == "mtp_m_nn2" ? std::string("mtp_m_n2") : name;
}

const char *const kHeadNames[] = {"linear", "mtp_m_li", "mtp_m_q2", "mtp_m_fs", "mtp_m_n1",
                                  "mtp_m_n2"};
const char *const kActNames[] = {"TANH", "RELU", "SIGMOID", "LINEAR"};

int head_index(const std::string &model)
{
    for (int k = 0; k < 6; ++k)
        if (model == kHeadNames[k])
            return k;
    return -1;
}

// Tag::validate (tools/mtp_metadata.h:133-204) with MTPMetadata::require_model
// (:520-529) for the short-range models.
bool validate(const std::map<std::string, Json> &f, int Z, std::string &err)
{
    auto get = [&](const char *k) -> const Json * {
        auto it = f.find(k);
        return it == f.end() ? nullptr : &it->second;
    };
    const Json *schema = get("schema"), *version = get("version"), *type = get("type"),
               *model = get("model");
    if (!schema || !nonempty_text(*schema) || schema->str != "gpml.mtp.metadata")
        return fail(err, "unknown schema");
    if (!version || version->kind != Json::Num || version->num != 1.0)
        return fail(err, "unsupported or missing metadata version");
    if (!type || !model)
        return fail(err, "type and model are required");
    if (!nonempty_text(*type) || !nonempty_text(*model))
        return fail(err, "type and model must be nonempty strings");
    if (type->str == "MTP_LES")
        return fail(err, "long-range terms are not supported");
    if (type->str != "MTP" && type->str != "MTP_M")
        return fail(err, "unknown model type");
    const std::string name = canonical_model(model->str);
    if (head_index(name) < 0)
        return fail(err, "unknown model");
    if (type->str != "MTP_M" && name != "linear")
        return fail(err, "ordinary MTP cannot declare an external head");
    if (get("long_range"))
        return fail(err, "long-range terms are not supported");
    if (const Json *e = get("elements")) {
        if (e->kind != Json::Arr)
            return fail(err, "elements must be an array");
        if ((int)e->arr.size() != Z)
            return fail(err, "elements count does not match species_count");
        std::set<std::string> seen;
        for (const Json &x : e->arr) {
            if (!nonempty_text(x) || !is_element(x.str))
                return fail(err, "invalid element symbol");
            if (!seen.insert(x.str).second)
                return fail(err, "duplicate element '" + x.str + "'");
        }
    }
    int v;
    if (const Json *c = get("q"))
        if (!json_int(*c, 1, v))
            return fail(err, "q is outside the integer range");
    if (const Json *c = get("model_coeffs_count"))
        if (!json_int(*c, 0, v))
            return fail(err, "model_coeffs_count is outside the integer range");
    if (type->str == "MTP_M") {
        const Json *q = get("q");
        if (!q)
            return fail(err, "MTP_M requires q");
        json_int(*q, 1, v);
        if (name == "linear")
            return fail(err, "MTP_M requires an external model");
        if (name == "mtp_m_li" && v != 1)
            return fail(err, "linear head requires q=1");
        if ((name == "mtp_m_q2" || name == "mtp_m_fs") && v != 2)
            return fail(err, "analytic head requires q=2");
    } else if (get("q") || get("nn")) {
        return fail(err, "ordinary MTP cannot declare an external head");
    }
    if (const Json *nn = get("nn")) {
        if (nn->kind != Json::Obj)
            return fail(err, "nn must be an object");
        auto a = nn->obj.find("activation");
        auto h = nn->obj.find("hidden_layers");
        if (a == nn->obj.end() || !nonempty_text(a->second))
            return fail(err, "nn.activation must be a nonempty string");
        if (h == nn->obj.end() || h->second.kind != Json::Arr)
            return fail(err, "nn.hidden_layers must be an array");
        const size_t expected = name == "mtp_m_n1" ? 1 : name == "mtp_m_n2" ? 2 : 0;
        if (h->second.arr.size() != expected || expected == 0)
            return fail(err, "nn.hidden_layers conflicts with model");
        const std::string act = upper(a->second.str);
        if (act != "TANH" && act != "RELU" && act != "SIGMOID" && act != "LINEAR")
            return fail(err, "unknown activation");
        for (const Json &layer : h->second.arr)
            if (!json_int(layer, 1, v))
                return fail(err, "nn.hidden_layers is outside the integer range");
    }
    return true;
}

// Head-field values of read_mtp_gpu_metadata (runtime/mtp/mlip.cpp:120-201):
// "mtp_<key>" -> value text, merged from the tag and the file's lines.
using Fields = std::map<std::string, std::string>;

// MTPMetadata::merge_legacy with normalize_legacy (tools/mtp_metadata.h:
// 400-421).
bool merge_field(Fields &f, const std::string &key, std::string value, std::string &err)
{
    if (key == "mtp_model") {
        value = canonical_model(value);
        if (value == "mtp")
            value = "linear";
    }
    if (key == "mtp_activation")
        value = upper(value);
    auto it = f.find(key);
    if (it != f.end() && it->second != value) {
        err = "Invalid MTP metadata: MTP metadata: conflicting JSON/footer metadata for " + key;
        return false;
    }
    f[key] = value;
    return true;
}

// std::stoi over the whole value (mlip.cpp:169-176)
bool whole_int(const std::string &s, int &out)
{
    if (s.empty())
        return false;
    char *e = nullptr;
    errno = 0;
    const long v = std::strtol(s.c_str(), &e, 10);
    if (e != s.c_str() + s.size() || errno || v < INT_MIN || v > INT_MAX ||
        std::isspace((unsigned char)s[0]))
        return false;
    out = (int)v;
    return true;
}

}  // namespace

bool json_parse(const std::string &text, Json &out, std::string &err)
{
    Reader r(text);
    out = Json();
    if (!r.value(out, 0) || !r.at_end()) {
        err = "invalid JSON";
        return false;
    }
    return true;
}

std::string json_serialize(const Json &v)
{
    std::string out;
    write_value(v, out);
    return out;
}

// Tag::parse (tools/mtp_metadata.h:206-333) for the forms PotMTP::Load
// admits: empty, plain text (kept as the legacy text) and structured JSON.
bool tag_parse(const std::string &raw, int Z, MetaTag &tag, std::string &err)
{
    tag = MetaTag();
    if (raw.size() > 65536)
        return fail(err, "tag exceeds 64 KiB");
    std::string source = trim(raw);
    if (!source.empty() && source[0] == '=')
        source = trim(source.substr(1));
    tag.legacy = source;
    if (source.empty() || source[0] != '{') {
        if (source.find("imrmlp_meta_v") != std::string::npos)
            return fail(err, "imrmlp_meta_v1 potential tags are not supported");
        return true;
    }
    Json v;
    std::string jerr;
    if (!json_parse(source, v, jerr)) {
        if (source.find("gpml.mtp.metadata") != std::string::npos)
            return fail(err, "invalid potential_tag JSON");
        return true;  // other text: kept as the legacy text
    }
    auto sc = v.obj.find("schema");
    if (v.kind != Json::Obj || sc == v.obj.end() || sc->second.kind != Json::Str ||
        sc->second.str != "gpml.mtp.metadata")
        return true;
    tag.fields = v.obj;
    auto lg = tag.fields.find("legacy_tag");
    if (lg != tag.fields.end() && !nonempty_text(lg->second))
        return fail(err, "legacy_tag must be a nonempty string");
    tag.legacy = lg != tag.fields.end() ? lg->second.str : "";
    if (!validate(tag.fields, Z, err))
        return false;
    // Tag::parse's canonical forms (tools/mtp_metadata.h:319-329)
    tag.fields["model"].str = canonical_model(tag.fields["model"].str);
    auto nn = tag.fields.find("nn");
    if (nn != tag.fields.end())
        nn->second.obj["activation"].str = upper(nn->second.obj["activation"].str);
    return true;
}

// read_mtp_gpu_metadata (runtime/mtp/mlip.cpp:70-296): the head fields of
// the tag (MTPMetadata::legacy_model_fields, tools/mtp_metadata.h:374-398)
// merged with the "mtp_<key> = value" lines of the text before any
// "#MVS_v1.1" payload, then checked against the head's dimensions.
bool head_parse(const std::string &text, const MetaTag &tag, Head &head, std::string &err)
{
    head = Head();
    Fields f;
    bool model_coeffs = false;
    const std::string pre = "Invalid MTP metadata: ";
    if (!tag.fields.empty()) {
        f["mtp_model"] = canonical_model(tag.fields.at("model").str);
        int v;
        auto q = tag.fields.find("q");
        if (q != tag.fields.end() && json_int(q->second, 0, v))
            f["mtp_descriptor_count"] = std::to_string(v);
        auto c = tag.fields.find("model_coeffs_count");
        if (c != tag.fields.end() && json_int(c->second, 0, v))
            f["mtp_model_coeffs_count"] = std::to_string(v);
        auto nn = tag.fields.find("nn");
        if (nn != tag.fields.end()) {
            const Json &o = nn->second;
            f["mtp_activation"] = upper(o.obj.at("activation").str);
            const std::vector<Json> &layers = o.obj.at("hidden_layers").arr;
            json_int(layers[0], 1, v);
            f["mtp_hidden1"] = std::to_string(v);
            if (layers.size() == 2)
                json_int(layers[1], 1, v);
            f["mtp_hidden2"] = layers.size() == 2 ? std::to_string(v) : "0";
        }
    }
    size_t pos = 0;
    while (pos <= text.size()) {
        size_t eol = text.find('\n', pos);
        if (eol == std::string::npos)
            eol = text.size();
        std::string line = trim(text.substr(pos, eol - pos));
        pos = eol + 1;
        if (line.rfind("#MVS_v1.1", 0) == 0)
            break;
        if (line.rfind("les_", 0) == 0 || line.rfind("sog_", 0) == 0 ||
            line.rfind("lr_les", 0) == 0 || line.rfind("long_range", 0) == 0)
            return fail(err, "long-range payload is unsupported by the short-range runtime");
        if (line.rfind("model_coeffs", 0) == 0)
            model_coeffs = true;
        if (!line.empty() && line[0] == '#')
            line = trim(line.substr(1));
        if (line.rfind("mtp_", 0) != 0)
            continue;
        const size_t eq = line.find('=');
        if (eq == std::string::npos)
            continue;
        if (!merge_field(f, trim(line.substr(0, eq)), trim(line.substr(eq + 1)), err))
            return false;
    }
    // a value that does not parse reports "invalid value for <key>", the
    // model and activation names included (mlip.cpp:196-200 catches their
    // own errors)
    int model = kHeadNone, q = 0, mcc = 0, h1 = 0, h2 = 0, act = kActTanh;
    for (const auto &kv : f) {
        const std::string &k = kv.first, &v = kv.second;
        bool ok = true;
        if (k == "mtp_model") {
            model = head_index(v);
            ok = model >= 0;
        } else if (k == "mtp_descriptor_count") {
            ok = whole_int(v, q);
        } else if (k == "mtp_model_coeffs_count") {
            ok = whole_int(v, mcc);
        } else if (k == "mtp_hidden1") {
            ok = whole_int(v, h1);
        } else if (k == "mtp_hidden2") {
            ok = whole_int(v, h2);
        } else if (k == "mtp_activation") {
            act = -1;
            for (int a = 0; a < 4; ++a)
                if (v == kActNames[a])
                    act = a;
            ok = act >= 0;
        }
        if (!ok) {
            err = pre + "invalid value for " + k + ": '" + v + "'";
            return false;
        }
    }
    if (q < 0 || mcc < 0 || h1 < 0 || h2 < 0) {
        err = pre + "model dimensions and coefficient counts must be nonnegative";
        return false;
    }
    for (int d : {q, mcc, h1, h2})
        if ((size_t)d > text.size()) {
            err = pre + "model dimension exceeds the serialized model size";
            return false;
        }
    auto bad = [&](const char *msg) {
        err = pre + msg;
        return false;
    };
    const bool neural = model == kHeadNn1 || model == kHeadNn2;
    if (!neural && (h1 != 0 || h2 != 0))
        return bad("non-neural models require zero hidden dimensions");
    if (model == kHeadNn1 && h2 != 0)
        return bad("NN1 requires zero hidden2");
    if (model == kHeadNone) {
        if (model_coeffs)
            return bad("model_coeffs is present but mtp_model metadata is missing");
        return true;
    }
    if (!model_coeffs)
        return bad("nonlinear mtp_model requires a model_coeffs section");
    if (model == kHeadLi) {
        if (q == 0)
            q = 1;
        if (q != 1 || mcc != 0)
            return bad("linear MTP-M requires one descriptor and no head coefficients");
    } else if (model == kHeadQ2 || model == kHeadFs) {
        if (q == 0)
            q = 2;
        else if (q != 2)
            return bad("analytic q2/fs models require descriptor_count 2");
        const int expected = model == kHeadQ2 ? 5 : 1;
        if (mcc == 0)
            mcc = expected;
        else if (mcc != expected)
            return bad("analytic model coefficient count does not match model type");
    } else {
        if (q <= 0 || h1 <= 0)
            return bad("neural model requires positive descriptor_count and hidden1");
        if (model == kHeadNn2 && h2 <= 0)
            return bad("NN2 model requires positive hidden2");
        const long long expected =
            model == kHeadNn1 ? (long long)h1 * ((long long)q + 2)
                              : (long long)q * h1 + h1 + (long long)h1 * h2 + 2LL * h2;
        if (expected > INT_MAX)
            return bad("neural coefficient count overflows the model index type");
        if (model == kHeadNn2 && act == kActLinear)
            return bad("NN2 does not support LINEAR activation");
        if (mcc == 0)
            mcc = (int)expected;
        else if (mcc != expected)
            return bad("neural model coefficient count does not match dimensions");
    }
    head.kind = model;
    head.P = q;
    head.h1 = neural ? h1 : 0;
    head.h2 = model == kHeadNn2 ? h2 : 0;
    head.act = act;
    head.Mc = mcc;
    return true;
}

// Tag::output(model_metadata()) serialised (tools/mtp_metadata.h:353-370;
// PotMTP::model_metadata potentials/potential_mtp.h:127-130 for the linear
// MTP, PotMTP_M::model_metadata potentials/potential_mtp_m.h:1564-1589 with a
// head).
std::string tag_output(const MetaTag &tag, const Head &head)
{
    Json v;
    v.kind = Json::Obj;
    v.obj = tag.fields;
    for (const char *k : {"type", "model", "q", "nn", "model_coeffs_count", "long_range"})
        v.obj.erase(k);
    auto number = [](double x) {
        Json n;
        n.kind = Json::Num;
        n.num = x;
        return n;
    };
    if (head.kind != kHeadNone) {
        v.obj["type"] = text_value("MTP_M");
        v.obj["model"] = text_value(kHeadNames[head.kind]);
        v.obj["q"] = number(head.P);
        v.obj["model_coeffs_count"] = number(head.Mc);
        if (head.kind == kHeadNn1 || head.kind == kHeadNn2) {
            Json nn, layers;
            nn.kind = Json::Obj;
            layers.kind = Json::Arr;
            layers.arr.push_back(number(head.h1));
            if (head.kind == kHeadNn2)
                layers.arr.push_back(number(head.h2));
            nn.obj["activation"] = text_value(kActNames[head.act]);
            nn.obj["hidden_layers"] = layers;
            v.obj["nn"] = nn;
        }
    } else {
        v.obj["type"] = text_value("MTP");
        v.obj["model"] = text_value("linear");
    }
    v.obj["schema"] = text_value("gpml.mtp.metadata");
    Json one;
    one.kind = Json::Num;
    one.num = 1.0;
    v.obj["version"] = one;
    if (!tag.legacy.empty())
        v.obj["legacy_tag"] = text_value(tag.legacy.c_str());
    return json_serialize(v);
}

}  // namespace mtpx
