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
// reads and writes that form; only the linear-MTP subset of the schema is
// accepted (type "MTP", model "linear"), which is what PotMTP::Load admits
// (MTPMetadata::require_model, tools/mtp_metadata.h:520-529).
#include "mtpx_internal.hpp"

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

// Tag::validate for the linear MTP (tools/mtp_metadata.h:133-204, with
// MTPMetadata::require_model, :520-529).
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
    if (type->str != "MTP")
        return fail(err, "model type '" + type->str + "' is not a linear MTP");
    if (model->str != "linear")
        return fail(err, "this potential does not support the model '" + model->str + "'");
    if (get("q") || get("nn"))
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
    if (const Json *c = get("model_coeffs_count")) {
        double ip;
        if (c->kind != Json::Num || c->num < 0 || c->num > 2147483647.0 ||
            std::modf(c->num, &ip) != 0)
            return fail(err, "model_coeffs_count is outside the integer range");
    }
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
    return validate(tag.fields, Z, err);
}

// Tag::output(model_metadata()) serialised (tools/mtp_metadata.h:353-370,
// PotMTP::model_metadata potentials/potential_mtp.h:127-130).
std::string tag_output(const MetaTag &tag)
{
    Json v;
    v.kind = Json::Obj;
    v.obj = tag.fields;
    for (const char *k : {"type", "model", "q", "nn", "model_coeffs_count", "long_range"})
        v.obj.erase(k);
    v.obj["type"] = text_value("MTP");
    v.obj["model"] = text_value("linear");
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
