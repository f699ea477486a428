// GPM v2 model bundles for MTP and MTP-M potentials (host code).
//
// A bundle (tools/gpm_container.h) is a 64-byte preamble -- "GPMLMODL",
// major version 2 (u16 at 8), required flags 0 (u32 at 12), the JSON header
// length (u64 at 16) and the data start, the header end rounded up to 64
// (u64 at 24) -- then the JSON manifest, then the data blocks, each at a
// 64-aligned offset from the data start.  The manifest's "blocks" directory
// gives each block's id, dtype, shape, codec ("none" or "zstd"), offset,
// stored and raw size, sizes as decimal strings.  Its "models" hold the
// root model node: for an MTP, "configuration" (dimensions, the
// potential_tag metadata, the named settings of each radial basis and the
// head fields) and "parameters" (coefficient and index blocks), written by
// encode_mtp (potentials/gpm_codec.cpp:190-312) and read back through
// GPM::mtp_text (tools/gpm_mtp.h:160-289), which rebuilds the .mtp text the
// ordinary reader parses.  This file restates both directions for the
// library's models; zstd blocks go through the system's libzstd, opened at
// run time.
#include "mtpx_internal.hpp"

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

namespace mtpx {

namespace {

using Bytes = std::vector<unsigned char>;

struct GpmError {
    std::string msg;
};

[[noreturn]] void gpm_fail(const std::string &why) { throw GpmError{"GPM: " + why}; }
void require(bool ok, const std::string &why)
{
    if (!ok)
        gpm_fail(why);
}

uint64_t checked_add(uint64_t a, uint64_t b)
{
    require(b <= UINT64_MAX - a, "size overflow");
    return a + b;
}
uint64_t checked_mul(uint64_t a, uint64_t b)
{
    require(!a || b <= UINT64_MAX / a, "size overflow");
    return a * b;
}
uint64_t align64(uint64_t x) { return checked_add(x, 63) & ~uint64_t(63); }

uint64_t get_le(const unsigned char *p, unsigned bytes)
{
    uint64_t n = 0;
    for (unsigned i = 0; i < bytes; ++i)
        n |= uint64_t(p[i]) << (8 * i);
    return n;
}
void put_le(unsigned char *p, uint64_t n, unsigned bytes)
{
    for (unsigned i = 0; i < bytes; ++i) {
        p[i] = (unsigned char)n;
        n >>= 8;
    }
}

// ---- JSON access (GPM::object / array / at / string / integer / decimal)
const std::map<std::string, Json> &object(const Json &v)
{
    require(v.kind == Json::Obj, "expected JSON object");
    return v.obj;
}
const std::vector<Json> &array(const Json &v)
{
    require(v.kind == Json::Arr, "expected JSON array");
    return v.arr;
}
const Json &at(const std::map<std::string, Json> &o, const std::string &key)
{
    auto it = o.find(key);
    require(it != o.end(), "missing field " + key);
    return it->second;
}
const std::string &text(const Json &v)
{
    require(v.kind == Json::Str, "expected string");
    return v.str;
}
int integer(const Json &v)
{
    require(v.kind == Json::Num, "expected integer");
    const double x = v.num;
    require(std::isfinite(x) && x >= 0 && x <= 2147483647.0 && std::floor(x) == x,
            "invalid integer");
    return (int)x;
}
// a count written as a decimal string: digits, no leading zero
uint64_t decimal(const Json &v)
{
    const std::string &s = text(v);
    require(!s.empty() && (s.size() == 1 || s[0] != '0'), "invalid uint64");
    uint64_t n = 0;
    for (char c : s) {
        require(c >= '0' && c <= '9' && n <= (UINT64_MAX - (uint64_t)(c - '0')) / 10,
                "invalid uint64");
        n = n * 10 + (uint64_t)(c - '0');
    }
    return n;
}
Json str_value(const std::string &s)
{
    Json v;
    v.kind = Json::Str;
    v.str = s;
    return v;
}
Json num_value(double x)
{
    Json v;
    v.kind = Json::Num;
    v.num = x;
    return v;
}
Json count_value(uint64_t n) { return str_value(std::to_string(n)); }
Json obj_value() { Json v; v.kind = Json::Obj; return v; }
Json arr_value() { Json v; v.kind = Json::Arr; return v; }

// The UTF-8 check of GPM::parse (tools/gpm_container.h:287-330): well
// formed, shortest form, no surrogates.
void check_utf8(const std::string &s)
{
    for (size_t i = 0; i < s.size();) {
        const unsigned char lead = (unsigned char)s[i++];
        if (lead < 0x80)
            continue;
        unsigned tails;
        uint32_t code;
        if (lead >= 0xc2 && lead <= 0xdf) {
            tails = 1;
            code = lead & 31;
        } else if (lead >= 0xe0 && lead <= 0xef) {
            tails = 2;
            code = lead & 15;
        } else if (lead >= 0xf0 && lead <= 0xf4) {
            tails = 3;
            code = lead & 7;
        } else {
            gpm_fail("invalid UTF-8");
        }
        require(tails <= s.size() - i, "truncated UTF-8");
        for (unsigned k = 0; k < tails; ++k) {
            const unsigned char next = (unsigned char)s[i++];
            require((next & 0xc0) == 0x80, "invalid UTF-8 continuation");
            code = (code << 6) | (next & 63);
        }
        require(code >= (tails == 1 ? 0x80u : tails == 2 ? 0x800u : 0x10000u) &&
                    code <= 0x10ffffu && !(code >= 0xd800u && code <= 0xdfffu),
                "invalid UTF-8 code point");
    }
}

unsigned width(const std::string &dtype)
{
    if (dtype == "f64" || dtype == "i64" || dtype == "u64")
        return 8;
    if (dtype == "i32" || dtype == "u32")
        return 4;
    if (dtype == "u8")
        return 1;
    gpm_fail("unsupported dtype " + dtype);
}

// ---- zstd, from the system library at run time --------------------------
struct Zstd {
    using Decompress = size_t (*)(void *, size_t, const void *, size_t);
    using Compress = size_t (*)(void *, size_t, const void *, size_t, int);
    using Bound = size_t (*)(size_t);
    using IsError = unsigned (*)(size_t);
    Decompress decompress = nullptr;
    Compress compress = nullptr;
    Bound bound = nullptr;
    IsError is_error = nullptr;
    bool ok = false;
    static const Zstd &get()
    {
        static const Zstd z = [] {
            Zstd r;
            void *h = dlopen("libzstd.so.1", RTLD_NOW | RTLD_LOCAL);
            if (!h)
                return r;
            r.decompress = (Decompress)dlsym(h, "ZSTD_decompress");
            r.compress = (Compress)dlsym(h, "ZSTD_compress");
            r.bound = (Bound)dlsym(h, "ZSTD_compressBound");
            r.is_error = (IsError)dlsym(h, "ZSTD_isError");
            r.ok = r.decompress && r.compress && r.bound && r.is_error;
            return r;
        }();
        return z;
    }
};

// ---- reader (GPM::Reader, tools/gpm_container.h:393-542) ----------------
struct Block {
    std::string dtype, codec;
    std::vector<uint64_t> shape;
    uint64_t offset = 0, stored = 0, raw = 0;
};

struct Reader {
    const unsigned char *p;
    uint64_t size, data = 0;
    Json manifest;
    std::map<std::string, Block> blocks;

    Reader(const void *bytes, size_t n) : p((const unsigned char *)bytes), size(n)
    {
        require(size >= 64, "truncated preamble");
        require(std::memcmp(p, "GPMLMODL", 8) == 0, "invalid magic");
        require(get_le(p + 8, 2) == 2, "unsupported major version");
        require(get_le(p + 12, 4) == 0, "unsupported required flags");
        const uint64_t length = get_le(p + 16, 8);
        data = get_le(p + 24, 8);
        require(length <= 64 * 1024 * 1024 && data == align64(checked_add(64, length)) &&
                    data <= size,
                "invalid header size");
        const std::string json((const char *)p + 64, (size_t)length);
        check_utf8(json);
        std::string err;
        require(json_parse(json, manifest, err), "invalid JSON: " + err);
        const auto &m = object(manifest);
        require(text(at(m, "schema")) == "gpml.model", "unknown schema");
        if (m.count("required_features"))
            require(array(m.at("required_features")).empty(), "unsupported required features");
        std::vector<std::pair<uint64_t, uint64_t>> spans;
        for (const Json &e : array(at(m, "blocks"))) {
            const auto &o = object(e);
            Block b;
            const std::string id = text(at(o, "id"));
            b.dtype = text(at(o, "dtype"));
            b.codec = text(at(o, "codec"));
            b.offset = decimal(at(o, "offset"));
            b.stored = decimal(at(o, "stored_size"));
            b.raw = decimal(at(o, "raw_size"));
            uint64_t elements = 1;
            for (const Json &x : array(at(o, "shape"))) {
                const uint64_t d = decimal(x);
                elements = checked_mul(elements, d);
                b.shape.push_back(d);
            }
            require(checked_mul(elements, width(b.dtype)) == b.raw,
                    "block shape/size mismatch: " + id);
            require(!id.empty() && b.offset % 64 == 0 && b.offset <= size - data &&
                        b.stored <= size - data - b.offset,
                    "invalid block bounds: " + id);
            require(b.codec != "none" || b.stored == b.raw, "invalid uncompressed block size");
            require(blocks.emplace(id, b).second, "duplicate block id");
            if (b.stored)
                spans.emplace_back(b.offset, checked_add(b.offset, b.stored));
        }
        std::sort(spans.begin(), spans.end());
        for (size_t i = 1; i < spans.size(); ++i)
            require(spans[i - 1].second <= spans[i].first, "overlapping blocks");
    }

    const Block &info(const std::string &id) const
    {
        auto it = blocks.find(id);
        require(it != blocks.end(), "missing block " + id);
        return it->second;
    }

    // Reader::read's default limit (tools/gpm_container.h:512-515): neither
    // size of a block may pass 8 GiB, checked before anything is allocated.
    static constexpr uint64_t kReadLimit = uint64_t(8) << 30;

    Bytes read(const std::string &id) const
    {
        const Block &b = info(id);
        require(b.raw <= kReadLimit && b.stored <= kReadLimit, "block exceeds read limit: " + id);
        require(b.codec == "none" || b.codec == "zstd", "unsupported codec " + b.codec);
        const unsigned char *s = p + data + b.offset;
        if (b.codec == "none")
            return Bytes(s, s + b.stored);
        const Zstd &z = Zstd::get();
        require(z.ok, "zstd support is not enabled (libzstd.so.1 not found)");
        Bytes raw((size_t)b.raw);
        const size_t n = z.decompress(raw.data(), raw.size(), s, (size_t)b.stored);
        require(!z.is_error(n) && n == raw.size(), "invalid zstd block " + id);
        return raw;
    }

    // GPM::values / GPM::indices (tools/gpm_mtp.h:52-85): an empty array is
    // {"dtype", "shape"} with a zero dimension; otherwise a block reference
    std::vector<double> values(const Json &ref) const
    {
        const auto &o = object(ref);
        if (!o.count("block")) {
            uint64_t n = 1;
            for (const Json &d : array(at(o, "shape")))
                n = checked_mul(n, decimal(d));
            require(n == 0 && text(at(o, "dtype")) == "f64", "invalid empty numeric array");
            return {};
        }
        const std::string id = text(at(o, "block"));
        require(info(id).dtype == "f64", "expected FP64 block");
        const Bytes b = read(id);
        std::vector<double> out(b.size() / 8);
        for (size_t i = 0; i < out.size(); ++i) {
            const uint64_t x = get_le(b.data() + 8 * i, 8);
            std::memcpy(&out[i], &x, 8);
        }
        return out;
    }
    std::vector<int32_t> indices(const Json &ref) const
    {
        const auto &o = object(ref);
        if (!o.count("block")) {
            uint64_t n = 1;
            for (const Json &d : array(at(o, "shape")))
                n = checked_mul(n, decimal(d));
            require(n == 0 && text(at(o, "dtype")) == "i32", "invalid empty index array");
            return {};
        }
        const std::string id = text(at(o, "block"));
        require(info(id).dtype == "i32", "expected index block");
        const Bytes b = read(id);
        std::vector<int32_t> out(b.size() / 4);
        for (size_t i = 0; i < out.size(); ++i) {
            const uint32_t x = (uint32_t)get_le(b.data() + 4 * i, 4);
            std::memcpy(&out[i], &x, 4);
        }
        return out;
    }
};

std::string g17(double v)
{
    char buf[64];
    std::snprintf(buf, sizeof buf, "%.17g", v);
    return buf;
}

// GPM::print_basis (tools/gpm_mtp.h:128-156): the four leading fields,
// then the optional selectors in their dependency order, then the rest in
// key order ("scaling" and "polynomial" are not basis lines).
void print_basis(std::string &out, const std::map<std::string, Json> &basis)
{
    for (const char *name : {"radial_basis_type", "min_dist", "max_dist", "radial_basis_size"})
        out += std::string(name) + " = " + text(at(basis, name)) + "\n";
    std::set<std::string> done{"radial_basis_type", "min_dist", "max_dist",
                               "radial_basis_size", "scaling",  "polynomial"};
    for (const char *name : {"rb_b", "basis_function_type", "cutoff_type", "cutoff_power",
                             "cutoff_coefficients", "cutoff_b", "cutoff_r1", "cutoff_r2",
                             "shift_type", "shift_lambda"}) {
        auto it = basis.find(name);
        if (it != basis.end()) {
            out += std::string(name) + " = " + text(it->second) + "\n";
            done.insert(name);
        }
    }
    for (const auto &kv : basis)
        if (!done.count(kv.first))
            out += kv.first + " = " + text(kv.second) + "\n";
}

// The root node's .mtp text (GPM::mtp_text with standalone = false, and
// the checks of MLIPCore::read_model_text, runtime/mtp/mlip.cpp:354-383).
std::string node_text(const Reader &r, std::vector<double> &scalings)
{
    const auto &m = object(r.manifest);
    const auto &node = object(at(object(at(m, "models")), text(at(m, "root_model"))));
    const std::string type = text(at(node, "type"));
    require(type == "mtp" || type == "mtp_m", "this library reads mtp and mtp_m models, not " + type);
    require(integer(at(node, "version")) == 1, "unsupported model version");
    if (node.count("required_features"))
        require(array(node.at("required_features")).empty(),
                "unsupported required model capability");
    const auto &units = object(at(m, "units"));
    require(text(at(units, "length")) == "angstrom" && text(at(units, "energy")) == "eV" &&
                text(at(units, "charge")) == "e" && text(at(units, "stress")) == "virial_eV",
            "unsupported GPM units");
    const auto &c = object(at(node, "configuration")), &p = object(at(node, "parameters"));
    require(integer(at(c, "radial_mode")) == 0, "unsupported radial mode");
    const int ns = integer(at(c, "species_count")), nf = integer(at(c, "radial_functions")),
              nb = integer(at(c, "radial_size")), nm = integer(at(c, "moments_count"));
    require(ns > 0 && nf > 0 && nb > 0 && nm > 0, "invalid MTP dimensions");
    const auto &bases = array(at(c, "radial_bases"));
    require(bases.size() == 1 || bases.size() == checked_mul(ns, ns), "invalid radial bases");
    const std::vector<double> radial = r.values(at(p, "radial")), species = r.values(at(p, "species")),
                              moments = r.values(at(p, "moments"));
    const std::vector<int32_t> basic = r.indices(at(p, "basic_indices")),
                               times = r.indices(at(p, "product_indices")),
                               mapping = r.indices(at(p, "scalar_mapping"));
    require(radial.size() == checked_mul(checked_mul(ns, ns), checked_mul(nf, nb)) &&
                basic.size() % 4 == 0 && times.size() % 4 == 0,
            "invalid MTP array sizes");
    require(!mapping.empty() && species.size() % ns == 0 && moments.size() % mapping.size() == 0,
            "invalid MTP coefficient dimensions");
    require(basic.size() / 4 <= (size_t)nm, "too many basic moments");
    for (size_t i = 0; i < basic.size(); i += 4) {
        require(basic[i] >= 0 && basic[i] < nf, "radial index out of bounds");
        for (int k = 1; k < 4; ++k)
            require(basic[i + k] >= 0 && basic[i + k] <= 128, "invalid angular degree");
    }
    for (size_t i = 0; i < times.size(); i += 4) {
        require(times[i] >= 0 && times[i] < nm && times[i + 1] >= 0 && times[i + 1] < nm &&
                    times[i + 3] >= int(basic.size() / 4) && times[i + 3] < nm,
                "invalid product rule");
        require(times[i] < times[i + 3] && times[i + 1] < times[i + 3], "cyclic moment rule");
    }
    for (int32_t x : mapping)
        require(x >= 0 && x < nm, "invalid scalar index");
    const Json &metadata = at(c, "metadata");
    require(!object(metadata).count("long_range"), "long-range GPM models are not supported");
    scalings.clear();
    for (const Json &b : bases) {
        const std::string &s = text(at(object(b), "scaling"));
        char *e = nullptr;
        const double v = std::strtod(s.c_str(), &e);
        require(e != s.c_str() && std::isfinite(v), "nonfinite basis scale");
        scalings.push_back(v);
    }
    std::string out = "MTP\nversion = 1.1.0\npotential_name = GPM\nscaling = " +
                      text(at(object(bases[0]), "scaling")) + "\nspecies_count = " +
                      std::to_string(ns) + "\npotential_tag = " + json_serialize(metadata) + "\n";
    if (bases.size() > 1)
        out += "radial_basis_split = 1\n";
    for (size_t i = 0; i < bases.size(); ++i) {
        if (bases.size() > 1)
            out += "pair " + std::to_string(i / ns) + " " + std::to_string(i % ns) + "\n";
        print_basis(out, object(bases[i]));
    }
    out += "radial_funcs_count = " + std::to_string(nf) + "\nradial_coeffs\n";
    size_t j = 0;
    for (int a = 0; a < ns; ++a)
        for (int b = 0; b < ns; ++b) {
            out += std::to_string(a) + "-" + std::to_string(b) + "\n";
            for (int f = 0; f < nf; ++f) {
                out += "{";
                for (int k = 0; k < nb; ++k)
                    out += (k ? ", " : "") + g17(radial[j++]);
                out += "}\n";
            }
        }
    auto rules = [&](const std::vector<int32_t> &v) {
        for (size_t i = 0; i < v.size(); i += 4) {
            if (i)
                out += ", ";
            out += "{";
            for (int k = 0; k < 4; ++k)
                out += (k ? ", " : "") + std::to_string(v[i + k]);
            out += "}";
        }
        out += "}\n";
    };
    out += "alpha_moments_count = " + std::to_string(nm) +
           "\nalpha_index_basic_count = " + std::to_string(basic.size() / 4) +
           "\nalpha_index_basic = {";
    rules(basic);
    out += "alpha_index_times_count = " + std::to_string(times.size() / 4) +
           "\nalpha_index_times = {";
    rules(times);
    out += "alpha_scalar_moments = " + std::to_string(mapping.size()) +
           "\nalpha_moment_mapping = {";
    for (size_t i = 0; i < mapping.size(); ++i)
        out += (i ? ", " : "") + std::to_string(mapping[i]);
    out += "}\n";
    auto coefficients = [&](const std::string &name, const std::vector<double> &v) {
        out += name + " = {";
        for (size_t i = 0; i < v.size(); ++i) {
            require(std::isfinite(v[i]), "nonfinite MTP coefficient");
            out += (i ? ", " : "") + g17(v[i]);
        }
        out += "}\n";
    };
    coefficients("species_coeffs", species);
    coefficients("moment_coeffs", moments);
    for (const Json &entry : array(at(c, "head_fields"))) {
        const auto &field = object(entry);
        const std::string &name = text(at(field, "name"));
        if (field.count("array"))
            coefficients(name, r.values(field.at("array")));
        else
            out += name + " = " + text(at(field, "value")) + "\n";
    }
    return out;
}

// ---- writer (GPM::Writer::save, tools/gpm_container.h:563-735) ----------
struct Writer {
    struct Entry {
        std::string dtype;
        std::vector<uint64_t> shape;
        Bytes raw;
    };
    std::map<std::string, Entry> data;  // written in id order, as Writer's std::map

    // vector_block / index_block (tools/gpm_mtp.h:35-50, :87-102): an empty
    // array is described in place, any other becomes a block
    Json add(const std::string &id, const std::string &dtype, std::vector<uint64_t> shape,
             Bytes raw)
    {
        if (raw.empty()) {
            Json o = obj_value(), dims = arr_value();
            for (uint64_t n : shape)
                dims.arr.push_back(count_value(n));
            o.obj["dtype"] = str_value(dtype);
            o.obj["shape"] = dims;
            return o;
        }
        require(!data.count(id), "duplicate block " + id);
        data[id] = Entry{dtype, std::move(shape), std::move(raw)};
        Json o = obj_value();
        o.obj["block"] = str_value(id);
        return o;
    }
    Json f64(const std::string &id, const double *v, size_t n, std::vector<uint64_t> shape = {})
    {
        if (shape.empty())
            shape = {n};
        Bytes b(checked_mul(n, 8));
        for (size_t i = 0; i < n; ++i) {
            uint64_t x;
            std::memcpy(&x, v + i, 8);
            put_le(b.data() + 8 * i, x, 8);
        }
        return add(id, "f64", std::move(shape), std::move(b));
    }
    Json i32(const std::string &id, const int *v, size_t n, std::vector<uint64_t> shape)
    {
        Bytes b(checked_mul(n, 4));
        for (size_t i = 0; i < n; ++i)
            put_le(b.data() + 4 * i, (uint32_t)v[i], 4);
        return add(id, "i32", std::move(shape), std::move(b));
    }

    std::string save(Json manifest, int zstd_level) const
    {
        const Zstd &z = Zstd::get();
        require(zstd_level <= 0 || z.ok, "zstd support is not enabled (libzstd.so.1 not found)");
        Bytes payload;
        Json directory = arr_value();
        for (const auto &kv : data) {
            const Entry &e = kv.second;
            Bytes stored;
            std::string codec = "none";
            if (zstd_level > 0) {
                stored.resize(z.bound(e.raw.size()));
                const size_t n = z.compress(stored.data(), stored.size(), e.raw.data(),
                                            e.raw.size(), zstd_level);
                require(!z.is_error(n), "compression failed");
                stored.resize(n);
                codec = "zstd";
            } else {
                stored = e.raw;
            }
            const uint64_t offset = align64(payload.size());
            payload.resize(offset);
            payload.insert(payload.end(), stored.begin(), stored.end());
            Json b = obj_value(), dims = arr_value();
            for (uint64_t n : e.shape)
                dims.arr.push_back(count_value(n));
            b.obj["id"] = str_value(kv.first);
            b.obj["dtype"] = str_value(e.dtype);
            b.obj["shape"] = dims;
            b.obj["codec"] = str_value(codec);
            b.obj["offset"] = count_value(offset);
            b.obj["stored_size"] = count_value(stored.size());
            b.obj["raw_size"] = count_value(e.raw.size());
            directory.arr.push_back(b);
        }
        manifest.obj["blocks"] = directory;
        const std::string json = json_serialize(manifest);
        require(json.size() <= 64 * 1024 * 1024, "header exceeds limit");
        const uint64_t start = align64(64 + json.size());
        std::string out((size_t)start, '\0');
        std::memcpy(&out[0], "GPMLMODL", 8);
        put_le((unsigned char *)&out[8], 2, 2);
        put_le((unsigned char *)&out[16], json.size(), 8);
        put_le((unsigned char *)&out[24], start, 8);
        std::memcpy(&out[64], json.data(), json.size());
        out.append((const char *)payload.data(), payload.size());
        return out;
    }
};

}  // namespace

bool gpm_is_bundle(const void *bytes, size_t n)
{
    return n >= 8 && std::memcmp(bytes, "GPMLMODL", 8) == 0;
}

bool gpm_read(const void *bytes, size_t n, std::string &out, std::vector<double> &scalings,
              std::string &err)
{
    try {
        Reader r(bytes, n);
        out = node_text(r, scalings);
        return true;
    } catch (const GpmError &e) {
        err = e.msg;
        return false;
    } catch (const std::exception &e) {
        err = std::string("GPM: ") + e.what();
        return false;
    }
}

// encode_builtin + encode_mtp (potentials/gpm_codec.cpp:701-742, :190-312)
// in ModelBundle::encode's manifest (potentials/model_bundle.cpp:23-30).
bool gpm_write(const Model &m, int zstd_level, std::string &out, std::string &err)
{
    try {
        Writer w;
        const std::string id = "root";
        const int Z = m.Z;
        Json node = obj_value();
        node.obj["type"] = str_value(m.linear() ? "mtp" : "mtp_m");
        node.obj["version"] = num_value(1);
        node.obj["children"] = obj_value();
        // AnyPotential's common fields (gpm_codec.cpp common): the pair
        // cutoffs and minimum distances of the bases, zero regularisation
        // vectors of every coefficient (PotMTP::Load, potential_mtp.cpp:
        // 224-291, :643-644)
        std::vector<double> cut((size_t)Z * Z), rmin((size_t)Z * Z), reg((size_t)m.ncoef(), 0.0);
        for (int a = 0; a < Z; ++a)
            for (int b = 0; b < Z; ++b) {
                cut[(size_t)a * Z + b] = m.pair_basis(a, b).rmax;
                rmin[(size_t)a * Z + b] = m.pair_basis(a, b).rmin;
            }
        Json common = obj_value();
        common.obj["species_count"] = num_value(Z);
        common.obj["cutoff"] = num_value(m.rmax);
        common.obj["cutoffs"] = w.f64(id + "/common/cutoffs", cut.data(), cut.size(),
                                      {(uint64_t)Z, (uint64_t)Z});
        common.obj["r_mins"] = w.f64(id + "/common/r_mins", rmin.data(), rmin.size(),
                                     {(uint64_t)Z, (uint64_t)Z});
        Json no;
        no.kind = Json::Bool;
        no.b = false;
        common.obj["add_efs"] = no;
        common.obj["reg_L1"] = w.f64(id + "/common/reg_L1", reg.data(), reg.size());
        common.obj["reg_L2"] = w.f64(id + "/common/reg_L2", reg.data(), reg.size());
        node.obj["common"] = common;
        // species table, with the element symbols of the tag
        std::vector<std::string> names;
        auto el = m.tag.fields.find("elements");
        if (el != m.tag.fields.end() && el->second.kind == Json::Arr)
            for (const Json &x : el->second.arr)
                names.push_back(x.str);
        Json species = arr_value();
        for (int i = 0; i < Z; ++i) {
            Json e = obj_value();
            e.obj["id"] = num_value(i);
            if (i < (int)names.size())
                e.obj["symbol"] = str_value(names[i]);
            species.arr.push_back(e);
        }
        node.obj["species_mode"] = str_value("indexed");
        node.obj["species"] = species;
        // configuration
        Json c = obj_value();
        c.obj["species_count"] = num_value(Z);
        c.obj["radial_functions"] = num_value(m.M);
        c.obj["radial_mode"] = num_value(0);
        c.obj["radial_size"] = num_value(m.R);
        c.obj["moments_count"] = num_value(m.K);
        Json meta;
        std::string jerr;
        require(json_parse(tag_output(m.tag, m.head), meta, jerr), "invalid metadata");
        c.obj["metadata"] = meta;
        Json bases = arr_value();
        for (const RadialBasis &b : m.bases) {
            Json o = obj_value();
            for (const auto &kv : basis_settings(b, m.R))
                o.obj[kv.first] = str_value(kv.second);
            o.obj["scaling"] = str_value(g17(b.scaling));
            bases.arr.push_back(o);
        }
        c.obj["radial_bases"] = bases;
        // the fields PotMTP_M::Save writes after moment_coeffs (its comment
        // lines are not fields)
        Json head = arr_value();
        const double *coef = m.coef.data();
        const int sp = m.nradial(), mo = sp + m.nspecies(), hc = mo + m.nmoment();
        if (!m.linear()) {
            Json f = obj_value();
            f.obj["name"] = str_value("model_coeffs");
            f.obj["array"] = w.f64(id + "/head/model_coeffs", coef + hc, (size_t)m.head.Mc);
            head.arr.push_back(f);
        }
        c.obj["head_fields"] = head;
        node.obj["configuration"] = c;
        // parameters
        Json p = obj_value();
        p.obj["radial"] = w.f64(id + "/radial", coef, (size_t)sp);
        p.obj["species"] = w.f64(id + "/species", coef + sp, (size_t)m.nspecies());
        p.obj["moments"] = w.f64(id + "/moments", coef + mo, (size_t)m.nmoment());
        p.obj["basic_indices"] =
            w.i32(id + "/basic_indices", m.basic.data(), m.basic.size(), {(uint64_t)m.B, 4});
        p.obj["product_indices"] =
            w.i32(id + "/product_indices", m.times.data(), m.times.size(), {(uint64_t)m.T, 4});
        p.obj["scalar_mapping"] =
            w.i32(id + "/scalar_mapping", m.map.data(), m.map.size(), {(uint64_t)m.S});
        node.obj["parameters"] = p;
        // manifest (Writer's defaults and ModelBundle::encode's species)
        Json manifest = obj_value(), units = obj_value(), models = obj_value();
        units.obj["length"] = str_value("angstrom");
        units.obj["energy"] = str_value("eV");
        units.obj["charge"] = str_value("e");
        units.obj["stress"] = str_value("virial_eV");
        manifest.obj["schema"] = str_value("gpml.model");
        manifest.obj["units"] = units;
        manifest.obj["species"] = species;
        manifest.obj["root_model"] = str_value(id);
        models.obj[id] = node;
        manifest.obj["models"] = models;
        out = w.save(manifest, zstd_level);
        return true;
    } catch (const GpmError &e) {
        err = e.msg;
        return false;
    } catch (const std::exception &e) {
        err = std::string("GPM: ") + e.what();
        return false;
    }
}

}  // namespace mtpx
