// mtpx_calc_efs: the calc_efs front end (apps/calc_efs.cpp:179-389, the
// --device=hip branch) over the C ABI.  Reads structures in the text MLIP
// configuration format (io/gpio_read_cfg.cpp:319-615) or a VASP POSCAR
// (GPIO::read_vasp_poscar, io/gpio_read_vasp.cpp:1108-1234), evaluates
// energy, forces, stress and site energies on the device in
// structure-preserving chunks (mtpx_set_structures + mtpx_compute_batch, or
// mtpx_energy with --energy-only), and writes the configurations back
// (GPIO::write_next_mlpcfg, io/gpio_write.cpp:224-380).
//
//   mtpx_calc_efs --pot potential.mtp|.gpm --in input.cfg|POSCAR --out output-efs.cfg
//       [--input-format cfg|POSCAR|bin] [--index index.map]
//       [--energy-only] [--no-site-energy] [--lossless] [--show-progress]
//       [--gpu-id K] [--gpu-batch-atoms N] [--gpu-batch-structures N]
//       [--deterministic]
//
// Binary configurations (io/gpio_binary.h, GPIO::load_next_from_mlpcfg_binary,
// io/gpio_read_cfg.cpp:38-316) are read too.  The input format is the one
// named (cfg, POSCAR, bin), else bin when the file starts with GPMLBIN2, cfg
// when it holds BEGIN_CFG, else POSCAR.  POSCAR element names become species through the
// reference's species map (GPIO::install_species_map, io/gpio.cpp:103-200):
// the index file (one element per line, in species order; index.map by
// default) when it exists, else the element order the potential declares
// (its potential_tag "elements"), else the periodic table (an element's
// species is its atomic number); a named index file that is missing is an
// error unless the potential declares its elements.
//
// Read: BEGIN_CFG, Size, an optional Supercell of three rows (periodic in
// all three directions; without it the structure is a cluster), AtomData
// with the columns id, type, cartes_x/y/z (or x/y/z) and any others (kept
// by name), Energy, PlusStress (xx yy zz yz xz xy), Feature lines (kept
// verbatim), END_CFG.  Types are species indices 0 .. Z-1.
// Written: the reference's fixed-width form ({:>15.8g}, printf "%15.8g"),
// or with --lossless numbers that read back to the same doubles ("%.17g";
// the reference prints the shortest such form).  Energy, forces, stress and
// site energies are replaced by the computed ones; --energy-only writes the
// energy and drops forces, stress and site energies, --no-site-energy drops
// the site energies.
#include "mtpx.h"

#include <algorithm>
#include <climits>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

namespace {

struct Config {
    int n = 0;
    bool periodic = false;  // all three axes (text cfg with a Supercell, POSCAR)
    int pbc[3] = {0, 0, 0};
    double cell[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    std::vector<int> type;
    std::vector<double> pos;              // [n][3]
    std::vector<std::string> extra_names; // other AtomData columns
    std::vector<double> extra;            // [n][extra]
    std::vector<std::string> features;    // "Feature ..." lines, verbatim
    double energy = 0;
    double stress[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    std::vector<double> force, site;      // computed
};

[[noreturn]] void die(const std::string &msg)
{
    std::fprintf(stderr, "mtpx_calc_efs: %s\n", msg.c_str());
    std::exit(1);
}

std::vector<std::string> split(const std::string &line)
{
    std::istringstream is(line);
    std::vector<std::string> out;
    std::string t;
    while (is >> t)
        out.push_back(t);
    return out;
}

bool number(const std::string &s, double &v)
{
    char *end = nullptr;
    v = std::strtod(s.c_str(), &end);
    return end && *end == 0 && end != s.c_str() && std::isfinite(v);
}

// GPIO::load_next_from_mlpcfg: false at a clean end of input, dies on a
// malformed configuration.
bool read_config(std::istream &is, Config &c, int index)
{
    std::string line;
    bool begin = false;
    while (std::getline(is, line))
        if (line.find("BEGIN_CFG") != std::string::npos) {
            begin = true;
            break;
        }
    if (!begin)
        return false;
    const std::string where = "configuration " + std::to_string(index) + ": ";
    double v = 0;
    if (!std::getline(is, line) || !std::getline(is, line))
        die(where + "missing Size");
    {
        auto t = split(line);
        if (t.empty() || !number(t[0], v) || v < 0 || v != std::floor(v) || v > INT_MAX)
            die(where + "invalid Size");
        c.n = (int)v;
    }
    if (!std::getline(is, line))
        die(where + "truncated");
    if (line.find("Supercell") != std::string::npos) {
        c.periodic = true;
        c.pbc[0] = c.pbc[1] = c.pbc[2] = 1;
        for (int a = 0; a < 3; ++a) {
            if (!std::getline(is, line))
                die(where + "truncated Supercell");
            auto t = split(line);
            if (t.size() < 3)
                die(where + "invalid Supercell row");
            for (int b = 0; b < 3; ++b)
                if (!number(t[b], c.cell[3 * a + b]))
                    die(where + "invalid Supercell row");
        }
        if (!std::getline(is, line))
            die(where + "truncated");
    }
    auto head = split(line);
    if (head.empty() || head[0] != "AtomData:")
        die(where + "missing AtomData");
    int col_id = -1, col_type = -1, col_x = -1, col_y = -1, col_z = -1;
    std::vector<int> extra_cols;
    const std::vector<std::string> computed = {"fx", "fy", "fz", "site_en"};
    for (size_t k = 1; k < head.size(); ++k) {
        const std::string &h = head[k];
        const int col = (int)k - 1;
        if (h == "id")
            col_id = col;
        else if (h == "type")
            col_type = col;
        else if (h == "cartes_x" || h == "x")
            col_x = col;
        else if (h == "cartes_y" || h == "y")
            col_y = col;
        else if (h == "cartes_z" || h == "z")
            col_z = col;
        else if (std::find(computed.begin(), computed.end(), h) == computed.end()) {
            c.extra_names.push_back(h);
            extra_cols.push_back(col);
        }
    }
    if (col_x < 0 || col_y < 0 || col_z < 0)
        die(where + "AtomData needs cartes_x cartes_y cartes_z");
    const int ncol = (int)head.size() - 1;
    c.type.assign(c.n, 0);
    c.pos.assign(3 * (size_t)c.n, 0.0);
    c.extra.assign((size_t)c.n * extra_cols.size(), 0.0);
    std::vector<char> seen(c.n, 0);
    for (int i = 0; i < c.n; ++i) {
        if (!std::getline(is, line))
            die(where + "truncated AtomData");
        auto t = split(line);
        if ((int)t.size() < ncol)
            die(where + "short AtomData row");
        std::vector<double> val(ncol);
        for (int k = 0; k < ncol; ++k)
            if (!number(t[k], val[k]))
                die(where + "invalid AtomData value");
        int id = i;
        if (col_id >= 0) {
            const double d = val[col_id];
            if (d != std::floor(d) || d < 1 || d > c.n || seen[(int)d - 1])
                die(where + "invalid atom id");
            id = (int)d - 1;
        }
        seen[id] = 1;
        if (col_type >= 0) {
            const double d = val[col_type];
            if (d != std::floor(d) || d < 0 || d > 1e9)
                die(where + "invalid atom type");
            c.type[id] = (int)d;
        }
        c.pos[3 * (size_t)id] = val[col_x];
        c.pos[3 * (size_t)id + 1] = val[col_y];
        c.pos[3 * (size_t)id + 2] = val[col_z];
        for (size_t e = 0; e < extra_cols.size(); ++e)
            c.extra[(size_t)id * extra_cols.size() + e] = val[extra_cols[e]];
    }
    while (std::getline(is, line)) {
        auto t = split(line);
        if (t.empty())
            continue;
        if (t[0] == "END_CFG")
            return true;
        if (t[0] == "Energy" || t[0] == "energy" || t[0] == "PlusStress:" ||
            t[0] == "plusstress:" || t[0] == "Stress:" || t[0] == "stress:") {
            if (!std::getline(is, line))  // the label values are replaced
                die(where + "truncated");
        } else if (t[0] == "Feature" || t[0] == "feature") {
            c.features.push_back(line);
        }
    }
    die(where + "missing END_CFG");
}

// ---- POSCAR --------------------------------------------------------------

// Element symbols by atomic number ("X" for 0), the periodic-table map.
const char *const kElements[] = {
    "X",  "H",  "He", "Li", "Be", "B",  "C",  "N",  "O",  "F",  "Ne", "Na", "Mg", "Al", "Si",
    "P",  "S",  "Cl", "Ar", "K",  "Ca", "Sc", "Ti", "V",  "Cr", "Mn", "Fe", "Co", "Ni", "Cu",
    "Zn", "Ga", "Ge", "As", "Se", "Br", "Kr", "Rb", "Sr", "Y",  "Zr", "Nb", "Mo", "Tc", "Ru",
    "Rh", "Pd", "Ag", "Cd", "In", "Sn", "Sb", "Te", "I",  "Xe", "Cs", "Ba", "La", "Ce", "Pr",
    "Nd", "Pm", "Sm", "Eu", "Gd", "Tb", "Dy", "Ho", "Er", "Tm", "Yb", "Lu", "Hf", "Ta", "W",
    "Re", "Os", "Ir", "Pt", "Au", "Hg", "Tl", "Pb", "Bi", "Po", "At", "Rn", "Fr", "Ra", "Ac",
    "Th", "Pa", "U",  "Np", "Pu", "Am", "Cm", "Bk", "Cf", "Es", "Fm", "Md", "No", "Lr", "Rf",
    "Db", "Sg", "Bh", "Hs", "Mt", "Ds", "Rg", "Cn", "Nh", "Fl", "Mc", "Lv", "Ts", "Og"};

// The element list of a potential_tag's "elements" array in .mtp text
// (empty when there is none).
std::vector<std::string> model_elements(const std::string &mtp_text)
{
    std::vector<std::string> out;
    const size_t tag = mtp_text.find("potential_tag");
    if (tag == std::string::npos)
        return out;
    const size_t eol = mtp_text.find('\n', tag);
    const std::string line = mtp_text.substr(tag, eol == std::string::npos ? std::string::npos
                                                                             : eol - tag);
    const size_t key = line.find("\"elements\"");
    if (key == std::string::npos)
        return out;
    const size_t open = line.find('[', key), close = line.find(']', key);
    if (open == std::string::npos || close == std::string::npos || close < open)
        return out;
    const std::string body = line.substr(open + 1, close - open - 1);
    for (size_t q = body.find('"'); q != std::string::npos;) {
        const size_t e = body.find('"', q + 1);
        if (e == std::string::npos)
            break;
        out.push_back(body.substr(q + 1, e - q - 1));
        q = body.find('"', e + 1);
    }
    return out;
}

// install_species_map: element name -> species.
std::vector<std::string> species_names(const std::string &index, bool index_named,
                                       const std::vector<std::string> &declared)
{
    std::ifstream f(index);
    if (f) {
        // GPIO::readmap: the first word of each line, species in line order
        std::vector<std::string> names;
        std::string line;
        while (std::getline(f, line)) {
            auto t = split(line);
            if (t.empty())
                break;
            names.push_back(t[0]);
        }
        if (names.empty())
            die("cannot read species map: " + index);
        return names;
    }
    bool valid = !declared.empty();
    for (size_t k = 0; k < declared.size() && valid; ++k) {
        valid = std::find(std::begin(kElements) + 1, std::end(kElements), declared[k]) !=
                std::end(kElements);
        for (size_t q = 0; q < k && valid; ++q)
            valid = declared[q] != declared[k];
    }
    if (valid) {
        if (index_named)
            std::fprintf(stderr,
                         "mtpx_calc_efs: index file \"%s\" not found; using the element order "
                         "declared by the model\n",
                         index.c_str());
        return declared;
    }
    if (index_named)
        die("index file \"" + index +
            "\" not found and the model does not declare an element order");
    std::fprintf(stderr,
                 "mtpx_calc_efs: index file \"%s\" not found; using the periodic table\n",
                 index.c_str());
    return std::vector<std::string>(std::begin(kElements), std::end(kElements));
}

// GPIO::read_vasp_poscar: one periodic structure.  The scale multiplies the
// cell, or, negative, sets its volume; an optional "Selective dynamics" line
// (its per-atom flags are read and dropped) precedes Cartesian (C, K) or
// Direct (D, F) coordinates; direct coordinates are turned into Cartesian
// ones (row vector times the cell, rows the lattice vectors).
Config read_poscar(std::istream &is, const std::vector<std::string> &names)
{
    Config c;
    c.periodic = true;
    c.pbc[0] = c.pbc[1] = c.pbc[2] = 1;
    std::string line;
    auto need = [&](const char *what) {
        if (!std::getline(is, line))
            die(std::string("POSCAR: missing ") + what);
    };
    need("comment line");
    need("scale");
    double scale = 0;
    {
        bool found = false;
        for (const auto &t : split(line))
            if (number(t, scale)) {
                found = true;
                break;
            }
        if (!found)
            die("POSCAR: invalid scale");
    }
    for (int a = 0; a < 3; ++a) {
        need("lattice vector");
        auto t = split(line);
        if (t.size() < 3)
            die("POSCAR: invalid lattice vector");
        for (int b = 0; b < 3; ++b)
            if (!number(t[b], c.cell[3 * a + b]))
                die("POSCAR: invalid lattice vector");
    }
    double f = scale;
    if (scale <= 0) {
        const double *m = c.cell;
        const double det = m[0] * (m[4] * m[8] - m[5] * m[7]) -
                           m[1] * (m[3] * m[8] - m[5] * m[6]) +
                           m[2] * (m[3] * m[7] - m[4] * m[6]);
        f = std::pow(-scale / std::fabs(det), 1.0 / 3.0);
    }
    for (double &v : c.cell)
        v *= f;
    need("element names");
    std::vector<int> chem;
    for (const auto &t : split(line)) {
        const auto it = std::find(names.begin(), names.end(), t);
        if (it == names.end())
            die("POSCAR: element " + t + " is not in the species map");
        chem.push_back((int)(it - names.begin()));
    }
    need("element counts");
    {
        auto t = split(line);
        if (t.size() < chem.size())
            die("POSCAR: missing element counts");
        for (size_t k = 0; k < chem.size(); ++k) {
            double v = 0;
            if (!number(t[k], v) || v < 0 || v != std::floor(v) || c.n + v > INT_MAX)
                die("POSCAR: invalid element count");
            c.type.insert(c.type.end(), (size_t)v, chem[k]);
            c.n += (int)v;
        }
    }
    need("coordinate mode");
    auto mode = [&]() {
        auto t = split(line);
        return t.empty() ? '?' : (char)std::toupper((unsigned char)t[0][0]);
    };
    char flag = mode();
    const bool selective = flag == 'S';
    if (selective) {
        need("coordinate mode");
        flag = mode();
    }
    bool direct;
    if (flag == 'C' || flag == 'K')
        direct = false;
    else if (flag == 'D' || flag == 'F')
        direct = true;
    else
        die("POSCAR: unknown POSCAR format");
    c.pos.assign(3 * (size_t)c.n, 0.0);
    for (int i = 0; i < c.n; ++i) {
        need("position");
        auto t = split(line);
        if (t.size() < (selective ? 6u : 3u))
            die(selective ? "POSCAR: no selective dynamics info given" : "POSCAR: short position");
        double p[3];
        for (int a = 0; a < 3; ++a)
            if (!number(t[a], p[a]))
                die("POSCAR: invalid position");
        for (int a = 3; selective && a < 6; ++a) {
            const char q = (char)std::toupper((unsigned char)t[a][0]);
            if (q != 'T' && q != 'F')
                die("POSCAR: unknown selective dynamics info " + t[a]);
        }
        for (int b = 0; b < 3; ++b)
            c.pos[3 * (size_t)i + b] =
                direct ? (p[0] * c.cell[b] + p[1] * c.cell[3 + b]) + p[2] * c.cell[6 + b] : p[b];
    }
    return c;
}

// ---- binary configurations ---------------------------------------------
//
// GPIO::load_next_from_mlpcfg_binary (io/gpio_read_cfg.cpp:38-316) over the
// frame layout of io/gpio_binary.h: "GPMLBIN2", a uint32 version (2 or 3)
// and an int32 atom count, then tagged records up to '#'.  The cell is
// written as Eigen stores a 3 x 3 matrix (column-major, the rows of the
// reference's cell being lattice vectors); positions are 3 doubles per atom,
// types an int32 per atom, the periodicity three bytes (version 2 has none
// and is periodic).  The other records (forces, energies, stresses, per-atom
// and global attributes) are read past; Feature records are kept.
template <class T>
bool get(std::istream &is, T &v)
{
    return (bool)is.read(reinterpret_cast<char *>(&v), sizeof v);
}

bool skip(std::istream &is, long long bytes)
{
    if (bytes < 0)
        return false;
    is.ignore(bytes);
    return is.gcount() == bytes;
}

bool get_string(std::istream &is, std::string &v)
{
    int32_t n = 0;
    if (!get(is, n) || n < 0 || n > (1 << 20))
        return false;
    v.resize((size_t)n);
    return n == 0 || (bool)is.read(&v[0], n);
}

// false at a clean end of input; dies on a malformed frame.
bool read_binary(std::istream &is, Config &c, int index)
{
    if (is.peek() == std::char_traits<char>::eof())
        return false;
    const std::string where = "binary configuration " + std::to_string(index) + ": ";
    char magic[8];
    uint32_t version = 0;
    int32_t natoms = 0;
    if (!is.read(magic, 8) || std::memcmp(magic, "GPMLBIN2", 8) != 0 || !get(is, version) ||
        !get(is, natoms) || version < 2 || version > 3 || natoms < 0 || natoms > (1 << 28) / 3)
        die(where + "invalid binary mlpcfg header");
    c.n = natoms;
    c.type.assign((size_t)natoms, 0);
    c.pos.assign(3 * (size_t)natoms, 0.0);
    bool has_cell = false, has_pos = false, has_pbc = false;
    const long long n = natoms;
    for (;;) {
        char tag = 0;
        if (!get(is, tag))
            die(where + "truncated");
        bool ok = true;
        std::string name, value;
        int32_t rows = 0;
        switch (tag) {
        case 'l': {
            double m[9];
            ok = (bool)is.read(reinterpret_cast<char *>(m), sizeof m);
            for (int i = 0; i < 3; ++i)
                for (int j = 0; j < 3; ++j)
                    c.cell[3 * i + j] = m[i + 3 * j];
            has_cell = true;
            break;
        }
        case 'p':
            ok = n == 0 || (bool)is.read(reinterpret_cast<char *>(c.pos.data()),
                                         (std::streamsize)(sizeof(double) * 3 * n));
            has_pos = true;
            break;
        case 't':
            ok = n == 0 || (bool)is.read(reinterpret_cast<char *>(c.type.data()),
                                         (std::streamsize)(sizeof(int32_t) * n));
            break;
        case 'b': {
            uint8_t f[3];
            ok = (bool)is.read(reinterpret_cast<char *>(f), 3);
            for (int d = 0; d < 3 && ok; ++d) {
                ok = f[d] <= 1;
                c.pbc[d] = f[d];
            }
            has_pbc = true;
            break;
        }
        case 'f': case 'm': case 'u': ok = skip(is, 24 * n); break;      // 3 doubles per atom
        case 'v': case 'M': case 'c': ok = skip(is, 8 * n); break;       // a double per atom
        case 'i': ok = skip(is, 4 * n); break;                           // an int per atom
        case 'h': case 'e': ok = skip(is, 8); break;
        case 's': ok = skip(is, 72); break;
        case 'F':
            ok = get_string(is, name) && get_string(is, value);
            if (ok)
                c.features.push_back("Feature   " + name + "\t" + value);
            break;
        case 'A': ok = get_string(is, name) && skip(is, 8 * n); break;
        case 'H': ok = get_string(is, name) && skip(is, 4 * n); break;
        case 'B': case 'I':
            ok = get_string(is, name) && get(is, rows) && rows >= 0 && rows <= (1 << 28) &&
                 (n == 0 || rows <= (1 << 28) / n) &&
                 skip(is, (tag == 'B' ? 8LL : 4LL) * rows * n);
            break;
        case 'C': ok = get_string(is, name) && skip(is, 8); break;
        case 'E': ok = get_string(is, name) && skip(is, 4); break;
        case 'D': case 'G':
            ok = get_string(is, name) && get(is, rows) && rows >= 0 && rows <= (1 << 28) &&
                 skip(is, (tag == 'D' ? 8LL : 4LL) * rows);
            break;
        case '#':
            if (!has_cell || !has_pos)
                die(where + "no cell or positions");
            if (!has_pbc)  // version 2: periodic
                c.pbc[0] = c.pbc[1] = c.pbc[2] = 1;
            c.periodic = c.pbc[0] && c.pbc[1] && c.pbc[2];
            return true;
        default:
            die(where + "unsupported binary mlpcfg tag " + std::string(1, tag));
        }
        if (!ok)
            die(where + "truncated or invalid record '" + std::string(1, tag) + "'");
    }
}

void write_num(std::ostream &os, double v, bool lossless, bool lead_space = true)
{
    char buf[64];
    std::snprintf(buf, sizeof buf, lossless ? "%.17g" : "%15.8g", v);
    if (lead_space)
        os << ' ';
    os << buf;
}

// GPIO::write_next_mlpcfg (io/gpio_write.cpp:224-380).
void write_config(std::ostream &os, const Config &c, bool lossless, bool energy_only,
                  bool site_energy)
{
    os << "BEGIN_CFG\nSize\n" << c.n << "\nSupercell\n";
    for (int a = 0; a < 3; ++a) {
        for (int b = 0; b < 3; ++b)
            write_num(os, c.cell[3 * a + b], lossless, b > 0);
        os << '\n';
    }
    const bool forces = !energy_only, site = !energy_only && site_energy;
    os << "AtomData: id type  cartes_x cartes_y cartes_z";
    if (site)
        os << " site_en";
    if (forces)
        os << " fx fy fz";
    for (const auto &name : c.extra_names)
        os << ' ' << name;
    os << '\n';
    const size_t ne = c.extra_names.size();
    for (int i = 0; i < c.n; ++i) {
        char buf[64];
        if (lossless)
            std::snprintf(buf, sizeof buf, "%d %d", i + 1, c.type[i]);
        else
            std::snprintf(buf, sizeof buf, " %-6d %-6d", i + 1, c.type[i]);
        os << buf;
        for (int a = 0; a < 3; ++a)
            write_num(os, c.pos[3 * (size_t)i + a], lossless);
        if (site)
            write_num(os, c.site[i], lossless);
        if (forces)
            for (int a = 0; a < 3; ++a)
                write_num(os, c.force[3 * (size_t)i + a], lossless);
        for (size_t e = 0; e < ne; ++e)
            write_num(os, c.extra[(size_t)i * ne + e], lossless);
        os << '\n';
    }
    os << "Energy\n";
    write_num(os, c.energy, lossless, !lossless);
    os << '\n';
    if (!energy_only) {
        os << "PlusStress: xx yy zz yz xz xy\n";
        const int order[6] = {0, 4, 8, 5, 2, 1};
        for (int k = 0; k < 6; ++k)
            write_num(os, c.stress[order[k]], lossless, k > 0 || !lossless);
        os << '\n';
    }
    for (const auto &f : c.features)
        os << f << '\n';
    os << "END_CFG\n\n";
}

void check(mtpx_context *ctx, int rc, const char *what)
{
    if (rc != MTPX_OK)
        die(std::string(what) + ": " + (ctx ? mtpx_last_error(ctx) : "error"));
}

}  // namespace

int main(int argc, char **argv)
{
    std::string pot = "potential.mtp", in = "POSCAR", out = "output-efs.cfg";
    std::string informat, index = "index.map";
    bool index_named = false;
    bool energy_only = false, site_energy = true, lossless = false, progress = false;
    bool deterministic = false;
    int gpu = 0;
    long batch_atoms = 0, batch_structures = 0;
    for (int k = 1; k < argc; ++k) {
        const std::string a = argv[k];
        auto value = [&]() -> std::string {
            if (k + 1 >= argc)
                die("missing value for " + a);
            return argv[++k];
        };
        if (a == "--pot" || a == "--potfile")
            pot = value();
        else if (a == "--in" || a == "--input")
            in = value();
        else if (a == "--out" || a == "--output")
            out = value();
        else if (a == "--input-format" || a == "--if")
            informat = value();
        else if (a == "--index" || a == "--id") {
            index = value();
            index_named = true;
        }
        else if (a == "--energy-only")
            energy_only = true;
        else if (a == "--no-site-energy")
            site_energy = false;
        else if (a == "--lossless")
            lossless = true;
        else if (a == "--show-progress")
            progress = true;
        else if (a == "--deterministic")
            deterministic = true;
        else if (a == "--gpu-id")
            gpu = std::atoi(value().c_str());
        else if (a == "--gpu-batch-atoms")
            batch_atoms = std::atol(value().c_str());
        else if (a == "--gpu-batch-structures")
            batch_structures = std::atol(value().c_str());
        else if (a == "-h" || a == "--help") {
            std::puts("mtpx_calc_efs --pot F.mtp --in F.cfg|POSCAR --out F.cfg "
                      "[--input-format cfg|POSCAR|bin] [--index index.map] [--energy-only] "
                      "[--no-site-energy] [--lossless] [--show-progress] [--deterministic] "
                      "[--gpu-id K] [--gpu-batch-atoms N] [--gpu-batch-structures N]");
            return 0;
        } else
            die("unknown option " + a);
    }
    if (batch_atoms < 0 || batch_structures < 0)
        die("GPU batch limits must be zero (automatic) or positive");
    if (gpu < 0)
        gpu = 0;

    std::ifstream pf(pot, std::ios::binary);
    if (!pf)
        die("cannot read " + pot);
    const std::string text((std::istreambuf_iterator<char>(pf)), {});
    std::ifstream inf(in);
    if (!inf)
        die("cannot read " + in);
    std::string fmt = informat;
    for (char &ch : fmt)
        ch = (char)std::tolower((unsigned char)ch);
    if (fmt.empty()) {
        // the format by content: a binary configuration starts with its
        // magic, a text one holds BEGIN_CFG, anything else is a POSCAR
        std::string head(4096, '\0');
        inf.read(&head[0], (std::streamsize)head.size());
        head.resize((size_t)inf.gcount());
        fmt = head.compare(0, 8, "GPMLBIN2") == 0        ? "bin"
              : head.find("BEGIN_CFG") != std::string::npos ? "cfg"
                                                           : "poscar";
        inf.clear();
        inf.seekg(0);
    }
    const bool poscar = fmt == "poscar" || fmt == "vasp" || fmt == "contcar";
    const bool binary = fmt == "bin" || fmt == "binary" || fmt == "cfgbin";
    if (!poscar && !binary && fmt != "cfg" && fmt != "mlip" && fmt != "mlp")
        die("unknown input format " + informat);

    mtpx_context *ctx = nullptr;
    check(nullptr, mtpx_create(gpu, &ctx), "mtpx_create");
    // a GPM bundle (by its magic, as GPM::is_file) or .mtp text
    const bool gpm = text.size() >= 8 && text.compare(0, 8, "GPMLMODL") == 0;
    if (gpm)
        check(ctx, mtpx_load_model_gpm(ctx, text.data(), text.size()), "load potential");
    else
        check(ctx, mtpx_load_model_text(ctx, text.c_str()), "load potential");

    std::vector<Config> cfgs;
    if (poscar) {
        // the element order the model declares, from its saved text
        size_t len = 0;
        check(ctx, mtpx_save_model_text(ctx, nullptr, 0, &len), "model text");
        std::string saved(len + 1, '\0');
        check(ctx, mtpx_save_model_text(ctx, &saved[0], saved.size(), &len), "model text");
        saved.resize(len);
        cfgs.push_back(read_poscar(inf, species_names(index, index_named, model_elements(saved))));
    } else {
        for (;;) {
            Config c;
            if (!(binary ? read_binary(inf, c, (int)cfgs.size())
                         : read_config(inf, c, (int)cfgs.size())))
                break;
            cfgs.push_back(std::move(c));
        }
    }
    int info[8];
    check(ctx, mtpx_model_info(ctx, info), "model info");
    double cutoff = 0;
    check(ctx, mtpx_model_cutoff(ctx, &cutoff), "model cutoff");
    for (size_t c = 0; c < cfgs.size(); ++c)
        for (int t : cfgs[c].type)
            if (t >= info[0])
                die("configuration " + std::to_string(c) + ": type " + std::to_string(t) +
                    " but the potential has " + std::to_string(info[0]) + " species");

    // structure-preserving chunks: at most batch_atoms atoms (2^21 by
    // default) and batch_structures structures
    const long max_atoms = batch_atoms > 0 ? batch_atoms : (1L << 21);
    size_t done = 0, chunks = 0, total_atoms = 0;
    for (size_t c0 = 0; c0 < cfgs.size();) {
        size_t c1 = c0;
        long atoms = 0;
        while (c1 < cfgs.size() && (c1 == c0 || atoms + cfgs[c1].n <= max_atoms) &&
               (batch_structures == 0 || (long)(c1 - c0) < batch_structures))
            atoms += cfgs[c1++].n;
        const int nconf = (int)(c1 - c0);
        std::vector<int> off(nconf + 1, 0), pbc(3 * (size_t)nconf), types;
        std::vector<double> cells(9 * (size_t)nconf), pos;
        for (int k = 0; k < nconf; ++k) {
            Config &c = cfgs[c0 + k];
            off[k + 1] = off[k] + c.n;
            for (int q = 0; q < 9; ++q)
                cells[9 * (size_t)k + q] = c.cell[q];
            for (int a = 0; a < 3; ++a)
                pbc[3 * (size_t)k + a] = c.pbc[a] ? 1 : 0;
            // Atoms::wrap before the lists (calc_efs.cpp:195), along the
            // periodic axes, as the reference writes the wrapped positions back
            if (c.pbc[0] || c.pbc[1] || c.pbc[2])
                check(ctx, mtpx_wrap(c.cell, &pbc[3 * (size_t)k], c.n, c.pos.data()), "wrap");
            pos.insert(pos.end(), c.pos.begin(), c.pos.end());
            types.insert(types.end(), c.type.begin(), c.type.end());
        }
        check(ctx, mtpx_set_structures(ctx, nconf, off.data(), cells.data(), pbc.data(),
                                       pos.data(), types.data(), cutoff),
              "neighbour lists");
        std::vector<double> E(nconf), F(3 * (size_t)atoms), S(9 * (size_t)nconf), se(atoms);
        if (energy_only)
            check(ctx, mtpx_energy(ctx, E.data(), nullptr), "energy");
        else
            check(ctx, mtpx_compute_batch(ctx, deterministic ? 1 : 0, E.data(), F.data(),
                                          S.data(), se.data()),
                  "evaluation");
        for (int k = 0; k < nconf; ++k) {
            Config &c = cfgs[c0 + k];
            c.energy = E[k];
            if (!energy_only) {
                c.force.assign(F.begin() + 3 * (size_t)off[k], F.begin() + 3 * (size_t)off[k + 1]);
                c.site.assign(se.begin() + off[k], se.begin() + off[k + 1]);
                std::memcpy(c.stress, &S[9 * (size_t)k], sizeof c.stress);
            }
        }
        total_atoms += (size_t)atoms;
        ++chunks;
        done += nconf;
        if (progress)
            std::fprintf(stderr, "Calculated EFS %zu/%zu\n", done, cfgs.size());
        c0 = c1;
    }
    std::ofstream of(out);
    if (!of)
        die("cannot write " + out);
    for (const Config &c : cfgs)
        write_config(of, c, lossless, energy_only, site_energy);
    of.close();
    if (!of)
        die("error writing " + out);
    std::fprintf(stderr, "mtpx_calc_efs: %zu structures, %zu atoms in %zu chunk(s)\n",
                 cfgs.size(), total_atoms, chunks);
    mtpx_destroy(ctx);
    return 0;
}
