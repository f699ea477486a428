// Driver for the reference MTP-M site executor (runtime/mtp/cpu/mtp_cpu.cpp,
// over the core reader runtime/mtp/mlip.cpp and
// runtime/mtp/radial_basis_setup.cpp), compiled from the reference sources by
// oracle/Makefile into oracle/_ref/mtpm_ref.  Test infrastructure only.
//
// MLIPCore::setup reads the potential with its MTP-M metadata and head
// coefficients; Cpu::Executor::evaluate_site gives each centre's energy and
// the gradient of that energy with respect to each neighbour's displacement.
// The driver lists neighbours by brute force over owned atoms and periodic
// images (ghosts), folds ghost forces back onto their owners and sums the
// virial as MLIPCore::compute does (mlip.cpp:1164-1190): v = -sum g (x) r,
// symmetrised, in the order xx yy zz xy xz yz.
//
// usage: mtpm_ref <model.mtp> <in.bin> <out.bin>
//   in : int32 Z | int32 npts | int32 n | f64 cutoff | f64 pts[npts][3] |
//        int32 type[npts] | int32 orig[npts]
//   out: f64 energy | f64 site_energy[n] | f64 force[n][3] | f64 virial[6]
#include "mtp_cpu.h"

#include <cstdint>
#include <cstdio>
#include <exception>
#include <vector>

int main(int argc, char **argv)
try
{
    if (argc != 4)
        return 2;
    FILE *f = std::fopen(argv[2], "rb");
    if (!f)
        return 3;
    int32_t Z, npts, n;
    double cutoff;
    if (std::fread(&Z, 4, 1, f) != 1 || std::fread(&npts, 4, 1, f) != 1 ||
        std::fread(&n, 4, 1, f) != 1 || std::fread(&cutoff, 8, 1, f) != 1)
        return 4;
    std::vector<double> pts(3 * (size_t)npts);
    std::vector<int32_t> type(npts), orig(npts);
    if (std::fread(pts.data(), 8, pts.size(), f) != pts.size() ||
        std::fread(type.data(), 4, type.size(), f) != type.size() ||
        std::fread(orig.data(), 4, orig.size(), f) != orig.size())
        return 5;
    std::fclose(f);

    std::vector<int> sp(Z);
    for (int t = 0; t < Z; ++t)
        sp[t] = t;
    double model_cutoff = 0;
    MLIPCore::Cpu::Model pot(MLIPCore::setup(argv[1], sp.data(), &model_cutoff, (std::size_t)Z));
    MLIPCore::Cpu::Executor exec(*pot);
    MLIPCore::Cpu::Workspace ws(*pot);

    const double rc2 = cutoff * cutoff;
    std::vector<const double *> x(npts);
    for (int p = 0; p < npts; ++p)
        x[p] = &pts[3 * p];
    std::vector<int> list;
    std::vector<double> site(n, 0.0), fold(3 * (size_t)n, 0.0);
    double energy = 0, vir[6] = {0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n; ++i)
    {
        list.clear();
        for (int p = 0; p < npts; ++p)
        {
            if (p == i)
                continue;
            const double d0 = pts[3 * p] - pts[3 * i], d1 = pts[3 * p + 1] - pts[3 * i + 1],
                         d2 = pts[3 * p + 2] - pts[3 * i + 2];
            if (d0 * d0 + d1 * d1 + d2 * d2 < rc2)
                list.push_back(p);
        }
        ws.reserve(*pot, list.size(), MLIPCore::Cpu::DerivativeMode::Cached);
        const double e = exec.evaluate_site(i, (int)list.size(), list.data(), type.data(),
                                            x.data(), sp.data(), true, true, ws);
        site[i] = e;
        energy += e;
        for (int k = 0; k < ws.edge_count(); ++k)
        {
            const int j = orig[ws.neighbor(k)];
            const double *g = ws.gradient(k), *r = ws.displacement(k);
            for (int a = 0; a < 3; ++a)
            {
                fold[3 * (size_t)i + a] += g[a];
                fold[3 * (size_t)j + a] -= g[a];
            }
            vir[0] -= g[0] * r[0];
            vir[1] -= g[1] * r[1];
            vir[2] -= g[2] * r[2];
            vir[3] -= 0.5 * (g[1] * r[0] + g[0] * r[1]);
            vir[4] -= 0.5 * (g[2] * r[0] + g[0] * r[2]);
            vir[5] -= 0.5 * (g[2] * r[1] + g[1] * r[2]);
        }
    }
    FILE *o = std::fopen(argv[3], "wb");
    if (!o)
        return 6;
    std::fwrite(&energy, 8, 1, o);
    std::fwrite(site.data(), 8, n, o);
    std::fwrite(fold.data(), 8, 3 * (size_t)n, o);
    std::fwrite(vir, 8, 6, o);
    std::fclose(o);
    return 0;
}
catch (const std::exception &e)
{
    std::fprintf(stderr, "%s\n", e.what());
    return 7;
}
