// Driver for the reference standalone MTP core (runtime/mtp/mlip.cpp,
// runtime/mtp/radial_basis_setup.cpp), compiled from the reference sources
// by oracle/Makefile into oracle/_ref/mlip_ref.  Test infrastructure only.
//
// The core evaluates LAMMPS-style full lists over owned + ghost atoms.  The
// driver receives the periodic images as ghost atoms, builds full lists by
// brute force and folds ghost forces back onto their owners.
//
// usage: mlip_ref <model.mtp> <in.bin> <out.bin>
//   in : int32 Z | int32 npts | int32 n | f64 cutoff | f64 pts[npts][3] |
//        int32 type[npts] | int32 orig[npts]
//   out: f64 energy | f64 site_energy[n] | f64 force[n][3] | f64 virial[6]
#include "mlip.h"
#include <cstdint>
#include <cstdio>
#include <vector>

int main(int argc, char **argv)
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
    MLIPCore::mlip *pot = MLIPCore::setup(argv[1], sp.data(), &model_cutoff, (std::size_t)Z);
    MLIPCore::mlip_buffers *buf = MLIPCore::create_mlip_buffer(pot);

    const double rc2 = cutoff * cutoff;
    std::vector<std::vector<int>> lists(n);
    for (int i = 0; i < n; ++i)
        for (int p = 0; p < npts; ++p)
        {
            if (p == i)
                continue;
            double d0 = pts[3 * p] - pts[3 * i], d1 = pts[3 * p + 1] - pts[3 * i + 1],
                   d2 = pts[3 * p + 2] - pts[3 * i + 2];
            if (d0 * d0 + d1 * d1 + d2 * d2 < rc2)
                lists[i].push_back(p);
        }
    std::vector<int> ilist(n), numneigh(npts, 0);
    std::vector<int *> firstneigh(npts, nullptr);
    for (int i = 0; i < n; ++i)
    {
        ilist[i] = i;
        numneigh[i] = (int)lists[i].size();
        firstneigh[i] = lists[i].data();
    }
    std::vector<double *> x(npts), fptr(npts), vptr(npts);
    std::vector<double> force(3 * (size_t)npts, 0.0), virial(6 * (size_t)npts, 0.0);
    for (int p = 0; p < npts; ++p)
    {
        x[p] = &pts[3 * p];
        fptr[p] = &force[3 * p];
        vptr[p] = &virial[6 * p];
    }
    std::vector<double> site(npts, 0.0);
    double energy = 0;
    MLIPCore::compute(pot, buf, ilist.data(), numneigh.data(), n, type.data(), x.data(),
                      firstneigh.data(), &energy, site.data(), vptr.data(), fptr.data());

    std::vector<double> fold(3 * (size_t)n, 0.0);
    double vir[6] = {0, 0, 0, 0, 0, 0};
    for (int p = 0; p < npts; ++p)
    {
        for (int a = 0; a < 3; ++a)
            fold[3 * orig[p] + a] += force[3 * p + a];
        for (int q = 0; q < 6; ++q)
            vir[q] += virial[6 * p + q];
    }
    FILE *o = std::fopen(argv[3], "wb");
    if (!o)
        return 6;
    std::fwrite(&energy, 8, 1, o);
    std::fwrite(site.data(), 8, n, o);
    std::fwrite(fold.data(), 8, 3 * (size_t)n, o);
    std::fwrite(vir, 8, 6, o);
    std::fclose(o);
    MLIPCore::destroy_mlip_buffer(buf);
    MLIPCore::destroy_mlip(pot);
    return 0;
}
