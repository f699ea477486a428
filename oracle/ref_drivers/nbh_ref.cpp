// Driver for the reference BOXED neighbour builder (base/neighborhood.cpp,
// base/neighborhoods_base.h), compiled from the reference sources by
// oracle/Makefile into oracle/_ref/nbh_ref.  Test infrastructure only.
//
// usage: nbh_ref <in.bin> <out.bin>
//   in : int32 n | f64 cell[9] (rows = lattice vectors) | int32 pbc[3] |
//        f64 cutoff | f64 pos[n][3] | int32 types[n]
//   out: int32 n | int64 P | int32 offsets[n+1] | int32 idx[P] |
//        int32 types[P] | f64 vec[P][3] | f64 dist[P] | int32 centertype[n]
#include "neighborhood.h"
#include <cstdio>
#include <cstdint>
#include <vector>

int main(int argc, char **argv)
{
    if (argc != 3)
        return 2;
    FILE *f = std::fopen(argv[1], "rb");
    if (!f)
        return 3;
    int32_t n;
    double cell[9], cutoff;
    int32_t pbc[3];
    if (std::fread(&n, 4, 1, f) != 1 || std::fread(cell, 8, 9, f) != 9 ||
        std::fread(pbc, 4, 3, f) != 3 || std::fread(&cutoff, 8, 1, f) != 1)
        return 4;
    std::vector<double> pos(3 * (size_t)n);
    std::vector<int32_t> types(n);
    if (std::fread(pos.data(), 8, pos.size(), f) != pos.size() ||
        std::fread(types.data(), 4, types.size(), f) != types.size())
        return 5;
    std::fclose(f);

    Atoms atom;
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c)
            atom.cell_(r, c) = cell[3 * r + c];
    atom.pbc_ = {pbc[0] != 0, pbc[1] != 0, pbc[2] != 0};
    atom.pos_.resize(n);
    atom.chemmap_.resize(n);
    for (int i = 0; i < n; ++i)
    {
        atom.pos_[i] = Eigen::RowVector3d(pos[3 * i], pos[3 * i + 1], pos[3 * i + 2]);
        atom.chemmap_[i] = types[i];
    }
    Neighborhoods nbhs(atom, cutoff);

    std::vector<int32_t> offsets(n + 1, 0);
    for (int i = 0; i < n; ++i)
        offsets[i + 1] = offsets[i] + nbhs[i].nbhcount_;
    int64_t P = offsets[n];
    FILE *o = std::fopen(argv[2], "wb");
    if (!o)
        return 6;
    std::fwrite(&n, 4, 1, o);
    std::fwrite(&P, 8, 1, o);
    std::fwrite(offsets.data(), 4, offsets.size(), o);
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < nbhs[i].nbhcount_; ++j)
            std::fwrite(&nbhs[i].indices_[j], 4, 1, o);
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < nbhs[i].nbhcount_; ++j)
            std::fwrite(&nbhs[i].chemmap_[j], 4, 1, o);
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < nbhs[i].nbhcount_; ++j)
            std::fwrite(nbhs[i].pos_[j].data(), 8, 3, o);
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < nbhs[i].nbhcount_; ++j)
            std::fwrite(&nbhs[i].distances_[j], 8, 1, o);
    for (int i = 0; i < n; ++i)
        std::fwrite(&nbhs[i].centertype, 4, 1, o);
    std::fclose(o);
    return 0;
}
