// Host geometry: Atoms::wrap (base/structures.cpp:1282-1305) and the 3x3
// helpers shared with the neighbour builder.  Compiled with
// -ffp-contract=off: the products below reproduce the evaluation order of
// the Eigen expressions the reference uses (RowVector3d * Matrix3d summed
// left to right; Matrix3d::inverse by cofactors, det = (c00 m00 + c10 m10) +
// c20 m20), so wrapped coordinates agree with the reference bit for bit.
#include "mtpx.h"
#include "mtpx_geometry.hpp"

#include <cmath>

namespace mtpx {

static double cofactor(const double *m, int i, int j)
{
    const int i1 = (i + 1) % 3, i2 = (i + 2) % 3, j1 = (j + 1) % 3, j2 = (j + 2) % 3;
    return m[i1 * 3 + j1] * m[i2 * 3 + j2] - m[i1 * 3 + j2] * m[i2 * 3 + j1];
}

bool cell_inverse(const double *m, double *inv)
{
    const double c0 = cofactor(m, 0, 0), c1 = cofactor(m, 1, 0), c2 = cofactor(m, 2, 0);
    const double det = (c0 * m[0] + c1 * m[3]) + c2 * m[6];
    if (det == 0 || !std::isfinite(det))
        return false;
    const double invdet = 1.0 / det;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            inv[j * 3 + i] = cofactor(m, i, j) * invdet;
    return true;
}

void row_times(const double *p, const double *M, double *out)
{
    double r[3];
    for (int j = 0; j < 3; ++j) {
        const double a0 = p[0] * M[j], a1 = p[1] * M[3 + j], a2 = p[2] * M[6 + j];
        r[j] = (a0 + a1) + a2;
    }
    out[0] = r[0];
    out[1] = r[1];
    out[2] = r[2];
}

}  // namespace mtpx

extern "C" int mtpx_wrap(const double cell[9], const int pbc[3], int n, double *pos)
{
    if (!cell || !pbc || n < 0 || (n > 0 && !pos))
        return MTPX_E_INVALID;
    if (!pbc[0] && !pbc[1] && !pbc[2])
        return MTPX_OK;
    double inv[9];
    if (!mtpx::cell_inverse(cell, inv))
        return MTPX_E_INVALID;
    for (int i = 0; i < n; ++i) {
        double f[3];
        mtpx::row_times(pos + 3 * i, inv, f);
        for (int j = 0; j < 3; ++j)
            if (pbc[j])
                f[j] -= std::floor(f[j]);
        mtpx::row_times(f, cell, pos + 3 * i);
    }
    return MTPX_OK;
}
