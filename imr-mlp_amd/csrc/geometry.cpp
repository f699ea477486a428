// Host geometry: Atoms::wrap (base/structures.cpp:1282-1305) with its
// singular-cell branch (:97-130) and the 3x3 helpers shared with the
// neighbour builder.  Compiled with
// -ffp-contract=off: the products below reproduce the evaluation order of
// the Eigen expressions the reference uses (RowVector3d * Matrix3d summed
// left to right; Matrix3d::inverse by cofactors, det = (c00 m00 + c10 m10) +
// c20 m20), so wrapped coordinates agree with the reference bit for bit.
#include "mtpx.h"
#include "mtpx_geometry.hpp"

#include <cmath>
#include <limits>
#include <utility>

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

// Eigen's FullPivLU of an n x n row-major matrix (n <= 3), as far as its
// rank test and solve need it (Eigen/src/LU/FullPivLU.h computeInPlace):
// the pivot is the first largest |a_ij| of the remaining corner in
// column-major order; elimination stops at an exactly zero corner; a pivot
// counts towards the rank when |u_kk| > n eps max|pivot|.
struct FullPivLu {
    int n = 0, nonzero = 0;
    double lu[9], maxpivot = 0;
    int rowt[3], colt[3];  // transpositions of step k
    double at(int i, int j) const { return lu[i * 3 + j]; }
    void factor(const double *m, int dim)
    {
        n = dim;
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < n; ++j)
                lu[i * 3 + j] = m[i * 3 + j];
        nonzero = n;
        maxpivot = 0;
        for (int k = 0; k < n; ++k) {
            double big = -1;
            int bi = k, bj = k;
            for (int j = k; j < n; ++j)
                for (int i = k; i < n; ++i)
                    if (std::fabs(lu[i * 3 + j]) > big) {
                        big = std::fabs(lu[i * 3 + j]);
                        bi = i;
                        bj = j;
                    }
            if (big == 0) {
                nonzero = k;
                for (int i = k; i < n; ++i)
                    rowt[i] = colt[i] = i;
                break;
            }
            if (big > maxpivot)
                maxpivot = big;
            rowt[k] = bi;
            colt[k] = bj;
            if (bi != k)
                for (int j = 0; j < n; ++j)
                    std::swap(lu[k * 3 + j], lu[bi * 3 + j]);
            if (bj != k)
                for (int i = 0; i < n; ++i)
                    std::swap(lu[i * 3 + k], lu[i * 3 + bj]);
            for (int i = k + 1; i < n; ++i)
                lu[i * 3 + k] /= lu[k * 3 + k];
            for (int j = k + 1; j < n; ++j)
                for (int i = k + 1; i < n; ++i)
                    lu[i * 3 + j] -= lu[i * 3 + k] * lu[k * 3 + j];
        }
    }
    int rank() const
    {
        const double thr = maxpivot * (std::numeric_limits<double>::epsilon() * n);
        int r = 0;
        for (int i = 0; i < nonzero; ++i)
            r += std::fabs(lu[i * 3 + i]) > thr;
        return r;
    }
    // X = A^-1 B for B [n][3] (row-major), FullPivLU::_solve_impl: rows
    // permuted by P, unit-lower then upper triangular solves (the upper one
    // multiplies by 1 / u_ii), rows placed by Q.
    void solve(const double *B, double *X) const
    {
        double c[9];
        int perm[3] = {0, 1, 2};
        for (int k = 0; k < n; ++k)
            std::swap(perm[k], perm[rowt[k]]);
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < 3; ++j)
                c[i * 3 + j] = B[perm[i] * 3 + j];
        for (int k = 0; k < n; ++k)
            for (int i = k + 1; i < n; ++i)
                for (int j = 0; j < 3; ++j)
                    c[i * 3 + j] -= c[k * 3 + j] * at(i, k);
        const int r = rank();
        for (int k = r - 1; k >= 0; --k) {
            const double a = 1.0 / at(k, k);
            for (int j = 0; j < 3; ++j)
                c[k * 3 + j] *= a;
            for (int i = 0; i < k; ++i)
                for (int j = 0; j < 3; ++j)
                    c[i * 3 + j] -= c[k * 3 + j] * at(i, k);
        }
        int q[3] = {0, 1, 2};
        for (int k = 0; k < n; ++k)
            std::swap(q[k], q[colt[k]]);
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < 3; ++j)
                X[q[i] * 3 + j] = i < r ? c[i * 3 + j] : 0.0;
    }
};

// wrap_singular_cell (base/structures.cpp:97-130): a cell that Eigen's
// FullPivLU finds singular wraps along its periodic rows only.  The rank
// periodic rows form the basis B, G = B B^T its metric, D = G^-1 B its dual;
// each position p loses floor(D p)_k B_k for every periodic row k.
// Returns false for a full cell (the caller takes the fractional path) and
// sets bad for the reference's errors (non-finite or dependent rows).
bool wrap_singular(const double *cell, const int *pbc, int n, double *pos, bool &bad)
{
    bad = false;
    FullPivLu cl;
    cl.factor(cell, 3);
    if (cl.rank() == 3)
        return false;
    int rank = 0;
    double B[9];
    for (int a = 0; a < 3; ++a)
        if (pbc[a]) {
            for (int j = 0; j < 3; ++j)
                B[rank * 3 + j] = cell[a * 3 + j];
            ++rank;
        }
    if (rank == 0)
        return true;
    for (int q = 0; q < rank * 3; ++q)
        if (!std::isfinite(B[q])) {
            bad = true;
            return true;
        }
    double G[9];
    for (int i = 0; i < rank; ++i)
        for (int j = 0; j < rank; ++j)
            G[i * 3 + j] = (B[i * 3] * B[j * 3] + B[i * 3 + 1] * B[j * 3 + 1]) +
                           B[i * 3 + 2] * B[j * 3 + 2];
    for (int i = 0; i < rank; ++i)
        for (int j = 0; j < rank; ++j)
            if (!std::isfinite(G[i * 3 + j])) {
                bad = true;
                return true;
            }
    FullPivLu gl;
    gl.factor(G, rank);
    if (gl.rank() != rank) {
        bad = true;
        return true;
    }
    double D[9];
    gl.solve(B, D);
    for (int q = 0; q < rank * 3; ++q)
        if (!std::isfinite(D[q])) {
            bad = true;
            return true;
        }
    for (int i = 0; i < n; ++i) {
        double *p = pos + 3 * i;
        double c[3];
        for (int k = 0; k < rank; ++k)
            c[k] = (D[k * 3] * p[0] + D[k * 3 + 1] * p[1]) + D[k * 3 + 2] * p[2];
        for (int k = 0; k < rank; ++k) {
            const double f = std::floor(c[k]);
            for (int j = 0; j < 3; ++j)
                p[j] -= f * B[k * 3 + j];
        }
    }
    return true;
}

}  // namespace mtpx

extern "C" int mtpx_wrap(const double cell[9], const int pbc[3], int n, double *pos)
{
    if (!cell || !pbc || n < 0 || (n > 0 && !pos))
        return MTPX_E_INVALID;
    if (!pbc[0] && !pbc[1] && !pbc[2])
        return MTPX_OK;
    bool bad = false;
    if (mtpx::wrap_singular(cell, pbc, n, pos, bad))
        return bad ? MTPX_E_INVALID : MTPX_OK;
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
