// 3x3 cell helpers with the reference's evaluation order (geometry.cpp).
#pragma once

namespace mtpx {
// Matrix3d::inverse() by cofactors; false for a singular cell.
bool cell_inverse(const double *cell, double *inv);
// RowVector3d * Matrix3d, each component summed left to right.
void row_times(const double *p, const double *M, double *out);
}  // namespace mtpx
