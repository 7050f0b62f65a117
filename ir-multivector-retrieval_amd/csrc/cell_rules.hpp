// cell_rules.hpp — the scalar rules of the cell-list encode, shared by the
// GPU kernels (cell_kernels.hpp) and a host-side check
// (tests/native/cell_rules_check.cpp).  Plain C++ when compiled by a host
// compiler; compile with -ffp-contract=off either way.
//
// A uniform grid of G cells per dimension covers a box [lo, lo + G / s) of a
// subspace.  A vector's cell comes from f = fl(fl(x - lo) * s) per dimension
// (two roundings, no contraction); it is inside the grid when 0 <= f < G in
// every dimension (NaN never is).  cell_interval gives, per dimension, a real
// interval that holds every fp32 x mapped to a range of cells, so each cell
// has a box B that holds all of its vectors.
//
// Each cell lists the codewords that can be the reference's first-index
// argmin (src/util/vec.zig:271-283 over the fold of vec.zig:109-175) for
// some point of B.  With T the exact squared distance, the reference fold
// satisfies |ref(p, c) - T(p, c)| <= g T(p, c) + eta (g = gamma_{D+2}, eta
// < 1e-43 for underflow).  For an anchor c0 and any codeword c,
//   T(p, c) - T(p, c0) = sum_j (c_j - c0_j) (c_j + c0_j - 2 p_j),
// linear in p, so its minimum over B sits at a corner; if that minimum
// exceeds g (max_B T(., c) + max_B T(., c0)) + 2 eta then ref(p, c) >
// ref(p, c0) everywhere in B and c is never the argmin there.  A cell's
// list keeps every codeword that this test does not exclude (c0 itself is
// never excluded), so the reference's argmin of any vector of the cell is
// in it, and the lexicographic (distance bits, index) minimum over the list
// is that argmin.  Excluding against a coarse cell's anchor over the coarse
// box holds for every fine cell inside it, so fine lists are built from the
// coarse list.
#pragma once

#include <stdint.h>

#ifndef TAC_HD
#if defined(__HIPCC__)
#define TAC_HD __host__ __device__
#else
#define TAC_HD
#endif
#endif

namespace tacgpu {

// Coarse cells per dimension and fine cells per coarse cell per dimension:
// G = Gc * Gs fine cells per dimension, at most 65,536 fine cells and 4,096
// coarse cells per subspace.  Sub-dimensions past 4 keep the anchored
// candidate encode.
TAC_HD constexpr uint32_t cell_coarse_side(int D) {
  return D == 1 ? 4096u : D == 2 ? 64u : D == 3 ? 12u : 8u;
}
TAC_HD constexpr uint32_t cell_sub_side(int D) {
  return D == 1 ? 16u : D == 2 ? 4u : D == 3 ? 3u : 2u;
}
TAC_HD constexpr uint32_t cell_pow(uint32_t b, int e) { return e == 0 ? 1u : b * cell_pow(b, e - 1); }
TAC_HD constexpr uint32_t cell_side(int D) { return cell_coarse_side(D) * cell_sub_side(D); }
TAC_HD constexpr uint32_t cell_count(int D) { return cell_pow(cell_side(D), D); }
TAC_HD constexpr uint32_t cell_coarse_count(int D) { return cell_pow(cell_coarse_side(D), D); }
TAC_HD constexpr uint32_t cell_fine_per_coarse(int D) { return cell_pow(cell_sub_side(D), D); }

constexpr uint32_t kCellItem = 4;       // list entries per work item (lists are padded to whole items)
constexpr uint32_t kCellMaxItems = 32;  // items per cell list; longer lists defer
constexpr double kCellTame = 1e15;      // box and codeword magnitudes the rules accept

// Cell of one coordinate: f = fl(fl(x - lo) * s); *inside is false outside
// [0, G) and on NaN.  The kernels use this exact expression.
TAC_HD inline uint32_t cell_coord(float x, float lo, float s, uint32_t G, bool* inside) {
  const float f = (x - lo) * s;
  const bool in = f >= 0.0f && f < (float)G;
  *inside = in;
  return in ? (uint32_t)f : 0u;
}

// Fine cell id of in-grid coordinates k[0..D): coarse-major, so the fine
// cells of one coarse cell are contiguous.
template <int D>
TAC_HD inline uint32_t cell_id(const uint32_t (&k)[D]) {
  constexpr uint32_t Gc = cell_coarse_side(D), Gs = cell_sub_side(D);
  uint32_t coarse = 0, sub = 0;
  for (int j = D - 1; j >= 0; --j) {
    coarse = coarse * Gc + k[j] / Gs;
    sub = sub * Gs + k[j] % Gs;
  }
  return coarse * cell_fine_per_coarse(D) + sub;
}

// Real interval [*a, *b] holding every fp32 x whose coordinate cell_coord
// lies in [k0, k1), for the fp32 values lo and s > 0 (finite).
//   f = fd * s (1 + d2), fd = (x - lo)(1 + d1), |d| <= u = 2^-24 (normal
//   results), so for fd >= 0: x - lo in [k0 / (s (1+u)^2), k1 / (s (1-u)^2)].
//   A negative fd gives f <= 0, inside only as -0.0 after an underflow of
//   fd * s, when |x - lo| < 2^-148 / s; subnormal roundings add at most
//   2^-149 to fd and 2^-149 to f.  The reciprocals and the double arithmetic
//   (relative errors near 2^-53) are covered by widening the interval by a
//   relative 2^-40 of its ends.
struct CellAxis {
  double lo, rlo, rhi, tiny;
};
TAC_HD inline CellAxis cell_axis(float lo, float s) {
  const double u = 5.9604644775390625e-8;  // 2^-24
  const double sd = (double)s;
  CellAxis ax;
  ax.lo = (double)lo;
  ax.rlo = 1.0 / (sd * (1.0 + u) * (1.0 + u));
  ax.rhi = 1.0 / (sd * (1.0 - u) * (1.0 - u));
  ax.tiny = 3.0e-45 / sd + 2.0e-45;  // subnormal roundings of f and fd
  return ax;
}
TAC_HD inline void cell_interval_axis(const CellAxis& ax, uint32_t k0, uint32_t k1, double* a,
                                      double* b) {
  double lo_off = (double)k0 * ax.rlo - ax.tiny;
  if (k0 == 0) lo_off = -2.0 * ax.tiny - 6.0e-45 * ax.rhi;  // the -0.0 case
  const double hi_off = (double)k1 * ax.rhi + ax.tiny;
  const double lo_x = ax.lo + lo_off, hi_x = ax.lo + hi_off;
  const double w = 9.094947017729282e-13 * (lo_x < 0 ? -lo_x : lo_x) +
                   9.094947017729282e-13 * (hi_x < 0 ? -hi_x : hi_x);  // 2^-40
  *a = lo_x - w;
  *b = hi_x + w;
}
TAC_HD inline void cell_interval(float lo, float s, uint32_t k0, uint32_t k1, double* a,
                                 double* b) {
  cell_interval_axis(cell_axis(lo, s), k0, k1, a, b);
}

// Grid origin and scale of a subspace from a box [lo, hi] (doubles): the
// fp32 origin and s = G / width, the width kept above a relative 2^-20 of
// the magnitudes.  False when the grid would not be tame (non-finite, or
// past kCellTame); every vector of the subspace then takes the full search.
// The box only decides how long the lists are: the rules above hold for
// any origin and scale.
TAC_HD inline bool cell_grid_params(double lo, double hi, uint32_t G, float* lo_f, float* s_f) {
  if (!(lo <= hi) || !(lo >= -kCellTame) || !(hi <= kCellTame)) return false;
  const double mag = (lo < 0 ? -lo : lo) + (hi < 0 ? -hi : hi);
  double w = hi - lo;
  const double wmin = mag * 9.5367431640625e-7 + 1e-30;  // 2^-20
  if (w < wmin) w = wmin;
  const float l = (float)lo;
  const float s = (float)((double)G / w);
  if (!(s > 0.0f) || !(s < 3.0e38f)) return false;
  const double top = (double)l + (double)G / (double)s * 1.001;
  if (!(top <= kCellTame) || !(top >= -kCellTame)) return false;
  *lo_f = l;
  *s_f = s;
  return true;
}

// gamma_{D+2} in double, rounded up.
TAC_HD inline double cell_gamma(int D) {
  const double nu = (double)(D + 2) * 5.9604644775390625e-8;
  return nu / (1.0 - nu) * (1.0 + 1e-9);
}

// max over the box of the exact squared distance to c.
template <int D>
TAC_HD inline double cell_max_t(const double (&c)[D], const double (&a)[D], const double (&b)[D]) {
  double t = 0.0;
  for (int j = 0; j < D; ++j) {
    const double p = a[j] - c[j], q = b[j] - c[j];
    const double pp = p * p, qq = q * q;
    t += pp > qq ? pp : qq;
  }
  return t;
}

// True when c can be dropped from the list of a box [a, b] with anchor c0
// (mt0 = cell_max_t(c0, a, b)): ref(p, c) > ref(p, c0) for every p of the
// box.  The double evaluation is covered by a relative 2^-40 of the
// magnitudes involved.
template <int D>
TAC_HD inline bool cell_excluded(const double (&c)[D], const double (&c0)[D], double mt0,
                                 const double (&a)[D], const double (&b)[D], double g) {
  double lin = 0.0, mag = 0.0;
  for (int j = 0; j < D; ++j) {
    const double dc = c[j] - c0[j];
    const double p = dc > 0.0 ? b[j] : a[j];  // the corner that minimises the term
    const double t = dc * ((c[j] + c0[j]) - 2.0 * p);
    lin += t;
    mag += t < 0 ? -t : t;
  }
  const double mt = cell_max_t<D>(c, a, b);
  const double bound = g * (mt + mt0) + 1e-40 + 9.094947017729282e-13 * (mag + mt + mt0);
  return lin > bound;
}

}  // namespace tacgpu
