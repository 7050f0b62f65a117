// screen_rules.hpp — the scalar rules of the matrix-core screen
// (screen_kernels.hpp), shared by the GPU kernel and a host-side check
// (tests/native/screen_rules_check.cpp).  Plain C++ when compiled by a host
// compiler; compile with -ffp-contract=off either way.
//
// The screen ranks codewords by s~(c), which is within
//   E(x, c) = 2^-14 (1.07 ||x|| ||c|| + 0.04 ||c||^2) + 2^-123 (2 ||c|| + ||x||) + 2^-120
// of s(c) = ||c||^2 - 2 x.c (the derivation is in screen_kernels.hpp).
// screen_err gives twice that, with the codebook's largest norm cmax, and
// screen_separates decides from the two smallest block minima b1 <= b2
// whether the reference's first-index argmin (the fold of squared
// differences, gamma_{D+2} relative, src/util/vec.zig:109-175) must lie in
// the block of b1.
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

constexpr float kScreenTame = 1.329227995784916e36f;  // 2^120: ||x||^2 and cmax^2 at most this

// Twice the screen's error bound for a vector of norm at most nx against a
// codebook whose norms are at most cmax (cmax2 = cmax^2):
// 2^-13 (1.07 nx cmax + 0.04 cmax^2) + 2^-122 (2 cmax + nx) + 2^-119.
TAC_HD inline float screen_err(float nx, float cmax, float cmax2) {
  constexpr float kxc = 1.31e-4f;                 // >= 1.07 * 2^-13
  constexpr float kcc = 4.9e-6f;                  // >= 0.04 * 2^-13
  constexpr float k122 = 1.880790961315660e-37f;  // 2^-122
  constexpr float k119 = 1.504632769052528e-36f;  // 2^-119
  return kxc * nx * cmax + kcc * cmax2 + k122 * (2.0f * cmax + nx) + k119;
}

// Whether the smallest block minimum b1 is separated from every other
// block's (b2 the second smallest, +inf when every other block holds
// padding only): with s~ within ea / 2 of s, the reference distances (within
// gamma_{D+2} of s + ||x||^2, x2 = fl(||x||^2)) of the winning block's best
// codeword and of any codeword outside it cannot cross.  The margins are
// doubled again, and 1e-30 covers the reference distance's underflow.
// False on NaN.
template <int D>
TAC_HD inline bool screen_separates(float b1, float b2, float x2, float ea) {
  constexpr float u = 5.9604644775390625e-8f;  // 2^-24
  constexpr float gR = (float)(D + 2) * u / (1.0f - (float)(D + 2) * u);
  float thr = 2.0f * ea * (1.0f + gR) + gR * ((b2 + x2 < 0.0f ? -(b2 + x2) : b2 + x2) +
                                              (b1 + x2 < 0.0f ? -(b1 + x2) : b1 + x2));
  thr = 2.0f * thr + 1e-30f;
  return b2 == __builtin_inff() || (b2 - b1) > thr;
}

}  // namespace tacgpu
