// fold_rules.hpp — exact chunked evaluation of a serial fp32 sum of
// non-negative terms, s_{i+1} = fl(s_i + e_i) from s_0 = 0 (the wcss fold of
// src/tac/kmeans.zig:179).  Shared by the GPU kernels and a CPU check.
//
// While the accumulator s lies in one binade [2^k, 2^(k+1)), the floats there
// are exactly the multiples of U = 2^(k-23), so
//   fl(s + e) = s + U * round(e / U)
// whenever e / U is not exactly halfway between two integers (the tie would
// be broken by the parity of s) and the exact sum stays below 2^(k+1) - U/2.
// A chunk of terms therefore adds U * Q with Q = sum of round(e_i / U), an
// integer sum that can be formed in parallel, provided
//   - every term is finite, >= 0, and no e_i / U is a tie;
//   - s is normal and positive, and s + U * Q <= 2^(k+1) - U (every partial
//     sum is then below 2^(k+1) - U/2, so no step rounds across the binade).
// Terms are quantized for three candidate binades per chunk (around the
// chunk's approximate start, from an f64 prefix); a chunk that meets none of
// the conditions is folded term by term.
#pragma once

#include <math.h>
#include <stdint.h>

#ifndef TAC_HD
#if defined(__HIPCC__)
#define TAC_HD __host__ __device__
#else
#define TAC_HD
#endif
#endif

namespace tacgpu {

constexpr uint32_t kFoldChunk = 1024;  // terms per chunk
constexpr int kFoldCands = 3;          // candidate binades per chunk

struct FoldChunk {
  int32_t k0;          // candidate binade exponents k0, k0 + 1, k0 + 2
  uint32_t clean;      // bit c: candidate c is usable
  uint64_t q[kFoldCands];
};

TAC_HD inline int32_t fold_exponent(float s) {  // k with 2^k <= s < 2^(k+1), s normal > 0
  union {
    float f;
    uint32_t u;
  } v;
  v.f = s;
  return (int32_t)((v.u >> 23) & 0xFFu) - 127;
}

TAC_HD inline bool fold_is_normal_positive(float s) {
  union {
    float f;
    uint32_t u;
  } v;
  v.f = s;
  const uint32_t ex = (v.u >> 23) & 0xFFu;
  return (v.u >> 31) == 0 && ex != 0 && ex != 0xFFu;
}

constexpr uint64_t kFoldBad = ~0ull;  // fold_quantize: the term spoils the binade

// round(e / 2^(k-23)) for one term and one binade k, or kFoldBad when the
// term spoils the chunk for that binade (k outside [-126, 127], e not finite,
// negative, a tie, or so large that it alone would leave the binade).
// Written without early returns: callers OR the failure into a mask and add
// the value branch-free (a short-circuit `if (ok && quantize(&q)) ... else
// ok = 0` form was compiled for gfx950 such that a failing term left `ok`
// set).
TAC_HD inline uint64_t fold_quantize(float e, int32_t k) {
  const bool k_ok = k >= -126 && k <= 127;
  const bool e_ok = e >= 0.0f && e <= 3.402823466e38f;  // excludes NaN, negative, inf
  // e / U exactly, in double: e has 24 significant bits and U is a power of
  // two, and e * 2^(23-k) stays within double's normal range for every
  // float e and every k in [-126, 127].
  const double t = ldexp(e_ok ? (double)e : 0.0, k_ok ? 23 - k : 0);
  const bool small = t < 16777216.0;  // < 2^24 units: cannot leave the binade alone
  const double fl = floor(small ? t : 0.0);
  const double frac = t - fl;
  const bool tie = frac == 0.5;  // would depend on the parity of s
  const uint64_t q = (uint64_t)fl + (frac > 0.5 ? 1u : 0u);
  return (k_ok && e_ok && small && !tie) ? q : kFoldBad;
}

// Applies a chunk with quantized sums: true (and *out) when the chunk adds
// exactly U * Q without leaving the accumulator's binade.
TAC_HD inline bool fold_apply(float s, const FoldChunk& ch, float* out) {
  if (!fold_is_normal_positive(s)) return false;
  const int32_t k = fold_exponent(s);
  const int32_t c = k - ch.k0;
  if (c < 0 || c >= kFoldCands || !((ch.clean >> c) & 1u)) return false;
  const uint64_t Q = ch.q[c];
  // units of U: s = m * U with 2^23 <= m < 2^24; the binade ends at 2^24 U
  union {
    float f;
    uint32_t u;
  } v;
  v.f = s;
  const uint64_t m = (uint64_t)((v.u & 0x7FFFFFu) | 0x800000u);
  if (Q > (1ull << 24) || m + Q > (1ull << 24) - 1) return false;
  v.u = (v.u & 0xFF800000u) | (uint32_t)((m + Q) & 0x7FFFFFu);
  *out = v.f;
  return true;
}

}  // namespace tacgpu
