// fold_rules.hpp — exact chunked evaluation of a serial sum of non-negative
// float terms, s_{i+1} = fl(s_i + e_i) from s_0 = 0, with an fp32
// accumulator (the wcss fold of src/tac/kmeans.zig:179) or an f64 one (the
// weight folds of weightedSample, src/util/rng.zig:60-81).  Shared by the GPU
// kernels and a CPU check.
//
// Let the accumulator type carry F fraction bits (23 for fp32, 52 for f64).
// While the accumulator s lies in one binade [2^k, 2^(k+1)), the values
// there are exactly the multiples of U = 2^(k-F), so
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

constexpr uint32_t kFoldChunk = 256;  // terms per chunk
constexpr int kFoldCands = 3;          // candidate binades per chunk
constexpr uint64_t kFoldBad = ~0ull;   // fold_quantize: the term spoils the binade

struct FoldChunk {
  int32_t k0;          // candidate binade exponents k0, k0 + 1, k0 + 2
  uint32_t clean;      // bit c: candidate c is usable
  uint64_t q[kFoldCands];
};

template <typename Acc>
struct FoldTraits;
template <>
struct FoldTraits<float> {
  using Bits = uint32_t;
  static constexpr int kFrac = 23, kExpBits = 8, kBias = 127;
};
template <>
struct FoldTraits<double> {
  using Bits = uint64_t;
  static constexpr int kFrac = 52, kExpBits = 11, kBias = 1023;
};

template <typename Acc>
TAC_HD inline typename FoldTraits<Acc>::Bits fold_bits(Acc s) {
  union {
    Acc f;
    typename FoldTraits<Acc>::Bits u;
  } v;
  v.f = s;
  return v.u;
}

template <typename Acc>
TAC_HD inline Acc fold_from_bits(typename FoldTraits<Acc>::Bits u) {
  union {
    Acc f;
    typename FoldTraits<Acc>::Bits u;
  } v;
  v.u = u;
  return v.f;
}

// k with 2^k <= s < 2^(k+1), for a normal s > 0.
template <typename Acc>
TAC_HD inline int32_t fold_exponent(Acc s) {
  using T = FoldTraits<Acc>;
  const uint32_t ex = (uint32_t)(fold_bits(s) >> T::kFrac) & ((1u << T::kExpBits) - 1u);
  return (int32_t)ex - T::kBias;
}

template <typename Acc>
TAC_HD inline bool fold_is_normal_positive(Acc s) {
  using T = FoldTraits<Acc>;
  const auto u = fold_bits(s);
  const uint32_t ex = (uint32_t)(u >> T::kFrac) & ((1u << T::kExpBits) - 1u);
  return (u >> (T::kFrac + T::kExpBits)) == 0 && ex != 0 && ex != (1u << T::kExpBits) - 1u;
}

// round(e / 2^(k-F)) for one float term and one binade k of the accumulator,
// or kFoldBad when the term spoils the chunk for that binade (k outside the
// normal range, e not finite, negative, a tie, or so large that it alone
// would leave the binade).  Written without early returns: callers OR the
// failure into a mask and add the value branch-free (a short-circuit
// `if (ok && quantize(&q)) ... else ok = 0` form was compiled for gfx950
// such that a failing term left `ok` set).
template <typename Acc>
TAC_HD inline uint64_t fold_quantize(float e, int32_t k) {
  using T = FoldTraits<Acc>;
  constexpr int32_t kMin = 1 - T::kBias, kMax = T::kBias;
  const bool k_ok = k >= kMin && k <= kMax;
  const bool e_ok = e >= 0.0f && e <= 3.402823466e38f;  // excludes NaN, negative, inf
  // e / U in double.  e has 24 significant bits and U is a power of two, so
  // the scaling is exact unless it overflows (then t = inf: a term far
  // beyond the binade) or underflows (then e / U < 2^-1022, which rounds to
  // 0 and is no tie, and t rounds to a value below 0.5 as well).
  const double t = ldexp(e_ok ? (double)e : 0.0, k_ok ? T::kFrac - k : 0);
  const bool small = t < (double)(1ull << (T::kFrac + 1));  // cannot leave the binade alone
  const double fl = floor(small ? t : 0.0);
  const double frac = t - fl;  // exact: t < 2^53
  const bool tie = frac == 0.5;  // would depend on the parity of s
  const uint64_t q = (uint64_t)fl + (frac > 0.5 ? 1u : 0u);
  return (k_ok && e_ok && small && !tie) ? q : kFoldBad;
}

// The accumulator in units of its ulp U: s = m * U with 2^F <= m < 2^(F+1)
// (s normal and positive).
template <typename Acc>
TAC_HD inline uint64_t fold_units(Acc s) {
  using T = FoldTraits<Acc>;
  using Bits = typename T::Bits;
  constexpr uint64_t kOne = 1ull << T::kFrac;
  return (uint64_t)(fold_bits(s) & (Bits)(kOne - 1)) | kOne;
}

// m * U in the binade of s, for 2^F <= m < 2^(F+1).
template <typename Acc>
TAC_HD inline Acc fold_with_units(Acc s, uint64_t m) {
  using T = FoldTraits<Acc>;
  using Bits = typename T::Bits;
  constexpr uint64_t kOne = 1ull << T::kFrac;
  return fold_from_bits<Acc>((Bits)((fold_bits(s) & ~(Bits)(kOne - 1)) | (Bits)(m & (kOne - 1))));
}

// The chunk's quantized sum for the binade of s (normal, positive), or
// kFoldBad when the chunk has no clean candidate there or the sum alone
// would leave the binade.
template <typename Acc>
TAC_HD inline uint64_t fold_chunk_q(Acc s, const FoldChunk& ch) {
  using T = FoldTraits<Acc>;
  constexpr uint64_t kOne = 1ull << T::kFrac;
  const int32_t c = fold_exponent(s) - ch.k0;
  if (c < 0 || c >= kFoldCands || !((ch.clean >> c) & 1u)) return kFoldBad;
  const uint64_t Q = c == 0 ? ch.q[0] : c == 1 ? ch.q[1] : ch.q[2];
  return Q > 2 * kOne ? kFoldBad : Q;
}

// A run of chunks from s: with P_i the prefix sums of their fold_chunk_q,
// chunk i adds U * Q_i exactly while fold_units(s) + P_i <= 2^(F+1) - 1, so
// the run's partial sums are fold_with_units(s, fold_units(s) + P_i) and a
// wave applies 64 chunks with one prefix sum (each Q_i <= 2^(F+1), so P
// stays below 2^60).
template <typename Acc>
TAC_HD inline bool fold_run_fits(uint64_t m, uint64_t P) {
  using T = FoldTraits<Acc>;
  return m + P <= 2 * (1ull << T::kFrac) - 1;
}

// Applies a chunk with quantized sums: true (and *out) when the chunk adds
// exactly U * Q without leaving the accumulator's binade.
template <typename Acc>
TAC_HD inline bool fold_apply(Acc s, const FoldChunk& ch, Acc* out) {
  using T = FoldTraits<Acc>;
  using Bits = typename T::Bits;
  if (!fold_is_normal_positive(s)) return false;
  const int32_t c = fold_exponent(s) - ch.k0;
  if (c < 0 || c >= kFoldCands || !((ch.clean >> c) & 1u)) return false;
  const uint64_t Q = ch.q[c];
  // units of U: s = m * U with 2^F <= m < 2^(F+1); the binade ends at 2^(F+1) U
  constexpr uint64_t kOne = 1ull << T::kFrac;
  const Bits u = fold_bits(s);
  const uint64_t m = (uint64_t)(u & (Bits)(kOne - 1)) | kOne;
  if (Q > 2 * kOne || m + Q > 2 * kOne - 1) return false;
  *out = fold_from_bits<Acc>((Bits)((u & ~(Bits)(kOne - 1)) | (Bits)((m + Q) & (kOne - 1))));
  return true;
}

}  // namespace tacgpu
