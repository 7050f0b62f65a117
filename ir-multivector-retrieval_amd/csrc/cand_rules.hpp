// cand_rules.hpp — the scalar rules of the exact candidate-set assignment,
// shared by the GPU kernels (cand_kernels.hpp) and a host-side check
// (tests/native/cand_rules_check.cpp).  Plain C++ when compiled by a host
// compiler; compile with -ffp-contract=off either way.
//
// For an anchor codeword a and U2 = ref(x, c_a), the reference distance
// (src/util/vec.zig:109-175: D squares and D-1 adds, separately rounded):
//   * R2 = cand_radius(U2) >= 4 (U2 + eta) / (1 - g), g = gamma_{D+2};
//   * a neighbour key stores cand_lower_bound(ref(c_a, c)) <= ||c_a - c||^2
//     in its value bits and c << 4 in its low 14 bits (K <= 1024);
//   * every codeword that ties or beats c_a under ref() has a key value
//     <= R2, so the reference's first-index argmin lies in
//     {a} + {c : value(key(a, c)) <= R2}.
#pragma once

#include <stdint.h>
#include <string.h>

#ifndef TAC_HD
#if defined(__HIPCC__)
#define TAC_HD __host__ __device__
#else
#define TAC_HD
#endif
#endif

namespace tacgpu {

constexpr uint32_t kCandList = 128;   // neighbours kept per codeword (Lloyd iterations, dsub <= 4)
constexpr uint32_t kCandListWide = 64;  // the same past dsub 4, where items cost more
constexpr uint32_t kCandListEncode = 64;  // the same for encode (grid anchors)
constexpr uint32_t kCandSamples = 16; // row samples: entries 0, 7, 15, ..., 119
constexpr uint32_t kCandItem = 8;   // candidates per work item
constexpr uint32_t kCandMaxK = 1024; // codeword ids fit the key's low 14 bits as id << 4

TAC_HD inline uint32_t cand_f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
TAC_HD inline float cand_u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// gamma_n = n u / (1 - n u) with n = D + 2, u = 2^-24: relative error bound
// of the reference fold at sub-dimension D.
TAC_HD constexpr float cand_gamma(int D) {
  return (float)(D + 2) * 5.9604644775390625e-8f / (1.0f - (float)(D + 2) * 5.9604644775390625e-8f);
}

// Radius of the candidate ball: R2 >= 4 (U2 + eta) / (1 - g).  The x4 is
// exact, the factor covers g and the rounding of the product, the addend
// covers eta (< 1e-43).  Valid for 0 <= U2 < 1e37 (cand_tame).
TAC_HD inline float cand_radius(float U2, float g) { return (U2 * 4.0f) * (1.0f + 8.0f * g) + 1e-38f; }

// The bound arithmetic stays finite; false on NaN and inf.
TAC_HD inline bool cand_tame(float U2) { return U2 < 1e37f; }

// Lower bound of ||c_a - c||^2 from s = ref(c_a, c): >= (s - eta) / (1 + g)
// >= s (1 - 2g) - 1e-38 after rounding; clamped at 0 (NaN -> 0).
TAC_HD inline float cand_lower_bound(float s, float g) {
  const float lo = s * (1.0f - 2.0f * g) - 1e-38f;
  return lo > 0.0f ? lo : 0.0f;
}

// Key of neighbour c: the bound's bits with the low 14 bits replaced by
// c << 4 (the bound keeps 9 mantissa bits).  Clearing low bits of a
// non-negative float lowers it, so the value part stays a lower bound, and
// sorting keys sorts by bound, then by id.
constexpr uint32_t kCandValueMask = 0xFFFFC000u;
constexpr uint32_t kCandIdField = 0x3FF0u;  // c << 4
TAC_HD inline uint32_t cand_key(float lo, uint32_t c) {
  return (cand_f2u(lo) & kCandValueMask) | (c << 4);
}
TAC_HD inline float cand_key_value(uint32_t key) { return cand_u2f(key & kCandValueMask); }
TAC_HD inline uint32_t cand_key_code(uint32_t key) { return (key & kCandIdField) >> 4; }
constexpr uint32_t kCandNoKey = 0xFFFFFFFFu;  // value part is NaN: never inside R2
// Padding entry of anchor a's stored row: its value part is NaN, so no
// sample counts it, and its code is a, a real codeword, so an item that
// reads it evaluates a valid (distance, index) key.
TAC_HD inline uint32_t cand_pad_key(uint32_t a) { return kCandValueMask | (a << 4); }

// Row position of sample q: 0, 7, 15, ..., 119.  With b samples inside R2,
// every row entry inside R2 lies in [0, 8b): item q covers [8q, 8q + 8).
// Sample values never decrease along a row (keys are sorted, padding is NaN),
// so when sample 7 lies outside R2 so do samples 8-15.
TAC_HD inline uint32_t cand_sample_pos(uint32_t q) { return q ? 8u * q - 1u : 0u; }

// Value bits of sample q of a row of L kept keys (all-ones past the row).
TAC_HD inline uint32_t cand_sample(const uint32_t* row, uint32_t L, uint32_t q) {
  const uint32_t pos = cand_sample_pos(q);
  return pos < L ? row[pos] & kCandValueMask : kCandNoKey;
}

// Sample q as the top 16 bits of its value bits.  Clearing low bits of a
// non-negative float lowers it, so the truncated sample is a lower bound of
// the entry's value (NaN padding stays NaN): a count of truncated samples
// inside R2 is never below the count of the samples themselves.
TAC_HD inline uint16_t cand_sample16(const uint32_t* row, uint32_t L, uint32_t q) {
  return (uint16_t)(cand_sample(row, L, q) >> 16);
}
TAC_HD inline float cand_u16f(uint16_t h) { return cand_u2f((uint32_t)h << 16); }

// Samples a row of L kept keys has (positions below L): 1 + L / 8, at most
// kCandSamples.  Its items, 8 per sample, cover the stored row.
TAC_HD constexpr uint32_t cand_row_samples(uint32_t L) {
  return 1u + L / 8u < kCandSamples ? 1u + L / 8u : kCandSamples;
}

// Number of kCandItem-candidate items a vector needs from its anchor's row,
// given the row's kCandSamples truncated samples.  When b truncated samples
// are inside R2, at most b of the samples themselves are, so every row entry
// inside R2 lies in [0, 8b).  *deferred when every sample the row has counts
// as inside and the row is missing codewords (L + 1 < K): the candidate set
// may then extend past the row.
TAC_HD inline uint32_t cand_items16(const uint16_t (&samples)[kCandSamples], float R2,
                                    uint32_t L, bool row_complete, bool* deferred) {
  uint32_t nit = 0;
  for (uint32_t q = 0; q < kCandSamples; ++q) nit += cand_u16f(samples[q]) <= R2 ? 1u : 0u;
  *deferred = nit >= cand_row_samples(L) && !row_complete;
  return *deferred ? 0u : nit;
}

// The same count from the 8 words that hold the samples two to a word
// (sample 2w in the low half of word w).  A truncated sample h is inside R2
// exactly when h <= bits(R2) >> 16: h << 16 is a non-negative float or the
// NaN padding (0xFFFF, never inside), non-negative floats order as their
// bits, and R2 is finite and non-negative.  Samples never decrease along a
// row, so the count is found by a binary search: four probes find it up to
// 15, a fifth tells 15 from 16.  Every probe picks its word with selects on
// the bits found so far (no indexed register reads).
TAC_HD inline uint32_t cand_items_words(const uint32_t (&w)[8], float R2, uint32_t L,
                                        bool row_complete, bool* deferred) {
  const uint32_t lim = cand_f2u(R2) >> 16;
  uint32_t b = (w[3] >> 16) <= lim ? 8u : 0u;                     // sample 7
  const uint32_t w2 = b ? w[5] : w[1];                            // sample b + 3
  b += (w2 >> 16) <= lim ? 4u : 0u;
  const uint32_t lo3 = (b & 4u) ? w[2] : w[0], hi3 = (b & 4u) ? w[6] : w[4];
  const uint32_t w3 = (b & 8u) ? hi3 : lo3;                       // sample b + 1
  b += (w3 >> 16) <= lim ? 2u : 0u;
  const uint32_t a0 = (b & 2u) ? w[1] : w[0], a1 = (b & 2u) ? w[3] : w[2];
  const uint32_t a2 = (b & 2u) ? w[5] : w[4], a3 = (b & 2u) ? w[7] : w[6];
  const uint32_t a01 = (b & 4u) ? a1 : a0, a23 = (b & 4u) ? a3 : a2;
  const uint32_t w4 = (b & 8u) ? a23 : a01;                       // sample b
  b += (w4 & 0xFFFFu) <= lim ? 1u : 0u;
  b += (b == 15u && (w[7] >> 16) <= lim) ? 1u : 0u;               // sample 15
  *deferred = b >= cand_row_samples(L) && !row_complete;
  return *deferred ? 0u : b;
}

// Entry j of the row is a candidate when j < L and its value is inside R2.
TAC_HD inline bool cand_is_candidate(uint32_t key, uint32_t j, uint32_t L, float R2) {
  return j < L && cand_key_value(key) <= R2;
}

// Stored row length: the L kept keys padded with cand_pad_key to the end of
// the last item that the samples can select (16 items when L >= 120), so
// every item reads 8 entries without a bound check.
TAC_HD constexpr uint32_t cand_row_len(uint32_t L) {
  return 8u * (L / 8u + 1u < kCandSamples ? L / 8u + 1u : kCandSamples);
}

// True when a codeword whose anchor bound is lo (cand_lower_bound of its
// reference distance to c_a) cannot tie or beat c_a for a vector with
// U2 = ref(x, c_a): then ref(x, c) > U2.  k-means++ uses it to keep a weight
// without reading the vector.
TAC_HD inline bool cand_cannot_beat(float lo, float U2, float g) {
  return cand_tame(U2) && lo > cand_radius(U2, g);
}

// Lexicographic (distance bits, index) key, the index stored as c << 4 as
// in the neighbour keys: its minimum is the first-index argmin among
// non-negative distances.  The minimum over any set of codewords that holds
// the candidate set is the same, so evaluating extra codewords is harmless.
TAC_HD inline uint64_t cand_best_key(float d, uint32_t c) {
  return ((uint64_t)cand_f2u(d) << 32) | (c << 4);
}
TAC_HD inline uint32_t cand_best_code(uint64_t key) { return (uint32_t)key >> 4; }

}  // namespace tacgpu
