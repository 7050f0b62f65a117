// kpp_rules.hpp — the scalar rules of k-means++ seeding, shared by the GPU
// kernels (kmeanspp.hpp) and a host-side check: the restated Zig std.Random
// stream (src/util/rng.zig:22-44 over std.Random.DefaultPrng) and the band
// test that decides weightedSample (src/util/rng.zig:57-82) from parallel
// prefix sums.  Plain C++ when compiled by a host compiler.
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

// ---- Zig std.Random restated: SplitMix64 seeding, Xoshiro256++ --------------
TAC_HD inline uint64_t kpp_splitmix(uint64_t* s) {
  *s += 0x9e3779b97f4a7c15ull;
  uint64_t z = *s;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

TAC_HD inline uint64_t kpp_rotl(uint64_t x, int k) {
  return (x << k) | (x >> (64 - k));
}

TAC_HD inline uint64_t kpp_next(uint64_t* s) {
  const uint64_t out = kpp_rotl(s[0] + s[3], 23) + s[0];
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = kpp_rotl(s[3], 45);
  return out;
}

TAC_HD inline uint64_t kpp_mulhi(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(a, b);
#else
  return (uint64_t)(((unsigned __int128)a * b) >> 64);
#endif
}

TAC_HD inline int kpp_clz(uint64_t x) {
#ifdef __HIP_DEVICE_COMPILE__
  return x == 0 ? 64 : __clzll((long long)x);
#else
  return x == 0 ? 64 : __builtin_clzll(x);
#endif
}

// Random.uintLessThan over 64 bits (multiply-shift with threshold rejection).
TAC_HD inline uint64_t kpp_uint_less_than(uint64_t* s, uint64_t less_than) {
  uint64_t x = kpp_next(s);
  uint64_t hi = kpp_mulhi(x, less_than), lo = x * less_than;
  if (lo < less_than) {
    uint64_t t = (uint64_t)0 - less_than;
    if (t >= less_than) {
      t -= less_than;
      if (t >= less_than) t %= less_than;
    }
    while (lo < t) {
      x = kpp_next(s);
      hi = kpp_mulhi(x, less_than);
      lo = x * less_than;
    }
  }
  return hi;
}

// Random.float(f64): 52 mantissa bits, geometric exponent from leading zeros.
TAC_HD inline double kpp_float64(uint64_t* s) {
  const uint64_t rnd = kpp_next(s);
  int64_t lz = kpp_clz(rnd);
  if (lz >= 12) {
    lz = 12;
    for (;;) {
      const int64_t add = kpp_clz(kpp_next(s));
      lz += add;
      if (add != 64) break;
      if (lz >= 1022) {
        lz = 1022;
        break;
      }
    }
  }
  const uint64_t bits = ((uint64_t)(1022 - lz) << 52) | (rnd & 0xFFFFFFFFFFFFFull);
  double out;
  memcpy(&out, &bits, sizeof out);
  return out;
}

// ---- the decision rule, shared by the kernel and the host-side unit test ---

// Half-width of the band around a rounded prefix sum of i + 1 non-negative
// terms whose (approximate) value is p: both the reference's sequential f64
// fold and any other summation order sit within (i + 1) 2^-53 p of the exact
// sum; 2.1 covers the two of them plus the rounding of this expression.
TAC_HD inline double kpp_band(uint64_t i, double p) {
  return 2.1 * (double)(i + 1) * 1.1102230246251565e-16 * p + 1e-300;
}

// Given the draw r, the approximate total t over n terms, the candidate i
// (first index with r * t < p_i) and the approximate prefixes p_prev = P_{i-1}
// (0 when i == 0) and p_i, decide whether the reference's weightedSample
// must return i: u = fl(r * T_seq) must lie below every possible cum_i and at
// or above every possible cum_{i-1}.
TAC_HD inline bool kpp_decides(double r, double t, uint64_t n, uint64_t i,
                                            double p_prev, double p_i) {
  const double bt = kpp_band(n, t);
  const double u_lo = r * (t - bt) * (1.0 - 4.5e-16);  // covers fl(r * T) rounding
  const double u_hi = r * (t + bt) * (1.0 + 4.5e-16);
  const bool below_i = u_hi < p_i - kpp_band(i, p_i);
  const bool above_prev = (i == 0) ? true : (u_lo >= p_prev + kpp_band(i - 1, p_prev));
  return below_i && above_prev;
}

}  // namespace tacgpu
