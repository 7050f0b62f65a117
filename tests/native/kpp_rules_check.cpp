// Host check of the k-means++ rules used by the GPU seeding kernels
// (ir-multivector-retrieval_amd/csrc/kpp_rules.hpp):
//   1. the restated Zig PRNG (stream, uintLessThan, float(f64)) agrees with
//      the oracle's independent restatement (oracle/pq_oracle.c);
//   2. whenever kpp_decides() accepts a candidate computed from prefix sums
//      in a different summation order, it is the index the reference's
//      sequential f64 weightedSample (src/util/rng.zig:57-82) returns —
//      including draws aimed at the cumulative boundaries themselves.
#include <cmath>
#include <cstdio>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/kpp_rules.hpp"
#include "../../oracle/pq_oracle.h"

using namespace tacgpu;

static uint64_t lcg = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {
  lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
  return lcg ^ (lcg >> 29);
}
static double unit() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }

// rng.zig:57-82 with the draw given
static uint64_t reference_pick(const std::vector<float>& w, double r) {
  double total = 0.0;
  for (float x : w) total += (double)x;
  const double u = r * total;
  double cum = 0.0;
  for (size_t i = 0; i < w.size(); ++i) {
    cum += (double)w[i];
    if (u < cum) return i;
  }
  size_t last = w.size() - 1;
  while (last > 0 && w[last] == 0.0f) --last;
  return last;
}

// prefix sums in another order: pairwise within blocks of 64, blocks in order
static std::vector<double> other_order_prefix(const std::vector<float>& w) {
  std::vector<double> p(w.size());
  double base = 0.0;
  for (size_t b = 0; b < w.size(); b += 64) {
    const size_t e = std::min(w.size(), b + 64);
    double run = 0.0;
    for (size_t i = b; i < e; ++i) {  // local running sum, then offset
      run += (double)w[i];
      p[i] = base + run;
    }
    double tree[64] = {0};
    for (size_t i = b; i < e; ++i) tree[i - b] = (double)w[i];
    for (int s = 1; s < 64; s <<= 1)
      for (int i = 0; i + s < 64; i += 2 * s) tree[i] += tree[i + s];
    base += tree[0];
  }
  return p;
}

int main() {
  int bad = 0;
  // 1. PRNG agreement with the oracle's restatement
  const uint64_t seeds[] = {0, 1, 42, 0xa1b2c3d4ull + 7, ~0ull, 0x52017};
  for (uint64_t seed : seeds) {
    uint64_t s[4];
    uint64_t sm = seed;
    for (int q = 0; q < 4; ++q) s[q] = kpp_splitmix(&sm);
    orc_xoshiro r;
    orc_zig_prng_init(&r, seed);
    for (int k = 0; k < 2000; ++k) {
      const int what = k % 3;
      if (what == 0) bad += kpp_next(s) != orc_zig_next(&r);
      if (what == 1) {
        const uint64_t n = 1 + (next_u64() % 5000000);
        bad += kpp_uint_less_than(s, n) != orc_zig_uint_less_than(&r, n);
      }
      if (what == 2) {
        const double a = kpp_float64(s), b = orc_zig_float_f64(&r);
        bad += memcmp(&a, &b, sizeof a) != 0;
      }
    }
  }
  std::printf("prng: %s\n", bad ? "MISMATCH" : "agrees with the oracle restatement");

  // 2. decision rule
  uint64_t decided = 0, undecided = 0, wrong = 0, aimed = 0;
  for (int trial = 0; trial < 3000; ++trial) {
    const size_t n = 1 + next_u64() % (trial % 10 == 0 ? 20000 : 300);
    std::vector<float> w(n);
    const int kind = trial % 4;
    for (auto& x : w) {
      if (kind == 0) x = (float)unit();
      if (kind == 1) x = (float)std::pow(10.0, -30.0 + 60.0 * unit());  // 60 decades
      if (kind == 2) x = (next_u64() % 3 == 0) ? 0.0f : (float)unit();
      if (kind == 3) x = (next_u64() % 2) ? 1.0f : 1e-9f;
    }
    if (kind == 2) w[next_u64() % n] = 1.0f;  // at least one positive
    const std::vector<double> p = other_order_prefix(w);
    const double t = p[n - 1];
    for (int d = 0; d < 8; ++d) {
      double r = unit();
      if (d >= 4) {  // aim the draw at a cumulative boundary
        const size_t k = next_u64() % n;
        r = p[k] / t;
        if (d == 5) r = std::nextafter(r, 0.0);
        if (d == 6) r = std::nextafter(r, 2.0);
        if (r >= 1.0) r = std::nextafter(1.0, 0.0);
        ++aimed;
      }
      const double u = r * t;
      size_t i = n;
      for (size_t q = 0; q < n; ++q)
        if (u < p[q]) {
          i = q;
          break;
        }
      if (i == n) {
        ++undecided;  // the kernel falls back on the tail rule
        continue;
      }
      const double prev = i ? p[i - 1] : 0.0;
      if (kpp_decides(r, t, n, i, prev, p[i])) {
        ++decided;
        if (reference_pick(w, r) != i) {
          ++wrong;
          if (wrong < 5) std::printf("wrong: trial %d n %zu i %zu ref %llu\n", trial, n, i,
                                     (unsigned long long)reference_pick(w, r));
        }
      } else {
        ++undecided;
      }
    }
  }
  std::printf("decision: %llu decided, %llu to the sequential fallback (%llu aimed draws), %llu wrong\n",
              (unsigned long long)decided, (unsigned long long)undecided, (unsigned long long)aimed,
              (unsigned long long)wrong);
  bad += (int)wrong;
  std::printf("%s\n", bad ? "kpp rules check FAILED" : "kpp rules check passed");
  return bad ? 1 : 0;
}
