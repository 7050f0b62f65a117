// Host check of the candidate-set rules used by the GPU assignment and encode
// kernels (ir-multivector-retrieval_amd/csrc/cand_rules.hpp).  For random and
// adversarial codebooks and vectors, and for any anchor codeword, the
// candidate set that the rules select (neighbour rows of rounded-down bounds,
// 16 row samples truncated to 16 bits, item counts, the R2 radius, deferral)
// must contain the
// reference's first-index argmin (src/util/vec.zig:271-283 over the
// unfused fold of vec.zig:109-175), and the lexicographic (distance bits,
// index) minimum over it must equal that argmin and its distance bit for
// bit.  As the kernels do, every entry of every selected item is evaluated,
// candidate or not, with rows padded to cand_row_len(L) by cand_pad_key.  Two planted mistakes must fail: a radius of rho instead of 2 rho, and
// a tie rule that ignores the codeword index.  The k-means++ skip
// (cand_cannot_beat) is checked directly: whenever it holds for a codeword,
// that codeword's reference distance is strictly greater than the anchor's.
// Build with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/cand_rules.hpp"

using namespace tacgpu;

static uint64_t lcg = 0x2545F4914F6CDD1Dull;
static uint64_t next_u64() {
  lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
  return lcg ^ (lcg >> 29);
}
static double unit() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
static float gauss() {
  const double u1 = unit() + 1e-300, u2 = unit();
  return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

// The reference distance: left fold, every operation rounded separately.
static float fold(const float* x, const float* c, int D) {
  float t = x[0] - c[0];
  float s = t * t;
  for (int k = 1; k < D; ++k) {
    const float u = x[k] - c[k];
    const float q = u * u;
    s = s + q;
  }
  return s;
}

struct Counts {
  long checks = 0, deferred = 0, wrong = 0, planted_radius = 0, planted_ties = 0;
  long skip_checks = 0, skips = 0, skip_wrong = 0;
  long row_overrun = 0;
  long search_mismatch = 0, search_checks = 0;
};

// The binary search against the linear count on sorted sample rows built to
// put R2 on, just below and just above every sample (and NaN tails).
static void search_cases(Counts& ct) {
  for (int rep = 0; rep < 200000; ++rep) {
    uint16_t sv[kCandSamples];
    const uint32_t valid = (uint32_t)(next_u64() % 17);  // samples before the NaN tail
    uint16_t v = (uint16_t)(next_u64() % 0x7F00);
    for (uint32_t q = 0; q < kCandSamples; ++q) {
      if (q < valid) {
        v = (uint16_t)std::min<uint32_t>(0x7F7Fu, v + (uint32_t)(next_u64() % 3 == 0 ? 0 : next_u64() % 300));
        sv[q] = v;
      } else {
        sv[q] = 0xFFFF;
      }
    }
    const uint32_t pick = (uint32_t)(next_u64() % kCandSamples);
    const uint32_t base = valid ? sv[std::min(pick, valid - 1)] : (uint32_t)(next_u64() % 0x7F00);
    const int delta = (int)(next_u64() % 3) - 1;
    const uint32_t hi = (uint32_t)std::min<int64_t>(0x7F7F, std::max<int64_t>(0, (int64_t)base + delta));
    const float R2 = cand_u2f((hi << 16) | (uint32_t)(next_u64() & 0xFFFF));
    const uint32_t L = (uint32_t)(next_u64() % 200);
    const bool complete = next_u64() % 4 == 0;
    bool d1 = false, d2 = false;
    const uint32_t n1 = cand_items16(sv, R2, L, complete, &d1);
    uint32_t words[8];
    for (uint32_t q = 0; q < 8; ++q) words[q] = (uint32_t)sv[2 * q] | ((uint32_t)sv[2 * q + 1] << 16);
    const uint32_t n2 = cand_items_words(words, R2, L, complete, &d2);
    ++ct.search_checks;
    if (n1 != n2 || d1 != d2) ++ct.search_mismatch;
  }
}

static void run_case(const std::vector<float>& cb, int K, int D, const std::vector<float>& xs,
                     int n, uint32_t Lmax, Counts& ct) {
  const float g = cand_gamma(D);
  const uint32_t L = std::min<uint32_t>(Lmax, (uint32_t)K - 1);
  const bool row_complete = L + 1 >= (uint32_t)K;
  const uint32_t Lr = cand_row_len(L);
  std::vector<uint32_t> rows((size_t)K * Lr);
  std::vector<uint16_t> samples((size_t)K * kCandSamples);
  for (int a = 0; a < K; ++a) {
    std::vector<uint32_t> keys;
    for (int c = 0; c < K; ++c)
      if (c != a) keys.push_back(cand_key(cand_lower_bound(fold(&cb[a * D], &cb[c * D], D), g), c));
    std::sort(keys.begin(), keys.end());
    for (uint32_t j = 0; j < Lr; ++j) rows[(size_t)a * Lr + j] = j < L ? keys[j] : cand_pad_key(a);
    for (uint32_t q = 0; q < kCandSamples; ++q)
      samples[(size_t)a * kCandSamples + q] = cand_sample16(&rows[(size_t)a * Lr], L, q);
  }
  for (int i = 0; i < n; ++i) {
    const float* x = &xs[(size_t)i * D];
    // kmeans argmin: best = dists[0], strict < (vec.zig:271-283)
    float best = fold(x, &cb[0], D);
    int bi = 0;
    for (int c = 1; c < K; ++c) {
      const float d = fold(x, &cb[c * D], D);
      if (d < best) {
        best = d;
        bi = c;
      }
    }
    for (int rep = 0; rep < 3; ++rep) {
      const int a = rep == 0 ? (int)(next_u64() % K) : rep == 1 ? bi : (int)cand_key_code(rows[(size_t)bi * Lr]);
      const float U2 = fold(x, &cb[a * D], D);
      ++ct.checks;
      if (rep == 0)  // the k-means++ skip against every other codeword
        for (int c = 0; c < K; ++c) {
          if (c == a) continue;
          ++ct.skip_checks;
          if (cand_cannot_beat(cand_lower_bound(fold(&cb[a * D], &cb[c * D], D), g), U2, g)) {
            ++ct.skips;
            if (!(fold(x, &cb[c * D], D) > U2)) ++ct.skip_wrong;
          }
        }
      if (!cand_tame(U2)) {
        ++ct.deferred;
        continue;
      }
      const uint32_t* row = &rows[(size_t)a * Lr];
      uint16_t sv[kCandSamples];
      for (uint32_t q = 0; q < kCandSamples; ++q) sv[q] = samples[(size_t)a * kCandSamples + q];
      const float R2 = cand_radius(U2, g);
      bool deferred = false;
      const uint32_t nit = cand_items16(sv, R2, L, row_complete, &deferred);
      {  // the kernels' binary search over the packed words gives the same count
        uint32_t words[8];
        for (uint32_t q = 0; q < 8; ++q) words[q] = (uint32_t)sv[2 * q] | ((uint32_t)sv[2 * q + 1] << 16);
        bool d2 = false;
        const uint32_t n2 = cand_items_words(words, R2, L, row_complete, &d2);
        if (n2 != nit || d2 != deferred) ++ct.search_mismatch;
      }
      if (nit * kCandItem > Lr) ++ct.row_overrun;  // items must stay inside the stored row
      if (deferred) {
        ++ct.deferred;
        continue;
      }
      // Every entry of every selected item, candidate or not (the kernels).
      uint64_t key = cand_best_key(U2, a);
      for (uint32_t j = 0; j < nit * kCandItem && j < Lr; ++j) {
        const uint32_t c = cand_key_code(row[j]);
        const uint64_t kk = cand_best_key(fold(x, &cb[c * D], D), c);
        key = kk < key ? kk : key;
      }
      if ((int)cand_best_code(key) != bi || (uint32_t)(key >> 32) != cand_f2u(best)) ++ct.wrong;
      // Planted: radius rho^2 instead of 4 rho^2.
      {
        const float R2w = U2;
        uint64_t kw = cand_best_key(U2, a);
        for (uint32_t j = 0; j < L; ++j)
          if (cand_key_value(row[j]) <= R2w) {
            const uint32_t c = cand_key_code(row[j]);
            const uint64_t kk = cand_best_key(fold(x, &cb[c * D], D), c);
            kw = kk < kw ? kk : kw;
          }
        if ((int)cand_best_code(kw) != bi) ++ct.planted_radius;
      }
      // Planted: ties resolved by scan order (row order) instead of the index.
      {
        float bd = U2;
        uint32_t bc = a;
        for (uint32_t j = 0; j < nit * kCandItem; ++j) {
          const uint32_t k = row[j];
          if (!cand_is_candidate(k, j, L, R2)) continue;
          const uint32_t c = cand_key_code(k);
          const float d = fold(x, &cb[c * D], D);
          if (d < bd) {
            bd = d;
            bc = c;
          }
        }
        if ((int)bc != bi) ++ct.planted_ties;
      }
    }
  }
}

int main() {
  Counts ct;
  const int Ks[] = {2, 3, 17, 64, 65, 100, 256, 300, 1024};
  const double scales[] = {1.0, 1e-19, 1e-12, 1e15, 1e18};
  for (int D = 1; D <= 8; ++D)
    for (int K : Ks)
      for (double sc : scales)
        for (int pattern = 0; pattern < 3; ++pattern) {
          std::vector<float> cb((size_t)K * D);
          for (auto& v : cb) v = (float)(gauss() * 0.1 * sc);
          if (pattern == 1)  // duplicates: the second half repeats the first
            for (int c = K / 2; c < K; ++c)
              for (int k = 0; k < D; ++k) cb[c * D + k] = cb[(c - K / 2) * D + k];
          if (pattern == 2)  // few distinct points: many exact ties
            for (int c = 0; c < K; ++c)
              for (int k = 0; k < D; ++k) cb[c * D + k] = cb[(c % 5) * D + k];
          const int n = 300;
          std::vector<float> xs((size_t)n * D);
          for (int i = 0; i < n; ++i) {
            const int kind = i % 5;
            for (int k = 0; k < D; ++k) {
              float v = (float)(gauss() * 0.1 * sc);
              if (kind == 1) v = cb[(next_u64() % K) * D + k];                       // on a codeword
              if (kind == 2) v = (float)(cb[(i % K) * D + k] + gauss() * 1e-6 * sc);  // near one
              if (kind == 3) v = (float)(v * 1e3);                                    // outlier
              xs[(size_t)i * D + k] = v;
            }
          }
          // the Lloyd iterations' rows and encode's shorter ones
          run_case(cb, K, D, xs, n, kCandList, ct);
          run_case(cb, K, D, xs, n, kCandListEncode, ct);
        }
  std::printf("cand rules: %ld checks, %ld deferred, %ld wrong; planted radius: %ld wrong, "
              "planted ties: %ld wrong\n",
              ct.checks, ct.deferred, ct.wrong, ct.planted_radius, ct.planted_ties);
  std::printf("kmeans++ skip: %ld checks, %ld skips, %ld skip_wrong\n", ct.skip_checks, ct.skips,
              ct.skip_wrong);
  search_cases(ct);
  std::printf("items: row_overrun %ld\n", ct.row_overrun);
  std::printf("binary search: %ld checks, %ld search_mismatch\n", ct.search_checks, ct.search_mismatch);
  return ct.wrong == 0 && ct.skip_wrong == 0 && ct.skips > 0 && ct.planted_radius > 0 &&
                 ct.planted_ties > 0 && ct.row_overrun == 0 && ct.search_mismatch == 0
             ? 0
             : 1;
}
