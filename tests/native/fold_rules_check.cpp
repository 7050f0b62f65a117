// CPU check of fold_rules.hpp: the chunked evaluation of a serial fp32 sum of
// non-negative terms must equal the plain serial fold bit for bit, on random
// and adversarial sequences (exact ties, zeros, huge and tiny terms, NaN and
// inf, long absorbed tails).  Built with -ffp-contract=off.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/fold_rules.hpp"

using namespace tacgpu;

static float serial(const std::vector<float>& e) {
  float s = 0.0f;
  for (float v : e) s = s + v;
  return s;
}

// Host emulation of the GPU passes: f64 chunk prefix -> candidate binades ->
// quantized sums -> sequential application with term-by-term fallback.
static float chunked(const std::vector<float>& e, uint64_t* fallbacks) {
  const size_t n = e.size();
  const size_t nc = (n + kFoldChunk - 1) / kFoldChunk;
  std::vector<double> pre(nc);
  double acc = 0.0;
  for (size_t j = 0; j < nc; ++j) {
    pre[j] = acc;
    for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) acc += (double)e[i];
  }
  float s = 0.0f;
  for (size_t j = 0; j < nc; ++j) {
    FoldChunk ch{};
    const float ps = (float)pre[j];
    ch.k0 = fold_is_normal_positive(ps) ? fold_exponent(ps) - 1 : -1000;
    uint32_t bad = 0;  // as the quantize kernel: every term, bad bits OR-ed
    for (int c = 0; c < kFoldCands; ++c) {
      uint64_t q = 0;
      for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) {
        const uint64_t qi = fold_quantize(e[i], ch.k0 + c);
        bad |= qi == kFoldBad ? 1u << c : 0u;
        q += qi == kFoldBad ? 0 : qi;
      }
      ch.q[c] = q;
    }
    ch.clean = ~bad & ((1u << kFoldCands) - 1u);
    float out;
    if (fold_apply(s, ch, &out)) {
      s = out;
    } else {
      ++*fallbacks;
      for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) s = s + e[i];
    }
  }
  return s;
}

static bool same(float a, float b) {
  uint32_t x, y;
  std::memcpy(&x, &a, 4);
  std::memcpy(&y, &b, 4);
  return x == y;
}

int main() {
  std::mt19937_64 rng(12345);
  int bad = 0;
  uint64_t fb = 0, chunks = 0;
  auto run = [&](const char* what, const std::vector<float>& e) {
    const float a = serial(e), b = chunked(e, &fb);
    chunks += (e.size() + kFoldChunk - 1) / kFoldChunk;
    if (!same(a, b)) {
      std::printf("MISMATCH %s n=%zu serial=%a chunked=%a\n", what, e.size(), a, b);
      ++bad;
    }
  };
  std::exponential_distribution<float> ex(1.0f);
  std::uniform_real_distribution<float> un(0.0f, 1.0f);
  for (int trial = 0; trial < 60; ++trial) {
    const size_t n = 1 + rng() % 300000;
    const float scale = std::ldexp(1.0f, (int)(rng() % 40) - 30);
    std::vector<float> e(n);
    for (auto& v : e) v = ex(rng) * scale;
    run("exponential", e);
    // exact ties: multiples of a power of two that land on half ulps
    for (auto& v : e) v = std::ldexp((float)(rng() % 64), (int)(rng() % 6) - 12);
    run("dyadic", e);
    // zeros and a few huge terms
    for (size_t i = 0; i < n; ++i) e[i] = (rng() % 5 == 0) ? 0.0f : un(rng) * scale;
    e[rng() % n] = 1e30f;
    run("huge", e);
    // subnormal start, then growth
    for (size_t i = 0; i < n; ++i) e[i] = i < 100 ? 1e-44f : un(rng);
    run("subnormal", e);
  }
  {
    std::vector<float> e(50000, 1.0f);
    e[30000] = std::nanf("");
    run("nan", e);
    e[30000] = INFINITY;
    run("inf", e);
    std::vector<float> z(70000, 0.0f);
    run("zeros", z);
    std::vector<float> t(300000, 1e-8f);  // absorbed once s is large enough
    t[0] = 1.0f;
    run("absorbed", t);
    std::vector<float> h(300000, 0.5f);  // every term a half-ulp tie at 2^24
    h[0] = 16777216.0f;
    run("half-ulp", h);
  }
  std::printf("%d mismatches; %llu of %llu chunks folded term by term\n", bad,
              (unsigned long long)fb, (unsigned long long)chunks);
  std::printf("%s\n", bad ? "fold rules check FAILED" : "fold rules check passed");
  return bad ? 1 : 0;
}
