// CPU check of fold_rules.hpp: the chunked evaluation of a serial sum of
// non-negative float terms, with an fp32 or an f64 accumulator, must equal
// the plain serial fold bit for bit, on random and adversarial sequences
// (exact ties, zeros, huge and tiny terms, NaN and inf, long absorbed
// tails).  The chunk descriptors are applied both one by one and in runs of
// 64 with one prefix sum per run, as the GPU wave applies them; the two must
// agree with each other, chunk starts included, and with the serial fold.
// The f64 case also mirrors the k-means++ fallback's search (first u < cum
// through the exact chunk start values) against the plain weightedSample
// loop.  Built with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/fold_rules.hpp"

using namespace tacgpu;

template <typename Acc>
static Acc serial(const std::vector<float>& e) {
  Acc s = 0;
  for (float v : e) s = s + (Acc)v;
  return s;
}

// Host restatement of the GPU passes: f64 chunk prefix -> candidate binades
// -> quantized sums (every term, spoiled candidates OR-ed into a mask, as
// the quantize waves do).
template <typename Acc>
static std::vector<FoldChunk> describe(const std::vector<float>& e) {
  const size_t n = e.size();
  const size_t nc = (n + kFoldChunk - 1) / kFoldChunk;
  std::vector<double> pre(nc);
  double acc = 0.0;
  for (size_t j = 0; j < nc; ++j) {
    pre[j] = acc;
    for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) acc += (double)e[i];
  }
  std::vector<FoldChunk> out(nc);
  for (size_t j = 0; j < nc; ++j) {
    FoldChunk ch{};
    const Acc ps = (Acc)pre[j];
    ch.k0 = fold_is_normal_positive(ps) ? fold_exponent(ps) - 1 : -100000;
    uint32_t bad = 0;
    for (int c = 0; c < kFoldCands; ++c) {
      uint64_t q = 0;
      for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) {
        const uint64_t qi = fold_quantize<Acc>(e[i], ch.k0 + c);
        bad |= qi == kFoldBad ? 1u << c : 0u;
        q += qi == kFoldBad ? 0 : qi;
      }
      ch.q[c] = q;
    }
    ch.clean = ~bad & ((1u << kFoldCands) - 1u);
    out[j] = ch;
  }
  return out;
}

// Sequential application with term-by-term fallback; `starts` receives the
// exact value before every chunk.
template <typename Acc>
static Acc chunked(const std::vector<float>& e, uint64_t* fallbacks, std::vector<Acc>* starts) {
  const size_t n = e.size();
  const std::vector<FoldChunk> chs = describe<Acc>(e);
  const size_t nc = chs.size();
  if (starts) starts->assign(nc, 0);
  Acc s = 0;
  for (size_t j = 0; j < nc; ++j) {
    if (starts) (*starts)[j] = s;
    Acc out;
    if (fold_apply(s, chs[j], &out)) {
      s = out;
    } else {
      ++*fallbacks;
      for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) s = s + (Acc)e[i];
    }
  }
  return s;
}

// The wave's procedure: from s, up to 64 chunks at once through the prefix
// sums of fold_chunk_q while fold_run_fits holds; the first chunk that does
// not fit (or any chunk while s is not normal) is folded term by term.
template <typename Acc>
static Acc chunked_runs(const std::vector<float>& e, std::vector<Acc>* starts) {
  const size_t n = e.size();
  const std::vector<FoldChunk> chs = describe<Acc>(e);
  const size_t nc = chs.size();
  if (starts) starts->assign(nc, 0);
  Acc s = 0;
  size_t j = 0;
  while (j < nc) {
    const size_t cnt = std::min<size_t>(64, nc - j);
    size_t b = 0;
    if (fold_is_normal_positive(s)) {
      const uint64_t m = fold_units(s);
      uint64_t P = 0;
      for (; b < cnt; ++b) {
        const uint64_t Q = fold_chunk_q(s, chs[j + b]);
        if (Q == kFoldBad || !fold_run_fits<Acc>(m, P + Q)) break;
        if (starts) (*starts)[j + b] = fold_with_units(s, m + P);
        P += Q;
      }
      if (b > 0) s = fold_with_units(s, m + P);
    }
    j += b;
    if (b < cnt) {
      if (starts) (*starts)[j] = s;
      for (size_t i = j * kFoldChunk; i < std::min(n, (j + 1) * kFoldChunk); ++i) s = s + (Acc)e[i];
      ++j;
    }
  }
  return s;
}

// weightedSample after its checks (rng.zig:70-81), given the draw r.
static size_t sample_serial(const std::vector<float>& w, double r) {
  const double total = serial<double>(w);
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

// The fallback kernel's steps: exact total and chunk starts, first chunk
// whose end exceeds u, term-by-term fold inside it.
static size_t sample_chunked(const std::vector<float>& w, double r, uint64_t* fb) {
  std::vector<double> starts;
  const double total = chunked<double>(w, fb, &starts);
  const double u = r * total;
  const size_t nc = starts.size();
  for (size_t j = 0; j < nc; ++j) {
    const double end = j + 1 < nc ? starts[j + 1] : total;
    if (u < end) {
      double cum = starts[j];
      for (size_t i = j * kFoldChunk; i < std::min(w.size(), (j + 1) * kFoldChunk); ++i) {
        cum += (double)w[i];
        if (u < cum) return i;
      }
      return ~(size_t)0;  // unreachable when the starts are exact
    }
  }
  size_t last = w.size() - 1;
  while (last > 0 && w[last] == 0.0f) --last;
  return last;
}

template <typename T>
static bool same(T a, T b) {
  return std::memcmp(&a, &b, sizeof(T)) == 0;
}

int main() {
  std::mt19937_64 rng(12345);
  int bad = 0;
  uint64_t fb32 = 0, fb64 = 0, chunks = 0;
  auto run = [&](const char* what, const std::vector<float>& e) {
    chunks += (e.size() + kFoldChunk - 1) / kFoldChunk;
    const float a = serial<float>(e), b = chunked<float>(e, &fb32, nullptr);
    if (!same(a, b)) {
      std::printf("MISMATCH f32 %s n=%zu serial=%a chunked=%a\n", what, e.size(), a, b);
      ++bad;
    }
    const double c = serial<double>(e), d = chunked<double>(e, &fb64, nullptr);
    if (!same(c, d)) {
      std::printf("MISMATCH f64 %s n=%zu serial=%a chunked=%a\n", what, e.size(), c, d);
      ++bad;
    }
    // runs of 64 chunks, with the chunk starts
    std::vector<float> s32a, s32b;
    std::vector<double> s64a, s64b;
    uint64_t unused = 0;
    (void)chunked<float>(e, &unused, &s32a);
    (void)chunked<double>(e, &unused, &s64a);
    const float r32 = chunked_runs<float>(e, &s32b);
    const double r64 = chunked_runs<double>(e, &s64b);
    bool starts_ok = s32a.size() == s32b.size() && s64a.size() == s64b.size();
    for (size_t j = 0; starts_ok && j < s32a.size(); ++j) starts_ok = same(s32a[j], s32b[j]);
    for (size_t j = 0; starts_ok && j < s64a.size(); ++j) starts_ok = same(s64a[j], s64b[j]);
    if (!same(a, r32) || !same(c, r64) || !starts_ok) {
      std::printf("MISMATCH runs %s n=%zu\n", what, e.size());
      ++bad;
    }
  };
  std::exponential_distribution<float> ex(1.0f);
  std::uniform_real_distribution<float> un(0.0f, 1.0f);
  for (int trial = 0; trial < 40; ++trial) {
    const size_t n = 1 + rng() % 300000;
    const float scale = std::ldexp(1.0f, (int)(rng() % 40) - 30);
    std::vector<float> e(n);
    for (auto& v : e) v = ex(rng) * scale;
    run("exponential", e);
    // exact ties: multiples of a power of two that land on half ulps
    for (auto& v : e) v = std::ldexp((float)(rng() % 64), (int)(rng() % 6) - 12);
    run("dyadic", e);
    // f64 ties: tiny dyadic terms after a large first term
    for (size_t i = 0; i < n; ++i) e[i] = i == 0 ? 1e9f : std::ldexp(1.0f, -(int)(rng() % 30) - 1);
    run("dyadic-f64", e);
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
    std::vector<float> g(300000, 0x1p-30f);  // f64 half-ulp ties at 2^23
    g[0] = 0x1p23f;
    run("half-ulp-f64", g);
  }
  // weightedSample through the chunk starts
  uint64_t fbs = 0;
  int draws = 0;
  for (int trial = 0; trial < 30; ++trial) {
    const size_t n = 1 + rng() % 200000;
    std::vector<float> w(n);
    for (auto& v : w) v = (rng() % 7 == 0) ? 0.0f : ex(rng) * 0.01f;
    if (trial % 5 == 0)  // a zero tail
      for (size_t i = n - n / 3; i < n; ++i) w[i] = 0.0f;
    w[0] = trial % 3 == 0 ? 0.0f : w[0];
    if (serial<double>(w) <= 0.0) continue;
    for (int d = 0; d < 40; ++d) {
      const double r = d == 0 ? std::nextafter(1.0, 0.0)
                       : d == 1 ? 0.0
                                : std::uniform_real_distribution<double>(0.0, 1.0)(rng);
      const size_t a = sample_serial(w, r), b = sample_chunked(w, r, &fbs);
      ++draws;
      if (a != b) {
        std::printf("MISMATCH sample n=%zu r=%a serial=%zu chunked=%zu\n", n, r, a, b);
        ++bad;
      }
    }
  }
  std::printf("%d mismatches; of %llu chunks, %llu (f32) and %llu (f64) folded term by term; "
              "%d draws\n",
              bad, (unsigned long long)chunks, (unsigned long long)fb32, (unsigned long long)fb64,
              draws);
  std::printf("%s\n", bad ? "fold rules check FAILED" : "fold rules check passed");
  return bad ? 1 : 0;
}
