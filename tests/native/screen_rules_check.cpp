// Host check of the matrix-core screen's rules
// (ir-multivector-retrieval_amd/csrc/screen_rules.hpp, screen_kernels.hpp).
//
// 1. The bound.  The screen value of a vector x against a codeword c is the
//    fp32 sum of the accumulator input n = fl(sum_d c_d^2) and the 32 bf16
//    products (a_hi + a_lo) (x_hi + x_lo), a = -2 c, in an order the matrix
//    core chooses.  For random and adversarial pairs, with the pieces rounded
//    to nearest even (and, separately, with subnormal pieces flushed) and the
//    sum taken in several orders (slot order, reversed, pairwise, the
//    accumulator first or last, random permutations), |s~ - s| stays within
//    E = 2^-14 (1.07 ||x|| ||c|| + 0.04 ||c||^2) + 2^-123 (2 ||c|| + ||x||) + 2^-120,
//    s = ||c||^2 - 2 x.c in long double; a bound of E / 16 must fail.
// 2. The decision.  For random and adversarial codebooks (dsub 5-8, K 2-256,
//    duplicate and near-duplicate codewords, vectors on bisectors, far from
//    the codebook, scales 1e-30 to 1e17), the kernel's blocks of 8 codewords
//    and its test (screen_err, screen_separates): whenever the test settles
//    a vector, the reference's first-index argmin (the left fold of squared
//    differences, src/util/vec.zig:109-175, 271-283; also the 4-lane form at
//    dsub 8) lies in the winning block, and the (distance bits, index)
//    minimum over that block equals it.  Two planted mistakes must settle
//    some vector wrongly: a threshold of a thirty-second (the kernel's is
//    eight times the bound on one screen value, and the error of a
//    difference of two reaches about 0.6 of that bound), and a test without
//    the reference distance's rounding term.
// Build with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/screen_rules.hpp"

using namespace tacgpu;

static uint64_t lcg = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {
  lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
  return lcg ^ (lcg >> 29);
}
static double unit() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
static float gauss() {
  const double u1 = unit() + 1e-300, u2 = unit();
  return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

static float from_bits(uint32_t b) {
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
static uint32_t bits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return b;
}

// fp32 -> bf16 (round to nearest even) as a float; flush: subnormal inputs
// become 0 (the other behaviour the matrix core's conversion may have).
static float bf16r(float v, bool flush) {
  if (flush && v != 0.0f && std::fabs(v) < 1.17549435e-38f) return 0.0f;
  uint32_t b = bits(v);
  if ((b & 0x7F800000u) == 0x7F800000u) return v;
  b += 0x7FFFu + ((b >> 16) & 1u);
  return from_bits(b & 0xFFFF0000u);
}

// The screen's 33 terms for x against c (D dims): the accumulator input and
// the four products per dimension, each product formed in fp32 (exact but for
// underflow).
static void terms(const float* x, const float* c, int D, bool flush, float* t) {
  float n2 = c[0] * c[0];
  for (int d = 1; d < D; ++d) n2 = n2 + c[d] * c[d];
  t[0] = n2;
  int k = 1;
  for (int d = 0; d < D; ++d) {
    const float a = -2.0f * c[d];
    const float ah = bf16r(a, flush), al = bf16r(a - ah, flush);
    const float xh = bf16r(x[d], flush), xl = bf16r(x[d] - xh, flush);
    t[k++] = ah * xh;
    t[k++] = al * xh;
    t[k++] = ah * xl;
    t[k++] = al * xl;
  }
  for (; k < 33; ++k) t[k] = 0.0f;
}

// fp32 sums of the terms in one of several orders.
static float sum_order(const float* t, int order) {
  float s = 0.0f;
  switch (order) {
    case 0:  // accumulator first, slot order
      for (int k = 0; k < 33; ++k) s = s + t[k];
      return s;
    case 1:  // products first, the accumulator last
      for (int k = 1; k < 33; ++k) s = s + t[k];
      return s + t[0];
    case 2:  // reversed
      for (int k = 32; k >= 0; --k) s = s + t[k];
      return s;
    case 3: {  // pairwise over the products, then the accumulator
      float v[32];
      for (int k = 0; k < 32; ++k) v[k] = t[k + 1];
      for (int w = 32; w > 1; w /= 2)
        for (int k = 0; k < w / 2; ++k) v[k] = v[2 * k] + v[2 * k + 1];
      return t[0] + v[0];
    }
    case 4: {  // two chained halves (as two 16-slot instructions), each pairwise
      float v[16], w16[16];
      for (int k = 0; k < 16; ++k) {
        v[k] = t[1 + k];
        w16[k] = t[17 + k];
      }
      for (int w = 16; w > 1; w /= 2)
        for (int k = 0; k < w / 2; ++k) {
          v[k] = v[2 * k] + v[2 * k + 1];
          w16[k] = w16[2 * k] + w16[2 * k + 1];
        }
      return (t[0] + v[0]) + w16[0];
    }
    default: {  // a random permutation
      int p[33];
      for (int k = 0; k < 33; ++k) p[k] = k;
      for (int k = 32; k > 0; --k) std::swap(p[k], p[next_u64() % (k + 1)]);
      for (int k = 0; k < 33; ++k) s = s + t[p[k]];
      return s;
    }
  }
}

// s = ||c||^2 - 2 x.c, and the norms, in long double.
static long double exact_s(const float* x, const float* c, int D, long double* nx,
                           long double* nc) {
  long double c2 = 0, x2 = 0, xc = 0;
  for (int d = 0; d < D; ++d) {
    c2 += (long double)c[d] * c[d];
    x2 += (long double)x[d] * x[d];
    xc += (long double)x[d] * c[d];
  }
  *nx = std::sqrt(x2);
  *nc = std::sqrt(c2);
  return c2 - 2 * xc;
}

static long double bound_E(long double nx, long double nc) {
  return std::ldexp(1.07L * nx * nc + 0.04L * nc * nc, -14) + std::ldexp(2 * nc + nx, -123) +
         std::ldexp(1.0L, -120);
}

// The reference distance: the left fold (16 lanes, D <= 8), or at D = 8 the
// 4-lane form (lanes j and j + 4 paired, then the lane sums in order).
static float ref_dist(const float* x, const float* c, int D, bool lanes4) {
  if (lanes4 && D == 8) {
    float l[4];
    for (int j = 0; j < 4; ++j) {
      const float t0 = x[j] - c[j], t1 = x[j + 4] - c[j + 4];
      l[j] = t0 * t0;
      l[j] = l[j] + t1 * t1;
    }
    return ((l[0] + l[1]) + l[2]) + l[3];
  }
  float t = x[0] - c[0];
  float s = t * t;
  for (int k = 1; k < D; ++k) {
    const float u = x[k] - c[k];
    s = s + u * u;
  }
  return s;
}

// The kernel's block of codeword c: 32-codeword groups g, in each the lane
// half h = (c % 8) / 4 and the pair of 8-rows s = (c % 32) / 16.
static int block_of(int c) {
  const int g = c / 32, r = c % 32, h = (r / 4) % 2, s = (r / 8) / 2;
  return (2 * g + s) * 2 + h;
}

template <int D>
static bool separates_no_gamma(float b1, float b2, float x2, float ea) {
  float thr = 2.0f * ea;
  thr = 2.0f * thr + 1e-30f;
  (void)x2;
  return b2 == __builtin_inff() || (b2 - b1) > thr;
}

struct Counts {
  long bound_checks = 0, over = 0, planted_over = 0;
  double max_ratio = 0;
  long decisions = 0, deferred = 0, wrong = 0, planted_small = 0, planted_gamma = 0;
};

// One vector against one codebook: the screen's decision and, when it
// settles the vector, the check against the reference.  mode 0: the rules;
// 1: a thirty-second of the bound; 2: no rounding term.
template <int D>
static long decide(const float* x, const std::vector<float>& cb, int K, int order, bool flush,
                   bool lanes4, int mode) {
  float cmax2 = 0.0f;
  for (int c = 0; c < K; ++c) {
    float n2 = cb[c * D] * cb[c * D];
    for (int d = 1; d < D; ++d) n2 = n2 + cb[c * D + d] * cb[c * D + d];
    cmax2 = std::max(cmax2, n2);
  }
  if (!(cmax2 <= kScreenTame)) return -1;
  float x2 = x[0] * x[0];
  for (int d = 1; d < D; ++d) x2 = std::fma(x[d], x[d], x2);
  if (!(x2 <= kScreenTame)) return -1;
  const float cmax = std::sqrt(cmax2);
  const float nx = std::sqrt(std::max(x2, 7.888609052210118e-31f)) * 1.000001f;
  const int nblocks = ((K + 31) / 32) * 4;
  std::vector<float> bmin(nblocks, __builtin_inff());
  for (int c = 0; c < K; ++c) {
    float t[33];
    terms(x, &cb[c * D], D, flush, t);
    const float sv = sum_order(t, order);
    const int b = block_of(c);
    bmin[b] = std::min(bmin[b], sv);
  }
  float b1 = __builtin_inff(), b2 = __builtin_inff();
  int bb = 0;
  for (int b = 0; b < nblocks; ++b) {
    const float v = bmin[b];
    b2 = std::min(b2, std::max(b1, v));
    if (v < b1) bb = b;
    b1 = std::min(b1, v);
  }
  float ea = screen_err(nx, cmax, cmax2);
  bool ok;
  if (mode == 1) ea = ea / 32.0f;
  if (mode == 2)
    ok = separates_no_gamma<D>(b1, b2, x2, ea);
  else
    ok = screen_separates<D>(b1, b2, x2, ea);
  if (!ok) return -1;
  // the reference's first-index argmin over all codewords
  float best = ref_dist(x, &cb[0], D, lanes4);
  int bi = 0;
  for (int c = 1; c < K; ++c) {
    const float d = ref_dist(x, &cb[c * D], D, lanes4);
    if (d < best) {
      best = d;
      bi = c;
    }
  }
  // the (distance bits, index) minimum over the winning block
  uint64_t key = ~0ull;
  for (int c = 0; c < K; ++c)
    if (block_of(c) == bb) {
      const uint64_t k = ((uint64_t)bits(ref_dist(x, &cb[c * D], D, lanes4)) << 32) | (uint32_t)c;
      key = std::min(key, k);
    }
  const bool right = key != ~0ull && (int)(uint32_t)key == bi &&
                     (uint32_t)(key >> 32) == bits(best);
  return right ? 0 : 1;
}

// A component of magnitude scale (a power of two) times 1 + 2^-9 + j 2^-16 +
// 2^-17 - k 2^-23 (j < 128, k = 1, 2), random sign: its bf16 pieces are scale
// and scale (2^-9 + j 2^-16), missing it by scale (2^-17 - k 2^-23), about the
// most that two pieces can miss (half a unit of the second piece's last place).
static float aligned_component(float scale) {
  const int jj = (int)(next_u64() % 128), k = 1 + (int)(next_u64() % 2);
  const float f = 1.0f + std::ldexp(1.0f, -9) + std::ldexp((float)jj, -16) +
                  std::ldexp(1.0f, -17) - std::ldexp((float)k, -23);  // exact
  return f * scale * ((next_u64() & 1) ? -1.0f : 1.0f);
}

// The bound for one pair, in every summation order, where the screen applies
// (fl(||x||^2) and fl(||c||^2) at most 2^120).
template <int D>
static void check_bound(const float* x, const float* c, bool flush, Counts& ct) {
  float x2 = x[0] * x[0], c2 = c[0] * c[0];
  for (int d = 1; d < D; ++d) {
    x2 = std::fma(x[d], x[d], x2);
    c2 = c2 + c[d] * c[d];
  }
  if (!(x2 <= kScreenTame) || !(c2 <= kScreenTame)) return;
  float t[33];
  terms(x, c, D, flush, t);
  long double nx, nc;
  const long double s = exact_s(x, c, D, &nx, &nc);
  const long double E = bound_E(nx, nc);
  for (int o = 0; o < 7; ++o) {
    const long double err = std::fabs((long double)sum_order(t, o) - s);
    ++ct.bound_checks;
    if (err > E) ++ct.over;
    if (err > E / 16) ++ct.planted_over;
    ct.max_ratio = std::max(ct.max_ratio, (double)(err / E));
  }
}

template <int D>
static void check_decisions(const float* x, const std::vector<float>& cb, int K, int order,
                            bool flush, bool lanes4, Counts& ct) {
  const long r = decide<D>(x, cb, K, order, flush, lanes4, 0);
  ++ct.decisions;
  if (r < 0) ++ct.deferred;
  if (r > 0) ++ct.wrong;
  if (decide<D>(x, cb, K, order, flush, lanes4, 1) > 0) ++ct.planted_small;
  if (decide<D>(x, cb, K, order, flush, lanes4, 2) > 0) ++ct.planted_gamma;
}

template <int D>
static void run_dim(Counts& ct) {
  const int Ks[] = {2, 17, 31, 64, 100, 256};
  for (int K : Ks) {
    for (int rep = 0; rep < 60; ++rep) {
      const int kind = rep % 6;
      const float scale = std::pow(10.0f, -30.0f + 47.0f * (float)unit());
      std::vector<float> cb(K * D);
      for (auto& v : cb) v = gauss() * scale;
      if (kind == 1)  // duplicate codewords
        for (int c = K / 2; c < K; ++c)
          for (int d = 0; d < D; ++d) cb[c * D + d] = cb[(c - K / 2) * D + d];
      if (kind == 2)  // near-duplicates: the last bits differ
        for (int c = 1; c < K; c += 2)
          for (int d = 0; d < D; ++d)
            cb[c * D + d] = from_bits(bits(cb[(c - 1) * D + d]) + (uint32_t)(next_u64() % 5));
      float off[8] = {0};
      if (kind == 3)  // the codebook far from the origin (cancellation in the screen)
        for (int d = 0; d < D; ++d) off[d] = gauss() * scale * 300.0f;
      for (int c = 0; c < K; ++c)
        for (int d = 0; d < D; ++d) cb[c * D + d] += off[d];
      for (int q = 0; q < 40; ++q) {
        float x[8] = {0};
        const int vk = q % 4;
        if (vk == 0) {  // near a codeword
          const int c = (int)(next_u64() % K);
          for (int d = 0; d < D; ++d) x[d] = cb[c * D + d] + gauss() * scale * 0.1f;
        } else if (vk == 1) {  // near the bisector of two codewords
          const int a = (int)(next_u64() % K), b = (int)(next_u64() % K);
          for (int d = 0; d < D; ++d)
            x[d] = 0.5f * (cb[a * D + d] + cb[b * D + d]) + gauss() * scale * 1e-6f;
        } else if (vk == 2) {  // far from the codebook (the reference's rounding matters)
          for (int d = 0; d < D; ++d) x[d] = off[d] + gauss() * scale * 2000.0f;
        } else {
          for (int d = 0; d < D; ++d) x[d] = off[d] + gauss() * scale;
        }
        const int order = (int)(next_u64() % 7);
        const bool flush = (q & 8) != 0;
        const bool lanes4 = (q & 16) != 0;
        for (int c = 0; c < K; c += std::max(1, K / 8)) check_bound<D>(x, &cb[c * D], flush, ct);
        check_decisions<D>(x, cb, K, order, flush, lanes4, ct);
      }
    }
  }
  // Aligned pieces: every component of x loses close to the most that two
  // bf16 pieces can lose (2^-17 of it), with its own sign, so the screen
  // value of a x (a a power of two) is 4 a (sum_d x_d e_d) ~ 2^-15 a ||x||^2
  // above s.  c1 = 4 x (index 0) and c2 = -2 x (index 4, another block) are
  // at the same distance from x (9 ||x||^2, the same rounding), so the
  // reference takes c1, while the screen puts c1 about 3 2^-14 ||x||^2 above
  // c2: 0.6 of the bound at cmax = 4 ||x||, so a threshold a thirty-second
  // of the kernel's settles on c2.  Also c1 = 2 x, c2 = 0.  The other
  // codewords point away from x, with norms below ||x||.
  for (int rep = 0; rep < 400; ++rep) {
    const int K = 5 + (int)(next_u64() % 252);
    const float scale = std::ldexp(1.0f, -66 + (int)(next_u64() % 120));  // 2^-66 .. 2^53
    float x[8] = {0};
    for (int d = 0; d < D; ++d) x[d] = aligned_component(scale);
    std::vector<float> cb(K * D);
    for (int c = 0; c < K; ++c) {
      float g[8], dot = 0.0f;
      for (int d = 0; d < D; ++d) {
        g[d] = gauss();
        dot += g[d] * x[d];
      }
      for (int d = 0; d < D; ++d) cb[c * D + d] = (dot > 0 ? -g[d] : g[d]) * scale * 0.3f;
    }
    const float a1 = (rep & 4) ? 2.0f : 4.0f;
    for (int d = 0; d < D; ++d) {
      cb[0 * D + d] = a1 * x[d];
      cb[4 * D + d] = (2.0f - a1) * x[d];
    }
    const bool flush = (rep & 1) != 0, lanes4 = (rep & 2) != 0;
    const int order = (int)(next_u64() % 7);
    check_bound<D>(x, &cb[0], flush, ct);
    check_decisions<D>(x, cb, K, order, flush, lanes4, ct);
  }
  // Far vectors: ||x|| 2^15 to 2^21 times the codebook's scale, so the
  // reference distances round on a grid coarser than the screen's error and
  // near ties between codewords flip there (a test without that rounding
  // term settles some of them wrongly).
  for (int rep = 0; rep < 600; ++rep) {
    const int K = 8 + (int)(next_u64() % 249);
    const float scale = std::pow(10.0f, -12.0f + 20.0f * (float)unit());
    std::vector<float> cb(K * D);
    for (auto& v : cb) v = gauss() * scale;
    const float far = scale * std::ldexp(1.0f, 15 + (int)(next_u64() % 7));
    for (int q = 0; q < 40; ++q) {
      float x[8] = {0};
      for (int d = 0; d < D; ++d) x[d] = gauss() * far;
      const bool flush = (q & 1) != 0, lanes4 = (q & 2) != 0;
      const int order = (int)(next_u64() % 7);
      check_bound<D>(x, &cb[(q % K) * D], flush, ct);
      check_decisions<D>(x, cb, K, order, flush, lanes4, ct);
    }
  }
}

int main() {
  Counts ct;
  run_dim<5>(ct);
  run_dim<6>(ct);
  run_dim<7>(ct);
  run_dim<8>(ct);
  std::printf("screen_rules: %ld bound checks, %ld over the bound (largest error %.3f of it), "
              "%ld over a sixteenth; %ld decisions, %ld deferred, %ld wrong; planted: "
              "a thirty-second of the bound %ld wrong, no rounding term %ld wrong\n",
              ct.bound_checks, ct.over, ct.max_ratio, ct.planted_over, ct.decisions,
              ct.deferred, ct.wrong, ct.planted_small, ct.planted_gamma);
  const bool good = ct.over == 0 && ct.wrong == 0 && ct.planted_over > 0 &&
                    ct.planted_small > 0 && ct.planted_gamma > 0;
  return good ? 0 : 1;
}
