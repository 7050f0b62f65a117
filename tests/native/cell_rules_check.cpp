// Host check of the cell-list encode rules (ir-multivector-retrieval_amd/
// csrc/cell_rules.hpp).  Grids are set up from a box as the build kernels do,
// coarse and fine lists are built as the build kernels build them (coarse
// anchor = the nearest codeword to the coarse box's centre, fine anchor = the
// nearest coarse-list codeword to the fine box's centre), and for random and
// adversarial vectors (on codewords, near bisectors of codeword pairs, on and
// around cell edges, subnormal and large scales, duplicate and lattice
// codebooks) two things must hold:
//   * a vector that cell_coord places in a cell lies inside the cell's
//     cell_interval box;
//   * the cell's list holds the reference's first-index argmin
//     (src/util/vec.zig:271-283 over the fold of vec.zig:109-175), and the
//     lexicographic (distance bits, index) minimum over the list, padded with
//     the fine anchor to whole items as the kernels pad it, equals it bit for
//     bit.
// Two planted mistakes must fail: exclusion without the rounding margin
// (g = 0, no slack), and cell intervals without the (1 +- u)^2 widening.
// Build with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/cell_rules.hpp"

using namespace tacgpu;

static uint64_t lcg = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {
  lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
  return lcg ^ (lcg >> 29);
}
static double unit() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
static double gauss() {
  const double u1 = unit() + 1e-300, u2 = unit();
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}
static uint32_t f2u(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

// The reference distance at D <= 4: left fold, every operation rounded.
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
  long checks = 0, outside = 0, box_miss = 0, wrong = 0, planted_margin = 0,
       planted_interval = 0, entries = 0, cells = 0;
};

template <int D>
struct Grid {
  const std::vector<float>& cb;
  int K;
  float lo[D], s[D];
  double g;
  bool planted_margin;
  std::map<uint32_t, std::vector<int>> coarse;   // coarse id -> list
  std::map<uint32_t, std::vector<int>> fine;     // fine id -> list (anchor first)
  Grid(const std::vector<float>& cb_, int K_, bool pm) : cb(cb_), K(K_), planted_margin(pm) {
    g = pm ? 0.0 : cell_gamma(D);
  }
  void box(const uint32_t (&k0)[D], const uint32_t (&k1)[D], double (&a)[D], double (&b)[D]) {
    for (int j = 0; j < D; ++j) cell_interval(lo[j], s[j], k0[j], k1[j], &a[j], &b[j]);
  }
  bool excluded(const double (&c)[D], const double (&c0)[D], double mt0, const double (&a)[D],
                const double (&b)[D]) {
    if (!planted_margin) return cell_excluded<D>(c, c0, mt0, a, b, g);
    double lin = 0.0;
    for (int j = 0; j < D; ++j) {
      const double dc = c[j] - c0[j];
      const double p = dc > 0.0 ? b[j] : a[j];
      lin += dc * ((c[j] + c0[j]) - 2.0 * p);
    }
    return lin > 0.0;
  }
  void cw(int c, double (&v)[D]) {
    for (int j = 0; j < D; ++j) v[j] = (double)cb[(size_t)c * D + j];
  }
  int nearest(const double (&p)[D], const std::vector<int>* among) {
    int best = -1;
    double bd = 0;
    const int n = among ? (int)among->size() : K;
    for (int q = 0; q < n; ++q) {
      const int c = among ? (*among)[q] : q;
      double v[D], t = 0;
      cw(c, v);
      for (int j = 0; j < D; ++j) t += (p[j] - v[j]) * (p[j] - v[j]);
      if (best < 0 || t < bd) {
        bd = t;
        best = c;
      }
    }
    return best;
  }
  const std::vector<int>& coarse_list(const uint32_t (&kc)[D]) {
    constexpr uint32_t Gc = cell_coarse_side(D), Gs = cell_sub_side(D);
    uint32_t id = 0;
    for (int j = D - 1; j >= 0; --j) id = id * Gc + kc[j];
    auto it = coarse.find(id);
    if (it != coarse.end()) return it->second;
    uint32_t k0[D], k1[D];
    for (int j = 0; j < D; ++j) {
      k0[j] = kc[j] * Gs;
      k1[j] = k0[j] + Gs;
    }
    double a[D], b[D], m[D];
    box(k0, k1, a, b);
    for (int j = 0; j < D; ++j) m[j] = 0.5 * (a[j] + b[j]);
    const int c0 = nearest(m, nullptr);
    double v0[D];
    cw(c0, v0);
    const double mt0 = cell_max_t<D>(v0, a, b);
    std::vector<int> out;
    for (int c = 0; c < K; ++c) {
      double v[D];
      cw(c, v);
      if (!excluded(v, v0, mt0, a, b)) out.push_back(c);
    }
    return coarse[id] = out;
  }
  const std::vector<int>& fine_list(const uint32_t (&k)[D]) {
    constexpr uint32_t Gs = cell_sub_side(D);
    const uint32_t id = cell_id<D>(k);
    auto it = fine.find(id);
    if (it != fine.end()) return it->second;
    uint32_t kc[D], k1[D];
    for (int j = 0; j < D; ++j) {
      kc[j] = k[j] / Gs;
      k1[j] = k[j] + 1;
    }
    const std::vector<int> cl = coarse_list(kc);
    double a[D], b[D], m[D];
    box(k, k1, a, b);
    for (int j = 0; j < D; ++j) m[j] = 0.5 * (a[j] + b[j]);
    const int c0 = nearest(m, &cl);
    double v0[D];
    cw(c0, v0);
    const double mt0 = cell_max_t<D>(v0, a, b);
    std::vector<int> out{c0};
    for (int c : cl) {
      double v[D];
      cw(c, v);
      if (c != c0 && !excluded(v, v0, mt0, a, b)) out.push_back(c);
    }
    return fine[id] = out;
  }
};

template <int D>
static void run_case(const std::vector<float>& cb, int K, double scale, Counts& ct) {
  // The grid box: the codebook box widened three times about its centre
  // (as mean +- 3 sigma of data would widen it).
  double lo[D], hi[D];
  for (int j = 0; j < D; ++j) {
    lo[j] = hi[j] = cb[j];
    for (int c = 1; c < K; ++c) {
      lo[j] = std::min(lo[j], (double)cb[(size_t)c * D + j]);
      hi[j] = std::max(hi[j], (double)cb[(size_t)c * D + j]);
    }
    const double mid = 0.5 * (lo[j] + hi[j]), half = 0.5 * (hi[j] - lo[j]);
    lo[j] = mid - 3 * half - 0.05 * scale;
    hi[j] = mid + 3 * half + 0.05 * scale;
  }
  Grid<D> grid(cb, K, false), bad(cb, K, true);
  for (int j = 0; j < D; ++j) {
    if (!cell_grid_params(lo[j], hi[j], cell_side(D), &grid.lo[j], &grid.s[j])) return;
    bad.lo[j] = grid.lo[j];
    bad.s[j] = grid.s[j];
  }
  const int n = 600;
  for (int i = 0; i < n; ++i) {
    float x[D];
    const int kind = i % 6;
    const int c1 = (int)(next_u64() % K), c2 = (int)(next_u64() % K);
    for (int j = 0; j < D; ++j) {
      double v = lo[j] + (hi[j] - lo[j]) * unit();
      if (kind == 1) v = cb[(size_t)c1 * D + j];
      if (kind == 2)  // near the bisector of two codewords
        v = 0.5 * ((double)cb[(size_t)c1 * D + j] + cb[(size_t)c2 * D + j]) +
            gauss() * 1e-7 * scale;
      if (kind == 3 || kind == 4) {  // on or beside a cell edge
        const uint32_t k = (uint32_t)(next_u64() % (cell_side(D) + 1));
        float e = grid.lo[j] + (float)k / grid.s[j];
        const int steps = kind == 3 ? 0 : (int)(next_u64() % 5) - 2;
        for (int q = 0; q < std::abs(steps); ++q) e = std::nextafter(e, steps > 0 ? 1e30f : -1e30f);
        v = e;
      }
      if (kind == 5) v = (double)cb[(size_t)c1 * D + j] + gauss() * 0.02 * scale;
      x[j] = (float)v;
    }
    uint32_t k[D];
    bool inside = true;
    for (int j = 0; j < D; ++j) {
      bool in;
      k[j] = cell_coord(x[j], grid.lo[j], grid.s[j], cell_side(D), &in);
      inside = inside && in;
    }
    if (!inside) {
      ++ct.outside;
      continue;
    }
    ++ct.checks;
    // the vector lies in its cell's box, and in the planted box?
    for (int j = 0; j < D; ++j) {
      double a, b;
      cell_interval(grid.lo[j], grid.s[j], k[j], k[j] + 1, &a, &b);
      if (!((double)x[j] >= a && (double)x[j] <= b)) ++ct.box_miss;
      const double pa = (double)grid.lo[j] + (double)k[j] / (double)grid.s[j];
      const double pb = (double)grid.lo[j] + (double)(k[j] + 1) / (double)grid.s[j];
      if (!((double)x[j] >= pa && (double)x[j] <= pb)) ++ct.planted_interval;
    }
    float best = fold(x, &cb[0], D);
    int bi = 0;
    for (int c = 1; c < K; ++c) {
      const float d = fold(x, &cb[(size_t)c * D], D);
      if (d < best) {
        best = d;
        bi = c;
      }
    }
    const std::vector<int>& L = grid.fine_list(k);
    ct.entries += (long)L.size();
    ++ct.cells;
    // the kernels' evaluation: every entry, padded with the anchor to whole items
    const size_t padded = (L.size() + kCellItem - 1) / kCellItem * kCellItem;
    uint64_t key = ~0ull;
    for (size_t q = 0; q < padded; ++q) {
      const int c = q < L.size() ? L[q] : L[0];
      const uint64_t kk = ((uint64_t)f2u(fold(x, &cb[(size_t)c * D], D)) << 32) | (uint32_t)c;
      key = kk < key ? kk : key;
    }
    if ((int)(uint32_t)key != bi || (uint32_t)(key >> 32) != f2u(best)) ++ct.wrong;
    const std::vector<int>& P = bad.fine_list(k);
    if (std::find(P.begin(), P.end(), bi) == P.end()) ++ct.planted_margin;
  }
}

template <int D>
static void sweep(Counts& ct) {
  const int Ks[] = {2, 3, 17, 64, 256};
  const double scales[] = {1.0, 1e-19, 1e-12, 1e10, 1e14};
  for (int K : Ks)
    for (double sc : scales)
      for (int pattern = 0; pattern < 4; ++pattern) {
        std::vector<float> cb((size_t)K * D);
        for (auto& v : cb) v = (float)(gauss() * 0.1 * sc);
        if (pattern == 1)  // duplicates
          for (int c = K / 2; c < K; ++c)
            for (int j = 0; j < D; ++j) cb[(size_t)c * D + j] = cb[(size_t)(c - K / 2) * D + j];
        if (pattern == 2)  // few distinct points
          for (int c = 0; c < K; ++c)
            for (int j = 0; j < D; ++j) cb[(size_t)c * D + j] = cb[(size_t)(c % 5) * D + j];
        if (pattern == 3)  // a lattice: exact ties on the bisectors
          for (int c = 0; c < K; ++c)
            for (int j = 0; j < D; ++j)
              cb[(size_t)c * D + j] = (float)((double)((next_u64() % 4)) * 0.03125 * sc);
        run_case<D>(cb, K, sc, ct);
      }
}

int main() {
  Counts ct;
  sweep<1>(ct);
  sweep<2>(ct);
  sweep<3>(ct);
  sweep<4>(ct);
  std::printf("cell rules: %ld checks (%ld outside the grid), %ld box_miss, %ld wrong; "
              "mean list %.2f; planted margin: %ld wrong, planted interval: %ld box_miss\n",
              ct.checks, ct.outside, ct.box_miss, ct.wrong,
              ct.cells ? (double)ct.entries / (double)ct.cells : 0.0, ct.planted_margin,
              ct.planted_interval);
  return ct.wrong == 0 && ct.box_miss == 0 && ct.planted_margin > 0 && ct.planted_interval > 0 &&
                 ct.checks > 100000
             ? 0
             : 1;
}
