// CPU check of the library's host-side TAC budget phases
// (ir-multivector-retrieval_amd/csrc/tac_phases.hpp, whose phase 4 walks the
// eligible tokens in remainder order) against the oracle's literal
// restatement of src/tac/tac.zig:97-401 (one centroid per loop step), on
// random vocabularies, spreads and thresholds, including infeasible budgets
// and invalid thresholds: the status must agree, and kappa when it succeeds.
#include <cstdio>
#include <random>
#include <vector>

#include "../../ir-multivector-retrieval_amd/csrc/tac_phases.hpp"
extern "C" {
#include "../../oracle/pq_oracle.h"
}

int main() {
  std::mt19937_64 rng(2024);
  int bad = 0, ok_runs = 0, err_runs = 0;
  for (int trial = 0; trial < 4000; ++trial) {
    const size_t nd = 1 + rng() % (trial % 10 == 0 ? 3000 : 60);
    std::vector<uint32_t> f(nd);
    std::vector<float> s(nd);
    const uint32_t mu = 1 + rng() % 8, tau = mu + (rng() % 6 == 0 ? 0 : 1 + rng() % 20);
    for (size_t j = 0; j < nd; ++j) {
      const uint64_t r = rng() % 10;
      f[j] = r < 2 ? 0 : r < 5 ? (uint32_t)(rng() % (tau + 1)) : (uint32_t)(tau + rng() % 500);
      s[j] = rng() % 7 == 0 ? 0.0f : std::uniform_real_distribution<float>(0.0f, 3.0f)(rng);
      if (rng() % 40 == 0) s[j] = (float)(rng() % 4);  // ties in the weights
    }
    if (trial % 13 == 0)
      for (auto& x : s) x = 0.0f;  // uniform fallback of phase 2
    uint64_t tail = 0, caps = 0;
    const uint32_t eps = 1 + rng() % 4, theta = 1 + rng() % 4;
    for (size_t j = 0; j < nd; ++j) {
      tail += f[j] == 0 ? 0 : f[j] < mu ? 1 : f[j] < tau ? 2 : 0;
      caps += f[j] >= tau ? f[j] / theta : 0;
    }
    const uint64_t span = tail + caps + 10;
    const uint32_t kt = (uint32_t)(rng() % 5 == 0 ? rng() % (span + 1) : tail + rng() % (caps + 1));
    orc_tac_params op{kt, mu, tau, eps, theta, 25, 1e-4f, 0, 1};
    std::vector<uint32_t> k1(nd, 0), k2(nd, 0);
    std::vector<float> frac(nd, 0.0f);
    const int st1 = orc_tac_allocate_budgets(f.data(), s.data(), nd, k1.data(), frac.data(), &op);
    const tacgpu::tacphase::Params pp{kt, mu, tau, eps, theta};
    const int st2 = tacgpu::tacphase::allocate(f, s, k2, pp);
    if (st1 != st2 || (st1 == 0 && k1 != k2)) {
      if (bad < 5) std::printf("MISMATCH trial %d nd %zu status %d vs %d\n", trial, nd, st1, st2);
      ++bad;
    }
    (st1 == 0 ? ok_runs : err_runs) += 1;
  }
  std::printf("%d mismatches over %d successful and %d failing allocations\n", bad, ok_runs,
              err_runs);
  std::printf("%s\n", bad ? "tac phases check FAILED" : "tac phases check passed");
  return bad ? 1 : 0;
}
