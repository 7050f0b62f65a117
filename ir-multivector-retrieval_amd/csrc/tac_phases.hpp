// tac_phases.hpp — host side of token-aware clustering (src/tac/tac.zig):
// the CSR grouping of input rows by token id (:575-602) and the four budget
// phases (:97-401) that turn per-token frequencies and spreads into kappa_j.
// Plain C++, scalar: N_T is a vocabulary (tens of thousands of tokens).
#pragma once

#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

namespace tacgpu {
namespace tacphase {

enum Tier { kEmpty, kMicro, kSmall, kActive };

// Status values shared with include/tac_gpu.h.
constexpr int kOk = 0, kBudgetTooSmall = 21, kBudgetTooLarge = 22, kInvalidThresholds = 23;

// tac.zig:77-82
inline Tier classify(uint32_t n, uint32_t mu, uint32_t tau) {
  return n == 0 ? kEmpty : n < mu ? kMicro : n < tau ? kSmall : kActive;
}

struct Params {
  uint32_t kappa_total, mu, tau, epsilon, theta;
};

// Phase 1 (tac.zig:97-126): micro tokens get 1, small tokens 2; returns the
// budget left for active tokens in *active_budget.
inline int tail(const std::vector<uint32_t>& f, std::vector<uint32_t>& kappa, const Params& p,
                uint32_t* active_budget) {
  if (p.mu == 0 || p.tau == 0 || p.mu >= p.tau) return kInvalidThresholds;
  uint64_t used = 0;
  for (size_t j = 0; j < f.size(); ++j) {
    const Tier t = classify(f[j], p.mu, p.tau);
    kappa[j] = t == kMicro ? 1u : t == kSmall ? 2u : 0u;
    used += kappa[j];
  }
  if (used > p.kappa_total) return kBudgetTooSmall;
  *active_budget = p.kappa_total - (uint32_t)used;
  return kOk;
}

// Phase 2 (tac.zig:157-217): kappa_j = floor((w_j / sum w) * B) with the
// damped weight w_j = sqrt(f32(n_j)) * s_j (f32), sums and targets in f64,
// the fractional remainder kept (as f32) for phase 4.
inline int damped(const std::vector<uint32_t>& f, const std::vector<float>& s,
                  std::vector<uint32_t>& kappa, std::vector<float>& frac, uint32_t budget,
                  const Params& p) {
  for (auto& x : frac) x = 0.0f;
  double sum_w = 0.0;
  uint32_t n_active = 0;
  for (size_t j = 0; j < f.size(); ++j) {
    if (classify(f[j], p.mu, p.tau) != kActive) continue;
    const float w = sqrtf((float)f[j]) * s[j];
    if (!isfinite(w) || w < 0.0f) return kInvalidThresholds;
    sum_w += (double)w;
    ++n_active;
  }
  if (n_active == 0) return kOk;
  if (sum_w <= 0.0) {  // every active spread 0: equal shares, leftovers to the lowest ids
    const uint32_t base = budget / n_active;
    uint32_t left = budget - base * n_active;
    for (size_t j = 0; j < f.size(); ++j) {
      if (classify(f[j], p.mu, p.tau) != kActive) continue;
      kappa[j] = base + (left > 0 ? 1u : 0u);
      if (left > 0) --left;
    }
    return kOk;
  }
  for (size_t j = 0; j < f.size(); ++j) {
    if (classify(f[j], p.mu, p.tau) != kActive) continue;
    const double w = (double)(sqrtf((float)f[j]) * s[j]);
    const double target = (w / sum_w) * (double)budget;
    const uint32_t k = (uint32_t)floor(target);
    kappa[j] = k;
    frac[j] = (float)(target - (double)k);
  }
  return kOk;
}

// Phase 3 (tac.zig:236-258): epsilon <= kappa_j <= floor(n_j / theta).
inline int bound(const std::vector<uint32_t>& f, std::vector<uint32_t>& kappa, const Params& p) {
  if (p.epsilon == 0 || p.theta == 0) return kInvalidThresholds;
  if ((uint64_t)p.tau < (uint64_t)p.epsilon * p.theta) return kInvalidThresholds;
  for (size_t j = 0; j < f.size(); ++j) {
    if (classify(f[j], p.mu, p.tau) != kActive) continue;
    const uint32_t cap = f[j] / p.theta;
    if (kappa[j] < p.epsilon) kappa[j] = p.epsilon;
    if (kappa[j] > cap) kappa[j] = cap;
  }
  return kOk;
}

// Phase 4 (tac.zig:286-372): one centroid at a time to the active token with
// the largest remainder below its cap (surplus), or from the active token
// with the smallest remainder above the floor (deficit; then small 2 -> 1,
// then micro 1 -> 0, lowest id first).  Ties go to the lowest token id.
// The remainders never change and a token stays eligible until it reaches
// its cap (floor), so the token chosen first keeps being chosen until then:
// the loop is the same as walking the eligible tokens once, in order of
// remainder (then id), each taking as many steps as it has room for.
inline int reconcile(const std::vector<uint32_t>& f, std::vector<uint32_t>& kappa,
                     const std::vector<float>& frac, const Params& p) {
  uint64_t cur = 0;
  for (uint32_t k : kappa) cur += k;
  if (cur == p.kappa_total) return kOk;
  const size_t n = f.size();
  std::vector<uint32_t> order;
  if (cur < p.kappa_total) {
    uint64_t left = p.kappa_total - cur;
    for (size_t j = 0; j < n; ++j)
      if (classify(f[j], p.mu, p.tau) == kActive && kappa[j] < f[j] / p.theta)
        order.push_back((uint32_t)j);
    std::stable_sort(order.begin(), order.end(),
                     [&](uint32_t a, uint32_t b) { return frac[a] > frac[b]; });
    for (uint32_t j : order) {
      if (left == 0) break;
      const uint64_t room = f[j] / p.theta - kappa[j];
      const uint64_t take = room < left ? room : left;
      kappa[j] += (uint32_t)take;
      left -= take;
    }
    return left == 0 ? kOk : kBudgetTooLarge;
  }
  uint64_t excess = cur - p.kappa_total;
  for (size_t j = 0; j < n; ++j)
    if (classify(f[j], p.mu, p.tau) == kActive && kappa[j] > p.epsilon)
      order.push_back((uint32_t)j);
  std::stable_sort(order.begin(), order.end(),
                   [&](uint32_t a, uint32_t b) { return frac[a] < frac[b]; });
  for (uint32_t j : order) {
    if (excess == 0) break;
    const uint64_t room = kappa[j] - p.epsilon;
    const uint64_t take = room < excess ? room : excess;
    kappa[j] -= (uint32_t)take;
    excess -= take;
  }
  for (size_t j = 0; j < n && excess > 0; ++j)
    if (classify(f[j], p.mu, p.tau) == kSmall && kappa[j] == 2) {
      kappa[j] = 1;
      --excess;
    }
  for (size_t j = 0; j < n && excess > 0; ++j)
    if (classify(f[j], p.mu, p.tau) == kMicro && kappa[j] == 1) {
      kappa[j] = 0;
      --excess;
    }
  return excess == 0 ? kOk : kBudgetTooSmall;
}

// Phases 1-4 (tac.zig:388-401).
inline int allocate(const std::vector<uint32_t>& f, const std::vector<float>& s,
                    std::vector<uint32_t>& kappa, const Params& p) {
  std::vector<float> frac(f.size(), 0.0f);
  uint32_t budget = 0;
  int st = tail(f, kappa, p, &budget);
  if (st == kOk) st = damped(f, s, kappa, frac, budget, p);
  if (st == kOk) st = bound(f, kappa, p);
  if (st == kOk) st = reconcile(f, kappa, frac, p);
  return st;
}

}  // namespace tacphase
}  // namespace tacgpu
