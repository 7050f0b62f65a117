/*
 * tac_oracle.c — CPU restatement of the reference's token-aware clustering
 * (src/tac/tac.zig), test infrastructure only: the parity checker for the
 * HIP library's TAC path.  Nothing in the shipped library links it.
 *
 *   orc_tac_allocate_tail     tac.zig:97-126   (Phase 1, tail handling)
 *   orc_tac_damped_phase2     tac.zig:133-217  (Phase 2, damped weights)
 *   orc_tac_bound_phase3      tac.zig:236-258  (Phase 3, floor and cap)
 *   orc_tac_reconcile_phase4  tac.zig:286-372  (Phase 4, reconciliation)
 *   orc_tac_allocate_budgets  tac.zig:388-401
 *   orc_tac_spreads           tac.zig:604-638  (Welford, per token)
 *   orc_tac_cluster_flat      tac.zig:563-830  (driver; per-token kmeans.fit
 *                             through orc_kmeans_fit, runOneTokenKmeans
 *                             :458-513)
 *
 * Compiled with -ffp-contract=off: every operation rounds on its own.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "pq_oracle.h"

enum { TIER_EMPTY, TIER_MICRO, TIER_SMALL, TIER_ACTIVE };

/* tac.zig:77-82 */
static int classify(uint32_t n_j, uint32_t mu, uint32_t tau) {
  if (n_j == 0) return TIER_EMPTY;
  if (n_j < mu) return TIER_MICRO;
  if (n_j < tau) return TIER_SMALL;
  return TIER_ACTIVE;
}

int orc_tac_allocate_tail(const uint32_t *freqs, uint64_t n, uint32_t *kappa, uint32_t mu,
                          uint32_t tau, uint32_t kappa_total, uint32_t *budget_active) {
  if (mu == 0 || tau == 0 || mu >= tau) return ORC_INVALID_THRESHOLDS;
  uint32_t tail = 0; /* u32 as in the reference; a sum past 2^32 would trap there */
  for (uint64_t j = 0; j < n; ++j) {
    switch (classify(freqs[j], mu, tau)) {
      case TIER_MICRO: kappa[j] = 1; tail += 1; break;
      case TIER_SMALL: kappa[j] = 2; tail += 2; break;
      default: kappa[j] = 0; break;
    }
  }
  if (tail > kappa_total) return ORC_BUDGET_TOO_SMALL;
  *budget_active = kappa_total - tail;
  return ORC_OK;
}

/* tac.zig:133-135: sqrt(f32(n_j)) * s_j in f32. */
static float damped_weight(uint32_t n_j, float s_j) { return sqrtf((float)n_j) * s_j; }

int orc_tac_damped_phase2(const uint32_t *freqs, const float *spreads, uint64_t n,
                          uint32_t *kappa, float *frac, uint32_t budget_active, uint32_t mu,
                          uint32_t tau) {
  for (uint64_t j = 0; j < n; ++j) frac[j] = 0.0f;
  double sum_w = 0.0;
  uint32_t n_active = 0;
  for (uint64_t j = 0; j < n; ++j) {
    if (classify(freqs[j], mu, tau) != TIER_ACTIVE) continue;
    const float w = damped_weight(freqs[j], spreads[j]);
    if (!isfinite(w) || w < 0.0f) return ORC_INVALID_THRESHOLDS;
    sum_w += (double)w;
    n_active += 1;
  }
  if (n_active == 0) return ORC_OK;
  if (sum_w <= 0.0) { /* uniform fallback in token-id order (:188-200) */
    const uint32_t base = budget_active / n_active;
    uint32_t leftover = budget_active - base * n_active;
    for (uint64_t j = 0; j < n; ++j) {
      if (classify(freqs[j], mu, tau) != TIER_ACTIVE) continue;
      kappa[j] = base;
      if (leftover > 0) {
        kappa[j] += 1;
        leftover -= 1;
      }
    }
    return ORC_OK;
  }
  const double b = (double)budget_active;
  for (uint64_t j = 0; j < n; ++j) {
    if (classify(freqs[j], mu, tau) != TIER_ACTIVE) continue;
    const double w = (double)damped_weight(freqs[j], spreads[j]);
    const double target = (w / sum_w) * b;
    const double fl = floor(target);
    const uint32_t k = (uint32_t)fl;
    kappa[j] = k;
    frac[j] = (float)(target - (double)k);
  }
  return ORC_OK;
}

int orc_tac_bound_phase3(const uint32_t *freqs, uint64_t n, uint32_t *kappa, uint32_t mu,
                         uint32_t tau, uint32_t epsilon, uint32_t theta) {
  if (epsilon == 0 || theta == 0) return ORC_INVALID_THRESHOLDS;
  /* tau < epsilon * theta (u32 product; an overflow would trap in the reference) */
  if ((uint64_t)tau < (uint64_t)epsilon * theta) return ORC_INVALID_THRESHOLDS;
  for (uint64_t j = 0; j < n; ++j) {
    if (classify(freqs[j], mu, tau) != TIER_ACTIVE) continue;
    const uint32_t cap = freqs[j] / theta;
    if (kappa[j] < epsilon) kappa[j] = epsilon;
    if (kappa[j] > cap) kappa[j] = cap;
  }
  return ORC_OK;
}

int orc_tac_reconcile_phase4(const uint32_t *freqs, uint64_t n, uint32_t *kappa,
                             const float *frac, uint32_t kappa_total, uint32_t mu, uint32_t tau,
                             uint32_t epsilon, uint32_t theta) {
  uint64_t current = 0;
  for (uint64_t j = 0; j < n; ++j) current += kappa[j];
  if (current == kappa_total) return ORC_OK;
  if (current < kappa_total) { /* surplus: grow the largest remainder (:300-321) */
    uint32_t remaining = (uint32_t)(kappa_total - current);
    while (remaining > 0) {
      int64_t best = -1;
      float best_frac = -INFINITY;
      for (uint64_t j = 0; j < n; ++j) {
        if (classify(freqs[j], mu, tau) != TIER_ACTIVE) continue;
        const uint32_t cap = freqs[j] / theta;
        if (kappa[j] >= cap) continue;
        if (frac[j] > best_frac || (frac[j] == best_frac && best < 0)) {
          best = (int64_t)j;
          best_frac = frac[j];
        }
      }
      if (best < 0) return ORC_BUDGET_TOO_LARGE;
      kappa[best] += 1;
      remaining -= 1;
    }
    return ORC_OK;
  }
  uint32_t excess = (uint32_t)(current - kappa_total); /* deficit (:324-371) */
  while (excess > 0) {
    int64_t best = -1;
    float best_frac = INFINITY;
    for (uint64_t j = 0; j < n; ++j) { /* step 1: shrinkable actives, smallest remainder */
      if (classify(freqs[j], mu, tau) != TIER_ACTIVE) continue;
      if (kappa[j] <= epsilon) continue;
      if (frac[j] < best_frac) {
        best = (int64_t)j;
        best_frac = frac[j];
      }
    }
    if (best >= 0) {
      kappa[best] -= 1;
      excess -= 1;
      continue;
    }
    int64_t found = -1; /* step 2: the first small token at 2 drops to 1 */
    for (uint64_t j = 0; j < n && found < 0; ++j)
      if (classify(freqs[j], mu, tau) == TIER_SMALL && kappa[j] == 2) found = (int64_t)j;
    if (found >= 0) {
      kappa[found] = 1;
      excess -= 1;
      continue;
    }
    for (uint64_t j = 0; j < n && found < 0; ++j) /* step 3: the first micro token drops to 0 */
      if (classify(freqs[j], mu, tau) == TIER_MICRO && kappa[j] == 1) found = (int64_t)j;
    if (found >= 0) {
      kappa[found] = 0;
      excess -= 1;
      continue;
    }
    return ORC_BUDGET_TOO_SMALL;
  }
  return ORC_OK;
}

int orc_tac_allocate_budgets(const uint32_t *freqs, const float *spreads, uint64_t n,
                             uint32_t *kappa, float *frac, const orc_tac_params *p) {
  uint32_t b = 0;
  int st = orc_tac_allocate_tail(freqs, n, kappa, p->mu, p->tau, p->kappa_total, &b);
  if (st) return st;
  if ((st = orc_tac_damped_phase2(freqs, spreads, n, kappa, frac, b, p->mu, p->tau))) return st;
  if ((st = orc_tac_bound_phase3(freqs, n, kappa, p->mu, p->tau, p->epsilon, p->theta)))
    return st;
  return orc_tac_reconcile_phase4(freqs, n, kappa, frac, p->kappa_total, p->mu, p->tau,
                                  p->epsilon, p->theta);
}

void orc_tac_spreads(const float *vectors, uint32_t dim, const uint32_t *group_offsets,
                     const uint32_t *group_indices, uint64_t n_distinct, float *spreads) {
  float *mean = malloc(sizeof(float) * dim);
  float *m2 = malloc(sizeof(float) * dim);
  for (uint64_t j = 0; j < n_distinct; ++j) {
    spreads[j] = 0.0f;
    const uint32_t lo = group_offsets[j], hi = group_offsets[j + 1];
    if (hi == lo) continue;
    memset(mean, 0, sizeof(float) * dim);
    memset(m2, 0, sizeof(float) * dim);
    float count = 0.0f;
    for (uint32_t q = lo; q < hi; ++q) {
      const float *v = vectors + (uint64_t)group_indices[q] * dim;
      count = count + 1.0f;
      const float inv = 1.0f / count;
      for (uint32_t d = 0; d < dim; ++d) {
        const float x = v[d];
        const float old = mean[d];
        const float delta = x - old;
        mean[d] = old + delta * inv;
        m2[d] = m2[d] + delta * (x - mean[d]);
      }
    }
    float trace = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) trace = trace + m2[d];
    spreads[j] = trace / (float)(hi - lo);
  }
  free(mean);
  free(m2);
}

int orc_tac_cluster_flat(const uint32_t *token_ids, uint64_t n_tokens, const float *vectors,
                         uint64_t vectors_len, uint32_t dim, const orc_tac_params *p,
                         float *centroids,
                         uint32_t *assignments, uint32_t *kappa_per_token, float *wcss_total,
                         uint64_t *n_distinct_out) {
  if (n_tokens == 0) return ORC_EMPTY_TOKEN_DUMP;
  if (dim == 0) return ORC_INVALID_THRESHOLDS;
  if (vectors_len != n_tokens * (uint64_t)dim) return ORC_INVALID_THRESHOLDS;
  if (p->kappa_total == 0) return ORC_BUDGET_TOO_SMALL;
  uint32_t max_id = 0;
  for (uint64_t i = 0; i < n_tokens; ++i)
    if (token_ids[i] > max_id) max_id = token_ids[i];
  const uint64_t nd = (uint64_t)max_id + 1;
  if (n_distinct_out) *n_distinct_out = nd;
  int st = ORC_OK;
  uint32_t *freqs = calloc(nd, sizeof(uint32_t));
  uint32_t *offs = malloc(sizeof(uint32_t) * (nd + 1));
  uint32_t *idx = malloc(sizeof(uint32_t) * n_tokens);
  uint32_t *cursor = malloc(sizeof(uint32_t) * nd);
  float *spreads = malloc(sizeof(float) * nd);
  float *frac = malloc(sizeof(float) * nd);
  uint32_t *goff = malloc(sizeof(uint32_t) * (nd + 1));
  float *gather = NULL, *cent = NULL;
  uint32_t *asg = NULL;
  float *chunk_w = NULL;
  if (!freqs || !offs || !idx || !cursor || !spreads || !frac || !goff) {
    st = ORC_OUT_OF_MEMORY;
    goto done;
  }
  for (uint64_t i = 0; i < n_tokens; ++i) freqs[token_ids[i]] += 1;
  offs[0] = 0;
  for (uint64_t j = 0; j < nd; ++j) offs[j + 1] = offs[j] + freqs[j];
  memcpy(cursor, offs, sizeof(uint32_t) * nd);
  for (uint64_t i = 0; i < n_tokens; ++i) idx[cursor[token_ids[i]]++] = (uint32_t)i;
  orc_tac_spreads(vectors, dim, offs, idx, nd, spreads);
  if ((st = orc_tac_allocate_budgets(freqs, spreads, nd, kappa_per_token, frac, p))) goto done;
  for (uint64_t j = 0; j < nd; ++j)
    if (freqs[j] > 0 && kappa_per_token[j] == 0) {
      st = ORC_BUDGET_TOO_SMALL;
      goto done;
    }
  goff[0] = 0;
  for (uint64_t j = 0; j < nd; ++j) goff[j + 1] = goff[j] + kappa_per_token[j];
  if (goff[nd] != p->kappa_total) {
    st = ORC_BUDGET_TOO_SMALL;
    goto done;
  }
  uint32_t max_n = 0, max_k = 0;
  for (uint64_t j = 0; j < nd; ++j) {
    if (freqs[j] > max_n) max_n = freqs[j];
    if (kappa_per_token[j] > max_k) max_k = kappa_per_token[j];
  }
  gather = malloc(sizeof(float) * (uint64_t)max_n * dim);
  cent = malloc(sizeof(float) * (uint64_t)(max_k ? max_k : 1) * dim);
  asg = malloc(sizeof(uint32_t) * (max_n ? max_n : 1));
  /* wcss_total: the serial path folds the per-token wcss in token order
   * (:681-703); with n_threads > 1 each thread folds its contiguous slice of
   * token ids from 0 and the slices are folded in thread order (:806-811). */
  const uint32_t nt = p->n_threads > 1 ? p->n_threads : 1;
  const uint64_t chunk = nt > 1 ? (nd + nt - 1) / nt : nd;
  chunk_w = calloc(nt, sizeof(float));
  if (!gather || !cent || !asg || !chunk_w) {
    st = ORC_OUT_OF_MEMORY;
    goto done;
  }
  for (uint64_t j = 0; j < nd; ++j) {
    const uint32_t k = kappa_per_token[j], n = freqs[j];
    if (k == 0 || n == 0) continue;
    for (uint32_t w = 0; w < n; ++w)
      memcpy(gather + (uint64_t)w * dim, vectors + (uint64_t)idx[offs[j] + w] * dim,
             sizeof(float) * dim);
    float wcss = 0.0f;
    uint32_t iters = 0;
    st = orc_kmeans_fit(gather, n, dim, k, p->max_iters, p->tol, p->seed ^ (uint64_t)j, 1, NULL,
                        cent, asg, &wcss, &iters, NULL);
    if (st) goto done;
    memcpy(centroids + (uint64_t)goff[j] * dim, cent, sizeof(float) * (uint64_t)k * dim);
    for (uint32_t w = 0; w < n; ++w) assignments[idx[offs[j] + w]] = goff[j] + asg[w];
    const uint64_t t = nt > 1 ? j / chunk : 0;
    chunk_w[t] = chunk_w[t] + wcss;
  }
  float total = 0.0f;
  for (uint32_t t = 0; t < nt; ++t) total = total + chunk_w[t];
  *wcss_total = total;
  for (uint64_t i = 0; i < n_tokens; ++i)
    if (assignments[i] >= p->kappa_total) {
      st = ORC_INVALID_THRESHOLDS;
      goto done;
    }
done:
  free(freqs);
  free(offs);
  free(idx);
  free(cursor);
  free(spreads);
  free(frac);
  free(goff);
  free(gather);
  free(cent);
  free(asg);
  free(chunk_w);
  return st;
}
