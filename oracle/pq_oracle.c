/*
 * pq_oracle.c — CPU restatement of the reference PQ build path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker (tests/,
 * __graft_entry__.smoke) and the timed CPU baseline (bench.py cpu_baseline).
 * The product library never links, loads or calls it.
 *
 * Arithmetic contract (reference uses Zig's strict float mode, no @mulAdd):
 *   - every subtract, multiply and add is rounded separately; this file is
 *     compiled with -ffp-contract=off and without -ffast-math;
 *   - distance folds, cluster-sum folds and the wcss fold run in the exact
 *     order of the reference loops.
 */
#include "pq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* vec primitives: src/util/vec.zig                                          */
/* ------------------------------------------------------------------------ */

/* vec.lane_count (src/util/vec.zig:16), settable to the reference host's. */
static uint32_t g_lanes = 16;
int orc_set_lane_count(uint32_t lanes) {
  if (lanes != 4 && lanes != 8 && lanes != 16) return ORC_INVALID_ARGUMENT;
  g_lanes = lanes;
  return ORC_OK;
}
uint32_t orc_lane_count(void) { return g_lanes; }

/* src/util/vec.zig:109-175.  dim 2 and 4 are explicit left folds (:114-118,
 * :133-139); dims 64 and 128 use four vector lanes that accumulate chunk
 * after chunk and an ordered reduce (:142-155); other dims use the host
 * lane count L with an ordered reduce and a scalar tail (:159-175): lane j
 * accumulates elements j, j + L, ... of the whole L-chunks from 0.0, the
 * lanes are summed in order, then the tail elements one by one.  Below 2 L
 * elements that is the sequential fold (0 + x = x for a square). */
float orc_l2sq(const float *a, const float *b, uint32_t d) {
  if (d == 2) {
    const float d0 = a[0] - b[0];
    const float d1 = a[1] - b[1];
    return d0 * d0 + d1 * d1;
  }
  if (d == 4) {
    float s = 0.0f;
    for (int i = 0; i < 4; ++i) {
      const float t = a[i] - b[i];
      s += t * t;
    }
    return s;
  }
  if (d == 64 || d == 128) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t c = 0; c < d; c += 4) {
      for (int j = 0; j < 4; ++j) {
        const float t = a[c + j] - b[c + j];
        acc[j] += t * t;
      }
    }
    return ((acc[0] + acc[1]) + acc[2]) + acc[3];
  }
  const uint32_t L = g_lanes;
  float acc[ORC_MAX_LANES];
  for (uint32_t j = 0; j < L; ++j) acc[j] = 0.0f;
  uint32_t i = 0;
  while (i + L <= d) {
    for (uint32_t j = 0; j < L; ++j) {
      const float t = a[i + j] - b[i + j];
      acc[j] += t * t;
    }
    i += L;
  }
  float sum = acc[0];
  for (uint32_t j = 1; j < L; ++j) sum += acc[j];
  for (; i < d; ++i) {
    const float t = a[i] - b[i];
    sum += t * t;
  }
  return sum;
}

/* src/util/vec.zig:37-103 — same dispatch shape as l2sq. */
float orc_dot(const float *a, const float *b, uint32_t d) {
  if (d == 2) return a[0] * b[0] + a[1] * b[1];
  if (d == 4) {
    float s = 0.0f;
    for (int i = 0; i < 4; ++i) s += a[i] * b[i];
    return s;
  }
  if (d == 64 || d == 128) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t c = 0; c < d; c += 4)
      for (int j = 0; j < 4; ++j) acc[j] += a[c + j] * b[c + j];
    return ((acc[0] + acc[1]) + acc[2]) + acc[3];
  }
  const uint32_t L = g_lanes;
  float acc[ORC_MAX_LANES];
  for (uint32_t j = 0; j < L; ++j) acc[j] = 0.0f;
  uint32_t i = 0;
  while (i + L <= d) {
    for (uint32_t j = 0; j < L; ++j) acc[j] += a[i + j] * b[i + j];
    i += L;
  }
  float sum = acc[0];
  for (uint32_t j = 1; j < L; ++j) sum += acc[j];
  for (; i < d; ++i) sum += a[i] * b[i];
  return sum;
}

/* src/util/vec.zig:271-283: start at index 0, replace only on strict <. */
uint64_t orc_argmin(const float *v, uint64_t n) {
  uint64_t best = 0;
  float best_v = v[0];
  for (uint64_t i = 1; i < n; ++i) {
    if (v[i] < best_v) {
      best_v = v[i];
      best = i;
    }
  }
  return best;
}

/* src/util/vec.zig:287-299: start at index 0, replace only on strict >. */
uint64_t orc_argmax(const float *v, uint64_t n) {
  uint64_t best = 0;
  float best_v = v[0];
  for (uint64_t i = 1; i < n; ++i) {
    if (v[i] > best_v) {
      best_v = v[i];
      best = i;
    }
  }
  return best;
}

/* ------------------------------------------------------------------------ */
/* Distances to every codeword, the way the reference's loops write them     */
/* ------------------------------------------------------------------------ */

/* The reference's assignment writes dists[cc] = l2sq(v, c_cc) for every
 * codeword and then takes vec.argmin (src/tac/kmeans.zig:356-364); PQ.encode
 * scans the same distances from best = +inf (src/index/pq.zig:64-73).  For
 * d <= 8 every arm of l2sq is the sequential fold ((x0-c0)^2 + (x1-c1)^2)
 * + ..., except d = 8 at 4 lanes, whose lanes j = 0..3 hold
 * (x_j-c_j)^2 + (x_{j+4}-c_{j+4})^2 and are summed in order; the distances
 * below fold each codeword in that order, reading a transposed codebook
 * cbt[k][cc] (row stride kp): the loop over codewords vectorizes, and each
 * codeword's bits equal orc_l2sq's.  orc_set_scalar(1) forces the per-pair
 * orc_l2sq path, against which the tests compare this one. */
static int g_scalar = 0;
void orc_set_scalar(int on) { g_scalar = on; }

typedef void (*dists_fn)(const float *, const float *, uint32_t, uint32_t, float *);

#define ORC_DISTS(D)                                                            \
  static void dists_d##D(const float *x, const float *cbt, uint32_t k,        \
                         uint32_t kp, float *out) {                           \
    float xv[D];                                                              \
    for (int j = 0; j < D; ++j) xv[j] = x[j];                                 \
    for (uint32_t cc = 0; cc < k; ++cc) {                                     \
      float t = xv[0] - cbt[cc];                                              \
      float acc = t * t;                                                      \
      for (int j = 1; j < D; ++j) {                                           \
        t = xv[j] - cbt[(uint64_t)j * kp + cc];                               \
        acc = acc + t * t;                                                    \
      }                                                                       \
      out[cc] = acc;                                                          \
    }                                                                         \
  }
ORC_DISTS(1)
ORC_DISTS(2)
ORC_DISTS(3)
ORC_DISTS(4)
ORC_DISTS(5)
ORC_DISTS(6)
ORC_DISTS(7)
ORC_DISTS(8)

static void dists_d8_l4(const float *x, const float *cbt, uint32_t k, uint32_t kp, float *out) {
  float xv[8];
  for (int j = 0; j < 8; ++j) xv[j] = x[j];
  for (uint32_t cc = 0; cc < k; ++cc) {
    float lane[4];
    for (int j = 0; j < 4; ++j) {
      const float t0 = xv[j] - cbt[(uint64_t)j * kp + cc];
      const float t1 = xv[j + 4] - cbt[(uint64_t)(j + 4) * kp + cc];
      lane[j] = t0 * t0;
      lane[j] = lane[j] + t1 * t1;
    }
    out[cc] = ((lane[0] + lane[1]) + lane[2]) + lane[3];
  }
}

static dists_fn dists_for(uint32_t d) {
  if (g_scalar) return NULL;
  switch (d) {
    case 1: return dists_d1;
    case 2: return dists_d2;
    case 3: return dists_d3;
    case 4: return dists_d4;
    case 5: return dists_d5;
    case 6: return dists_d6;
    case 7: return dists_d7;
    case 8: return g_lanes == 4 ? dists_d8_l4 : dists_d8;
    default: return NULL;
  }
}

/* cbt[j][cc] = cb[cc][j] for k codewords of d floats. */
static void transpose_cb(const float *cb, uint32_t k, uint32_t d, float *cbt) {
  for (uint32_t cc = 0; cc < k; ++cc)
    for (uint32_t j = 0; j < d; ++j) cbt[(uint64_t)j * k + cc] = cb[(uint64_t)cc * d + j];
}

/* The scan `best = start; for i: if (v[i] < best) take i` (strict <, first
 * index kept) as two passes that vectorize: the smallest value below start
 * (NaN never compares below), then the first index holding a value equal to
 * it (== makes -0.0 and +0.0 one class, as < does).  No value below start:
 * index 0, which is where both of the reference's scans stay (vec.argmin
 * with start = v[0], PQ.encode with start = +inf). */
static uint64_t first_below(const float *v, uint64_t n, float start) {
  float lane[8];
  for (int j = 0; j < 8; ++j) lane[j] = start;
  uint64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) lane[j] = v[i + j] < lane[j] ? v[i + j] : lane[j];
  for (; i < n; ++i) lane[0] = v[i] < lane[0] ? v[i] : lane[0];
  float best = start;
  for (int j = 0; j < 8; ++j) best = lane[j] < best ? lane[j] : best;
  if (!(best < start)) return 0;
  for (i = 0; i < n; ++i)
    if (v[i] == best) return i;
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Zig std PRNG (parity unpinned: restated from the published algorithms    */
/* Xoshiro256++ / SplitMix64 and Zig std's Random helpers; no Zig toolchain   */
/* is available to check the stream).  Reference call sites:                 */
/* src/util/rng.zig:25-38 (init, nextIndex), :57-82 (weightedSample).        */
/* ------------------------------------------------------------------------ */

static uint64_t splitmix64_next(uint64_t *s) {
  *s += 0x9e3779b97f4a7c15ULL;
  uint64_t z = *s;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) {
  return (x << k) | (x >> (64 - k));
}

void orc_zig_prng_init(orc_xoshiro *r, uint64_t seed) {
  uint64_t sm = seed;
  for (int i = 0; i < 4; ++i) r->s[i] = splitmix64_next(&sm);
}

uint64_t orc_zig_next(orc_xoshiro *r) {
  uint64_t *s = r->s;
  const uint64_t out = rotl64(s[0] + s[3], 23) + s[0];
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return out;
}

/* Lemire's multiply-shift with the threshold refinement used by Zig's
 * Random.uintLessThan for a 64-bit range. */
uint64_t orc_zig_uint_less_than(orc_xoshiro *r, uint64_t less_than) {
  uint64_t x = orc_zig_next(r);
  unsigned __int128 m = (unsigned __int128)x * less_than;
  uint64_t l = (uint64_t)m;
  if (l < less_than) {
    uint64_t t = (uint64_t)0 - less_than;
    if (t >= less_than) {
      t -= less_than;
      if (t >= less_than) t %= less_than;
    }
    while (l < t) {
      x = orc_zig_next(r);
      m = (unsigned __int128)x * less_than;
      l = (uint64_t)m;
    }
  }
  return (uint64_t)(m >> 64);
}

/* Zig Random.float(f64): 52 random mantissa bits; the exponent is drawn
 * geometrically from the leading zeros of the remaining bits. */
double orc_zig_float_f64(orc_xoshiro *r) {
  const uint64_t rnd = orc_zig_next(r);
  uint64_t lz = rnd == 0 ? 64 : (uint64_t)__builtin_clzll(rnd);
  if (lz >= 12) {
    lz = 12;
    for (;;) {
      const uint64_t more = orc_zig_next(r);
      const uint64_t add = more == 0 ? 64 : (uint64_t)__builtin_clzll(more);
      lz += add;
      if (add != 64) break;
      if (lz >= 1022) {
        lz = 1022;
        break;
      }
    }
  }
  const uint64_t mant = rnd & 0xFFFFFFFFFFFFFULL;
  const uint64_t expo = (uint64_t)(1022 - lz) << 52;
  const uint64_t bits = expo | mant;
  double out;
  memcpy(&out, &bits, sizeof out);
  return out;
}

/* src/util/rng.zig:57-82 */
int orc_weighted_sample(orc_xoshiro *r, const float *w, uint64_t n,
                        uint64_t *out) {
  if (n == 0) return ORC_RNG_EMPTY_DISTRIBUTION;
  double total = 0.0;
  for (uint64_t i = 0; i < n; ++i) {
    if (!isfinite(w[i]) || w[i] < 0.0f) return ORC_RNG_NON_FINITE;
    total += (double)w[i];
  }
  if (total <= 0.0) return ORC_RNG_ALL_ZERO;
  const double u = orc_zig_float_f64(r) * total;
  double cum = 0.0;
  for (uint64_t i = 0; i < n; ++i) {
    cum += (double)w[i];
    if (u < cum) {
      *out = i;
      return ORC_OK;
    }
  }
  uint64_t last = n - 1;
  while (last > 0 && w[last] == 0.0f) --last;
  *out = last;
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* kmeans.fit: src/tac/kmeans.zig:67-365                                     */
/* ------------------------------------------------------------------------ */

typedef struct {
  const float *vectors;
  const float *centroids;
  uint32_t *assignments;
  float *min_to_any;
  float *dists;
  uint64_t lo, hi;
  uint32_t d, k;
  const float *cbt; /* transposed centroids [d][k] for the vectorized distances, or NULL */
} assign_ctx;

/* src/tac/kmeans.zig:344-365 */
static void assign_slice(const assign_ctx *c) {
  const dists_fn f = c->cbt ? dists_for(c->d) : NULL;
  for (uint64_t i = c->lo; i < c->hi; ++i) {
    const float *v = c->vectors + i * c->d;
    uint64_t a;
    if (f) {
      f(v, c->cbt, c->k, c->k, c->dists);
      a = first_below(c->dists, c->k, c->dists[0]);
    } else {
      for (uint32_t cc = 0; cc < c->k; ++cc)
        c->dists[cc] = orc_l2sq(v, c->centroids + (uint64_t)cc * c->d, c->d);
      a = orc_argmin(c->dists, c->k);
    }
    c->assignments[i] = (uint32_t)a;
    c->min_to_any[i] = c->dists[a];
  }
}

static void *assign_thread(void *p) {
  assign_slice((const assign_ctx *)p);
  return NULL;
}

/* src/tac/kmeans.zig:244-340: static chunks of ceil(n/T), T clamped to n. */
static int assign_vectors(const float *vectors, uint64_t n, uint32_t d,
                          uint32_t k, const float *centroids,
                          uint32_t *assignments, float *min_to_any,
                          uint32_t n_threads) {
  uint64_t real = n_threads <= 1 ? 1 : (n_threads < n ? n_threads : n);
  float *cbt = NULL;
  if (dists_for(d)) {
    cbt = (float *)malloc(sizeof(float) * (uint64_t)k * d);
    if (!cbt) return ORC_OUT_OF_MEMORY;
    transpose_cb(centroids, k, d, cbt);
  }
  if (real <= 1) {
    float *dists = (float *)malloc(sizeof(float) * k);
    if (!dists) {
      free(cbt);
      return ORC_OUT_OF_MEMORY;
    }
    assign_ctx c = {vectors, centroids, assignments, min_to_any, dists, 0, n, d, k, cbt};
    assign_slice(&c);
    free(dists);
    free(cbt);
    return ORC_OK;
  }
  assign_ctx *ctx = (assign_ctx *)calloc(real, sizeof(assign_ctx));
  pthread_t *th = (pthread_t *)calloc(real, sizeof(pthread_t));
  float *dists = (float *)malloc(sizeof(float) * k * real);
  if (!ctx || !th || !dists) {
    free(ctx);
    free(th);
    free(dists);
    free(cbt);
    return ORC_OUT_OF_MEMORY;
  }
  const uint64_t chunk = (n + real - 1) / real;
  uint64_t spawned = 0;
  for (uint64_t t = 0; t < real; ++t) {
    uint64_t lo = t * chunk;
    uint64_t hi = lo + chunk < n ? lo + chunk : n;
    if (lo > n) lo = n;
    ctx[t] = (assign_ctx){vectors, centroids, assignments, min_to_any,
                          dists + t * k, lo, hi, d, k, cbt};
    if (pthread_create(&th[t], NULL, assign_thread, &ctx[t]) != 0) break;
    ++spawned;
  }
  for (uint64_t t = 0; t < spawned; ++t) pthread_join(th[t], NULL);
  /* A failed spawn leaves its slice unassigned: finish it on this thread. */
  for (uint64_t t = spawned; t < real; ++t) assign_slice(&ctx[t]);
  free(ctx);
  free(th);
  free(dists);
  free(cbt);
  return ORC_OK;
}

int orc_kmeans_fit(const float *vectors, uint64_t n, uint32_t dim, uint32_t k,
                   uint32_t max_iters, float tol, uint64_t seed,
                   uint32_t n_threads, const float *init_centroids,
                   float *centroids, uint32_t *assignments, float *wcss_out,
                   uint32_t *iters_out, const orc_fit_extras *ex) {
  /* src/tac/kmeans.zig:73-76 */
  if (k == 0) return ORC_KMEANS_BUDGET_TOO_SMALL;
  if (dim == 0) return ORC_DIM_MISMATCH;
  if (n == 0) return ORC_EMPTY_VECTOR_SET;
  const uint64_t d = dim;

  /* Degenerate k >= n: src/tac/kmeans.zig:88-104 */
  if ((uint64_t)k >= n) {
    memcpy(centroids, vectors, sizeof(float) * n * d);
    for (uint64_t c = n; c < k; ++c)
      memcpy(centroids + c * d, vectors + (n - 1) * d, sizeof(float) * d);
    for (uint64_t i = 0; i < n; ++i) assignments[i] = (uint32_t)i;
    if (wcss_out) *wcss_out = 0.0f;
    if (iters_out) *iters_out = 0;
    return ORC_OK;
  }

  int st = ORC_OK;
  float *min_dist_sq = NULL, *sums = NULL, *min_to_any = NULL;
  uint32_t *counts = NULL;

  if (init_centroids) {
    memcpy(centroids, init_centroids, sizeof(float) * k * d);
  } else {
    /* k-means++: src/tac/kmeans.zig:106-136 */
    orc_xoshiro rng;
    orc_zig_prng_init(&rng, seed);
    min_dist_sq = (float *)malloc(sizeof(float) * n);
    if (!min_dist_sq) return ORC_OUT_OF_MEMORY;
    const uint64_t idx0 = orc_zig_uint_less_than(&rng, n);
    memcpy(centroids, vectors + idx0 * d, sizeof(float) * d);
    for (uint64_t i = 0; i < n; ++i)
      min_dist_sq[i] = orc_l2sq(vectors + i * d, centroids, dim);
    for (uint64_t c = 1; c < k; ++c) {
      uint64_t idx = 0;
      st = orc_weighted_sample(&rng, min_dist_sq, n, &idx);
      if (st != ORC_OK) goto done;
      memcpy(centroids + c * d, vectors + idx * d, sizeof(float) * d);
      for (uint64_t i = 0; i < n; ++i) {
        const float dist = orc_l2sq(vectors + i * d, centroids + c * d, dim);
        if (dist < min_dist_sq[i]) min_dist_sq[i] = dist;
      }
    }
  }

  sums = (float *)malloc(sizeof(float) * k * d);
  counts = (uint32_t *)malloc(sizeof(uint32_t) * k);
  min_to_any = (float *)malloc(sizeof(float) * n);
  if (!sums || !counts || !min_to_any) {
    st = ORC_OUT_OF_MEMORY;
    goto done;
  }

  float prev_wcss = INFINITY;
  float wcss = 0.0f;
  uint32_t iters_run = 0;
  uint32_t iter = 0;
  for (; iter < max_iters; ++iter) {
    wcss = 0.0f;
    memset(sums, 0, sizeof(float) * k * d);
    memset(counts, 0, sizeof(uint32_t) * k);
    st = assign_vectors(vectors, n, dim, k, centroids, assignments, min_to_any,
                        n_threads);
    if (st != ORC_OK) goto done;
    /* serial accumulation in vector order: src/tac/kmeans.zig:177-184 */
    for (uint64_t i = 0; i < n; ++i) {
      const uint64_t a = assignments[i];
      wcss += min_to_any[i];
      const float *v = vectors + i * d;
      float *slot = sums + a * d;
      for (uint64_t dd = 0; dd < d; ++dd) slot[dd] += v[dd];
      counts[a] += 1;
    }
    iters_run = iter + 1;
    /* update + empty reseed: src/tac/kmeans.zig:193-212 */
    uint32_t empties = 0;
    for (uint64_t cc = 0; cc < k; ++cc) {
      if (counts[cc] > 0) {
        const float inv = 1.0f / (float)counts[cc];
        float *slot = centroids + cc * d;
        const float *sum = sums + cc * d;
        for (uint64_t dd = 0; dd < d; ++dd) slot[dd] = sum[dd] * inv;
      } else {
        const uint64_t far = orc_argmax(min_to_any, n);
        memcpy(centroids + cc * d, vectors + far * d, sizeof(float) * d);
        min_to_any[far] = -INFINITY;
        ++empties;
      }
    }
    if (ex && ex->trace)
      memcpy(ex->trace + (uint64_t)iter * k * d, centroids,
             sizeof(float) * k * d);
    if (ex && ex->empties) ex->empties[iter] = empties;
    if (ex && ex->wcss_trace) ex->wcss_trace[iter] = wcss;
    /* convergence: src/tac/kmeans.zig:217-223 */
    if (iter > 0) {
      const float denom = prev_wcss > 0.0f ? prev_wcss : 1.0f;
      const float rel = (prev_wcss - wcss) / denom;
      if (rel < tol) break;
    }
    prev_wcss = wcss;
  }
  /* Iterations never run repeat the final centroids in the trace. */
  if (ex && ex->trace)
    for (uint32_t t = iters_run; t < max_iters; ++t) {
      memcpy(ex->trace + (uint64_t)t * k * d, centroids, sizeof(float) * k * d);
      if (ex->empties) ex->empties[t] = 0;
      if (ex->wcss_trace) ex->wcss_trace[t] = wcss;
    }
  if (wcss_out) *wcss_out = wcss;
  if (iters_out) *iters_out = iters_run;

done:
  free(min_dist_sq);
  free(sums);
  free(counts);
  free(min_to_any);
  return st;
}

/* ------------------------------------------------------------------------ */
/* pq.train: src/index/pq.zig:158-336                                        */
/* ------------------------------------------------------------------------ */

typedef struct {
  const float *residuals;
  uint64_t n;
  uint32_t dim, m, ksub, dsub, max_iters, inner_threads;
  float tol;
  uint64_t seed;
  const float *init;
  float *codebooks;
  const orc_train_extras *ex;
  _Atomic uint32_t *next;
  int status;
} train_ctx;

/* src/index/pq.zig:301-336: gather column block mm, run fit, copy out. */
static int train_one_subspace(const train_ctx *c, uint32_t mm, float *sub_buf) {
  const uint64_t dsub = c->dsub;
  for (uint64_t i = 0; i < c->n; ++i)
    memcpy(sub_buf + i * dsub, c->residuals + i * c->dim + mm * dsub,
           sizeof(float) * dsub);
  const uint64_t cb = (uint64_t)c->ksub * dsub;
  uint32_t *assign = (uint32_t *)malloc(sizeof(uint32_t) * c->n);
  float *trace = NULL;
  uint32_t *emp = NULL;
  float *wtr = NULL;
  if (!assign) return ORC_OUT_OF_MEMORY;
  if (c->ex && c->ex->trace && c->max_iters) {
    trace = (float *)malloc(sizeof(float) * cb * c->max_iters);
    if (!trace) {
      free(assign);
      return ORC_OUT_OF_MEMORY;
    }
  }
  if (c->ex && c->ex->empties && c->max_iters)
    emp = (uint32_t *)calloc(c->max_iters, sizeof(uint32_t));
  orc_fit_extras fx = {trace, emp, wtr};
  float wcss = 0.0f;
  uint32_t iters = 0;
  const int st = orc_kmeans_fit(
      sub_buf, c->n, c->dsub, c->ksub, c->max_iters, c->tol, c->seed + mm,
      c->inner_threads, c->init ? c->init + (uint64_t)mm * cb : NULL,
      c->codebooks + (uint64_t)mm * cb, assign, &wcss, &iters, &fx);
  if (st == ORC_OK && c->ex) {
    if (c->ex->iters_run) c->ex->iters_run[mm] = iters;
    if (c->ex->wcss) c->ex->wcss[mm] = wcss;
    if (trace) {
      if ((uint64_t)c->ksub >= c->n) /* degenerate: no iteration ran */
        for (uint32_t t = 0; t < c->max_iters; ++t)
          memcpy(trace + (uint64_t)t * cb, c->codebooks + (uint64_t)mm * cb,
                 sizeof(float) * cb);
      for (uint32_t t = 0; t < c->max_iters; ++t)
        memcpy(c->ex->trace + ((uint64_t)t * c->m + mm) * cb,
               trace + (uint64_t)t * cb, sizeof(float) * cb);
    }
    if (c->ex->empties) {
      uint32_t tot = 0;
      if (emp)
        for (uint32_t t = 0; t < c->max_iters; ++t) tot += emp[t];
      c->ex->empties[mm] = tot;
    }
  }
  free(assign);
  free(trace);
  free(emp);
  return st;
}

static void *train_worker(void *p) {
  train_ctx *c = (train_ctx *)p;
  float *sub_buf = (float *)malloc(sizeof(float) * c->n * c->dsub);
  if (!sub_buf) {
    c->status = ORC_OUT_OF_MEMORY;
    return NULL;
  }
  for (;;) {
    const uint32_t mm = atomic_fetch_add(c->next, 1);
    if (mm >= c->m) break;
    const int st = train_one_subspace(c, mm, sub_buf);
    if (st != ORC_OK) {
      c->status = st;
      break;
    }
  }
  free(sub_buf);
  return NULL;
}

int orc_pq_train(const float *residuals, uint64_t n, uint32_t dim, uint32_t m,
                 uint32_t ksub, const float *init_codebooks, uint64_t seed,
                 uint32_t max_iters, float tol, uint32_t n_threads,
                 float *codebooks, const orc_train_extras *ex) {
  /* src/index/pq.zig:165-168 */
  if (m == 0) return ORC_INVALID_ARGUMENT;
  if (dim == 0) return ORC_DIM_MISMATCH;
  if (dim % m != 0) return ORC_DIM_NOT_DIVISIBLE_BY_M;
  if (n == 0) return ORC_EMPTY_CORPUS;
  if (ksub == 0) return ORC_KMEANS_BUDGET_TOO_SMALL;
  _Atomic uint32_t next = 0;
  train_ctx base = {residuals, n, dim, m, ksub, dim / m, max_iters, 1,
                    tol, seed, init_codebooks, codebooks, ex, &next, ORC_OK};
  if (n_threads <= 1) {
    base.inner_threads = n_threads;
    train_worker(&base);
    return base.status;
  }
  /* work stealing over subspaces: src/index/pq.zig:236-283 */
  const uint32_t real = n_threads < m ? n_threads : m;
  const uint32_t inner = n_threads <= real ? 1 : (n_threads / real > 1 ? n_threads / real : 1);
  train_ctx *ctx = (train_ctx *)calloc(real, sizeof(train_ctx));
  pthread_t *th = (pthread_t *)calloc(real, sizeof(pthread_t));
  if (!ctx || !th) {
    free(ctx);
    free(th);
    return ORC_OUT_OF_MEMORY;
  }
  uint32_t spawned = 0;
  for (uint32_t t = 0; t < real; ++t) {
    ctx[t] = base;
    ctx[t].inner_threads = inner;
    if (pthread_create(&th[t], NULL, train_worker, &ctx[t]) != 0) break;
    ++spawned;
  }
  for (uint32_t t = 0; t < spawned; ++t) pthread_join(th[t], NULL);
  int st = spawned == 0 ? ORC_OUT_OF_MEMORY : ORC_OK;
  for (uint32_t t = 0; t < spawned; ++t)
    if (ctx[t].status != ORC_OK) st = ctx[t].status;
  free(ctx);
  free(th);
  return st;
}

/* ------------------------------------------------------------------------ */
/* PQ.encode / decode / buildDistanceTable                                   */
/* ------------------------------------------------------------------------ */

typedef struct {
  const float *residuals;
  const float *codebooks;
  void *codes;
  uint64_t lo, hi;
  uint32_t dim, m, ksub, dsub;
  float rel_tol;
  uint64_t near;
  const float *cbt; /* per subspace, the transposed codebook [dsub][ksub], or NULL */
} encode_ctx;

/* src/index/pq.zig:59-76: best_d starts at +inf, strict < keeps the first. */
static void encode_slice(encode_ctx *c) {
  const dists_fn f = c->cbt ? dists_for(c->dsub) : NULL;
  float *dists = f ? (float *)malloc(sizeof(float) * c->ksub) : NULL;
  const dists_fn fn = dists ? f : NULL;
  for (uint64_t i = c->lo; i < c->hi; ++i) {
    const float *r = c->residuals + i * c->dim;
    for (uint32_t mm = 0; mm < c->m; ++mm) {
      const float *sub = r + (uint64_t)mm * c->dsub;
      const float *cb = c->codebooks + (uint64_t)mm * c->ksub * c->dsub;
      uint32_t best_c = 0;
      if (fn) {
        fn(sub, c->cbt + (uint64_t)mm * c->ksub * c->dsub, c->ksub, c->ksub, dists);
        best_c = (uint32_t)first_below(dists, c->ksub, INFINITY);
      } else {
        float best_d = INFINITY;
        for (uint32_t cc = 0; cc < c->ksub; ++cc) {
          const float dd = orc_l2sq(sub, cb + (uint64_t)cc * c->dsub, c->dsub);
          if (dd < best_d) {
            best_d = dd;
            best_c = cc;
          }
        }
      }
      if (c->ksub <= 256)
        ((uint8_t *)c->codes)[i * c->m + mm] = (uint8_t)best_c;
      else
        ((uint16_t *)c->codes)[i * c->m + mm] = (uint16_t)best_c;
    }
  }
  free(dists);
}

static void near_slice(encode_ctx *c) {
  uint64_t near = 0;
  for (uint64_t i = c->lo; i < c->hi; ++i) {
    const float *r = c->residuals + i * c->dim;
    for (uint32_t mm = 0; mm < c->m; ++mm) {
      const float *sub = r + (uint64_t)mm * c->dsub;
      const float *cb = c->codebooks + (uint64_t)mm * c->ksub * c->dsub;
      float b1 = INFINITY, b2 = INFINITY;
      for (uint32_t cc = 0; cc < c->ksub; ++cc) {
        const float dd = orc_l2sq(sub, cb + (uint64_t)cc * c->dsub, c->dsub);
        if (dd < b1) {
          b2 = b1;
          b1 = dd;
        } else if (dd < b2) {
          b2 = dd;
        }
      }
      if (c->ksub > 1 && (double)(b2 - b1) <= (double)c->rel_tol * (double)b2)
        ++near;
    }
  }
  c->near = near;
}

static void *encode_thread(void *p) {
  encode_slice((encode_ctx *)p);
  return NULL;
}
static void *near_thread(void *p) {
  near_slice((encode_ctx *)p);
  return NULL;
}

/* Static-chunk fan-out of src/index/storage.zig:201-244 (serial when the
 * thread count is 1 or there are fewer than 1024 tokens). */
static int fan_out(encode_ctx base, uint32_t n_threads, void *(*fn)(void *),
                   uint64_t *near_total) {
  const uint64_t n = base.hi;
  if (n_threads <= 1 || n < 1024) {
    fn(&base);
    if (near_total) *near_total = base.near;
    return ORC_OK;
  }
  const uint64_t T = n_threads < n ? n_threads : n;
  encode_ctx *ctx = (encode_ctx *)calloc(T, sizeof(encode_ctx));
  pthread_t *th = (pthread_t *)calloc(T, sizeof(pthread_t));
  if (!ctx || !th) {
    free(ctx);
    free(th);
    return ORC_OUT_OF_MEMORY;
  }
  const uint64_t chunk = (n + T - 1) / T;
  uint64_t spawned = 0;
  for (uint64_t t = 0; t < T; ++t) {
    ctx[t] = base;
    ctx[t].lo = t * chunk < n ? t * chunk : n;
    ctx[t].hi = ctx[t].lo + chunk < n ? ctx[t].lo + chunk : n;
    if (pthread_create(&th[t], NULL, fn, &ctx[t]) != 0) break;
    ++spawned;
  }
  for (uint64_t t = 0; t < spawned; ++t) pthread_join(th[t], NULL);
  for (uint64_t t = spawned; t < T; ++t) fn(&ctx[t]);
  if (near_total) {
    uint64_t s = 0;
    for (uint64_t t = 0; t < T; ++t) s += ctx[t].near;
    *near_total = s;
  }
  free(ctx);
  free(th);
  return ORC_OK;
}

int orc_pq_encode(const float *residuals, uint64_t n, uint32_t dim, uint32_t m,
                  uint32_t ksub, const float *codebooks, void *codes,
                  uint32_t n_threads) {
  if (m == 0 || ksub == 0 || ksub > 65536) return ORC_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return ORC_DIM_MISMATCH;
  const uint32_t dsub = dim / m;
  float *cbt = NULL;
  if (dists_for(dsub)) {
    cbt = (float *)malloc(sizeof(float) * (uint64_t)m * ksub * dsub);
    if (!cbt) return ORC_OUT_OF_MEMORY;
    for (uint32_t mm = 0; mm < m; ++mm)
      transpose_cb(codebooks + (uint64_t)mm * ksub * dsub, ksub, dsub,
                   cbt + (uint64_t)mm * ksub * dsub);
  }
  encode_ctx base = {residuals, codebooks, codes, 0, n, dim, m, ksub, dsub, 0.0f, 0, cbt};
  const int st = fan_out(base, n_threads, encode_thread, NULL);
  free(cbt);
  return st;
}

int orc_pq_near_ties(const float *residuals, uint64_t n, uint32_t dim,
                     uint32_t m, uint32_t ksub, const float *codebooks,
                     float rel_tol, uint64_t *count, uint32_t n_threads) {
  if (m == 0 || ksub == 0) return ORC_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return ORC_DIM_MISMATCH;
  encode_ctx base = {residuals, codebooks, NULL, 0, n, dim, m, ksub, dim / m, rel_tol, 0, NULL};
  return fan_out(base, n_threads, near_thread, count);
}

/* src/index/pq.zig:79-88 */
int orc_pq_decode(const void *codes, uint64_t n, uint32_t dim, uint32_t m,
                  uint32_t ksub, const float *codebooks, float *out) {
  if (m == 0 || ksub == 0) return ORC_INVALID_ARGUMENT;
  if (dim == 0 || dim % m != 0) return ORC_DIM_MISMATCH;
  const uint32_t dsub = dim / m;
  for (uint64_t i = 0; i < n; ++i)
    for (uint32_t mm = 0; mm < m; ++mm) {
      const uint32_t code = ksub <= 256 ? ((const uint8_t *)codes)[i * m + mm]
                                        : ((const uint16_t *)codes)[i * m + mm];
      if (code >= ksub) return ORC_INVALID_ARGUMENT;
      memcpy(out + i * dim + (uint64_t)mm * dsub,
             codebooks + ((uint64_t)mm * ksub + code) * dsub,
             sizeof(float) * dsub);
    }
  return ORC_OK;
}

/* src/index/pq.zig:92-123 */
int orc_pq_distance_table(const float *queries, uint32_t n_q, uint32_t dim,
                          uint32_t m, uint32_t ksub, const float *codebooks,
                          float *table, uint64_t table_len) {
  if (m == 0 || ksub == 0) return ORC_INVALID_ARGUMENT;
  if (n_q == 0) return ORC_NQ_MISMATCH;
  if (dim == 0 || dim % m != 0) return ORC_DIM_MISMATCH;
  if (table_len != (uint64_t)m * ksub * n_q) return ORC_OUT_BUFFER_WRONG_SIZE;
  const uint32_t dsub = dim / m;
  for (uint32_t mm = 0; mm < m; ++mm)
    for (uint32_t c = 0; c < ksub; ++c) {
      const float *cv = codebooks + ((uint64_t)mm * ksub + c) * dsub;
      const uint64_t base = ((uint64_t)mm * ksub + c) * n_q;
      for (uint32_t i = 0; i < n_q; ++i)
        table[base + i] =
            orc_dot(queries + (uint64_t)i * dim + (uint64_t)mm * dsub, cv, dsub);
    }
  return ORC_OK;
}

/* src/index/storage.zig:255-278 (residualsAndNormsChunk).  Per token i with
 * centroid a = assignments[i]: diff_d = v_d - c_d is stored, sum_sq folds
 * diff_d * diff_d in ascending d from 0.0f, norm = sqrt(sum_sq) (correctly
 * rounded), and only when norm > 0 every diff_d is multiplied by
 * fl(1.0f / norm).  An assignment >= n_centroids (a bounds trap in the
 * reference) is ORC_INVALID_ARGUMENT here. */
int orc_residuals(const float *vectors, uint64_t n, uint32_t dim,
                  const float *centroids, uint32_t n_centroids,
                  const uint32_t *assignments, float *residuals, float *norms) {
  if (dim == 0) return ORC_DIM_MISMATCH;
  for (uint64_t i = 0; i < n; ++i)
    if (assignments[i] >= n_centroids) return ORC_INVALID_ARGUMENT;
  for (uint64_t i = 0; i < n; ++i) {
    const float *v = vectors + i * dim;
    const float *c = centroids + (uint64_t)assignments[i] * dim;
    float *r = residuals + i * dim;
    float sum_sq = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) {
      const float diff = v[d] - c[d];
      r[d] = diff;
      const float sq = diff * diff;
      sum_sq = sum_sq + sq;
    }
    const float norm = sqrtf(sum_sq);
    norms[i] = norm;
    if (norm > 0.0f) {
      const float inv = 1.0f / norm;
      for (uint32_t d = 0; d < dim; ++d) r[d] = r[d] * inv;
    }
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* .tac per-document layouts and footer checksum: src/index/storage.zig      */
/* ------------------------------------------------------------------------ */

static uint64_t align8(uint64_t x) { return (x + 7u) & ~(uint64_t)7u; }

/* storage.zig:674-686 (docPayloadSize), with m codes of code_bytes each per
 * token (the reference: m = PQ_M, one byte). */
uint64_t orc_doc_payload_bytes(const uint64_t *doc_offsets, uint64_t n_docs,
                               uint32_t m, uint32_t code_bytes) {
  uint64_t total = 0;
  for (uint64_t d = 0; d < n_docs; ++d) {
    const uint64_t n_d = doc_offsets[d + 1] - doc_offsets[d];
    total += align8(4 + n_d * 4 + n_d * (uint64_t)m * code_bytes);
  }
  return total;
}

/* storage.zig:705-749 (writeDocLayouts): doc_index[d] is the payload offset
 * of doc d (doc_index[n_docs] = total); each doc is u32 n_d (LE), the n_d
 * centroid ids (u32 LE), the n_d * m codes, zero padding to 8 bytes. */
int orc_write_doc_layouts(const uint64_t *doc_offsets, uint64_t n_docs,
                          const uint32_t *assignments, const void *codes,
                          uint32_t m, uint32_t code_bytes, uint64_t *doc_index,
                          uint8_t *payload, uint64_t payload_len) {
  if (m == 0 || (code_bytes != 1 && code_bytes != 2)) return ORC_INVALID_ARGUMENT;
  /* storage.zig:717: a payload buffer shorter than the layouts */
  if (payload_len < orc_doc_payload_bytes(doc_offsets, n_docs, m, code_bytes))
    return ORC_BUFFER_TOO_SMALL;
  uint64_t off = 0;
  for (uint64_t d = 0; d < n_docs; ++d) {
    doc_index[d] = off;
    const uint64_t lo = doc_offsets[d], n_d = doc_offsets[d + 1] - lo;
    const uint64_t bytes = align8(4 + n_d * 4 + n_d * (uint64_t)m * code_bytes);
    uint8_t *p = payload + off;
    const uint32_t nd32 = (uint32_t)n_d;
    for (int b = 0; b < 4; ++b) p[b] = (uint8_t)(nd32 >> (8 * b));
    for (uint64_t k = 0; k < n_d; ++k)
      for (int b = 0; b < 4; ++b) p[4 + 4 * k + b] = (uint8_t)(assignments[lo + k] >> (8 * b));
    const uint64_t cb = n_d * (uint64_t)m * code_bytes;
    memcpy(p + 4 + 4 * n_d, (const uint8_t *)codes + lo * (uint64_t)m * code_bytes, cb);
    memset(p + 4 + 4 * n_d + cb, 0, bytes - (4 + 4 * n_d + cb));
    off += bytes;
  }
  doc_index[n_docs] = off;
  return ORC_OK;
}

/* std.hash.Crc32 as used by storage.zig:612-617 and :782-786: CRC-32/ISO-HDLC
 * (reflected polynomial 0xEDB88320, register preset to all ones, result
 * complemented), one byte at a time. */
uint32_t orc_crc32(const uint8_t *bytes, uint64_t len) {
  uint32_t table[256];
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t r = i;
    for (int k = 0; k < 8; ++k) r = (r & 1u) ? (r >> 1) ^ 0xEDB88320u : r >> 1;
    table[i] = r;
  }
  uint32_t r = 0xFFFFFFFFu;
  for (uint64_t i = 0; i < len; ++i) r = table[(r ^ bytes[i]) & 0xFFu] ^ (r >> 8);
  return r ^ 0xFFFFFFFFu;
}

/* ------------------------------------------------------------------------ */
/* Query side: src/retrieval/refine.zig:83-145 for one candidate             */
/* ------------------------------------------------------------------------ */

int orc_refine(const float *query, uint32_t n_q, uint32_t dim,
               const float *centroids, uint32_t kappa, const float *table,
               uint64_t table_len, uint32_t m, uint32_t ksub,
               const uint64_t *doc_index, const uint8_t *payload,
               uint64_t payload_len, const uint64_t *doc_token_offsets,
               const float *norms, uint64_t n_tokens, uint64_t n_docs,
               uint64_t doc_id, float *score_out) {
  if (n_q == 0) return ORC_QUERY_SHAPE_MISMATCH;                      /* :99-101 */
  if (table_len != (uint64_t)m * ksub * n_q) return ORC_TABLE_SIZE_MISMATCH; /* :104 */
  if (doc_id >= n_docs) return ORC_DOC_OUT_OF_RANGE;                  /* :107 */
  const uint32_t code_bytes = ksub <= 256 ? 1 : 2;
  /* storage.zig:112-116 docLayout, refine.zig:51-65 decodeDocLayout */
  const uint64_t lo = doc_index[doc_id], hi = doc_index[doc_id + 1];
  if (hi < lo || hi > payload_len || hi - lo < 4) return ORC_DOC_LAYOUT_CORRUPT;
  const uint8_t *lay = payload + lo;
  const uint32_t n_d = (uint32_t)lay[0] | (uint32_t)lay[1] << 8 | (uint32_t)lay[2] << 16 |
                       (uint32_t)lay[3] << 24;
  if (hi - lo < 4 + (uint64_t)n_d * 4 + (uint64_t)n_d * m * code_bytes)
    return ORC_DOC_LAYOUT_CORRUPT;
  const uint64_t t_lo = doc_token_offsets[doc_id], t_hi = doc_token_offsets[doc_id + 1];
  if (t_hi - t_lo != n_d || t_hi > n_tokens) return ORC_DOC_LAYOUT_CORRUPT; /* :114 */
  const uint8_t *ids = lay + 4;
  const uint8_t *codes = lay + 4 + 4 * (uint64_t)n_d;
  float *best = (float *)malloc(sizeof(float) * n_q);
  if (!best) return ORC_OUT_OF_MEMORY;
  for (uint32_t i = 0; i < n_q; ++i) best[i] = -INFINITY;
  for (uint32_t k = 0; k < n_d; ++k) {
    const uint32_t c_id = (uint32_t)ids[4 * k] | (uint32_t)ids[4 * k + 1] << 8 |
                          (uint32_t)ids[4 * k + 2] << 16 | (uint32_t)ids[4 * k + 3] << 24;
    if (c_id >= kappa) {  /* a bounds trap in the reference */
      free(best);
      return ORC_DOC_LAYOUT_CORRUPT;
    }
    const float *c_vec = centroids + (uint64_t)c_id * dim;
    const float norm_k = norms[t_lo + k];
    for (uint32_t i = 0; i < n_q; ++i) {
      const float cent_term = orc_dot(query + (uint64_t)i * dim, c_vec, dim);
      float res = 0.0f;
      for (uint32_t mm = 0; mm < m; ++mm) {
        const uint64_t cpos = ((uint64_t)k * m + mm) * code_bytes;
        const uint32_t code = code_bytes == 1 ? codes[cpos]
                                              : (uint32_t)codes[cpos] | (uint32_t)codes[cpos + 1] << 8;
        if (code >= ksub) {
          free(best);
          return ORC_DOC_LAYOUT_CORRUPT;
        }
        res = res + table[((uint64_t)mm * ksub + code) * n_q + i];
      }
      const float scaled = norm_k * res;
      const float score = cent_term + scaled;
      if (score > best[i]) best[i] = score;
    }
  }
  float sum = 0.0f;
  if (n_d > 0)
    for (uint32_t i = 0; i < n_q; ++i) sum = sum + best[i];
  free(best);
  *score_out = sum;
  return ORC_OK;
}
