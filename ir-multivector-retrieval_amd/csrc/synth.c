/*
 * synth.c — deterministic synthetic residual generator for the PQ build
 * workloads (host C, no GPU).
 *
 * Every random draw is a pure function of (seed, stream, counter), so any
 * chunk of a corpus can be regenerated on its own and the output does not
 * depend on the thread count.
 *
 *   centres   c_j = normalize(z_j), z_j ~ N(0, I_dim)
 *   vector    v_i = normalize(c_{j_i} + sigma * N(0, I_dim))
 *   residual  r_i = v_i - c_{j_i}            (not re-normalised)
 *   j_i       uniform over centres, or Zipf(s): P(j) proportional to (j+1)^-s
 *
 * Normals come from Box-Muller in double precision; normalisation runs in
 * double and each residual component is rounded to float once.
 *
 * Initial codebooks: for subspace mm, the first ksub indices of a partial
 * Fisher-Yates shuffle of [0, n) seeded with seed + mm; codeword c is the
 * mm-th sub-vector of residual perm[c].
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define STREAM_CENTER 1u
#define STREAM_ASSIGN 2u
#define STREAM_NOISE 3u
#define STREAM_SHUFFLE 4u
#define STREAM_CODEBOOK 5u

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

static inline uint64_t draw(uint64_t seed, uint64_t stream, uint64_t ctr) {
  const uint64_t key = mix64(seed * 0x9e3779b97f4a7c15ULL + stream);
  return mix64(key ^ mix64(ctr + 0x632be59bd9b4e019ULL));
}

/* uniform in (0, 1) */
static inline double unit(uint64_t bits) {
  return ((double)(bits >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

static inline void normal_pair(uint64_t seed, uint64_t stream, uint64_t ctr,
                               double *z0, double *z1) {
  const double u1 = unit(draw(seed, stream, 2 * ctr));
  const double u2 = unit(draw(seed, stream, 2 * ctr + 1));
  const double r = sqrt(-2.0 * log(u1));
  const double th = 6.283185307179586 * u2;
  *z0 = r * cos(th);
  *z1 = r * sin(th);
}

/* N(0,1) draw for element (row, col) of a row-major matrix of width dim. */
static inline double normal_at(uint64_t seed, uint64_t stream, uint64_t row,
                               uint32_t dim, uint32_t col) {
  const uint64_t pairs = (dim + 1) / 2;
  double z0, z1;
  normal_pair(seed, stream, row * pairs + col / 2, &z0, &z1);
  return (col & 1) ? z1 : z0;
}

int tac_synth_centers(uint64_t seed, uint32_t n_centers, uint32_t dim,
                      float *centers) {
  if (!centers || dim == 0 || dim > 4096) return 14;
  double *w = (double *)malloc(sizeof(double) * dim);
  if (!w) return 11;
  for (uint64_t j = 0; j < n_centers; ++j) {
    double ss = 0.0;
    for (uint32_t d = 0; d < dim; ++d) {
      w[d] = normal_at(seed, STREAM_CENTER, j, dim, d);
      ss += w[d] * w[d];
    }
    const double inv = ss > 0.0 ? 1.0 / sqrt(ss) : 0.0;
    for (uint32_t d = 0; d < dim; ++d) centers[j * dim + d] = (float)(w[d] * inv);
  }
  free(w);
  return 0;
}

typedef struct {
  uint64_t seed, lo, hi, first;
  uint32_t dim, n_centers;
  const float *centers;
  const double *cdf; /* NULL: uniform popularity */
  double sigma;
  float *out;
  uint32_t *ids;
} gen_ctx;

static uint32_t pick_center(const gen_ctx *c, uint64_t gi) {
  const double u = unit(draw(c->seed, STREAM_ASSIGN, gi));
  if (!c->cdf) {
    uint64_t j = (uint64_t)(u * (double)c->n_centers);
    return (uint32_t)(j < c->n_centers ? j : c->n_centers - 1);
  }
  uint32_t lo = 0, hi = c->n_centers - 1; /* first j with u < cdf[j] */
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (u < c->cdf[mid]) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

static void *gen_worker(void *p) {
  const gen_ctx *c = (const gen_ctx *)p;
  double w[4096];
  for (uint64_t i = c->lo; i < c->hi; ++i) {
    const uint64_t gi = c->first + i;
    const uint32_t j = pick_center(c, gi);
    const float *cj = c->centers + (uint64_t)j * c->dim;
    double ss = 0.0;
    for (uint32_t d = 0; d < c->dim; ++d) {
      w[d] = (double)cj[d] + c->sigma * normal_at(c->seed, STREAM_NOISE, gi, c->dim, d);
      ss += w[d] * w[d];
    }
    const double inv = ss > 0.0 ? 1.0 / sqrt(ss) : 0.0;
    float *r = c->out + i * c->dim;
    for (uint32_t d = 0; d < c->dim; ++d) r[d] = (float)(w[d] * inv - (double)cj[d]);
    if (c->ids) c->ids[i] = j;
  }
  return NULL;
}

/* Generate residuals first_index .. first_index + n - 1 of a corpus.
 * zipf_s <= 0 selects uniform centre popularity. */
int tac_synth_residuals(uint64_t seed, uint64_t n, uint32_t dim,
                        uint32_t n_centers, const float *centers, double zipf_s,
                        float sigma, uint64_t first_index, float *out,
                        uint32_t *center_ids, uint32_t n_threads) {
  if (!out || !centers || dim == 0 || dim > 4096 || n_centers == 0) return 14;
  double *cdf = NULL;
  if (zipf_s > 0.0) {
    cdf = (double *)malloc(sizeof(double) * n_centers);
    if (!cdf) return 11;
    double acc = 0.0;
    for (uint32_t j = 0; j < n_centers; ++j) {
      acc += pow((double)j + 1.0, -zipf_s);
      cdf[j] = acc;
    }
    for (uint32_t j = 0; j < n_centers; ++j) cdf[j] /= acc;
    cdf[n_centers - 1] = 1.0;
  }
  uint32_t T = n_threads ? n_threads : 1;
  if (T > 256) T = 256;
  if ((uint64_t)T > n) T = n ? (uint32_t)n : 1;
  gen_ctx ctx[256];
  pthread_t th[256];
  const uint64_t chunk = (n + T - 1) / T;
  uint32_t spawned = 0;
  for (uint32_t t = 0; t < T; ++t) {
    uint64_t lo = (uint64_t)t * chunk, hi = lo + chunk;
    if (lo > n) lo = n;
    if (hi > n) hi = n;
    ctx[t] = (gen_ctx){seed, lo, hi, first_index, dim, n_centers, centers, cdf,
                       (double)sigma, out, center_ids};
    if (T == 1 || pthread_create(&th[t], NULL, gen_worker, &ctx[t]) != 0) {
      gen_worker(&ctx[t]);
      continue;
    }
    th[spawned++] = th[t];
  }
  for (uint32_t t = 0; t < spawned; ++t) pthread_join(th[t], NULL);
  free(cdf);
  return 0;
}

/* Partial Fisher-Yates over [0, n): the first ksub positions, with the
 * swapped-out entries kept in a small list instead of an n-sized array. */
static int shuffle_prefix(uint64_t seed, uint64_t n, uint32_t ksub,
                          uint64_t *prefix) {
  uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * 2 * ksub);
  uint64_t *vals = (uint64_t *)malloc(sizeof(uint64_t) * 2 * ksub);
  if (!keys || !vals) {
    free(keys);
    free(vals);
    return 11;
  }
  uint32_t used = 0;
  for (uint64_t t = 0; t < ksub; ++t) {
    const uint64_t range = n - t;
    const uint64_t r = (uint64_t)(((unsigned __int128)draw(seed, STREAM_SHUFFLE, t) * range) >> 64);
    const uint64_t j = t + r;
    uint64_t vt = t, vj = j;
    int it = -1, ij = -1;
    for (uint32_t q = 0; q < used; ++q) {
      if (keys[q] == t) it = (int)q;
      if (keys[q] == j) ij = (int)q;
    }
    if (it >= 0) vt = vals[it];
    if (ij >= 0) vj = vals[ij];
    prefix[t] = vj;
    /* position j now holds the old value of position t */
    if (ij >= 0) vals[ij] = vt;
    else {
      keys[used] = j;
      vals[used] = vt;
      ++used;
    }
    if (it >= 0) vals[it] = vj;
    else {
      keys[used] = t;
      vals[used] = vj;
      ++used;
    }
  }
  free(keys);
  free(vals);
  return 0;
}

/* The rows tac_synth_shuffle_init takes for subspace mm are
 * tac_synth_shuffle_prefix(seed + mm, n, ksub): for callers whose residuals
 * live in device memory. */
int tac_synth_shuffle_prefix(uint64_t seed, uint64_t n, uint32_t ksub, uint64_t *prefix) {
  if (!prefix || ksub == 0 || (uint64_t)ksub > n) return 14;
  return shuffle_prefix(seed, n, ksub, prefix);
}

int tac_synth_shuffle_init(const float *residuals, uint64_t n, uint32_t dim,
                           uint32_t m, uint32_t ksub, uint64_t seed,
                           float *codebooks) {
  if (!residuals || !codebooks || m == 0 || dim % m != 0 || ksub == 0) return 14;
  if ((uint64_t)ksub > n) return 14;
  const uint32_t dsub = dim / m;
  uint64_t *prefix = (uint64_t *)malloc(sizeof(uint64_t) * ksub);
  if (!prefix) return 11;
  for (uint32_t mm = 0; mm < m; ++mm) {
    const int st = shuffle_prefix(seed + mm, n, ksub, prefix);
    if (st) {
      free(prefix);
      return st;
    }
    for (uint32_t c = 0; c < ksub; ++c)
      memcpy(codebooks + ((uint64_t)mm * ksub + c) * dsub,
             residuals + prefix[c] * dim + (uint64_t)mm * dsub,
             sizeof(float) * dsub);
  }
  free(prefix);
  return 0;
}

/* Fixed codebooks with entries N(0, sigma^2), layout [m][ksub][dsub]. */
int tac_synth_gauss_codebooks(uint64_t seed, uint32_t m, uint32_t ksub,
                              uint32_t dsub, float sigma, float *out) {
  if (!out || m == 0 || ksub == 0 || dsub == 0) return 14;
  const uint64_t total = (uint64_t)m * ksub * dsub;
  for (uint64_t e = 0; e < total; ++e)
    out[e] = (float)(sigma * normal_at(seed, STREAM_CODEBOOK, e, 1, 0));
  return 0;
}
