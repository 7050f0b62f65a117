/*
 * pq_oracle.h — CPU restatement of the reference's product-quantization build
 * path (Lloyd k-means per subspace + PQ encode), used ONLY as test
 * infrastructure: the parity checker for the HIP library and the timed CPU
 * baseline.  Nothing in the shipped library links or calls this code.
 *
 * Every function follows a reference location (paths relative to the
 * reference repository root):
 *   orc_l2sq / orc_dot      src/util/vec.zig:37-175   (operation order, no FMA)
 *   orc_argmin / orc_argmax src/util/vec.zig:271-299  (first index wins ties)
 *   orc_zig_*               src/util/rng.zig:22-82 and Zig std 0.16
 *                           (std.Random.DefaultPrng = Xoshiro256++, SplitMix64
 *                           seeding, uintLessThan, float(f64)) — "parity
 *                           unpinned": no Zig toolchain exists here to check
 *                           the stream against.
 *   orc_kmeans_fit          src/tac/kmeans.zig:67-365
 *   orc_pq_train            src/index/pq.zig:158-336
 *   orc_pq_encode           src/index/pq.zig:59-76 driven as in
 *                           src/index/storage.zig:201-244,280-295
 *   orc_pq_decode           src/index/pq.zig:79-88
 *   orc_pq_distance_table   src/index/pq.zig:92-123
 *   orc_residuals           src/index/storage.zig:255-278
 *   orc_doc_payload_bytes   src/index/storage.zig:674-686
 *   orc_write_doc_layouts   src/index/storage.zig:705-749
 *   orc_crc32               std.hash.Crc32 (CRC-32/ISO-HDLC) as storage.zig
 *                           applies it to the image (:612-617, :782-786)
 *   orc_refine              src/retrieval/refine.zig:51-145 (one candidate)
 *   orc_tac_*               src/tac/tac.zig:77-330 (phases 1-4) and
 *                           :563-830 (clusterFlat), in tac_oracle.c
 *
 * Status codes share their numbering with include/tac_gpu.h.
 */
#ifndef PQ_ORACLE_H
#define PQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ORC_OK = 0,
  ORC_DIM_NOT_DIVISIBLE_BY_M = 1,
  ORC_DIM_MISMATCH = 2,
  ORC_EMPTY_CORPUS = 3,
  ORC_OUT_BUFFER_WRONG_SIZE = 4,
  ORC_NQ_MISMATCH = 5,
  ORC_KMEANS_BUDGET_TOO_SMALL = 6,
  ORC_EMPTY_VECTOR_SET = 7,
  ORC_RNG_EMPTY_DISTRIBUTION = 8,
  ORC_RNG_NON_FINITE = 9,
  ORC_RNG_ALL_ZERO = 10,
  ORC_OUT_OF_MEMORY = 11,
  ORC_INVALID_ARGUMENT = 14,
  ORC_QUERY_SHAPE_MISMATCH = 16,  /* RefineError (src/retrieval/refine.zig:37-42) */
  ORC_TABLE_SIZE_MISMATCH = 17,
  ORC_DOC_OUT_OF_RANGE = 18,
  ORC_DOC_LAYOUT_CORRUPT = 19,
  ORC_BUFFER_TOO_SMALL = 20,      /* StorageError (src/index/storage.zig:42-47) */
  ORC_BUDGET_TOO_SMALL = 21,      /* ClusteringError (src/tac/tac.zig:59-64) */
  ORC_BUDGET_TOO_LARGE = 22,
  ORC_INVALID_THRESHOLDS = 23,
  ORC_EMPTY_TOKEN_DUMP = 24,
};

/* Lane count of the reference's generic vec path, vec.lane_count =
 * std.simd.suggestVectorLength(f32) of the host it is built for
 * (src/util/vec.zig:16): 16 on AVX-512 x86-64 (the default here), 8 on AVX2,
 * 4 on NEON (aarch64).  orc_set_lane_count takes 4, 8 or 16 and returns 0,
 * or 14 (invalid argument) and keeps the current value. */
#define ORC_MAX_LANES 16
int orc_set_lane_count(uint32_t lanes);
uint32_t orc_lane_count(void);

/* 1: every distance goes through orc_l2sq pair by pair (the per-pair form);
 * 0 (default): for d <= 8 all K distances of a vector are formed at once from
 * a transposed codebook, in the same per-codeword order.  Test hook. */
void orc_set_scalar(int on);

float orc_l2sq(const float *a, const float *b, uint32_t d);
float orc_dot(const float *a, const float *b, uint32_t d);
uint64_t orc_argmin(const float *v, uint64_t n);
uint64_t orc_argmax(const float *v, uint64_t n);

/* Zig std PRNG restatement (parity unpinned). */
typedef struct { uint64_t s[4]; } orc_xoshiro;
void orc_zig_prng_init(orc_xoshiro *r, uint64_t seed);
uint64_t orc_zig_next(orc_xoshiro *r);
uint64_t orc_zig_uint_less_than(orc_xoshiro *r, uint64_t less_than);
double orc_zig_float_f64(orc_xoshiro *r);
int orc_weighted_sample(orc_xoshiro *r, const float *w, uint64_t n, uint64_t *out);

/* Optional per-iteration outputs. Any pointer may be NULL. */
typedef struct {
  float *trace;           /* [max_iters][k][dim]: centroids after iteration t */
  uint32_t *empties;      /* [max_iters]: empty clusters reseeded in iteration t */
  float *wcss_trace;      /* [max_iters]: wcss accumulated in iteration t */
} orc_fit_extras;

/* kmeans.fit. init_centroids == NULL selects k-means++ seeding with `seed`.
 * tol = -INFINITY never breaks early.  Outputs: centroids [k][dim],
 * assignments [n], wcss, iters_run. */
int orc_kmeans_fit(const float *vectors, uint64_t n, uint32_t dim, uint32_t k,
                   uint32_t max_iters, float tol, uint64_t seed,
                   uint32_t n_threads, const float *init_centroids,
                   float *centroids, uint32_t *assignments, float *wcss,
                   uint32_t *iters_run, const orc_fit_extras *extras);

typedef struct {
  float *trace;          /* [max_iters][m][ksub][dsub] */
  uint32_t *iters_run;   /* [m] */
  float *wcss;           /* [m]  final wcss per subspace */
  uint32_t *empties;     /* [m]  total empty reseeds per subspace */
} orc_train_extras;

/* pq.train with runtime m / ksub / iteration control.
 * init_codebooks [m][ksub][dsub] or NULL (k-means++ with seed +% subspace). */
int orc_pq_train(const float *residuals, uint64_t n, uint32_t dim, uint32_t m,
                 uint32_t ksub, const float *init_codebooks, uint64_t seed,
                 uint32_t max_iters, float tol, uint32_t n_threads,
                 float *codebooks, const orc_train_extras *extras);

/* Batched PQ.encode: codes token-major [n][m], u8 when ksub <= 256 else u16. */
int orc_pq_encode(const float *residuals, uint64_t n, uint32_t dim, uint32_t m,
                  uint32_t ksub, const float *codebooks, void *codes,
                  uint32_t n_threads);

/* Best-vs-second margin census of the exhaustive encode: number of
 * (vector, subspace) pairs whose (second - best) / second <= rel_tol. */
int orc_pq_near_ties(const float *residuals, uint64_t n, uint32_t dim,
                     uint32_t m, uint32_t ksub, const float *codebooks,
                     float rel_tol, uint64_t *count, uint32_t n_threads);

int orc_pq_decode(const void *codes, uint64_t n, uint32_t dim, uint32_t m,
                  uint32_t ksub, const float *codebooks, float *out);

/* table[((mm * ksub) + c) * n_q + i] = dot(query_i[mm], codebook[mm][c]) */
int orc_pq_distance_table(const float *queries, uint32_t n_q, uint32_t dim,
                          uint32_t m, uint32_t ksub, const float *codebooks,
                          float *table, uint64_t table_len);

/* Residuals and per-token norms (storage.build stage 2). */
int orc_residuals(const float *vectors, uint64_t n, uint32_t dim,
                  const float *centroids, uint32_t n_centroids,
                  const uint32_t *assignments, float *residuals, float *norms);

uint64_t orc_doc_payload_bytes(const uint64_t *doc_offsets, uint64_t n_docs,
                               uint32_t m, uint32_t code_bytes);
int orc_write_doc_layouts(const uint64_t *doc_offsets, uint64_t n_docs,
                          const uint32_t *assignments, const void *codes,
                          uint32_t m, uint32_t code_bytes, uint64_t *doc_index,
                          uint8_t *payload, uint64_t payload_len);
uint32_t orc_crc32(const uint8_t *bytes, uint64_t len);
int orc_refine(const float *query, uint32_t n_q, uint32_t dim,
               const float *centroids, uint32_t kappa, const float *table,
               uint64_t table_len, uint32_t m, uint32_t ksub,
               const uint64_t *doc_index, const uint8_t *payload,
               uint64_t payload_len, const uint64_t *doc_token_offsets,
               const float *norms, uint64_t n_tokens, uint64_t n_docs,
               uint64_t doc_id, float *score_out);


/* ---- TAC: token-aware clustering (src/tac/tac.zig) -------------------- */

typedef struct {
  uint32_t kappa_total, mu, tau, epsilon, theta, max_iters;
  float tol;
  uint64_t seed;
  uint32_t n_threads; /* wcss_total grouping only (tac.zig:688-820) */
} orc_tac_params;

/* Phase 1 (tac.zig:97-126): tail kappa; *budget_active = kappa_total - tail. */
int orc_tac_allocate_tail(const uint32_t *freqs, uint64_t n, uint32_t *kappa, uint32_t mu,
                          uint32_t tau, uint32_t kappa_total, uint32_t *budget_active);
/* Phase 2 (tac.zig:157-217). */
int orc_tac_damped_phase2(const uint32_t *freqs, const float *spreads, uint64_t n,
                          uint32_t *kappa, float *frac, uint32_t budget_active, uint32_t mu,
                          uint32_t tau);
/* Phase 3 (tac.zig:236-258). */
int orc_tac_bound_phase3(const uint32_t *freqs, uint64_t n, uint32_t *kappa, uint32_t mu,
                         uint32_t tau, uint32_t epsilon, uint32_t theta);
/* Phase 4 (tac.zig:286-372). */
int orc_tac_reconcile_phase4(const uint32_t *freqs, uint64_t n, uint32_t *kappa,
                             const float *frac, uint32_t kappa_total, uint32_t mu, uint32_t tau,
                             uint32_t epsilon, uint32_t theta);
/* Phases 1-4 (tac.zig:388-401). */
int orc_tac_allocate_budgets(const uint32_t *freqs, const float *spreads, uint64_t n,
                             uint32_t *kappa, float *frac, const orc_tac_params *p);
/* Per-token spread s_j by Welford (tac.zig:604-638); vectors grouped by token
 * through offsets / indices (CSR, ascending input order within a token). */
void orc_tac_spreads(const float *vectors, uint32_t dim, const uint32_t *group_offsets,
                     const uint32_t *group_indices, uint64_t n_distinct, float *spreads);
/* clusterFlat (tac.zig:563-830).  n_distinct = max(token_ids) + 1 is written
 * to *n_distinct_out; kappa_per_token must hold it (callers size it from the
 * ids).  centroids: kappa_total * dim; assignments: n_tokens. */
int orc_tac_cluster_flat(const uint32_t *token_ids, uint64_t n_tokens, const float *vectors,
                         uint64_t vectors_len, uint32_t dim, const orc_tac_params *p,
                         float *centroids,
                         uint32_t *assignments, uint32_t *kappa_per_token, float *wcss_total,
                         uint64_t *n_distinct_out);

#ifdef __cplusplus
}
#endif
#endif
