/*
 * tac_gpu.h — C ABI of the MI355X (gfx950) product-quantization build path.
 *
 * Drop-in boundary for the reference's `tac.index.pq` module (Zig):
 *   pq.train        src/index/pq.zig:158-291   -> tac_pq_train / tac_pq_train_device
 *   PQ.encode       src/index/pq.zig:59-76, batched the way storage.build drives
 *                   it (src/index/storage.zig:280-295, :384-401)
 *                                              -> tac_pq_encode / tac_pq_encode_device
 *   PQ.decode       src/index/pq.zig:79-88     -> tac_pq_decode
 *   kmeans.fit      src/tac/kmeans.zig:67-232  -> tac_kmeans_fit
 *   storage.build stage 2, residualsAndNormsChunk
 *                   src/index/storage.zig:255-278, :355-376
 *                                              -> tac_residuals / tac_residuals_device
 *   .tac doc layouts and footer checksum
 *                   src/index/storage.zig:674-686, :705-749, :612-617
 *                                              -> tac_doc_payload_bytes,
 *                                                 tac_write_doc_layouts[_device],
 *                                                 tac_crc32[_device]
 *   PQ.buildDistanceTable src/index/pq.zig:92-123 -> tac_pq_distance_table[_device]
 *   refine          src/retrieval/refine.zig:83-145 -> tac_refine / tac_refine_device
 *   TAC.clusterFlat src/tac/tac.zig:563-830    -> tac_cluster_flat
 *   RefineError / StorageError (src/retrieval/refine.zig:37-42,
 *   src/index/storage.zig:42-47) -> tac_status 16-20
 *   PqError / KMeansError / RngError (src/index/pq.zig:32-38,
 *   src/tac/kmeans.zig:56-60, src/util/rng.zig:14-18) -> tac_status
 *
 * Rules: plain C types; buffers are owned by the caller; the library never
 * returns memory it allocated; 0 means success; no exception crosses the ABI.
 * Calls are thread-safe and serialise per device.  Arguments are validated
 * (with the reference's error precedence) before any device is touched, so
 * argument errors are reported the same way on a host without a GPU.
 *
 * Shapes: `n` residual vectors of `dim` fp32 values, token-major [n][dim];
 * `m` subspaces of dsub = dim / m values (1 <= dsub <= 8); `ksub` codewords
 * per subspace (1 <= ksub <= 1024).  Codebooks are [m][ksub][dsub] fp32
 * (codebook[((mm * ksub) + c) * dsub + k], src/index/pq.zig:14-15).  Codes are
 * token-major [n][m], uint8_t when ksub <= 256 and uint16_t otherwise.
 *
 * Arithmetic is the reference's: distances are the unfused left fold of
 * (x_k - c_k)^2, argmin keeps the first index, cluster sums fold members in
 * ascending vector order from 0.0f and the centroid is sum * fl(1/fl(count)).
 * Results are bit-identical to the oracle's restatement of the reference for
 * the same inputs; they equal the reference's wherever that restatement's two
 * unverifiable assumptions hold: the Zig std PRNG stream behind k-means++
 * seeding, and 16 f32 lanes in the reference's generic distance path.
 */
#ifndef TAC_GPU_H
#define TAC_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum tac_status {
  TAC_OK = 0,
  TAC_ERR_DIM_NOT_DIVISIBLE_BY_M = 1,  /* PqError.DimNotDivisibleByM */
  TAC_ERR_DIM_MISMATCH = 2,            /* PqError.DimMismatch, KMeansError.DimMismatch */
  TAC_ERR_EMPTY_CORPUS = 3,            /* PqError.EmptyCorpus */
  TAC_ERR_OUT_BUFFER_WRONG_SIZE = 4,   /* PqError.OutBufferWrongSize */
  TAC_ERR_NQ_MISMATCH = 5,             /* PqError.NQMismatch */
  TAC_ERR_KMEANS_BUDGET_TOO_SMALL = 6, /* KMeansError.KmeansBudgetTooSmall */
  TAC_ERR_EMPTY_VECTOR_SET = 7,        /* KMeansError.EmptyVectorSet */
  TAC_ERR_RNG_EMPTY_DISTRIBUTION = 8,  /* RngError.EmptyDistribution */
  TAC_ERR_RNG_NON_FINITE = 9,          /* RngError.NonFinite */
  TAC_ERR_RNG_ALL_ZERO = 10,           /* RngError.AllZero */
  TAC_ERR_OUT_OF_MEMORY = 11,          /* Allocator.Error.OutOfMemory */
  TAC_ERR_NO_DEVICE = 12,              /* no usable HIP device */
  TAC_ERR_HIP = 13,                    /* HIP runtime error; see tac_gpu_last_error */
  TAC_ERR_INVALID_ARGUMENT = 14,       /* null pointer / shape outside the limits above */
  TAC_ERR_UNSUPPORTED = 15,            /* valid request this build does not implement */
  TAC_ERR_QUERY_SHAPE_MISMATCH = 16,   /* RefineError.QueryShapeMismatch */
  TAC_ERR_TABLE_SIZE_MISMATCH = 17,    /* RefineError.TableSizeMismatch */
  TAC_ERR_DOC_OUT_OF_RANGE = 18,       /* RefineError.DocOutOfRange */
  TAC_ERR_DOC_LAYOUT_CORRUPT = 19,     /* RefineError.DocLayoutCorrupt */
  TAC_ERR_BUFFER_TOO_SMALL = 20,       /* StorageError.BufferTooSmall */
  TAC_ERR_BUDGET_TOO_SMALL = 21,       /* ClusteringError.BudgetTooSmall */
  TAC_ERR_BUDGET_TOO_LARGE = 22,       /* ClusteringError.BudgetTooLarge */
  TAC_ERR_INVALID_THRESHOLDS = 23,     /* ClusteringError.InvalidThresholds */
  TAC_ERR_EMPTY_TOKEN_DUMP = 24        /* ClusteringError.EmptyTokenDump */
} tac_status;

/* Never-break iteration control: pass as `tol` to run exactly max_iters. */
#define TAC_TOL_NEVER (-__builtin_inff())

/* Human-readable name of a status ("DimNotDivisibleByM", ...). */
const char *tac_gpu_strerror(int status);
/* Detail of the last TAC_ERR_HIP / TAC_ERR_OUT_OF_MEMORY on this thread. */
const char *tac_gpu_last_error(void);

/* ---- devices and memory (helpers for callers without a HIP binding) ---- */
int tac_gpu_device_count(int *count);
typedef struct tac_gpu_device_info {
  char name[256];
  char arch[64];            /* e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int clock_khz;
  uint64_t global_mem_bytes;
  uint64_t lds_bytes_per_block;
} tac_gpu_device_info;
int tac_gpu_get_device_info(int device, tac_gpu_device_info *info);
/*
 * vec.lane_count of the host the reference is built for,
 * std.simd.suggestVectorLength(f32) (src/util/vec.zig:16): 16 on AVX-512
 * x86-64 (the default), 8 on AVX2, 4 on NEON (aarch64).  It orders the
 * reference's generic l2sq / dot (vec.zig:90-103, :159-175), used at PQ
 * sub-dimension 8 (4 lanes pair elements j and j + 4) and by token
 * clustering at dims other than 2, 4, 64 and 128; every other distance is
 * unaffected.  Process-wide; takes effect on a device at the next call there
 * (calls already running keep the value they started with).  lanes must be
 * 4, 8 or 16 (else TAC_ERR_INVALID_ARGUMENT).  No counterpart call in the
 * reference, where it is a build-time constant.
 */
int tac_gpu_set_lane_count(uint32_t lanes);
int tac_gpu_get_lane_count(uint32_t *lanes);

int tac_gpu_set_device(int device);
int tac_gpu_malloc(void **ptr, uint64_t bytes);
int tac_gpu_free(void *ptr);
int tac_gpu_memcpy_htod(void *dst, const void *src, uint64_t bytes);
int tac_gpu_memcpy_dtoh(void *dst, const void *src, uint64_t bytes);
int tac_gpu_memcpy_dtod(void *dst, const void *src, uint64_t bytes);
int tac_gpu_synchronize(void);
/* Release the per-device workspace the library caches between calls (device
 * buffers and the pinned host staging buffers of large uploads). */
int tac_gpu_release_workspace(void);

/* ---- optional outputs of training (every pointer may be NULL) ---------- */
typedef struct tac_pq_train_extras {
  uint32_t *iters_run; /* host [m]: Lloyd iterations run per subspace (KMeansResult.iters_run) */
  float *wcss;         /* host [m]: wcss of each subspace's last iteration (KMeansResult.wcss) */
  uint32_t *empties;   /* host [m]: empty clusters reseeded, summed over iterations */
  float *trace;        /* host [max_iters][m][ksub][dsub]: codebooks after each iteration;
                          iterations a subspace did not run repeat its final codebook */
} tac_pq_train_extras;

/*
 * pq.train (src/index/pq.zig:158-291) with runtime m / ksub and iteration
 * control.  Each subspace runs kmeans.fit with k = ksub
 * (src/index/pq.zig:301-336):
 *   - init_codebooks [m][ksub][dsub] seeds the Lloyd loop; NULL selects the
 *     reference's k-means++ seeding (src/tac/kmeans.zig:106-136) on the GPU,
 *     subspace m drawing from std.Random.DefaultPrng seeded with seed +% m;
 *     its errors are TAC_ERR_RNG_NON_FINITE and TAC_ERR_RNG_ALL_ZERO
 *     (src/util/rng.zig:57-82), reported for the lowest failing subspace;
 *   - tol = 1e-4f, max_iters = 25 are the reference's values
 *     (src/index/pq.zig:319-325); TAC_TOL_NEVER runs exactly max_iters;
 *   - n <= ksub takes the degenerate branch (src/tac/kmeans.zig:88-104).
 * Host pointers; the device copy of the residuals lives only for the call.
 */
int tac_pq_train(const float *residuals, uint64_t n, uint32_t dim, uint32_t m,
                 uint32_t ksub, const float *init_codebooks, uint64_t seed,
                 uint32_t max_iters, float tol, float *codebooks_out,
                 tac_pq_train_extras *extras);

/* Same, with residuals, init codebooks and the output in device memory.
 * `stream` is a hipStream_t (NULL: the library's stream for the device). */
int tac_pq_train_device(const float *d_residuals, uint64_t n, uint32_t dim,
                        uint32_t m, uint32_t ksub, const float *d_init_codebooks,
                        uint64_t seed, uint32_t max_iters, float tol,
                        float *d_codebooks_out, tac_pq_train_extras *extras,
                        void *stream);

/*
 * pq.train followed by PQ.encode of the same residuals, the way
 * storage.build chains them (src/index/storage.zig:380-401; train at :380,
 * the token-major encode loop at :384-401): d_codebooks_out as
 * tac_pq_train_device, and d_codes_out [n][m] (uint8_t, uint16_t past
 * ksub 256) equal to tac_pq_encode_device's codes for those codebooks.  The
 * encode runs as one more candidate pass anchored at the last Lloyd codes
 * (no grid anchors; the argmin is exact for any anchor); configurations
 * without the candidate tables (ksub > 1024, n < 16,384 with one
 * iteration, n <= ksub, max_iters 0) run tac_pq_encode_device's path.
 */
int tac_pq_train_encode_device(const float *d_residuals, uint64_t n, uint32_t dim,
                               uint32_t m, uint32_t ksub, const float *d_init_codebooks,
                               uint64_t seed, uint32_t max_iters, float tol,
                               float *d_codebooks_out, void *d_codes_out,
                               tac_pq_train_extras *extras, void *stream);

/*
 * PQ.encode (src/index/pq.zig:59-76) for n residuals at once, as
 * storage.build drives it (src/index/storage.zig:384-401): codes_out is
 * token-major [n][m] (uint8_t for ksub <= 256, else uint16_t).
 */
int tac_pq_encode(const float *residuals, uint64_t n, uint32_t dim, uint32_t m,
                  uint32_t ksub, const float *codebooks, void *codes_out);
int tac_pq_encode_device(const float *d_residuals, uint64_t n, uint32_t dim,
                         uint32_t m, uint32_t ksub, const float *d_codebooks,
                         void *d_codes_out, void *stream);

/*
 * tac_pq_encode_device without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, validation and codes as tac_pq_encode_device; stream NULL
 * is the device's null stream, and the call returns once the work is
 * enqueued.  Its scratch (counters, neighbour rows, grid anchors, deferred
 * lists) is one static 32 MiB device array per GPU, held until the process
 * ends; rows run in batches that fit it, so every n that
 * tac_pq_encode_device accepts is accepted (codebooks whose tables leave no
 * room for a 16,384-row batch take the full search).  All calls on one GPU
 * share its array: calls that overlap on a GPU (other threads or streams)
 * race, and the caller must serialise them.
 */
int tac_pq_encode_device_noalloc(const float *d_residuals, uint64_t n, uint32_t dim,
                                 uint32_t m, uint32_t ksub, const float *d_codebooks,
                                 void *d_codes_out, void *stream);

/* PQ.decode (src/index/pq.zig:79-88) for n code rows: out [n][dim]. */
int tac_pq_decode(const void *codes, uint64_t n, uint32_t dim, uint32_t m,
                  uint32_t ksub, const float *codebooks, float *out);

/*
 * kmeans.fit (src/tac/kmeans.zig:67-232) for one set of vectors:
 * centroids_out [k][dim], assignments_out [n] (the last iteration's
 * assignment, KMeansResult.assignments), wcss_out and iters_run_out.
 * init_centroids NULL selects k-means++ seeded with `seed`, as tac_pq_train.
 * Distances are vec.l2sq at the vectors' dim (src/util/vec.zig:109-175).
 * dim <= 8 (k <= 1024) runs on the PQ kernels; 9 <= dim <= 512 (any k) on
 * the token-clustering engine as one problem; wider rows are
 * TAC_ERR_UNSUPPORTED.
 */
int tac_kmeans_fit(const float *vectors, uint64_t n, uint32_t dim, uint32_t k,
                   uint32_t max_iters, float tol, uint64_t seed,
                   const float *init_centroids, float *centroids_out,
                   uint32_t *assignments_out, float *wcss_out,
                   uint32_t *iters_run_out);

/* ---- storage.build stage 2: residuals and norms -------------------------- */
/*
 * residualsAndNormsChunk (src/index/storage.zig:255-278), run over every
 * token as storage.build does at :355-376.  For token i with centroid
 * a = assignments[i]:
 *   diff_d = vectors[i][d] - centroids[a][d];
 *   norms_out[i] = sqrt(((0 + diff_0^2) + diff_1^2) + ...), each operation
 *                  rounded separately, in ascending d;
 *   residuals_out[i][d] = diff_d * fl(1 / norm) if norm > 0, else diff_d.
 * residuals_out may alias vectors.  An assignment >= n_centroids (a bounds
 * trap in the reference) is TAC_ERR_INVALID_ARGUMENT and leaves the outputs
 * unspecified.  dim <= 4096.
 */
int tac_residuals(const float *vectors, uint64_t n, uint32_t dim,
                  const float *centroids, uint32_t n_centroids,
                  const uint32_t *assignments, float *residuals_out,
                  float *norms_out);
/* Same on device buffers; ordered on `stream` (NULL: the library's stream).
 * Returns after the kernel has finished (it reads back the range check). */
int tac_residuals_device(const float *d_vectors, uint64_t n, uint32_t dim,
                         const float *d_centroids, uint32_t n_centroids,
                         const uint32_t *d_assignments, float *d_residuals_out,
                         float *d_norms_out, void *stream);

/* ---- .tac per-document layouts and image checksum ----------------------- */
/*
 * docPayloadSize (src/index/storage.zig:674-686) for m codes of code_bytes
 * (1: ksub <= 256, 2: ksub <= 65536, little-endian) per token; a host-only
 * computation over host doc_offsets [n_docs + 1].
 */
int tac_doc_payload_bytes(const uint64_t *doc_offsets, uint64_t n_docs, uint32_t m,
                          uint32_t code_bytes, uint64_t *bytes_out);
/*
 * writeDocLayouts (src/index/storage.zig:705-749): doc_index_out [n_docs + 1]
 * gets each document's payload offset (the last entry is the total) and
 * payload_out the layouts: u32 n_d | u32 centroid id x n_d | n_d x m codes |
 * zero padding to 8 bytes, all little-endian.  doc_offsets [n_docs + 1] must
 * be non-decreasing with doc_offsets[n_docs] <= n_tokens (else
 * TAC_ERR_INVALID_ARGUMENT); assignments [n_tokens]; codes [n_tokens][m].
 * payload_len smaller than the layouts: TAC_ERR_BUFFER_TOO_SMALL.
 */
int tac_write_doc_layouts(const uint64_t *doc_offsets, uint64_t n_docs, uint64_t n_tokens,
                          const uint32_t *assignments, const void *codes, uint32_t m,
                          uint32_t code_bytes, uint64_t *doc_index_out, uint8_t *payload_out,
                          uint64_t payload_len);
/* Same on device buffers (payload_out 8-byte aligned); returns when done. */
int tac_write_doc_layouts_device(const uint64_t *d_doc_offsets, uint64_t n_docs,
                                 uint64_t n_tokens, const uint32_t *d_assignments,
                                 const void *d_codes, uint32_t m, uint32_t code_bytes,
                                 uint64_t *d_doc_index_out, uint8_t *d_payload_out,
                                 uint64_t payload_len, void *stream);
/*
 * std.hash.Crc32 (CRC-32/ISO-HDLC) of len bytes, the footer checksum that
 * serialise writes and parse verifies (src/index/storage.zig:612-617,
 * :782-786).  tac_crc32 takes a host buffer, tac_crc32_device a device one;
 * both store the checksum in *crc_out (host memory) and return when done.
 */
int tac_crc32(const void *bytes, uint64_t len, uint32_t *crc_out);
int tac_crc32_device(const void *d_bytes, uint64_t len, uint32_t *crc_out, void *stream);

/* ---- query side: distance table and refine ------------------------------ */
/*
 * PQ.buildDistanceTable (src/index/pq.zig:92-123): table_out [m][ksub][n_q],
 * entry ((mm * ksub) + c) * n_q + i = dot(query_i[mm * dsub ..], codeword).
 * n_q == 0: TAC_ERR_NQ_MISMATCH; table_len != m * ksub * n_q:
 * TAC_ERR_OUT_BUFFER_WRONG_SIZE.
 */
int tac_pq_distance_table(const float *query_tokens, uint32_t n_q, uint32_t dim, uint32_t m,
                          uint32_t ksub, const float *codebooks, float *table_out,
                          uint64_t table_len);
int tac_pq_distance_table_device(const float *d_query_tokens, uint32_t n_q, uint32_t dim,
                                 uint32_t m, uint32_t ksub, const float *d_codebooks,
                                 float *d_table_out, uint64_t table_len, void *stream);

/* The parts of a parsed .tac Index (src/index/storage.zig:86-124) that refine
 * reads.  Pointers are host or device memory to match the entry point. */
typedef struct tac_doc_index {
  uint32_t dim;                      /* token dim */
  uint32_t kappa;                    /* centroids */
  uint32_t m;                        /* PQ codes per token */
  uint32_t ksub;                     /* codes are uint8 if <= 256, else uint16 LE */
  uint64_t n_docs;
  uint64_t n_tokens;
  uint64_t payload_len;
  const float *centroids;            /* [kappa][dim] */
  const uint64_t *doc_index;         /* [n_docs + 1] payload offsets */
  const uint8_t *doc_payload;        /* per-document layouts */
  const uint64_t *doc_token_offsets; /* [n_docs + 1] */
  const float *residual_norms;       /* [n_tokens] */
} tac_doc_index;

/*
 * refine (src/retrieval/refine.zig:83-145) for n_candidates documents of one
 * query: scores_out[j] = exact MaxSim of doc doc_ids[j],
 *   sum_i max_k ( dot(q_i, centroid[c_k]) + norm_k * sum_m table[m][code_km][i] ).
 * Errors, checked per candidate in order, return the first failing
 * candidate's RefineError (n_q == 0: QueryShapeMismatch; table_len !=
 * m * ksub * n_q: TableSizeMismatch; doc id >= n_docs: DocOutOfRange; a
 * layout, token range, centroid id or code out of bounds: DocLayoutCorrupt).
 * The query tokens (n_q * (dim + 1) floats) and per-wave staging must fit in
 * 64 KB of LDS (about n_q * dim <= 14,000), else TAC_ERR_UNSUPPORTED.
 */
int tac_refine(const tac_doc_index *index, const float *table, uint64_t table_len,
               const float *query_tokens, uint32_t n_q, const uint32_t *doc_ids,
               uint32_t n_candidates, float *scores_out);
int tac_refine_device(const tac_doc_index *d_index, const float *d_table, uint64_t table_len,
                      const float *d_query_tokens, uint32_t n_q, const uint32_t *d_doc_ids,
                      uint32_t n_candidates, float *d_scores_out, void *stream);


/* ---- token-aware clustering --------------------------------------------- */
/* ClusteringParams (src/tac/tac.zig:35-58).  The paper defaults are
 * mu 128, tau 256, epsilon 4, theta 39, max_iters 25, tol 1e-4
 * (src/constants.zig TAC_MU / TAC_TAU / TAC_EPSILON / TAC_THETA). */
typedef struct tac_cluster_params {
  uint32_t kappa_total;
  uint32_t mu, tau, epsilon, theta;
  uint32_t max_iters;
  float tol;
  uint64_t seed;
  uint32_t n_threads; /* only groups wcss_total: 1 folds the per-token wcss in token
                         order (the serial path); T > 1 folds each of T contiguous
                         slices of token ids, then the slices (tac.zig:688-820) */
} tac_cluster_params;

/*
 * TAC.clusterFlat (src/tac/tac.zig:563-830): groups the n_tokens vectors
 * (vectors_len = n_tokens * dim floats) by token id, computes every token's
 * spread (Welford), allocates the kappa_total centroids over tokens (phases
 * 1-4) and runs kmeans.fit per token with seed ^ token id, all tokens at once
 * on the device.  Outputs, bit-identical to the oracle (and to the reference
 * under the assumptions stated at the top of this file):
 *   centroids_out   kappa_total * dim, concatenated in token-id order;
 *   assignments_out n_tokens global centroid ids;
 *   kappa_per_token_out[j] for j < n_distinct = max(token id) + 1, written to
 *     *n_distinct_out (kappa_per_token_len smaller: TAC_ERR_BUFFER_TOO_SMALL);
 *   *wcss_total_out the per-token wcss folded as params->n_threads selects.
 * Errors follow the reference's order: no tokens EmptyTokenDump; dim 0 or a
 * length mismatch InvalidThresholds; kappa_total 0 BudgetTooSmall; then the
 * phases' errors, and the first failing token's kmeans error (RngError).
 * dim above 512 is TAC_ERR_UNSUPPORTED (rows are staged in LDS), as is a
 * plan of 2^24 or more row tiles, tokens with centroids or wcss chunks (one
 * block each).
 */
int tac_cluster_flat(const uint32_t *token_ids, uint64_t n_tokens, const float *vectors,
                     uint64_t vectors_len, uint32_t dim, const tac_cluster_params *params,
                     float *centroids_out, uint32_t *assignments_out,
                     uint32_t *kappa_per_token_out, uint64_t kappa_per_token_len,
                     float *wcss_total_out, uint64_t *n_distinct_out);
/* tac_cluster_flat over token vectors already resident on the device
 * (d_vectors: n_tokens * dim floats); token ids and every output stay in host
 * memory, results and errors are those of tac_cluster_flat.  No counterpart in
 * the reference: it is for callers whose token vectors are on the GPU already
 * (the storage build holds them there for the residual and encode stages), and
 * skips the n_tokens * dim * 4-byte upload. */
int tac_cluster_flat_device(const uint32_t *token_ids, uint64_t n_tokens,
                            const float *d_vectors, uint64_t vectors_len, uint32_t dim,
                            const tac_cluster_params *params, float *centroids_out,
                            uint32_t *assignments_out, uint32_t *kappa_per_token_out,
                            uint64_t kappa_per_token_len, float *wcss_total_out,
                            uint64_t *n_distinct_out);

/* ---- measurement -------------------------------------------------------- */
/* When enabled, the library brackets its kernels with HIP events on the
 * stream they run on and accumulates their durations. */
typedef struct tac_gpu_profile {
  double transpose_ms;   uint64_t transpose_launches;
  double assign_ms;      uint64_t assign_launches;   /* Lloyd assignment stage */
  double update_ms;      uint64_t update_iters;      /* sort + fold + reseed + convergence */
  double encode_ms;      uint64_t encode_launches;   /* encode kernel */
  uint64_t exact_rescans; /* (vector, subspace) searches the pruned pass left to a full
                             reference scan (near ties across codeword blocks) */
  double residual_ms;    uint64_t residual_launches; /* residual + norm kernel */
  double crc_ms;         uint64_t crc_launches;      /* CRC-32 kernels */
  double refine_ms;      uint64_t refine_launches;   /* refine kernel */
  double cluster_kpp_ms;   /* tac_cluster_flat: degenerate init + k-means++ seeding */
  double cluster_lloyd_ms; /* tac_cluster_flat: Lloyd iterations of every token */
  uint64_t cluster_calls;
  double cluster_prep_ms;  /* wall: grouping, upload, gather, spreads, budget phases, plan */
  double cluster_call_ms;  /* wall: the whole tac_cluster_flat call */
  uint64_t cand_vectors;   /* (vector, subspace) searches started from an anchor codeword:
                              the previous code (Lloyd iterations after the first) or a
                              grid cell's codeword (the first Lloyd iteration and encode,
                              on 16,384 vectors or more) */
  uint64_t cand_deferred;  /* of those, the ones left to the full search (candidate row
                              exhausted, non-finite or huge values) */
  double cand_assign_ms;   /* assignment stages that started from the previous codes
                              (included in assign_ms) */
  uint64_t cand_assign_iters;
  uint64_t train_streams;  /* streams the last training call split its subspaces over: 2 when
                              M is even (halves m < M/2 and m >= M/2 side by side), else 1.
                              With 2, assign_ms and update_ms time the first half while the
                              second runs beside it */
  uint64_t cell_subspaces; /* encode subspaces that took the cell-list pass (rows wider than
                              the codebook's box); the others took the anchored pass */
  uint64_t screen_vectors;  /* (vector, subspace) searches through the matrix-core screen
                               (sub-dimensions 5-8, K <= 256: Lloyd assignment and encode) */
  uint64_t screen_deferred; /* of those, the ones the screen could not settle (left to the
                               pruned exact search) */
} tac_gpu_profile;
int tac_gpu_profile_enable(int enable);
int tac_gpu_profile_read(tac_gpu_profile *out, int reset);

/* Per-kernel times: while profiling is enabled, training and encode bracket
 * each kernel launch with HIP events on the stream it runs on.  `name` is the
 * kernel as rocprofv3 reports it, without the namespace (for example
 * "cand_kernel<4, false, false, unsigned short>"). */
typedef struct tac_gpu_kernel_time {
  char name[96];
  double ms;          /* summed over launches */
  uint64_t launches;
} tac_gpu_kernel_time;
/* Writes up to cap entries to out (sorted by name) and the number of
 * distinct kernels timed to *count; reset clears the tallies. */
int tac_gpu_profile_kernels(tac_gpu_kernel_time *out, uint32_t cap, uint32_t *count, int reset);

#ifdef __cplusplus
}
#endif
#endif /* TAC_GPU_H */
