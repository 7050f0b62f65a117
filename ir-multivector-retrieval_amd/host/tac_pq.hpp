// tac_pq.hpp — C++ mirror of the reference's `tac.index.pq` and `tac.kmeans`
// over the gfx950 C ABI (include/tac_gpu.h).
//
//   tac::index::pq::train   <- pq.train       src/index/pq.zig:158-291
//   tac::index::pq::PQ      <- PQ             src/index/pq.zig:41-56
//     .encode / .decode     <- PQ.encode/decode  src/index/pq.zig:59-88
//     .encode_many          <- the storage.build encode loop
//                              src/index/storage.zig:280-295, :384-401
//   tac::kmeans::fit        <- kmeans.fit     src/tac/kmeans.zig:67-232
//   tac::index::storage::residualsAndNorms
//                           <- residualsAndNormsChunk over every token
//                              src/index/storage.zig:255-278, :355-376
//
// Zig error unions become exceptions of type tac::Error carrying the C-ABI
// status; error names follow PqError / KMeansError / RngError.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/tac_gpu.h"

namespace tac {

class Error : public std::runtime_error {
 public:
  explicit Error(int status)
      : std::runtime_error(message(status)), status_(status) {}
  int status() const noexcept { return status_; }

 private:
  static std::string message(int status) {
    std::string m = tac_gpu_strerror(status);
    if (status == TAC_ERR_HIP || status == TAC_ERR_OUT_OF_MEMORY || status == TAC_ERR_NO_DEVICE) {
      const char* detail = tac_gpu_last_error();
      if (detail && *detail) m += std::string(": ") + detail;
    }
    return m;
  }
  int status_;
};

inline void check(int status) {
  if (status != TAC_OK) throw Error(status);
}

namespace constants {
constexpr uint32_t PQ_M = 32;          // src/constants.zig:16
constexpr uint32_t PQ_BITS = 8;        // src/constants.zig:17
constexpr uint32_t PQ_CENTROIDS = 256; // src/constants.zig:18
}  // namespace constants

namespace index {
namespace pq {

struct TrainOptions {
  uint32_t m = constants::PQ_M;
  uint32_t ksub = constants::PQ_CENTROIDS;
  uint32_t max_iters = 25;     // src/index/pq.zig:321
  float tol = 1e-4f;           // src/index/pq.zig:322; TAC_TOL_NEVER for fixed iterations
  const float* init_codebooks = nullptr;  // [m][ksub][dsub]; nullptr: k-means++
};

struct PQ {
  uint32_t dim = 0;
  uint32_t sub_dim = 0;
  uint32_t m = constants::PQ_M;
  uint32_t ksub = constants::PQ_CENTROIDS;
  std::vector<float> codebooks;  // codebook[((mm * ksub) + c) * sub_dim + k]

  const float* codebook_entry(uint32_t mm, uint32_t c) const {
    return codebooks.data() + (static_cast<size_t>(mm) * ksub + c) * sub_dim;
  }

  // Codes of one residual, one byte per subspace (ksub <= 256).
  std::vector<uint8_t> encode(const std::vector<float>& residual) const {
    if (residual.size() != dim) throw Error(TAC_ERR_DIM_MISMATCH);
    return encode_many(residual.data(), 1);
  }

  // Token-major [n][m] codes for n residuals (ksub <= 256).
  std::vector<uint8_t> encode_many(const float* residuals, uint64_t n) const {
    if (ksub > 256) throw Error(TAC_ERR_UNSUPPORTED);
    std::vector<uint8_t> out(static_cast<size_t>(n) * m);
    if (n) check(tac_pq_encode(residuals, n, dim, m, ksub, codebooks.data(), out.data()));
    return out;
  }

  std::vector<float> decode(const std::vector<uint8_t>& codes) const {
    if (codes.size() != m) throw Error(TAC_ERR_DIM_MISMATCH);
    std::vector<float> out(dim);
    check(tac_pq_decode(codes.data(), 1, dim, m, ksub, codebooks.data(), out.data()));
    return out;
  }
};

// pq.train: n_threads is accepted for signature parity; the GPU trains every
// subspace at once.
inline PQ train(const std::vector<float>& residuals, uint32_t dim, uint64_t seed,
                uint32_t n_threads = 1, const TrainOptions& opt = {}) {
  (void)n_threads;
  // Order of src/index/pq.zig:165-168.
  if (dim == 0) throw Error(TAC_ERR_DIM_MISMATCH);
  if (opt.m == 0) throw Error(TAC_ERR_INVALID_ARGUMENT);
  if (dim % opt.m != 0) throw Error(TAC_ERR_DIM_NOT_DIVISIBLE_BY_M);
  if (residuals.empty()) throw Error(TAC_ERR_EMPTY_CORPUS);
  if (residuals.size() % dim != 0) throw Error(TAC_ERR_DIM_MISMATCH);
  PQ out;
  out.dim = dim;
  out.sub_dim = dim / opt.m;
  out.m = opt.m;
  out.ksub = opt.ksub;
  out.codebooks.resize(static_cast<size_t>(opt.m) * opt.ksub * out.sub_dim);
  check(tac_pq_train(residuals.data(), residuals.size() / dim, dim, opt.m, opt.ksub,
                     opt.init_codebooks, seed, opt.max_iters, opt.tol, out.codebooks.data(),
                     nullptr));
  return out;
}

}  // namespace pq

namespace storage {

struct Residuals {
  std::vector<float> residuals;  // [n][dim], unit norm where norm > 0
  std::vector<float> norms;      // [n]
};

// storage.build stage 2: residual = (vector - centroids[assignment]) scaled
// by fl(1 / norm) when norm > 0.  An assignment outside the centroid table
// throws InvalidArgument.
inline Residuals residualsAndNorms(const std::vector<float>& vectors, uint32_t dim,
                                   const std::vector<float>& centroids,
                                   const std::vector<uint32_t>& assignments) {
  if (dim == 0 || vectors.size() % dim != 0 || centroids.size() % dim != 0 ||
      vectors.size() / dim != assignments.size())
    throw Error(TAC_ERR_DIM_MISMATCH);
  Residuals out;
  out.residuals.resize(vectors.size());
  out.norms.resize(assignments.size());
  if (assignments.empty()) return out;
  check(tac_residuals(vectors.data(), assignments.size(), dim, centroids.data(),
                      static_cast<uint32_t>(centroids.size() / dim), assignments.data(),
                      out.residuals.data(), out.norms.data()));
  return out;
}

}  // namespace storage
}  // namespace index

namespace kmeans {

struct KMeansResult {
  std::vector<float> centroids;     // [k][dim]
  std::vector<uint32_t> assignments;
  float wcss = 0.0f;
  uint32_t iters_run = 0;
};

struct KMeansParams {  // src/tac/kmeans.zig:28-41
  uint32_t k = 0;
  uint32_t max_iters = 25;
  float tol = 1e-4f;
  uint64_t seed = 0;
  uint32_t n_threads = 1;
  const float* init_centroids = nullptr;  // [k][dim]; nullptr: k-means++
};

inline KMeansResult fit(const std::vector<float>& vectors, uint32_t dim, const KMeansParams& p) {
  // Order of src/tac/kmeans.zig:73-76.
  if (p.k == 0) throw Error(TAC_ERR_KMEANS_BUDGET_TOO_SMALL);
  if (dim == 0) throw Error(TAC_ERR_DIM_MISMATCH);
  if (vectors.empty()) throw Error(TAC_ERR_EMPTY_VECTOR_SET);
  if (vectors.size() % dim != 0) throw Error(TAC_ERR_DIM_MISMATCH);
  const uint64_t n = vectors.size() / dim;
  KMeansResult r;
  r.centroids.resize(static_cast<size_t>(p.k) * dim);
  r.assignments.resize(n);
  check(tac_kmeans_fit(vectors.data(), n, dim, p.k, p.max_iters, p.tol, p.seed, p.init_centroids,
                       r.centroids.data(), r.assignments.data(), &r.wcss, &r.iters_run));
  return r;
}

}  // namespace kmeans
}  // namespace tac
