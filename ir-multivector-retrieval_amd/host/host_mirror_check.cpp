// host_mirror_check.cpp — exercises the C++ mirror (tac_pq.hpp) through the
// static library, the way a compiled host links it.
//
//   host_mirror_check errors   argument errors map to the reference's error
//                              names (no GPU needed); without a device, a
//                              valid call reports NoDevice
//   host_mirror_check gpu      train -> encode -> decode round trip on GPU 0:
//                              decode(encode(x)) re-encodes to the same codes
//                              (src/index/pq.zig:372-413)
#include <cstdio>
#include <cstring>
#include <vector>

#include "tac_pq.hpp"

namespace {

int expect_error(const char* what, int status, void (*fn)()) {
  try {
    fn();
  } catch (const tac::Error& e) {
    if (e.status() == status) {
      std::printf("ok   %-34s -> %s\n", what, tac_gpu_strerror(status));
      return 0;
    }
    std::printf("FAIL %-34s -> %s (wanted %s)\n", what, tac_gpu_strerror(e.status()),
                tac_gpu_strerror(status));
    return 1;
  }
  std::printf("FAIL %-34s -> no error\n", what);
  return 1;
}

int errors_mode() {
  int bad = 0;
  bad += expect_error("train dim 33 (pq.zig:357-363)", TAC_ERR_DIM_NOT_DIVISIBLE_BY_M, [] {
    tac::index::pq::train(std::vector<float>(33, 0.0f), 33, 1);
  });
  bad += expect_error("train empty (pq.zig:365-370)", TAC_ERR_EMPTY_CORPUS, [] {
    tac::index::pq::train(std::vector<float>{}, 32, 1);
  });
  bad += expect_error("train dim 0", TAC_ERR_DIM_MISMATCH, [] {
    tac::index::pq::train(std::vector<float>(64, 0.0f), 0, 1);
  });
  bad += expect_error("train ragged length", TAC_ERR_DIM_MISMATCH, [] {
    tac::index::pq::train(std::vector<float>(65, 0.0f), 32, 1);
  });
  bad += expect_error("fit k == 0 (kmeans.zig:373-377)", TAC_ERR_KMEANS_BUDGET_TOO_SMALL, [] {
    tac::kmeans::KMeansParams p;
    tac::kmeans::fit(std::vector<float>{1, 0, 0, 1}, 2, p);
  });
  bad += expect_error("fit empty (kmeans.zig:379-383)", TAC_ERR_EMPTY_VECTOR_SET, [] {
    tac::kmeans::KMeansParams p;
    p.k = 1;
    tac::kmeans::fit(std::vector<float>{}, 2, p);
  });
  bad += expect_error("fit dim mismatch (kmeans.zig:385-389)", TAC_ERR_DIM_MISMATCH, [] {
    tac::kmeans::KMeansParams p;
    p.k = 1;
    tac::kmeans::fit(std::vector<float>{1, 2, 3}, 2, p);
  });
  bad += expect_error("residuals ragged input", TAC_ERR_DIM_MISMATCH, [] {
    tac::index::storage::residualsAndNorms(std::vector<float>(7, 0.0f), 2, {0.0f, 0.0f}, {0, 0});
  });
  int count = 0;
  if (tac_gpu_device_count(&count) == TAC_ERR_NO_DEVICE) {
    bad += expect_error("valid train without a device", TAC_ERR_NO_DEVICE, [] {
      tac::index::pq::TrainOptions o;
      o.m = 2;
      o.ksub = 4;
      std::vector<float> init(2 * 4 * 2, 0.0f);
      o.init_codebooks = init.data();
      tac::index::pq::train(std::vector<float>(40, 0.5f), 4, 1, 1, o);
    });
  }
  return bad;
}

int gpu_mode() {
  const uint32_t n = 3000, dim = 32;
  std::vector<float> x(static_cast<size_t>(n) * dim);
  uint64_t s = 0x52017;
  for (auto& v : x) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    v = static_cast<float>(static_cast<int64_t>(s >> 11) % 2001 - 1000) * 1e-3f;
  }
  tac::index::pq::TrainOptions o;  // m = 32, ksub = 256, dsub = 1
  std::vector<float> init(static_cast<size_t>(o.m) * o.ksub);
  for (uint32_t mm = 0; mm < o.m; ++mm)
    for (uint32_t c = 0; c < o.ksub; ++c) init[mm * o.ksub + c] = x[static_cast<size_t>(c) * dim + mm];
  o.init_codebooks = init.data();
  const auto pq = tac::index::pq::train(x, dim, 17, 1, o);
  const std::vector<float> first(x.begin(), x.begin() + dim);
  const auto codes_a = pq.encode(first);
  const auto decoded = pq.decode(codes_a);
  const auto codes_b = pq.encode(decoded);
  const bool same = codes_a == codes_b;
  std::printf("%s encode(decode(encode(x))) == encode(x) over %u subspaces\n", same ? "ok  " : "FAIL",
              pq.m);
  // residual stage: centroids 0 and 1 of a 2-row table, (3, 4) -> norm 5
  const auto res = tac::index::storage::residualsAndNorms({4, 6, 1, 1}, 2, {1, 2, 1, 1}, {0, 1});
  const bool res_ok = res.norms[0] == 5.0f && res.norms[1] == 0.0f &&
                      res.residuals[0] == 0.6f && res.residuals[1] == 0.8f &&
                      res.residuals[2] == 0.0f && res.residuals[3] == 0.0f;
  std::printf("%s residualsAndNorms (3,4) -> norm 5, zero row unscaled\n", res_ok ? "ok  " : "FAIL");
  return (same && res_ok) ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "errors";
  const int bad = std::strcmp(mode, "gpu") == 0 ? gpu_mode() : errors_mode();
  std::printf("%s\n", bad ? "host mirror check FAILED" : "host mirror check passed");
  return bad ? 1 : 0;
}
