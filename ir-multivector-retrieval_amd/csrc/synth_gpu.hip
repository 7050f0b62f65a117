// synth_gpu.hip — the synthetic residual generator of synth.c as a gfx950
// kernel, for benchmark inputs that are too large to generate on the host
// in reasonable time (60M and 200M residuals).  Not part of the PQ library.
//
// Same definition as synth.c: every draw is a pure function of (seed,
// stream, counter); centres c_j = normalize(z_j); vector v_i =
// normalize(c_{j_i} + sigma * N(0, I)); residual r_i = v_i - c_{j_i}; j_i
// uniform or Zipf(s) through the host-built CDF.  Normals are Box-Muller in
// double precision with the device's log / sqrt / sincos, so a value can
// differ from synth.c's in its last bit; callers that compare against the
// oracle feed the oracle these very bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr uint64_t kStreamAssign = 2u;
constexpr uint64_t kStreamNoise = 3u;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t draw(uint64_t seed, uint64_t stream, uint64_t ctr) {
  const uint64_t key = mix64(seed * 0x9e3779b97f4a7c15ULL + stream);
  return mix64(key ^ mix64(ctr + 0x632be59bd9b4e019ULL));
}

__device__ __forceinline__ double unit(uint64_t bits) {
  return ((double)(bits >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

// The normal pair number `pair` of row `gi` (dim (dim + 1) / 2 pairs a row).
__device__ __forceinline__ void normal_pair(uint64_t seed, uint64_t ctr, double* z0, double* z1) {
  const double u1 = unit(draw(seed, kStreamNoise, 2 * ctr));
  const double u2 = unit(draw(seed, kStreamNoise, 2 * ctr + 1));
  const double r = sqrt(-2.0 * log(u1));
  double s, c;
  sincos(6.283185307179586 * u2, &s, &c);
  *z0 = r * c;
  *z1 = r * s;
}

// One thread per row: the squared norm of centre + noise folded in dimension
// order, then the row written as (w * 1/|w|) - c, each component rounded once.
__global__ __launch_bounds__(256) void synth_rows_kernel(uint64_t seed, uint64_t n, uint32_t dim,
                                                          uint32_t n_centers,
                                                          const float* __restrict__ centers,
                                                          const double* __restrict__ cdf,
                                                          double sigma, uint64_t first,
                                                          float* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t gi = first + i;
  const double u = unit(draw(seed, kStreamAssign, gi));
  uint32_t j;
  if (!cdf) {
    const uint64_t q = (uint64_t)(u * (double)n_centers);
    j = (uint32_t)(q < n_centers ? q : n_centers - 1);
  } else {
    uint32_t lo = 0, hi = n_centers - 1;  // first j with u < cdf[j]
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if (u < cdf[mid]) hi = mid;
      else lo = mid + 1;
    }
    j = lo;
  }
  const float* cj = centers + (uint64_t)j * dim;
  const uint64_t pairs = (dim + 1) / 2;
  double ss = 0.0;
  for (uint32_t d = 0; d < dim; d += 2) {
    double z0, z1;
    normal_pair(seed, gi * pairs + d / 2, &z0, &z1);
    const double w0 = (double)cj[d] + sigma * z0;
    ss += w0 * w0;
    if (d + 1 < dim) {
      const double w1 = (double)cj[d + 1] + sigma * z1;
      ss += w1 * w1;
    }
  }
  const double inv = ss > 0.0 ? 1.0 / sqrt(ss) : 0.0;
  float* r = out + i * dim;
  for (uint32_t d = 0; d < dim; d += 2) {
    double z0, z1;
    normal_pair(seed, gi * pairs + d / 2, &z0, &z1);
    const double w0 = (double)cj[d] + sigma * z0;
    r[d] = (float)(w0 * inv - (double)cj[d]);
    if (d + 1 < dim) {
      const double w1 = (double)cj[d + 1] + sigma * z1;
      r[d + 1] = (float)(w1 * inv - (double)cj[d + 1]);
    }
  }
}

}  // namespace

// Residual rows first .. first + n - 1 into d_out [n][dim] (device memory);
// d_centers [n_centers][dim] as synth.c's tac_synth_centers makes them,
// d_cdf the normalised Zipf CDF [n_centers] or NULL for uniform popularity.
// Enqueued on `stream` (NULL: the null stream); 0 on success, 14 on bad
// arguments, 13 on a launch error.
extern "C" int tac_synth_residuals_device(uint64_t seed, uint64_t n, uint32_t dim,
                                          uint32_t n_centers, const float* d_centers,
                                          const double* d_cdf, float sigma, uint64_t first,
                                          float* d_out, void* stream) {
  if (!d_out || !d_centers || dim == 0 || dim > 4096 || n_centers == 0) return 14;
  if (n == 0) return 0;
  const uint64_t blocks = (n + 255) / 256;
  if (blocks > 0x7FFFFFFFull) return 14;
  synth_rows_kernel<<<(unsigned)blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      seed, n, dim, n_centers, d_centers, d_cdf, (double)sigma, first, d_out);
  return hipGetLastError() == hipSuccess ? 0 : 13;
}
