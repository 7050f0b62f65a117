// storage_kernels.hpp — gfx950 kernels of the storage.build stages around the
// PQ build: per-token residuals and norms.  Included once, by tac_gpu.hip.
//
// Arithmetic contract: compiled with -ffp-contract=off, so every subtract,
// multiply and add is rounded separately as in Zig's strict float mode;
// sqrtf and 1.0f / x are the correctly rounded IEEE operations (HIP's
// default for single precision).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tacgpu {

constexpr int kResBlock = 256;  // threads per residual block
constexpr uint32_t kBadRow = 0xFFFFFFFFu;

// Rows per residual block: one folding thread per row and an LDS tile of
// rows x (dim + 1) floats within 64 KB.
__host__ __device__ inline uint32_t residual_rows(uint32_t dim) {
  uint32_t r = 16000u / (dim + 1u);
  return r > 64u ? 64u : (r == 0u ? 1u : r);
}

// storage.zig:255-278 (residualsAndNormsChunk) over rows [row0, row0 + R):
//   1. all threads load the rows and their centroids in VW-float units,
//      coalesced, and park diff = v - c in an LDS tile [R][dim + 1];
//   2. thread r folds row r: sum = 0; sum = sum + diff_d * diff_d for d
//      ascending; norm = sqrt(sum); scale = 1 / norm if norm > 0;
//   3. all threads store diff * scale (or diff unchanged when norm is not
//      > 0) with coalesced stores.
// Every row is read before any row of the block is written, and blocks own
// disjoint rows, so `out` may alias `v`.  An assignment >= n_cent raises
// `status` and its row reads nothing (the outputs of such a call are
// unspecified; the host reports the error).
template <int VW>
__global__ __launch_bounds__(kResBlock) void residual_kernel(
    const float* v, const float* __restrict__ cent, const uint32_t* __restrict__ assign,
    float* out, float* __restrict__ norms, uint32_t* __restrict__ status, uint64_t n,
    uint32_t dim, uint32_t n_cent, uint32_t R) {
  extern __shared__ __attribute__((aligned(16))) float tile[];  // [R][dim + 1]
  const uint32_t ld = dim + 1;
  float* scale = tile + (size_t)R * ld;                          // [R]
  uint32_t* rowa = reinterpret_cast<uint32_t*>(scale + R);       // [R]
  const uint64_t row0 = (uint64_t)blockIdx.x * R;
  const uint32_t rows = (uint32_t)(n - row0 < R ? n - row0 : R);
  const uint32_t t = threadIdx.x;
  if (t < rows) {
    uint32_t a = assign[row0 + t];
    if (a >= n_cent) {
      atomicOr(status, 1u);
      a = kBadRow;
    }
    rowa[t] = a;
  }
  __syncthreads();

  const uint32_t q = dim / VW;        // units per row
  const uint32_t units = rows * q;
  constexpr int kUnroll = 4;
  for (uint32_t base = 0; base < units; base += kResBlock * kUnroll) {
    float dv[kUnroll][VW];
    uint32_t rr[kUnroll], cc[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t u = base + k * kResBlock + t;
      rr[k] = u / q;
      cc[k] = u % q;
      if (u < units && rowa[rr[k]] != kBadRow) {
        const float* vp = v + (row0 + rr[k]) * dim + (uint64_t)cc[k] * VW;
        const float* cp = cent + (uint64_t)rowa[rr[k]] * dim + (uint64_t)cc[k] * VW;
        if constexpr (VW == 4) {
          const float4 a = *reinterpret_cast<const float4*>(vp);
          const float4 b = *reinterpret_cast<const float4*>(cp);
          dv[k][0] = a.x - b.x;
          dv[k][1] = a.y - b.y;
          dv[k][2] = a.z - b.z;
          dv[k][3] = a.w - b.w;
        } else {
#pragma unroll
          for (int j = 0; j < VW; ++j) dv[k][j] = vp[j] - cp[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < VW; ++j) dv[k][j] = __builtin_nanf("");
      }
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint32_t u = base + k * kResBlock + t;
      if (u < units) {
#pragma unroll
        for (int j = 0; j < VW; ++j) tile[rr[k] * ld + cc[k] * VW + j] = dv[k][j];
      }
    }
  }
  __syncthreads();

  if (t < rows) {
    const float* row = tile + (size_t)t * ld;
    float sum = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) {
      const float x = row[d];
      const float sq = x * x;
      sum = sum + sq;
    }
    const float norm = sqrtf(sum);
    norms[row0 + t] = norm;
    // 1/norm >= +0 for every norm > 0 (+inf included); -1 marks "unscaled"
    scale[t] = norm > 0.0f ? 1.0f / norm : -1.0f;
  }
  __syncthreads();

  for (uint32_t base = 0; base < units; base += kResBlock) {
    const uint32_t u = base + t;
    if (u >= units) break;
    const uint32_t r = u / q, c = u % q;
    const float s = scale[r];
    float y[VW];
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float x = tile[r * ld + c * VW + j];
      y[j] = s >= 0.0f ? x * s : x;
    }
    float* op = out + (row0 + r) * dim + (uint64_t)c * VW;
    if constexpr (VW == 4) {
      *reinterpret_cast<float4*>(op) = make_float4(y[0], y[1], y[2], y[3]);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) op[j] = y[j];
    }
  }
}

}  // namespace tacgpu
