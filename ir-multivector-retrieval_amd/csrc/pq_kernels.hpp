// pq_kernels.hpp — gfx950 kernels for product-quantization training and
// encoding.  Included once, by tac_gpu.hip.
//
// Arithmetic contract (mirrors src/util/vec.zig:109-175 and
// src/tac/kmeans.zig:177-198 of the reference):
//   * a distance is the left fold s = (x0-c0)^2; s = s + (xk-ck)^2 ... with
//     every subtract, multiply and add rounded separately — this file is
//     compiled with -ffp-contract=off so nothing fuses into an FMA;
//   * argmin keeps the first (lowest) index on ties;
//   * a cluster sum is the fp32 fold, from 0.0f, of its members in ascending
//     vector index; a centroid is sum * fl(1 / fl(count)).
// No float atomics anywhere: every result is independent of scheduling.
//
// Data layout in HBM during training (n vectors, M subspaces, K codewords,
// D = dsub, DP = D rounded up to 1/2/4/8):
//   xs      [M][n][DP]   subspace-major copy of the residuals (pads = 0)
//   cb      [M][K][D]    codebooks, the caller's layout
//   codes   [M][n] u16   assignment of the current iteration
//   e       [M][n] f32   distance to the assigned codeword (min_to_any)
//   hist    [M][T][K]    per-tile histogram, then the tile's exclusive offset
//   counts  [M][K]       cluster sizes; start [M][K] bucket starts
//   sorted  [M][D][n]    residual components grouped by cluster, stable
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tacgpu {

constexpr int kBlock = 256;        // threads per block for the streaming kernels
constexpr int kScatterTile = 16384; // elements per stable-scatter tile (4 waves)
constexpr int kWave = 64;

template <int D>
struct Pad {
  static constexpr int value = D <= 1 ? 1 : D <= 2 ? 2 : D <= 4 ? 4 : 8;
};

// Load DP consecutive floats from an aligned LDS / global address.
template <int D>
__device__ __forceinline__ void load_padded(const float* __restrict__ p, float (&v)[D]) {
  constexpr int DP = Pad<D>::value;
  if constexpr (DP == 1) {
    v[0] = p[0];
  } else if constexpr (DP == 2) {
    const float2 a = *reinterpret_cast<const float2*>(p);
    v[0] = a.x;
    if constexpr (D > 1) v[1] = a.y;
  } else if constexpr (DP == 4) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float t[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < D; ++k) v[k] = t[k];
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < D; ++k) v[k] = t[k];
  }
}

// Reference distance: sequential left fold, separate roundings.  The fold
// starts from 0.0f in the reference; 0.0f + (x0-c0)^2 equals (x0-c0)^2
// bit for bit because a square is never -0.0.
template <int D>
__device__ __forceinline__ float exact_l2sq(const float (&x)[D], const float (&c)[D]) {
  float t = x[0] - c[0];
  float s = t * t;
#pragma unroll
  for (int k = 1; k < D; ++k) {
    const float u = x[k] - c[k];
    const float q = u * u;
    s = s + q;
  }
  return s;
}

// ---------------------------------------------------------------------------
// Layout transform: token-major residuals [n][dim] -> xs [M][n][DP].
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kBlock) void transpose_kernel(
    const float* __restrict__ x, float* __restrict__ xs, uint64_t n, uint32_t dim) {
  constexpr int DP = Pad<D>::value;
  const uint32_t m = blockIdx.y;
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const float* src = x + i * dim + (uint64_t)m * D;
  float v[DP];
#pragma unroll
  for (int k = 0; k < DP; ++k) v[k] = k < D ? src[k] : 0.0f;
  float* dst = xs + ((uint64_t)m * n + i) * DP;
  if constexpr (DP == 1) {
    dst[0] = v[0];
  } else if constexpr (DP == 2) {
    *reinterpret_cast<float2*>(dst) = make_float2(v[0], v[1]);
  } else if constexpr (DP == 4) {
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Stage one subspace codebook [K][D] into LDS as [K][DP] (pads = 0).
template <int D>
__device__ __forceinline__ void stage_codebook(float* lds, const float* __restrict__ cb,
                                               uint32_t K) {
  constexpr int DP = Pad<D>::value;
  for (uint32_t t = threadIdx.x; t < K * DP; t += blockDim.x) {
    const uint32_t c = t / DP, k = t % DP;
    lds[t] = k < (uint32_t)D ? cb[(uint64_t)c * D + k] : 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Lloyd assignment (src/tac/kmeans.zig:344-365).  One block = one subspace
// and kBlock*VPT consecutive vectors; every thread owns VPT vectors and
// scans all K codewords, read from LDS as wave-wide broadcasts.
// vec.argmin semantics: best starts at codeword 0, replaced on strict <.
// ---------------------------------------------------------------------------
template <int D, int VPT>
__global__ __launch_bounds__(kBlock) void assign_kernel(
    const float* __restrict__ xs, const float* __restrict__ cb,
    uint16_t* __restrict__ codes, float* __restrict__ e,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t K) {
  constexpr int DP = Pad<D>::value;
  extern __shared__ float lds[];
  const uint32_t m = blockIdx.y;
  if (done[m]) return;
  stage_codebook<D>(lds, cb + (uint64_t)m * K * D, K);
  __syncthreads();

  const uint64_t base = (uint64_t)blockIdx.x * (kBlock * VPT) + threadIdx.x;
  const float* xm = xs + (uint64_t)m * n * DP;
  float x[VPT][D];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint64_t i = base + (uint64_t)j * kBlock;
    if (i < n) {
      load_padded<D>(xm + i * DP, x[j]);
    } else {
#pragma unroll
      for (int k = 0; k < D; ++k) x[j][k] = 0.0f;
    }
  }
  float best[VPT];
  uint32_t bidx[VPT];
  {
    float c0[D];
    load_padded<D>(lds, c0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      best[j] = exact_l2sq<D>(x[j], c0);
      bidx[j] = 0;
    }
  }
  for (uint32_t c = 1; c < K; ++c) {
    float cv[D];
    load_padded<D>(lds + c * DP, cv);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const float d = exact_l2sq<D>(x[j], cv);
      const bool lt = d < best[j];
      best[j] = lt ? d : best[j];
      bidx[j] = lt ? c : bidx[j];
    }
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint64_t i = base + (uint64_t)j * kBlock;
    if (i < n) {
      codes[(uint64_t)m * n + i] = (uint16_t)bidx[j];
      e[(uint64_t)m * n + i] = best[j];
    }
  }
}

// ---------------------------------------------------------------------------
// Stable counting sort by code, step 1: per-tile histograms.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void hist_kernel(
    const uint16_t* __restrict__ codes, uint32_t* __restrict__ hist,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t K, uint32_t T) {
  extern __shared__ uint32_t h[];
  const uint32_t m = blockIdx.y, t = blockIdx.x;
  if (done[m]) return;
  for (uint32_t c = threadIdx.x; c < K; c += blockDim.x) h[c] = 0;
  __syncthreads();
  const uint64_t lo = (uint64_t)t * kScatterTile;
  const uint64_t hi = lo + kScatterTile < n ? lo + kScatterTile : n;
  const uint16_t* cm = codes + (uint64_t)m * n;
  for (uint64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) atomicAdd(&h[cm[i]], 1u);
  __syncthreads();
  uint32_t* out = hist + ((uint64_t)m * T + t) * K;
  for (uint32_t c = threadIdx.x; c < K; c += blockDim.x) out[c] = h[c];
}

// Step 2: per subspace, exclusive scan of every code's tile counts (in
// place), cluster sizes, and bucket starts (exclusive scan over codes).
// Block = 1024 threads = K codes x P tile ranges.
__global__ __launch_bounds__(1024) void scan_kernel(
    uint32_t* __restrict__ hist, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ start, const uint32_t* __restrict__ done, uint32_t K,
    uint32_t T) {
  __shared__ uint32_t part_sum[1024];
  __shared__ uint32_t cnt[1024];
  const uint32_t m = blockIdx.x;
  if (done[m]) return;
  const uint32_t P = blockDim.x / K;  // tile ranges per code (K <= 1024)
  const bool active = threadIdx.x < P * K;
  const uint32_t c = threadIdx.x % K, p = threadIdx.x / K;
  const uint32_t per = (T + P - 1) / P;
  const uint32_t t0 = p * per < T ? p * per : T;
  const uint32_t t1 = t0 + per < T ? t0 + per : T;
  uint32_t* hm = hist + (uint64_t)m * T * K;
  uint32_t s = 0;
  if (active)
    for (uint32_t t = t0; t < t1; ++t) s += hm[(uint64_t)t * K + c];
  part_sum[threadIdx.x] = s;
  __syncthreads();
  if (active) {
    uint32_t run = 0;
    for (uint32_t q = 0; q < p; ++q) run += part_sum[q * K + c];
    for (uint32_t t = t0; t < t1; ++t) {
      const uint32_t v = hm[(uint64_t)t * K + c];
      hm[(uint64_t)t * K + c] = run;
      run += v;
    }
    if (p == P - 1) cnt[c] = run;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (uint32_t q = 0; q < K; ++q) {
      start[(uint64_t)m * K + q] = acc;
      counts[(uint64_t)m * K + q] = cnt[q];
      acc += cnt[q];
    }
  }
}

// Step 3: stable scatter.  Each of the 4 waves owns a quarter of the tile,
// walks it in rounds of 64 in index order, and ranks equal codes inside a
// round with ballots (match on every code bit).  Values land in
// sorted[m][d][start[code] + tile offset + wave prefix + running rank].
template <int D>
__global__ __launch_bounds__(kBlock) void scatter_kernel(
    const float* __restrict__ xs, const uint16_t* __restrict__ codes,
    const uint32_t* __restrict__ hist, const uint32_t* __restrict__ start,
    float* __restrict__ sorted, const uint32_t* __restrict__ done, uint64_t n,
    uint32_t K, uint32_t T, uint32_t code_bits) {
  constexpr int DP = Pad<D>::value;
  extern __shared__ uint32_t run[];  // [4][K]
  const uint32_t m = blockIdx.y, t = blockIdx.x;
  if (done[m]) return;
  const uint32_t w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  constexpr uint32_t kQuarter = kScatterTile / 4;
  const uint64_t tile_lo = (uint64_t)t * kScatterTile;
  const uint64_t lo = tile_lo + (uint64_t)w * kQuarter;
  const uint64_t hi_tile = tile_lo + kScatterTile < n ? tile_lo + kScatterTile : n;
  const uint64_t hi = lo + kQuarter < hi_tile ? lo + kQuarter : hi_tile;
  const uint16_t* cm = codes + (uint64_t)m * n;

  for (uint32_t c = threadIdx.x; c < 4 * K; c += blockDim.x) run[c] = 0;
  __syncthreads();
  for (uint64_t i = lo + lane; i < hi; i += kWave) atomicAdd(&run[w * K + cm[i]], 1u);
  __syncthreads();
  const uint32_t* hm = hist + ((uint64_t)m * T + t) * K;
  for (uint32_t c = threadIdx.x; c < K; c += blockDim.x) {
    uint32_t acc = start[(uint64_t)m * K + c] + hm[c];
    for (uint32_t q = 0; q < 4; ++q) {
      const uint32_t v = run[q * K + c];
      run[q * K + c] = acc;
      acc += v;
    }
  }
  __syncthreads();

  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const float* xm = xs + (uint64_t)m * n * DP;
  float* sm = sorted + (uint64_t)m * D * n;
  uint32_t* myrun = run + w * K;
  for (uint64_t r = lo; r < hi; r += kWave) {
    const uint64_t i = r + lane;
    const bool valid = i < hi;
    const uint32_t code = valid ? cm[i] : 0u;
    uint64_t match = __ballot(valid);
    for (uint32_t b = 0; b < code_bits; ++b) {
      const bool bit = (code >> b) & 1u;
      const uint64_t bal = __ballot(bit);
      match &= bit ? bal : ~bal;
    }
    const uint32_t rank = __popcll(match & lt_mask);
    const uint32_t total = __popcll(match);
    uint32_t pos = 0;
    if (valid) pos = myrun[code] + rank;
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == total - 1) myrun[code] = pos + 1;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      float v[D];
      load_padded<D>(xm + i * DP, v);
#pragma unroll
      for (int k = 0; k < D; ++k) sm[(uint64_t)k * n + pos] = v[k];
    }
  }
}

// Step 4: one lane per (subspace, dim, cluster) chain folds the cluster's
// members in ascending vector order and writes the centroid component
// sum * fl(1 / fl(count)) (src/tac/kmeans.zig:177-198).  Empty clusters
// are left for reseed_kernel.
template <int D>
__global__ __launch_bounds__(kBlock) void fold_kernel(
    const float* __restrict__ sorted, const uint32_t* __restrict__ counts,
    const uint32_t* __restrict__ start, float* __restrict__ cb,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t M, uint32_t K) {
  const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (uint64_t)M * D * K) return;
  const uint32_t c = g % K;
  const uint32_t d = (g / K) % D;
  const uint32_t m = g / ((uint64_t)K * D);
  if (done[m]) return;
  const uint32_t cnt = counts[(uint64_t)m * K + c];
  if (cnt == 0) return;
  const float* p = sorted + ((uint64_t)m * D + d) * n + start[(uint64_t)m * K + c];
  float s = 0.0f;
  uint32_t j = 0;
  constexpr uint32_t U = 16;
  for (; j + U <= cnt; j += U) {
    float v[U];
#pragma unroll
    for (uint32_t q = 0; q < U; ++q) v[q] = p[j + q];
#pragma unroll
    for (uint32_t q = 0; q < U; ++q) s = s + v[q];
  }
  for (; j < cnt; ++j) s = s + p[j];
  const float inv = 1.0f / (float)cnt;
  cb[((uint64_t)m * K + c) * D + d] = s * inv;
}

// ---------------------------------------------------------------------------
// wcss = sequential fp32 fold of e over ascending vector index
// (src/tac/kmeans.zig:179).  One wave per subspace: the wave stages 1024
// values through LDS with coalesced loads, lane 0 folds them in order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWave) void wcss_kernel(
    const float* __restrict__ e, float* __restrict__ wcss, const uint32_t* __restrict__ done,
    uint64_t n) {
  __shared__ float buf[1024];
  const uint32_t m = blockIdx.x;
  if (done[m]) return;
  const float* em = e + (uint64_t)m * n;
  float s = 0.0f;
  for (uint64_t b = 0; b < n; b += 1024) {
    const uint64_t len = n - b < 1024 ? n - b : 1024;
    for (uint32_t q = threadIdx.x; q < len; q += kWave) buf[q] = em[b + q];
    __syncthreads();
    if (threadIdx.x == 0)
      for (uint32_t q = 0; q < len; ++q) s = s + buf[q];
    __syncthreads();
  }
  if (threadIdx.x == 0) wcss[m] = s;
}

// ---------------------------------------------------------------------------
// Empty-cluster reseed (src/tac/kmeans.zig:199-211): clusters visited in
// ascending order; each takes argmax(e) (first index on ties), copies that
// vector and marks it claimed with -inf.  One block per subspace.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(1024) void reseed_kernel(
    const float* __restrict__ xs, float* __restrict__ e, const uint32_t* __restrict__ counts,
    float* __restrict__ cb, uint32_t* __restrict__ empties, const uint32_t* __restrict__ done,
    uint64_t n, uint32_t K) {
  constexpr int DP = Pad<D>::value;
  __shared__ float sv[1024 / kWave];
  __shared__ uint64_t si[1024 / kWave];
  const uint32_t m = blockIdx.x;
  if (done[m]) return;
  float* em = e + (uint64_t)m * n;
  const uint32_t* cm = counts + (uint64_t)m * K;
  const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const uint32_t nw = blockDim.x / kWave;
  uint32_t found = 0;
  for (uint32_t c = 0; c < K; ++c) {
    if (cm[c] != 0) continue;  // uniform across the block
    ++found;
    float bv = -__builtin_inff();
    uint64_t bi = ~0ull;
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const float v = em[i];
      if (bi == ~0ull || v > bv) {
        bv = v;
        bi = i;
      }
    }
    for (int off = kWave / 2; off > 0; off /= 2) {
      const float ov = __shfl_down(bv, off, kWave);
      const uint64_t oi = __shfl_down(bi, off, kWave);
      if (oi != ~0ull && (bi == ~0ull || ov > bv || (ov == bv && oi < bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      sv[w] = bv;
      si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = sv[0];
      uint64_t idx = si[0];
      for (uint32_t q = 1; q < nw; ++q) {
        if (si[q] != ~0ull && (idx == ~0ull || sv[q] > v || (sv[q] == v && si[q] < idx))) {
          v = sv[q];
          idx = si[q];
        }
      }
      const float* src = xs + ((uint64_t)m * n + idx) * DP;
      for (int k = 0; k < D; ++k) cb[((uint64_t)m * K + c) * D + k] = src[k];
      em[idx] = -__builtin_inff();
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) empties[m] += found;
}

// Convergence bookkeeping (src/tac/kmeans.zig:186, :214-223), run after the
// update of iteration `iter`.
__global__ void converge_kernel(const float* __restrict__ wcss, float* __restrict__ prev,
                                uint32_t* __restrict__ done, uint32_t* __restrict__ iters_run,
                                uint32_t M, uint32_t iter, float tol, int check) {
  const uint32_t m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M || done[m]) return;
  iters_run[m] = iter + 1;
  if (!check) return;
  const float w = wcss[m];
  if (iter > 0) {
    const float p = prev[m];
    const float denom = p > 0.0f ? p : 1.0f;
    const float rel = (p - w) / denom;
    if (rel < tol) {
      done[m] = 1;
      return;
    }
  }
  prev[m] = w;
}

// Degenerate k >= n (src/tac/kmeans.zig:88-104): codeword c of subspace m is
// sub-vector min(c, n-1).
__global__ void degenerate_kernel(const float* __restrict__ x, float* __restrict__ cb,
                                  uint64_t n, uint32_t dim, uint32_t M, uint32_t K, uint32_t D) {
  const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (uint64_t)M * K * D) return;
  const uint32_t k = g % D;
  const uint32_t c = (g / D) % K;
  const uint32_t m = g / ((uint64_t)K * D);
  const uint64_t row = c < n ? c : n - 1;
  cb[g] = x[row * dim + (uint64_t)m * D + k];
}

// Final codes [M][n] u16 -> caller's u32 assignments for kmeans.fit (M = 1).
__global__ void widen_codes_kernel(const uint16_t* __restrict__ codes, uint32_t* __restrict__ out,
                                   uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = codes[i];
}

// ---------------------------------------------------------------------------
// PQ.encode (src/index/pq.zig:59-76) over token-major residuals.  A block
// owns kBlock*VPT consecutive vectors and walks the M subspaces, staging one
// codebook at a time in LDS; codes collect in LDS and leave as one
// contiguous [tile][M] row block.  best starts at +inf, strict <.
// ---------------------------------------------------------------------------
template <int D, int VPT, typename CodeT>
__global__ __launch_bounds__(kBlock) void encode_kernel(
    const float* __restrict__ x, const float* __restrict__ cb, CodeT* __restrict__ codes,
    uint64_t n, uint32_t dim, uint32_t M, uint32_t K) {
  constexpr int DP = Pad<D>::value;
  constexpr uint32_t kTile = kBlock * VPT;
  extern __shared__ float lds[];
  float* lcb = lds;
  CodeT* lcodes = reinterpret_cast<CodeT*>(lds + K * DP);  // [kTile][M]
  const uint64_t tile_lo = (uint64_t)blockIdx.x * kTile;
  for (uint32_t m = 0; m < M; ++m) {
    __syncthreads();
    stage_codebook<D>(lcb, cb + (uint64_t)m * K * D, K);
    __syncthreads();
    float xv[VPT][D];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const uint64_t i = tile_lo + (uint64_t)j * kBlock + threadIdx.x;
      const float* src = x + (i < n ? i : 0) * dim + (uint64_t)m * D;
#pragma unroll
      for (int k = 0; k < D; ++k) xv[j][k] = src[k];
    }
    float best[VPT];
    uint32_t bidx[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      best[j] = __builtin_inff();
      bidx[j] = 0;
    }
    for (uint32_t c = 0; c < K; ++c) {
      float cv[D];
      load_padded<D>(lcb + c * DP, cv);
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const float d = exact_l2sq<D>(xv[j], cv);
        const bool lt = d < best[j];
        best[j] = lt ? d : best[j];
        bidx[j] = lt ? c : bidx[j];
      }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      lcodes[((uint32_t)j * kBlock + threadIdx.x) * M + m] = (CodeT)bidx[j];
  }
  __syncthreads();
  const uint64_t rows = n - tile_lo < kTile ? n - tile_lo : kTile;
  const uint64_t total = rows * M;
  CodeT* dst = codes + tile_lo * M;
  for (uint64_t q = threadIdx.x; q < total; q += kBlock) dst[q] = lcodes[q];
}

// PQ.decode (src/index/pq.zig:79-88): out[i][m*D + k] = cb[m][code[i][m]][k].
template <typename CodeT>
__global__ void decode_kernel(const CodeT* __restrict__ codes, const float* __restrict__ cb,
                              float* __restrict__ out, uint64_t n, uint32_t M, uint32_t K,
                              uint32_t D) {
  const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t dim = (uint64_t)M * D;
  if (g >= n * dim) return;
  const uint64_t i = g / dim;
  const uint32_t r = g % dim;
  const uint32_t m = r / D, k = r % D;
  uint32_t code = codes[i * M + m];
  if (code >= K) code = K - 1;
  out[g] = cb[((uint64_t)m * K + code) * D + k];
}

}  // namespace tacgpu
