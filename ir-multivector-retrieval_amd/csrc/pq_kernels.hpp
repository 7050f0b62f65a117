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
//   sorted  [M][n][DP]   residual records grouped by cluster, stable order
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fold_rules.hpp"

namespace tacgpu {

constexpr int kBlock = 256;        // threads per block for the streaming kernels
constexpr int kSortTile = 2048;    // vectors per stable counting-sort tile (4 waves)
constexpr int kFoldBatch = 8;      // 64-record loads in flight per fold wave
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

// vec.lane_count of the host the reference is built for
// (std.simd.suggestVectorLength(f32), src/util/vec.zig:16): 16 on AVX-512,
// 8 on AVX2, 4 on NEON.  It sets the order of the generic vec path
// (:90-103, :159-175) and is set per device from the host
// (tac_gpu_set_lane_count).
__constant__ uint32_t c_vec_lanes = 16;

// The generic vec path at L lanes: lane j accumulates the products of
// elements j, j + L, ... of the whole L-element chunks from 0.0f, the lanes
// are added in order, then the tail elements one by one.
template <int L, bool DOT>
__device__ __forceinline__ float generic_vec_lanes(const float* a, const float* b, uint32_t d) {
  float acc[L];
#pragma unroll
  for (int j = 0; j < L; ++j) acc[j] = 0.0f;
  uint32_t i = 0;
  for (; i + L <= d; i += L) {
#pragma unroll
    for (int j = 0; j < L; ++j) {
      if constexpr (DOT) {
        acc[j] = acc[j] + a[i + j] * b[i + j];
      } else {
        const float t = a[i + j] - b[i + j];
        acc[j] = acc[j] + t * t;
      }
    }
  }
  float sum = acc[0];
#pragma unroll
  for (int j = 1; j < L; ++j) sum = sum + acc[j];
  for (; i < d; ++i) {
    if constexpr (DOT) {
      sum = sum + a[i] * b[i];
    } else {
      const float t = a[i] - b[i];
      sum = sum + t * t;
    }
  }
  return sum;
}

// vec.l2sqGeneric / vec.dotGeneric at the device's lane count.
template <bool DOT>
__device__ __forceinline__ float generic_vec(const float* a, const float* b, uint32_t d) {
  const uint32_t L = c_vec_lanes;
  if (L == 4) return generic_vec_lanes<4, DOT>(a, b, d);
  if (L == 8) return generic_vec_lanes<8, DOT>(a, b, d);
  return generic_vec_lanes<16, DOT>(a, b, d);
}

// Reference distance at sub-dimension D <= 8 (src/util/vec.zig:109-175):
// the sequential left fold with separate roundings (the reference's
// explicit dim 2 / dim 4 folds, and its generic path for every D below two
// lane widths); at D = 8 on a 4-lane host the generic path's lane j holds
// (x_j - c_j)^2 + (x_{j+4} - c_{j+4})^2 and the lanes are added in order.
// The fold starts from 0.0f in the reference; 0.0f + (x0-c0)^2 equals
// (x0-c0)^2 bit for bit because a square is never -0.0.
template <int D>
__device__ __forceinline__ float exact_l2sq(const float (&x)[D], const float (&c)[D]) {
  if constexpr (D == 8) {
    if (c_vec_lanes == 4) {
      float l[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float t0 = x[j] - c[j];
        const float t1 = x[j + 4] - c[j + 4];
        l[j] = t0 * t0;
        l[j] = l[j] + t1 * t1;
      }
      return ((l[0] + l[1]) + l[2]) + l[3];
    }
  }
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
// Layout transform: token-major residuals [n][dim] -> xs [M][n][DP].  A block
// moves `rows` consecutive rows: coalesced row loads into LDS, then one
// contiguous [rows][DP] slab per subspace.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kBlock) void transpose_kernel(
    const float* __restrict__ x, float* __restrict__ xs, uint64_t n, uint32_t dim,
    uint32_t rows) {
  constexpr int DP = Pad<D>::value;
  extern __shared__ float tile[];  // [rows][dim + 1]
  const uint32_t M = dim / D;
  const uint64_t row0 = (uint64_t)blockIdx.x * rows;
  const uint32_t nrows = row0 + rows <= n ? rows : (uint32_t)(n - row0);
  const uint32_t ld = dim + 1;
  const float* src = x + row0 * dim;
  for (uint32_t f = threadIdx.x; f < nrows * dim; f += blockDim.x)
    tile[(f / dim) * ld + f % dim] = src[f];
  __syncthreads();
  const uint32_t slab = nrows * DP;
  for (uint32_t f = threadIdx.x; f < M * slab; f += blockDim.x) {
    const uint32_t m = f / slab, r = (f % slab) / DP, k = f % DP;
    xs[((uint64_t)m * n + row0 + r) * DP + k] = k < (uint32_t)D ? tile[r * ld + m * D + k] : 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Exact nearest-codeword search, pruned.
//
// The reference scans every codeword with the unfused distance
// ref(c) = sum_k (x_k - c_k)^2 and keeps the first minimum.  Here a first
// pass evaluates the expanded form a(c) = ||c||^2 - 2 x.c with FMAs (dsub
// FMAs per pair) in blocks of kPruneBlock consecutive codewords and keeps,
// per vector, the smallest block minimum best1 (block bblk) and the
// smallest minimum of every other block best2.
//
// Rounding-error analysis bounds how far a(c) + ||x||^2 and ref(c) can each
// stray from the true T(c) = ||x - c||^2, with g_n = n u / (1 - n u),
// u = 2^-24:
//   |a(c) + ||x||^2 - T(c)| <= Ea = 2 g_D (1 + g_D) (cmax^2 + 2 |x| cmax)
//   |ref(c) - T(c)|         <= g_{D+2} T(c)
// (||c||^2 is computed with error <= g_D ||c||^2 and the FMA chain adds
// g_D (||c||^2 + sum |2 x_k c_k|), bounded by Cauchy-Schwarz).  Hence if
// best2 - best1 > 2 Ea (1 + g_{D+2}) + g_{D+2} (|best1 + |x|^2| +
// |best2 + |x|^2|) (the bound is doubled and given an absolute floor for
// underflow), every codeword outside block bblk is strictly farther under
// ref() than some codeword inside it, and the reference's first-index argmin
// is the first-index argmin of block bblk, recomputed with ref().  Otherwise
// (a near tie across blocks, or any non-finite or overflowing value) the
// vector is resolved by the full reference scan.  Either way the result
// equals the exhaustive reference scan bit for bit.
// ---------------------------------------------------------------------------
constexpr int kPruneBlock = 8;

// Stage codebook [K][D] into LDS as lcb [Kp][DP] (pads 0) and lnc [Kp]
// (squared norms, pads +inf); *lmax receives the bits of max ||c||^2 over
// the real codewords (>= 0x7f800000 when any codeword is not finite).  The
// caller zeroes *lmax and synchronises before, and synchronises after.
template <int D>
__device__ __forceinline__ void stage_pruned(float* lcb, float* lnc, uint32_t* lmax,
                                             const float* __restrict__ cb, uint32_t K,
                                             uint32_t Kp) {
  constexpr int DP = Pad<D>::value;
  for (uint32_t c = threadIdx.x; c < Kp; c += blockDim.x) {
    float v[DP];
#pragma unroll
    for (int k = 0; k < DP; ++k) v[k] = (c < K && k < D) ? cb[(uint64_t)c * D + k] : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) s = s + v[k] * v[k];
#pragma unroll
    for (int k = 0; k < DP; ++k) lcb[c * DP + k] = v[k];
    lnc[c] = c < K ? s : __builtin_inff();
    if (c < K) atomicMax(lmax, __float_as_uint(s));
  }
}

// Reference scan over all K codewords: vec.argmin when SEED_FIRST
// (src/util/vec.zig:271-283, best = dists[0]), PQ.encode otherwise
// (src/index/pq.zig:64-73, best_d = +inf).  Strict < keeps the first index.
template <int D, bool SEED_FIRST>
__device__ __forceinline__ void reference_scan(const float (&x)[D], const float* lcb, uint32_t K,
                                               uint32_t& idx, float& best) {
  constexpr int DP = Pad<D>::value;
  uint32_t c = 0;
  if (SEED_FIRST) {
    float c0[D];
    load_padded<D>(lcb, c0);
    best = exact_l2sq<D>(x, c0);
    c = 1;
  } else {
    best = __builtin_inff();
  }
  idx = 0;
  for (; c < K; ++c) {
    float cv[D];
    load_padded<D>(lcb + c * DP, cv);
    const float d = exact_l2sq<D>(x, cv);
    if (d < best) {
      best = d;
      idx = c;
    }
  }
}

template <int D, int VPT, bool SEED_FIRST>
__device__ __forceinline__ void pruned_argmin(const float (&x)[VPT][D], const float* lcb,
                                              const float* lnc, uint32_t K, uint32_t Kp,
                                              uint32_t maxbits, uint32_t (&bidx)[VPT],
                                              float (&bdist)[VPT], uint32_t& rescans) {
  constexpr int DP = Pad<D>::value;
  constexpr int B = kPruneBlock;
  if (maxbits >= 0x7f800000u) {  // a non-finite codeword: reference scan for all
#pragma unroll
    for (int j = 0; j < VPT; ++j) reference_scan<D, SEED_FIRST>(x[j], lcb, K, bidx[j], bdist[j]);
    rescans += VPT;
    return;
  }
  float xp[VPT][D];
#pragma unroll
  for (int j = 0; j < VPT; ++j)
#pragma unroll
    for (int k = 0; k < D; ++k) xp[j][k] = -2.0f * x[j][k];
  float best1[VPT], best2[VPT];
  uint32_t bblk[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    best1[j] = __builtin_inff();
    best2[j] = __builtin_inff();
    bblk[j] = 0;
  }
  const uint32_t nb = Kp / B;
  for (uint32_t b = 0; b < nb; ++b) {
    float mb[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) mb[j] = __builtin_inff();
#pragma unroll
    for (int t = 0; t < B; ++t) {
      const uint32_t c = b * B + t;
      float cv[D];
      load_padded<D>(lcb + c * DP, cv);
      const float nc = lnc[c];
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        float acc = nc;
#pragma unroll
        for (int k = 0; k < D; ++k) acc = __builtin_fmaf(xp[j][k], cv[k], acc);
        mb[j] = fminf(mb[j], acc);
      }
    }
    // Top-2 over block minima with compares and selects only (a min on these
    // loop-carried values would add NaN-quieting instructions).
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const bool lt1 = mb[j] < best1[j];
      const bool lt2 = mb[j] < best2[j];
      best2[j] = lt1 ? best1[j] : (lt2 ? mb[j] : best2[j]);
      best1[j] = lt1 ? mb[j] : best1[j];
      bblk[j] = lt1 ? b : bblk[j];
    }
  }
  constexpr float u = 5.9604644775390625e-8f;  // 2^-24
  constexpr float gD = (float)D * u / (1.0f - (float)D * u);
  constexpr float gR = (float)(D + 2) * u / (1.0f - (float)(D + 2) * u);
  const float cmax2 = __uint_as_float(maxbits);
  const float cmax = sqrtf(cmax2);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    float x2 = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) x2 = x2 + x[j][k] * x[j][k];
    const float nx = sqrtf(x2);
    const float ea = 2.0f * gD * (1.0f + gD) * (cmax2 + 2.0f * nx * cmax);
    float thr = 2.0f * ea * (1.0f + gR) + gR * (fabsf(best2[j] + x2) + fabsf(best1[j] + x2));
    thr = 2.0f * thr + 1e-30f;
    // Below this magnitude no product or sum of the first pass overflows.
    const bool tame = (cmax2 + 2.0f * nx * cmax) < 1e38f;
    const bool ok = tame && (best2[j] - best1[j]) > thr;  // false on NaN
    if (ok) {
      float best = __builtin_inff();
      uint32_t idx = bblk[j] * B;
#pragma unroll
      for (int t = 0; t < B; ++t) {
        const uint32_t c = bblk[j] * B + t;
        if (c < K) {
          float cv[D];
          load_padded<D>(lcb + c * DP, cv);
          const float d = exact_l2sq<D>(x[j], cv);
          if (d < best) {
            best = d;
            idx = c;
          }
        }
      }
      bidx[j] = idx;
      bdist[j] = best;
    } else {
      reference_scan<D, SEED_FIRST>(x[j], lcb, K, bidx[j], bdist[j]);
      ++rescans;
    }
  }
}

__device__ __forceinline__ void flush_rescans(uint32_t mine, uint32_t* lcount,
                                              unsigned long long* __restrict__ rescans) {
  if (mine) atomicAdd(lcount, mine);
  __syncthreads();
  if (threadIdx.x == 0 && *lcount) atomicAdd(rescans, (unsigned long long)*lcount);
}

// Exclusive scan of one value per thread over the block (all threads call).
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wsum) {
  const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off, kWave);
    if (lane >= (uint32_t)off) incl += o;
  }
  if (lane == kWave - 1) wsum[w] = incl;
  __syncthreads();
  uint32_t before = 0;
  for (uint32_t q = 0; q < w; ++q) before += wsum[q];
  __syncthreads();
  return before + incl - v;
}

// ---------------------------------------------------------------------------
// Lloyd assignment (src/tac/kmeans.zig:344-365).  One block = one subspace
// and kBlock*VPT consecutive vectors; every thread owns VPT vectors.
// vec.argmin semantics: the first index of the minimum.
// ---------------------------------------------------------------------------
template <int D, int VPT>
__global__ __launch_bounds__(kBlock) void assign_kernel(
    const float* __restrict__ xs, const float* __restrict__ cb,
    uint16_t* __restrict__ codes, float* __restrict__ e,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t K,
    unsigned long long* __restrict__ rescans) {
  constexpr int DP = Pad<D>::value;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t m = blockIdx.y;
  if (done[m]) return;
  const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
  float* lcb = lds;                 // [Kp][DP], 16-byte aligned records
  float* lnc = lds + Kp * DP;       // [Kp]
  uint32_t& lmax = *reinterpret_cast<uint32_t*>(lnc + Kp);
  uint32_t& lcount = *(&lmax + 1);
  if (threadIdx.x == 0) {
    lmax = 0;
    lcount = 0;
  }
  __syncthreads();
  stage_pruned<D>(lcb, lnc, &lmax, cb + (uint64_t)m * K * D, K, Kp);
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
  uint32_t bidx[VPT];
  float best[VPT];
  uint32_t mine = 0;
  pruned_argmin<D, VPT, true>(x, lcb, lnc, K, Kp, lmax, bidx, best, mine);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint64_t i = base + (uint64_t)j * kBlock;
    if (i < n) {
      codes[(uint64_t)m * n + i] = (uint16_t)bidx[j];
      e[(uint64_t)m * n + i] = best[j];
    }
  }
  flush_rescans(mine, &lcount, rescans);
}

// ---------------------------------------------------------------------------
// Stable counting sort by code.  The vectors of a subspace are cut into
// tiles of kSortTile consecutive indices; a cluster's members end up in
// sorted[m][start[c] ...] in ascending vector order.
//
// Step 1: per-tile histograms hist[m][t][c].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void hist_kernel(
    const uint16_t* __restrict__ codes, uint32_t* __restrict__ hist,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t K, uint32_t T) {
  extern __shared__ uint32_t h[];
  const uint32_t m = blockIdx.y, t = blockIdx.x;
  if (done[m]) return;
  for (uint32_t c = threadIdx.x; c < K; c += blockDim.x) h[c] = 0;
  __syncthreads();
  const uint64_t lo = (uint64_t)t * kSortTile;
  const uint64_t hi = lo + kSortTile < n ? lo + kSortTile : n;
  const uint16_t* cm = codes + (uint64_t)m * n;
  if (hi - lo == (uint64_t)kBlock * 8 && ((uintptr_t)(cm + lo) & 15) == 0) {
    // a full, 16-byte aligned tile: eight codes per thread in one load
    const uint4 v = reinterpret_cast<const uint4*>(cm + lo)[threadIdx.x];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      atomicAdd(&h[w[q] & 0xFFFFu], 1u);
      atomicAdd(&h[w[q] >> 16], 1u);
    }
  } else {
    for (uint64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) atomicAdd(&h[cm[i]], 1u);
  }
  __syncthreads();
  uint32_t* out = hist + ((uint64_t)m * T + t) * K;
  for (uint32_t c = threadIdx.x; c < K; c += blockDim.x) out[c] = h[c];
}

// Step 2: every code's tile counts become exclusive offsets over tiles (in
// place); cluster sizes and bucket starts (exclusive scan over codes) are
// written alongside.  The T tiles of a subspace split into G ranges:
// scan_partial_kernel sums each range per code, scan_apply_kernel adds the
// ranges before its own and rewrites its tiles; range 0 also writes counts
// and starts.
constexpr uint32_t kScanRanges = 32;

// The fold's launch order of one subspace, from the block that holds its
// cluster sizes (thread t holds codes c0 .. c0 + per_c - 1): clusters binned
// by size (bin = count / unit, kFoldOrderBins bins, the last taking every
// larger cluster) and listed from the largest bin down into order[0 .. K),
// so the longest serial chains of the fold start first and the short ones
// fill the SIMDs around them.  The sums do not depend on the order; within a
// bin it follows the atomics.
constexpr uint32_t kFoldOrderBins = 256;
__device__ inline void fold_order_block(const uint32_t (&tot)[4], uint32_t per_c, uint32_t c0,
                                        uint32_t K, uint32_t* __restrict__ order,
                                        uint32_t unit) {
  __shared__ uint32_t bins[kFoldOrderBins];
  __shared__ uint32_t osum[kBlock / kWave];
  auto bin_of = [&](uint32_t cnt) {  // 0 = the largest clusters
    const uint32_t b = cnt / unit;
    return kFoldOrderBins - 1u - (b < kFoldOrderBins - 1u ? b : kFoldOrderBins - 1u);
  };
  for (uint32_t j = threadIdx.x; j < kFoldOrderBins; j += blockDim.x) bins[j] = 0;
  __syncthreads();
  for (uint32_t q = 0; q < per_c; ++q)
    if (c0 + q < K) atomicAdd(&bins[bin_of(tot[q])], 1u);
  __syncthreads();
  const uint32_t first =
      block_exclusive_scan(threadIdx.x < kFoldOrderBins ? bins[threadIdx.x] : 0u, osum);
  __syncthreads();
  if (threadIdx.x < kFoldOrderBins) bins[threadIdx.x] = first;
  __syncthreads();
  for (uint32_t q = 0; q < per_c; ++q)
    if (c0 + q < K) order[atomicAdd(&bins[bin_of(tot[q])], 1u)] = c0 + q;
}

// Each thread of the scan kernels takes per_c = ceil(K / kBlock) <= PER
// consecutive codes c0 .. c0 + per_c - 1 (PER = 1, 2 or 4 by K), and the
// loads of all its codes go out together (per code one after another would
// pay every round trip per_c times at K = 1,024).
template <uint32_t PER>
__global__ __launch_bounds__(kBlock) void scan_partial_kernel(
    const uint32_t* __restrict__ hist, uint32_t* __restrict__ part,
    const uint32_t* __restrict__ done, uint32_t K, uint32_t T, uint32_t G) {
  const uint32_t m = blockIdx.y, g = blockIdx.x;
  if (done[m]) return;
  const uint32_t per = (T + G - 1) / G;
  const uint32_t t0 = g * per < T ? g * per : T;
  const uint32_t t1 = t0 + per < T ? t0 + per : T;
  const uint32_t* hm = hist + (uint64_t)m * T * K;
  const uint32_t per_c = (K + kBlock - 1) / kBlock;
  const uint32_t c0 = threadIdx.x * per_c;
  const uint32_t nq = c0 < K ? (K - c0 < per_c ? K - c0 : per_c) : 0u;
  if (nq == 0) return;
  constexpr uint32_t B = 8;
  uint32_t s[PER] = {};
  uint32_t t = t0;
  for (; t + B <= t1; t += B) {
    uint32_t v[B][PER];
#pragma unroll
    for (uint32_t j = 0; j < B; ++j)
#pragma unroll
      for (uint32_t q = 0; q < PER; ++q) v[j][q] = q < nq ? hm[(uint64_t)(t + j) * K + c0 + q] : 0u;
#pragma unroll
    for (uint32_t j = 0; j < B; ++j)
#pragma unroll
      for (uint32_t q = 0; q < PER; ++q) s[q] += v[j][q];
  }
  for (; t < t1; ++t)
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q)
      if (q < nq) s[q] += hm[(uint64_t)t * K + c0 + q];
#pragma unroll
  for (uint32_t q = 0; q < PER; ++q)
    if (q < nq) part[((uint64_t)m * G + g) * K + c0 + q] = s[q];
}

template <uint32_t PER>
__global__ __launch_bounds__(kBlock) void scan_apply_kernel(
    uint32_t* __restrict__ hist, const uint32_t* __restrict__ part,
    uint32_t* __restrict__ counts, uint32_t* __restrict__ start, uint32_t* __restrict__ order,
    const uint32_t* __restrict__ done, uint32_t K, uint32_t T, uint32_t G, uint32_t unit) {
  __shared__ uint32_t wsum[kBlock / kWave];
  const uint32_t m = blockIdx.y, g = blockIdx.x;
  if (done[m]) return;
  const uint32_t per = (T + G - 1) / G;
  const uint32_t t0 = g * per < T ? g * per : T;
  const uint32_t t1 = t0 + per < T ? t0 + per : T;
  uint32_t* hm = hist + (uint64_t)m * T * K;
  const uint32_t* pm = part + (uint64_t)m * G * K;
  const uint32_t per_c = (K + kBlock - 1) / kBlock;  // <= 4 codes per thread
  const uint32_t c0 = threadIdx.x * per_c;
  const uint32_t nq = c0 < K ? (K - c0 < per_c ? K - c0 : per_c) : 0u;
  uint32_t tot[4] = {0, 0, 0, 0}, before[PER] = {};
  for (uint32_t gg = 0; gg < G; ++gg)
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q) {
      const uint32_t v = q < nq ? pm[(uint64_t)gg * K + c0 + q] : 0u;
      before[q] += gg < g ? v : 0u;
      tot[q] += v;
    }
  uint32_t local = 0;
#pragma unroll
  for (uint32_t q = 0; q < PER; ++q) local += tot[q];
  uint32_t st = block_exclusive_scan(local, wsum);
  if (g == 0) fold_order_block(tot, per_c, c0, K, order + (uint64_t)m * K, unit);
  uint32_t run[PER];
#pragma unroll
  for (uint32_t q = 0; q < PER; ++q) {
    if (q < nq && g == 0) {
      start[(uint64_t)m * K + c0 + q] = st;
      counts[(uint64_t)m * K + c0 + q] = tot[q];
    }
    st += tot[q];
    run[q] = before[q];
  }
  // Eight tiles' counts of every code of the thread are loaded before any is
  // rewritten, so the loads overlap instead of waiting behind the stores.
  constexpr uint32_t B = 8;
  uint32_t t = t0;
  for (; t + B <= t1; t += B) {
    uint32_t v[B][PER];
#pragma unroll
    for (uint32_t j = 0; j < B; ++j)
#pragma unroll
      for (uint32_t q = 0; q < PER; ++q) v[j][q] = q < nq ? hm[(uint64_t)(t + j) * K + c0 + q] : 0u;
#pragma unroll
    for (uint32_t j = 0; j < B; ++j)
#pragma unroll
      for (uint32_t q = 0; q < PER; ++q)
        if (q < nq) {
          hm[(uint64_t)(t + j) * K + c0 + q] = run[q];
          run[q] += v[j][q];
        }
  }
  for (; t < t1; ++t)
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q)
      if (q < nq) {
        const uint32_t v = hm[(uint64_t)t * K + c0 + q];
        hm[(uint64_t)t * K + c0 + q] = run[q];
        run[q] += v;
      }
}


// Workgroups are dispatched round-robin over the 8 XCDs; hand each XCD a
// contiguous range of logical tiles so neighbouring tiles (which write
// neighbouring runs of the same clusters) share one L2.
__device__ __forceinline__ uint32_t xcd_contiguous(uint32_t linear, uint32_t total) {
  const uint32_t per = (total + 7) / 8;
  return (linear % 8) * per + linear / 8;
}

// Step 3: stable scatter through LDS.  Each of the 4 waves owns a quarter of
// the tile and walks it in rounds of 64 in index order, ranking equal codes
// inside a round with ballots (match on every code bit).  The tile is first
// sorted by code in LDS, then every cluster's run leaves as consecutive
// DP-float records: sorted[m][start[c] + tile offset + rank][0..DP).
template <int D>
__global__ __launch_bounds__(kBlock) void scatter_kernel(
    const float* __restrict__ xs, const uint16_t* __restrict__ codes,
    const uint32_t* __restrict__ hist, const uint32_t* __restrict__ start,
    float* __restrict__ sorted, const uint32_t* __restrict__ done, uint64_t n,
    uint32_t K, uint32_t T, uint32_t M, uint32_t code_bits) {
  constexpr int DP = Pad<D>::value;
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  float* sx = reinterpret_cast<float*>(smem);  // [kSortTile][DP]
  uint32_t* gdest = smem + kSortTile * DP;     // [kSortTile]
  uint32_t* run = gdest + kSortTile;           // [4][K]
  uint32_t* delta = run + 4 * K;               // [K]
  __shared__ uint32_t wsum[kBlock / kWave];
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  if (logical >= M * T) return;
  const uint32_t m = logical / T, t = logical % T;
  if (done[m]) return;
  const uint32_t w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  constexpr uint32_t kQuarter = kSortTile / 4;
  const uint64_t tile_lo = (uint64_t)t * kSortTile;
  const uint64_t tile_hi = tile_lo + kSortTile < n ? tile_lo + kSortTile : n;
  const uint64_t lo = tile_lo + (uint64_t)w * kQuarter;
  const uint64_t hi = lo + kQuarter < tile_hi ? lo + kQuarter : tile_hi;
  const uint16_t* cm = codes + (uint64_t)m * n;
  const float* xm = xs + (uint64_t)m * n * DP;

  // The wave's kRounds rounds of codes and records are loaded up front, so
  // all of them are in flight while the counters and the scan run; the codes
  // serve both the counting and the ranking pass.
  constexpr uint32_t kRounds = kQuarter / kWave;
  uint32_t code[kRounds];
  float xv[kRounds][DP];
#pragma unroll
  for (uint32_t r = 0; r < kRounds; ++r) {
    const uint64_t i = lo + (uint64_t)r * kWave + lane;
    code[r] = i < hi ? cm[i] : 0u;
    if (i < hi) {
      const float* src = xm + i * DP;
#pragma unroll
      for (int k = 0; k < DP; k += (DP >= 4 ? 4 : DP)) {
        if constexpr (DP >= 4) {
          const float4 a = *reinterpret_cast<const float4*>(src + k);
          xv[r][k] = a.x; xv[r][k + 1] = a.y; xv[r][k + 2] = a.z; xv[r][k + 3] = a.w;
        } else if constexpr (DP == 2) {
          const float2 a = *reinterpret_cast<const float2*>(src);
          xv[r][0] = a.x; xv[r][1] = a.y;
        } else {
          xv[r][0] = src[0];
        }
      }
    }
  }

  // This thread's codes' global run starts (start + the tile's offset),
  // loaded now so that the scan below does not wait for them.
  const uint32_t per_c = (K + blockDim.x - 1) / blockDim.x;
  const uint32_t c0 = threadIdx.x * per_c;
  const uint32_t* hm = hist + ((uint64_t)m * T + t) * K;
  constexpr uint32_t kPre = 4;
  uint32_t pre[kPre];
#pragma unroll
  for (uint32_t q = 0; q < kPre; ++q)
    pre[q] = q < per_c && c0 + q < K ? start[(uint64_t)m * K + c0 + q] + hm[c0 + q] : 0u;

  for (uint32_t c = threadIdx.x; c < 4 * K; c += blockDim.x) run[c] = 0;
  __syncthreads();
  // Ranking inside each round of 64: the lanes holding the same code (a
  // match on every code bit), this lane's rank among them and their number,
  // kept as rank | total << 16 for the placement pass.  The last lane of
  // each code adds the number to the wave's count: one plain add per
  // distinct code and round (the wave's LDS operations run in order).
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint32_t* myrun = run + w * K;
  uint32_t rk[kRounds];
#pragma unroll
  for (uint32_t r = 0; r < kRounds; ++r) {
    const bool valid = lo + (uint64_t)r * kWave + lane < hi;
    const uint32_t cd = code[r];
    uint64_t match = __ballot(valid);
    for (uint32_t b = 0; b < code_bits; ++b) {
      const bool bit = (cd >> b) & 1u;
      const uint64_t bal = __ballot(bit);
      match &= bit ? bal : ~bal;
    }
    const uint32_t rank = __popcll(match & lt_mask);
    const uint32_t total = __popcll(match);
    rk[r] = rank | (total << 16);
    if (valid && rank == total - 1) myrun[cd] += total;
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();

  // Per code: tile-local bucket start (scan over codes), wave prefixes, and
  // delta = global start of the tile's run - local start.
  uint32_t tot = 0;
  for (uint32_t q = 0; q < per_c; ++q)
    if (c0 + q < K)
      tot += run[c0 + q] + run[K + c0 + q] + run[2 * K + c0 + q] + run[3 * K + c0 + q];
  uint32_t ls = block_exclusive_scan(tot, wsum);
  for (uint32_t q = 0; q < per_c; ++q) {
    const uint32_t c = c0 + q;
    if (c >= K) break;
    uint32_t g0 = 0;
#pragma unroll
    for (uint32_t j = 0; j < kPre; ++j) g0 = j == q ? pre[j] : g0;
    delta[c] = (q < kPre ? g0 : start[(uint64_t)m * K + c] + hm[c]) - ls;
    uint32_t acc = ls;
    for (uint32_t ww = 0; ww < 4; ++ww) {
      const uint32_t v = run[ww * K + c];
      run[ww * K + c] = acc;
      acc += v;
    }
    ls = acc;
  }
  __syncthreads();

#pragma unroll
  for (uint32_t r = 0; r < kRounds; ++r) {
    const bool valid = lo + (uint64_t)r * kWave + lane < hi;
    const uint32_t cd = code[r];
    const uint32_t rank = rk[r] & 0xFFFFu;
    const uint32_t total = rk[r] >> 16;
    uint32_t lp = 0;
    if (valid) lp = myrun[cd] + rank;
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == total - 1) myrun[cd] = lp + 1;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      float* dst = sx + lp * DP;
#pragma unroll
      for (int k = 0; k < DP; k += (DP >= 4 ? 4 : DP)) {
        if constexpr (DP >= 4)
          *reinterpret_cast<float4*>(dst + k) =
              make_float4(xv[r][k], xv[r][k + 1], xv[r][k + 2], xv[r][k + 3]);
        else if constexpr (DP == 2)
          *reinterpret_cast<float2*>(dst) = make_float2(xv[r][0], xv[r][1]);
        else
          dst[0] = xv[r][0];
      }
      gdest[lp] = lp + delta[cd];
    }
  }
  __syncthreads();

  const uint32_t len = (uint32_t)(tile_hi - tile_lo);
  float* sm = sorted + (uint64_t)m * n * DP;
  for (uint32_t lp = threadIdx.x; lp < len; lp += blockDim.x) {
    const float* src = sx + lp * DP;
    float* dst = sm + (uint64_t)gdest[lp] * DP;
#pragma unroll
    for (int k = 0; k < DP; k += (DP >= 4 ? 4 : DP)) {
      if constexpr (DP >= 4)
        *reinterpret_cast<float4*>(dst + k) = *reinterpret_cast<const float4*>(src + k);
      else if constexpr (DP == 2)
        *reinterpret_cast<float2*>(dst) = *reinterpret_cast<const float2*>(src);
      else
        dst[0] = src[0];
    }
  }
}

// Step 4: one wave per (subspace, FP consecutive ranks of its size order):
// block g * M + m folds the clusters of ranks g FP .. g FP + FP - 1 in
// subspace m's size order (fold_order_block), so every subspace's largest
// clusters start first, and clusters that share a wave have similar sizes.
// FP = 8 / DP below four padded dimensions (four clusters at dsub 2, eight
// at dsub 1), else 1, so that lane p DP + d folds dimension d of the wave's
// cluster p and one add serves FP clusters.  The wave streams each
// cluster's contiguous records with coalesced loads (kFoldBatch x 64 records
// in flight, staged through LDS dimension-major) and each lane folds its
// dimension in ascending vector order from 0.0f, then writes
// sum * fl(1 / fl(count)) (src/tac/kmeans.zig:177-198).  Empty clusters are
// left for reseed_kernel.
template <int D>
constexpr uint32_t fold_per_wave() {
  return Pad<D>::value < 4 ? 8u / (uint32_t)Pad<D>::value : 1u;
}

template <int D>
__global__ __launch_bounds__(kWave) void fold_kernel(
    const float* __restrict__ sorted, const uint32_t* __restrict__ counts,
    const uint32_t* __restrict__ start, float* __restrict__ cb,
    const uint32_t* __restrict__ done, const uint32_t* __restrict__ order, uint64_t n,
    uint32_t M, uint32_t K) {
  constexpr int DP = Pad<D>::value;
  constexpr uint32_t FP = fold_per_wave<D>();
  constexpr uint32_t U = kFoldBatch;
  // Padded: the FP * DP columns start on distinct banks.
  constexpr uint32_t kCol = U * kWave + 36;
  __shared__ __attribute__((aligned(16))) float buf[kCol * DP * FP];
  const uint32_t m = blockIdx.x % M, r0 = (blockIdx.x / M) * FP;
  if (done[m]) return;
  const uint32_t lane = threadIdx.x;
  uint32_t cl[FP], cnt[FP];
  const float* src[FP];
  uint32_t most = 0;
#pragma unroll
  for (uint32_t f = 0; f < FP; ++f) {
    cl[f] = r0 + f < K ? order[(uint64_t)m * K + r0 + f] : 0u;
    cnt[f] = r0 + f < K ? counts[(uint64_t)m * K + cl[f]] : 0u;
    src[f] = sorted + ((uint64_t)m * n + (cnt[f] ? start[(uint64_t)m * K + cl[f]] : 0u)) * DP;
    most = cnt[f] > most ? cnt[f] : most;
  }
  if (most == 0) return;
  float v[FP][U][DP];
  auto load_batch = [&](uint32_t j0) {
#pragma unroll
    for (uint32_t f = 0; f < FP; ++f)
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) {
        const uint32_t j = j0 + u * kWave + lane;
        if (j < cnt[f]) {
          const float* q = src[f] + (uint64_t)j * DP;
#pragma unroll
          for (int k = 0; k < DP; k += (DP >= 4 ? 4 : DP)) {
            if constexpr (DP >= 4) {
              const float4 a = *reinterpret_cast<const float4*>(q + k);
              v[f][u][k] = a.x; v[f][u][k + 1] = a.y; v[f][u][k + 2] = a.z; v[f][u][k + 3] = a.w;
            } else if constexpr (DP == 2) {
              const float2 a = *reinterpret_cast<const float2*>(q);
              v[f][u][0] = a.x; v[f][u][1] = a.y;
            } else {
              v[f][u][0] = q[0];
            }
          }
        }
      }
  };
  // buf is column-major, [FP][DP][kCol]: lane f DP + d reads four
  // consecutive members of dimension d of cluster f with one 16-byte LDS
  // read.
  const uint32_t f_of = lane / DP, d_of = lane % DP;
  const bool folds = f_of < FP && d_of < (uint32_t)D;
  uint32_t mine = 0, my_cl = 0;  // this lane's cluster, by selects (no indexed registers)
#pragma unroll
  for (uint32_t f = 0; f < FP; ++f) {
    mine = f == f_of ? cnt[f] : mine;
    my_cl = f == f_of ? cl[f] : my_cl;
  }
  mine = folds ? mine : 0u;
  float acc = 0.0f;
  load_batch(0);
  for (uint32_t j0 = 0; j0 < most; j0 += U * kWave) {
#pragma unroll
    for (uint32_t f = 0; f < FP; ++f)
#pragma unroll
      for (uint32_t u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < DP; ++k) buf[(f * DP + k) * kCol + u * kWave + lane] = v[f][u][k];
    __syncthreads();
    if (j0 + U * kWave < most) load_batch(j0 + U * kWave);
    const uint32_t len = mine > j0 ? (mine - j0 < U * kWave ? mine - j0 : U * kWave) : 0u;
    if (folds) {
      // One dependent add per member, in ascending member order.  A step
      // issues the LDS reads of 128 members together (32 16-byte reads), so
      // their latency is paid once per 128 adds; then steps of 32, then one.
      const float* col = buf + lane * kCol;
      const float4* col4 = reinterpret_cast<const float4*>(col);
      uint32_t jj = 0;
      for (; jj + 128 <= len; jj += 128) {
        float4 a[32];
#pragma unroll
        for (int q = 0; q < 32; ++q) a[q] = col4[jj / 4 + q];
#pragma unroll
        for (int q = 0; q < 32; ++q) {
          acc = acc + a[q].x;
          acc = acc + a[q].y;
          acc = acc + a[q].z;
          acc = acc + a[q].w;
        }
      }
      for (; jj + 32 <= len; jj += 32) {
        float4 a[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) a[q] = col4[jj / 4 + q];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          acc = acc + a[q].x;
          acc = acc + a[q].y;
          acc = acc + a[q].z;
          acc = acc + a[q].w;
        }
      }
      for (; jj < len; ++jj) acc = acc + col[jj];
    }
    __syncthreads();
  }
  if (folds && mine > 0) cb[((uint64_t)m * K + my_cl) * D + d_of] = acc * (1.0f / (float)mine);
}

// ---------------------------------------------------------------------------
// wcss = sequential fp32 fold of e over ascending vector index
// (src/tac/kmeans.zig:179), evaluated exactly in chunks of kFoldChunk terms
// (fold_rules.hpp): f64 chunk sums -> prefix -> per-chunk quantized sums for
// three candidate binades -> one wave per subspace applies the chunks in
// order, folding term by term any chunk the rules do not cover.  The wave
// helpers also serve the f64 weight folds of k-means++ (kmeanspp.hpp).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_down(v, off, kWave);
  return v;
}
// v of the lane the DPP control CTRL names (0 where it names none or the
// row is outside ROW_MASK), both halves of a 64-bit value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK,
                                                            0xf, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL,
                                                            ROW_MASK, 0xf, true);
  return ((uint64_t)hi << 32) | lo;
}

// Inclusive prefix sum over the wave's lanes by DPP moves (VALU, no LDS
// round trips): shifts by 1, 2, 4, 8 inside each row of 16 lanes, then row
// 0's total into row 1 and row 2's into row 3 (row_bcast:15), then rows
// 0-1's into rows 2-3 (row_bcast:31).
__device__ __forceinline__ uint64_t wave_inclusive_sum_u64(uint64_t v) {
  v += dpp_u64<0x111, 0xf>(v);  // row_shr:1
  v += dpp_u64<0x112, 0xf>(v);  // row_shr:2
  v += dpp_u64<0x114, 0xf>(v);  // row_shr:4
  v += dpp_u64<0x118, 0xf>(v);  // row_shr:8
  v += dpp_u64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_u64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// v of lane `l` (uniform) in every lane.
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, uint32_t l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, (int)l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), (int)l);
  return ((uint64_t)hi << 32) | lo;
}

// The sum over the wave's lanes, in every lane.
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  return readlane_u64(wave_inclusive_sum_u64(v), kWave - 1);
}

// Orders one wave's LDS accesses before and after this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int32_t kFoldNoBinade = -100000;  // k0 of a chunk whose start is not normal

__host__ __device__ inline uint32_t fold_chunk_len(uint64_t n, uint32_t j) {
  const uint64_t lo = (uint64_t)j * kFoldChunk;
  return n - lo < kFoldChunk ? (uint32_t)(n - lo) : kFoldChunk;
}

// f64 sum of chunk j in any order (it only places the candidate binades);
// the total lands in lane 0.
__device__ inline double fold_chunk_sum_wave(const float* __restrict__ em, uint64_t n, uint32_t j) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint64_t lo = (uint64_t)j * kFoldChunk;
  const uint32_t len = fold_chunk_len(n, j);
  double acc = 0.0;
  for (uint32_t t = lane; t < len; t += kWave) acc += (double)em[lo + t];
  return wave_sum_f64(acc);
}

// Exclusive prefix of a[0 .. cnt) in place, by a block of kThreads threads
// (f64, any rounding: the values only place the candidate binades).
template <uint32_t kThreads>
__device__ inline void block_prefix_f64(double* __restrict__ a, uint32_t cnt, double* wsum,
                                        double* carry) {
  const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  if (threadIdx.x == 0) *carry = 0.0;
  __syncthreads();
  for (uint32_t j0 = 0; j0 < cnt; j0 += kThreads) {
    const uint32_t j = j0 + threadIdx.x;
    const double x = j < cnt ? a[j] : 0.0;
    double incl = x;
    for (int off = 1; off < kWave; off <<= 1) {
      const double o = __shfl_up(incl, off, kWave);
      if (lane >= (uint32_t)off) incl += o;
    }
    if (lane == kWave - 1) wsum[w] = incl;
    __syncthreads();
    double before = *carry;
    for (uint32_t q = 0; q < w; ++q) before += wsum[q];
    if (j < cnt) a[j] = before + (incl - x);
    __syncthreads();
    if (threadIdx.x == kThreads - 1) *carry = before + incl;
    __syncthreads();
  }
}

// One wave: the descriptor of chunk j (quantized sums for the binades
// around the approximate start `pre`), written by lane 0.
template <typename Acc>
__device__ inline void fold_quantize_chunk_wave(const float* __restrict__ em, uint64_t n,
                                                uint32_t j, double pre,
                                                FoldChunk* __restrict__ out) {
  const uint32_t lane = threadIdx.x % kWave;
  const Acc ps = (Acc)pre;
  const int32_t k0 = fold_is_normal_positive(ps) ? fold_exponent(ps) - 1 : kFoldNoBinade;
  const uint64_t lo = (uint64_t)j * kFoldChunk;
  const uint32_t len = fold_chunk_len(n, j);
  uint64_t q[kFoldCands] = {0, 0, 0};
  uint32_t bad = 0;  // bit c: candidate c spoiled by one of this lane's terms
  for (uint32_t t = lane; t < len; t += kWave) {
    const float v = em[lo + t];
#pragma unroll
    for (int c = 0; c < kFoldCands; ++c) {
      const uint64_t qi = fold_quantize<Acc>(v, k0 + c);
      bad |= qi == kFoldBad ? 1u << c : 0u;
      q[c] += qi == kFoldBad ? 0u : qi;
    }
  }
  for (int off = kWave / 2; off > 0; off >>= 1) bad |= __shfl_xor(bad, off, kWave);
#pragma unroll
  for (int c = 0; c < kFoldCands; ++c) q[c] = wave_sum_u64(q[c]);
  if (lane == 0) {
    FoldChunk ch;
    ch.k0 = k0;
    ch.clean = ~bad & ((1u << kFoldCands) - 1u);
#pragma unroll
    for (int c = 0; c < kFoldCands; ++c) ch.q[c] = q[c];
    *out = ch;
  }
}

// fold_chunk_sum_wave and fold_quantize_chunk_wave for the B chunks
// j0 .. j0 + B - 1 below nc at once (each chunk's terms in the same lanes and
// order), every load issued before any arithmetic: one wave working through
// many chunks pays a memory round trip per B chunks instead of per chunk.
template <uint32_t B>
__device__ inline void fold_load_chunks_wave(const float* __restrict__ em, uint64_t n,
                                             uint32_t j0, uint32_t nc,
                                             float (&v)[B][kFoldChunk / kWave],
                                             uint32_t (&len)[B]) {
  const uint32_t lane = threadIdx.x % kWave;
#pragma unroll
  for (uint32_t b = 0; b < B; ++b) {
    const uint32_t j = j0 + b;
    len[b] = j < nc ? fold_chunk_len(n, j) : 0u;
    const uint64_t lo = (uint64_t)j * kFoldChunk;
#pragma unroll
    for (uint32_t t = 0; t < kFoldChunk / kWave; ++t) {
      const uint32_t i = lane + t * kWave;
      v[b][t] = i < len[b] ? em[lo + i] : 0.0f;
    }
  }
}

template <uint32_t B>
__device__ inline void fold_chunk_sums_wave(const float* __restrict__ em, uint64_t n, uint32_t j0,
                                            uint32_t nc, double (&cs)[B]) {
  const uint32_t lane = threadIdx.x % kWave;
  float v[B][kFoldChunk / kWave];
  uint32_t len[B];
  fold_load_chunks_wave<B>(em, n, j0, nc, v, len);
#pragma unroll
  for (uint32_t b = 0; b < B; ++b) {
    double acc = 0.0;
#pragma unroll
    for (uint32_t t = 0; t < kFoldChunk / kWave; ++t)
      if (lane + t * kWave < len[b]) acc += (double)v[b][t];
    cs[b] = wave_sum_f64(acc);
  }
}

template <typename Acc, uint32_t B>
__device__ inline void fold_quantize_chunks_wave(const float* __restrict__ em, uint64_t n,
                                                 uint32_t j0, uint32_t nc,
                                                 const double (&pre)[B],
                                                 FoldChunk* __restrict__ out) {
  const uint32_t lane = threadIdx.x % kWave;
  float v[B][kFoldChunk / kWave];
  uint32_t len[B];
  fold_load_chunks_wave<B>(em, n, j0, nc, v, len);
#pragma unroll
  for (uint32_t b = 0; b < B; ++b) {
    const Acc ps = (Acc)pre[b];
    const int32_t k0 = fold_is_normal_positive(ps) ? fold_exponent(ps) - 1 : kFoldNoBinade;
    uint64_t q[kFoldCands] = {0, 0, 0};
    uint32_t bad = 0;  // bit c: candidate c spoiled by one of this lane's terms
#pragma unroll
    for (uint32_t t = 0; t < kFoldChunk / kWave; ++t) {
      if (lane + t * kWave >= len[b]) continue;
#pragma unroll
      for (int c = 0; c < kFoldCands; ++c) {
        const uint64_t qi = fold_quantize<Acc>(v[b][t], k0 + c);
        bad |= qi == kFoldBad ? 1u << c : 0u;
        q[c] += qi == kFoldBad ? 0u : qi;
      }
    }
    for (int off = kWave / 2; off > 0; off >>= 1) bad |= __shfl_xor(bad, off, kWave);
#pragma unroll
    for (int c = 0; c < kFoldCands; ++c) q[c] = wave_sum_u64(q[c]);
    if (lane == 0 && j0 + b < nc) {
      FoldChunk ch;
      ch.k0 = k0;
      ch.clean = ~bad & ((1u << kFoldCands) - 1u);
#pragma unroll
      for (int c = 0; c < kFoldCands; ++c) ch.q[c] = q[c];
      out[b] = ch;
    }
  }
}

// One wave folds chunks 0 .. nc-1 of em in order from 0 with their
// descriptors and returns the exact serial sum in every lane; every lane
// computes the same values.  While the sum is normal, lane i takes chunk
// j + i's quantized sum for the sum's binade and one prefix sum applies the
// chunks up to the first one that does not fit (fold_run_fits), up to 64 at
// a time.  That chunk, and any chunk while the sum is zero or subnormal, is
// staged in `buf` (kFoldChunk floats of LDS) and folded term by term.  With
// `starts`, the exact accumulator value before each chunk is stored.
template <typename Acc>
__device__ inline Acc fold_apply_wave(const float* __restrict__ em, uint64_t n,
                                      const FoldChunk* __restrict__ cm, uint32_t nc, float* buf,
                                      Acc* __restrict__ starts) {
  const uint32_t lane = threadIdx.x % kWave;
  Acc s = 0;
  uint32_t j = 0;
  while (j < nc) {
    const uint32_t cnt = nc - j < kWave ? nc - j : kWave;
    uint32_t b = 0;  // chunks applied through the prefix sum
    if (fold_is_normal_positive(s)) {
      const uint64_t m = fold_units(s);
      const uint64_t Q = lane < cnt ? fold_chunk_q(s, cm[j + lane]) : kFoldBad;
      const bool ok = Q != kFoldBad;
      const uint64_t P = wave_inclusive_sum_u64(ok ? Q : 0u);
      const uint64_t bad = __ballot(lane < cnt && !(ok && fold_run_fits<Acc>(m, P)));
      b = bad ? (uint32_t)__builtin_ctzll(bad) : cnt;
      if (starts != nullptr && lane < b) starts[j + lane] = fold_with_units(s, m + P - Q);
      if (b > 0) s = fold_with_units(s, m + readlane_u64(P, b - 1));
    }
    j += b;
    if (b < cnt) {
      if (starts != nullptr && lane == 0) starts[j] = s;
      const uint64_t lo = (uint64_t)j * kFoldChunk;
      const uint32_t len = fold_chunk_len(n, j);
      wave_lds_sync();
      for (uint32_t t = lane; t < len; t += kWave) buf[t] = em[lo + t];
      wave_lds_sync();
      Acc out = s;
#pragma unroll 16
      for (uint32_t t = 0; t < len; ++t) out = out + (Acc)buf[t];
      s = out;
      ++j;
    }
  }
  return s;
}

// Chunk sums, one wave per chunk, four chunks per block.
__global__ __launch_bounds__(kBlock) void wcss_chunk_sums_kernel(
    const float* __restrict__ e, double* __restrict__ csum, const uint32_t* __restrict__ done,
    uint64_t n, uint32_t nc) {
  const uint32_t m = blockIdx.y, j = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
  if (done[m] || j >= nc) return;
  const double s = fold_chunk_sum_wave(e + (uint64_t)m * n, n, j);
  if (threadIdx.x % kWave == 0) csum[(uint64_t)m * nc + j] = s;
}

// Exclusive prefix of the chunk sums (in place), one block per subspace.
__global__ __launch_bounds__(kBlock) void wcss_prefix_kernel(double* __restrict__ csum,
                                                             const uint32_t* __restrict__ done,
                                                             uint32_t nc) {
  __shared__ double ws[kBlock / kWave];
  __shared__ double carry;
  const uint32_t m = blockIdx.x;
  if (done[m]) return;
  block_prefix_f64<kBlock>(csum + (uint64_t)m * nc, nc, ws, &carry);
}

// Chunk descriptors, one wave per chunk, four chunks per block.
__global__ __launch_bounds__(kBlock) void wcss_quantize_kernel(
    const float* __restrict__ e, const double* __restrict__ pre, FoldChunk* __restrict__ chunks,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t nc) {
  const uint32_t m = blockIdx.y, j = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
  if (done[m] || j >= nc) return;
  const uint64_t at = (uint64_t)m * nc + j;
  fold_quantize_chunk_wave<float>(e + (uint64_t)m * n, n, j, pre[at], chunks + at);
}

// One wave per subspace applies the chunks in order.
__global__ __launch_bounds__(kWave) void wcss_apply_kernel(
    const float* __restrict__ e, const FoldChunk* __restrict__ chunks, float* __restrict__ wcss,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t nc) {
  __shared__ __attribute__((aligned(16))) float buf[kFoldChunk];
  const uint32_t m = blockIdx.x;
  if (done[m]) return;
  const float s = fold_apply_wave<float>(e + (uint64_t)m * n, n, chunks + (uint64_t)m * nc, nc,
                                         buf, static_cast<float*>(nullptr));
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
    float* __restrict__ cb, uint32_t* __restrict__ empties, uint32_t* __restrict__ done,
    const float* __restrict__ wcss, float* __restrict__ prev, uint32_t* __restrict__ iters_run,
    uint64_t n, uint32_t K, uint32_t iter, float tol, int check) {
  constexpr int DP = Pad<D>::value;
  __shared__ float sv[1024 / kWave];
  __shared__ uint64_t si[1024 / kWave];
  const uint32_t m = blockIdx.x;
  if (done[m]) return;
  float* em = e + (uint64_t)m * n;
  const uint32_t* cm = counts + (uint64_t)m * K;
  const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const uint32_t nw = blockDim.x / kWave;
  // Empty clusters, listed in ascending order (K <= blockDim.x).
  __shared__ uint32_t elist[1024];
  __shared__ uint32_t ewsum[1024 / kWave];
  const bool empty = threadIdx.x < K && cm[threadIdx.x] == 0;
  const uint32_t pos = block_exclusive_scan(empty ? 1u : 0u, ewsum);
  if (empty) elist[pos] = threadIdx.x;
  uint32_t found = 0;
  for (uint32_t q = 0; q < nw; ++q) found += ewsum[q];  // wave totals: the count
  __syncthreads();
  for (uint32_t q = 0; q < found; ++q) {
    const uint32_t c = elist[q];  // uniform across the block
    float bv = -__builtin_inff();
    uint64_t bi = ~0ull;
    // vec.argmax starts from values[0] and moves only on a strict >, so a NaN
    // past index 0 never wins and a NaN at index 0 keeps index 0: NaN terms
    // are never candidates here, and index 0 is settled after the merge.
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const float v = em[i];
      if ((bi == ~0ull || v > bv) && !(v != v)) {
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
      const float e0 = em[0];
      if (e0 != e0 || idx == ~0ull) idx = 0;  // values[0] NaN: the scan keeps index 0
      const float* src = xs + ((uint64_t)m * n + idx) * DP;
      for (int k = 0; k < D; ++k) cb[((uint64_t)m * K + c) * D + k] = src[k];
      em[idx] = -__builtin_inff();
    }
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  empties[m] += found;
  // Convergence bookkeeping (src/tac/kmeans.zig:186, :214-223) of iteration
  // `iter`, whose wcss the update computed before the reseed.
  iters_run[m] = iter + 1;
  if (!check) return;
  const float ws = wcss[m];
  if (iter > 0) {
    const float p = prev[m];
    const float denom = p > 0.0f ? p : 1.0f;
    const float rel = (p - ws) / denom;
    if (rel < tol) {
      done[m] = 1;
      return;
    }
  }
  prev[m] = ws;
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

// Clears n 32-bit words (a kernel rather than a memset, so the clear is an
// ordinary dispatch in any stream or captured graph).
__global__ void zero_words_kernel(uint32_t* __restrict__ p, uint32_t n) {
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

// Final codes [M][n] u16 -> caller's u32 assignments for kmeans.fit (M = 1).
__global__ void widen_codes_kernel(const uint16_t* __restrict__ codes, uint32_t* __restrict__ out,
                                   uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = codes[i];
}

// Codes [M][n] u16 -> token-major rows [n][M] of CodeT (PQ.encode's layout,
// src/index/storage.zig:384-401): reads coalesced per subspace, each thread
// writes its row's M codes.
template <typename CodeT>
__global__ void codes_to_tokens_kernel(const uint16_t* __restrict__ codes, CodeT* __restrict__ out,
                                       uint64_t n, uint32_t M) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  for (uint32_t m = 0; m < M; ++m) out[i * M + m] = (CodeT)codes[(uint64_t)m * n + i];
}

// ---------------------------------------------------------------------------
// PQ.encode (src/index/pq.zig:59-76) over token-major residuals.  One block =
// one subspace m and kBlock*VPT consecutive vectors (the assignment kernel's
// shape, reading sub-vector m of each row in place).  Block ids are laid out
// XCD-contiguously with the M subspaces of a row tile adjacent, so the M
// blocks that read the same rows run together on one XCD and share its L2:
// each row crosses HBM once instead of once per subspace.  best_d starts at
// +inf, strict <.
// ---------------------------------------------------------------------------
template <int D, int VPT, typename CodeT>
__global__ __launch_bounds__(kBlock) void encode_kernel(
    const float* __restrict__ x, const float* __restrict__ cb, CodeT* __restrict__ codes,
    uint64_t n, uint32_t dim, uint32_t M, uint32_t K, uint32_t tiles,
    unsigned long long* __restrict__ rescans) {
  constexpr uint32_t kTile = kBlock * VPT;
  constexpr int DP = Pad<D>::value;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  if (logical >= tiles * M) return;  // grid padding to a multiple of 8
  const uint32_t t = logical / M, m = logical % M;
  const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
  float* lcb = lds;                 // [Kp][DP], 16-byte aligned records
  float* lnc = lds + Kp * DP;       // [Kp]
  uint32_t& lmax = *reinterpret_cast<uint32_t*>(lnc + Kp);
  uint32_t& lcount = *(&lmax + 1);
  if (threadIdx.x == 0) {
    lmax = 0;
    lcount = 0;
  }
  __syncthreads();
  stage_pruned<D>(lcb, lnc, &lmax, cb + (uint64_t)m * K * D, K, Kp);
  __syncthreads();

  const uint64_t base = (uint64_t)t * kTile + threadIdx.x;
  float xv[VPT][D];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint64_t i = base + (uint64_t)j * kBlock;
    const float* src = x + (i < n ? i : 0) * dim + (uint64_t)m * D;
#pragma unroll
    for (int k = 0; k < D; ++k) xv[j][k] = src[k];
  }
  uint32_t bidx[VPT];
  float best[VPT];
  uint32_t mine = 0;
  pruned_argmin<D, VPT, false>(xv, lcb, lnc, K, Kp, lmax, bidx, best, mine);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint64_t i = base + (uint64_t)j * kBlock;
    if (i < n) codes[i * M + m] = (CodeT)bidx[j];
  }
  flush_rescans(mine, &lcount, rescans);
}

// PQ.decode (src/index/pq.zig:79-88): out[i][m*D + k] = cb[m][code[i][m]][k].
// A code >= K raises `status` and yields NaN instead of a read.
template <typename CodeT>
__global__ void decode_kernel(const CodeT* __restrict__ codes, const float* __restrict__ cb,
                              float* __restrict__ out, uint32_t* __restrict__ status,
                              uint64_t n, uint32_t M, uint32_t K, uint32_t D) {
  const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t dim = (uint64_t)M * D;
  if (g >= n * dim) return;
  const uint64_t i = g / dim;
  const uint32_t r = g % dim;
  const uint32_t m = r / D, k = r % D;
  const uint32_t code = codes[i * M + m];
  if (code >= K) {
    atomicOr(status, 1u);
    out[g] = __builtin_nanf("");
    return;
  }
  out[g] = cb[((uint64_t)m * K + code) * D + k];
}

}  // namespace tacgpu
