// kmeanspp.hpp — k-means++ seeding of every subspace at once
// (src/tac/kmeans.zig:106-136, src/util/rng.zig:22-82).  Included once, by
// tac_gpu.hip, after pq_kernels.hpp.
//
// Per subspace m the reference draws with std.Random.DefaultPrng seeded with
// seed +% m (src/index/pq.zig:323):
//   c0 = row intRangeLessThan(0, n); w_i = l2sq(x_i, c0)
//   for c = 1 .. K-1:  idx = weightedSample(w); c_c = row idx;
//                      w_i = min(w_i, l2sq(x_i, c_c))   (strict <)
// weightedSample folds the weights sequentially in f64 (total, then the
// running cum), draws u = float(f64) * total and returns the first i with
// u < cum_i (last positive index if none).
//
// The GPU sums the weights in parallel, in any order.  For non-negative
// terms every rounded sum (the reference's sequential fold or ours) lies
// within i * 2^-53 * P_i of the exact prefix P_i, so the two differ by at
// most band_i = 2.1 (i + 1) 2^-53 P_i.  When the draw clears the bands of the
// candidate index on both sides the reference's pick is determined;
// otherwise the subspace falls back to the exact sequential fold on one wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kpp_rules.hpp"

namespace tacgpu {

struct KppState {
  uint64_t s[4];
  double r;          // draw of the current round
  uint32_t chosen;   // row picked in the current round
  uint32_t fallback; // 1: the parallel decision was inconclusive this round
  int32_t err;       // 0 or a tac_status (NonFinite / AllZero)
  uint32_t pad;
};

constexpr int kKppBlock = 4096;  // weights per partial sum

// Round c: write codeword c of every subspace from the row chosen last round,
// update the weights w = min(w, l2sq(x, c_new)) (the first round assigns),
// validate them, and emit f64 partial sums per block of kKppBlock rows.
template <int D>
__global__ __launch_bounds__(256) void kpp_update_kernel(
    const float* __restrict__ xs, float* __restrict__ w, double* __restrict__ bsum,
    uint32_t* __restrict__ bad, const KppState* __restrict__ st, float* __restrict__ cb,
    uint64_t n, uint32_t K, uint32_t c, uint32_t NB) {
  constexpr int DP = Pad<D>::value;
  __shared__ double part[256 / 64];
  const uint32_t m = blockIdx.y, b = blockIdx.x;
  if (st[m].err) return;
  const uint32_t chosen = st[m].chosen;
  float cv[D];
  load_padded<D>(xs + ((uint64_t)m * n + chosen) * DP, cv);
  if (b == 0 && threadIdx.x < (uint32_t)D) cb[((uint64_t)m * K + c) * D + threadIdx.x] = cv[threadIdx.x];
  const uint64_t lo = (uint64_t)b * kKppBlock;
  const uint64_t hi = lo + kKppBlock < n ? lo + kKppBlock : n;
  float* wm = w + (uint64_t)m * n;
  const float* xm = xs + (uint64_t)m * n * DP;
  double acc = 0.0;
  bool invalid = false;
  for (uint64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    float xv[D];
    load_padded<D>(xm + i * DP, xv);
    const float d = exact_l2sq<D>(xv, cv);
    float wi = d;
    if (c > 0) {
      const float old = wm[i];
      wi = d < old ? d : old;  // kmeans.zig:134: replace on strict <
    }
    wm[i] = wi;
    invalid |= !(wi >= 0.0f && wi <= 3.402823466e38f);  // rng.zig:62 NonFinite
    acc += (double)wi;
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
  if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = acc;
  if (invalid) atomicOr(&bad[m], 1u);
  __syncthreads();
  if (threadIdx.x == 0) bsum[(uint64_t)m * NB + b] = (part[0] + part[1]) + (part[2] + part[3]);
}

// Round c draw: one block per subspace.  Checks the weights, draws u, finds
// the candidate with the partial sums and a block-local prefix, and either
// fixes `chosen` or raises `fallback`.
__global__ __launch_bounds__(1024) void kpp_select_kernel(
    const float* __restrict__ w, const double* __restrict__ bsum, uint32_t* __restrict__ bad,
    KppState* __restrict__ st, uint64_t n, uint32_t NB) {
  __shared__ double s_before, s_total;
  __shared__ uint32_t s_block, s_first, s_stop;
  __shared__ double wsum[1024 / 64];
  const uint32_t m = blockIdx.x;
  KppState& S = st[m];
  // Thread 0 alone reads and writes the subspace state before the barrier;
  // every thread then acts on the shared verdict.
  if (threadIdx.x == 0) {
    s_stop = 1;
    s_first = 0xFFFFFFFFu;
    if (!S.err) {
      S.fallback = 0;
      if (bad[m]) {
        S.err = 9;  // NonFinite
      } else {
        double tot = 0.0;
        for (uint32_t b = 0; b < NB; ++b) tot += bsum[(uint64_t)m * NB + b];
        if (!(tot > 0.0)) {
          S.err = 10;  // AllZero
        } else {
          S.r = kpp_float64(S.s);
          const double u = S.r * tot;
          double run = 0.0;
          uint32_t blk = NB;
          for (uint32_t b = 0; b < NB; ++b) {
            const double next = run + bsum[(uint64_t)m * NB + b];
            if (u < next) {
              blk = b;
              break;
            }
            run = next;
          }
          s_block = blk;
          s_before = run;
          s_total = tot;
          if (blk == NB) {
            S.fallback = 1;  // u at or beyond the total: the tail rule decides
          } else {
            s_stop = 0;
          }
        }
      }
    }
  }
  __syncthreads();
  if (s_stop) return;
  const double r = S.r;
  // Block-local inclusive prefix of kKppBlock weights: 4 per thread.
  const uint64_t lo = (uint64_t)s_block * kKppBlock;
  const float* wm = w + (uint64_t)m * n;
  double v[4];
  double local = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint64_t i = lo + threadIdx.x * 4 + q;
    v[q] = i < n ? (double)wm[i] : 0.0;
    local += v[q];
  }
  const uint32_t lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  double incl = local;
  for (int off = 1; off < 64; off <<= 1) {
    const double o = __shfl_up(incl, off, 64);
    if (lane >= (uint32_t)off) incl += o;
  }
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  double base = s_before;
  for (uint32_t q = 0; q < wv; ++q) base += wsum[q];
  base += incl - local;
  const double u = r * s_total;
  double p = base;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    p += v[q];
    const uint64_t i = lo + threadIdx.x * 4 + q;
    if (i < n && u < p) {
      atomicMin(&s_first, (uint32_t)(i - lo));
      break;
    }
  }
  __syncthreads();
  // The thread owning the candidate checks the bands.
  if (s_first == 0xFFFFFFFFu) {
    if (threadIdx.x == 0) S.fallback = 1;
    return;
  }
  const uint32_t owner = s_first / 4;
  if (threadIdx.x == owner) {
    double pp = base, prev = base;
    const uint32_t k = s_first % 4;
    for (uint32_t q = 0; q <= k; ++q) {
      prev = pp;
      pp += v[q];
    }
    const uint64_t i = lo + s_first;
    if (kpp_decides(r, s_total, n, i, prev, pp)) {
      S.chosen = (uint32_t)i;
    } else {
      S.fallback = 1;
    }
  }
}

// Exact weightedSample on one wave for subspaces whose parallel decision was
// inconclusive: lane 0 folds the weights in order, as rng.zig:60-81 does.
__global__ __launch_bounds__(64) void kpp_fallback_kernel(const float* __restrict__ w,
                                                          KppState* __restrict__ st, uint64_t n) {
  __shared__ float buf[2048];
  const uint32_t m = blockIdx.x;
  KppState& S = st[m];
  if (S.err || !S.fallback) return;
  const float* wm = w + (uint64_t)m * n;
  double total = 0.0;
  for (uint64_t b = 0; b < n; b += 2048) {
    const uint32_t len = n - b < 2048 ? (uint32_t)(n - b) : 2048u;
    for (uint32_t q = threadIdx.x; q < len; q += 64) buf[q] = wm[b + q];
    __syncthreads();
    if (threadIdx.x == 0)
      for (uint32_t q = 0; q < len; ++q) total += (double)buf[q];
    __syncthreads();
  }
  __shared__ uint32_t found;
  __shared__ double cum_s;
  if (threadIdx.x == 0) {
    found = 0xFFFFFFFFu;
    cum_s = 0.0;
  }
  __syncthreads();
  const double u = S.r * total;
  for (uint64_t b = 0; b < n && found == 0xFFFFFFFFu; b += 2048) {
    const uint32_t len = n - b < 2048 ? (uint32_t)(n - b) : 2048u;
    for (uint32_t q = threadIdx.x; q < len; q += 64) buf[q] = wm[b + q];
    __syncthreads();
    if (threadIdx.x == 0) {
      double cum = cum_s;
      for (uint32_t q = 0; q < len; ++q) {
        cum += (double)buf[q];
        if (u < cum) {
          found = (uint32_t)(b + q);
          break;
        }
      }
      cum_s = cum;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (found == 0xFFFFFFFFu) {  // rng.zig:79-81: last positive weight
      uint64_t last = n - 1;
      while (last > 0 && wm[last] == 0.0f) --last;
      found = (uint32_t)last;
    }
    S.chosen = found;
    S.fallback = 0;
  }
}

// Seeds every subspace's stream with seed +% m and draws the first row.
__global__ void kpp_init_kernel(KppState* __restrict__ st, uint32_t* __restrict__ bad,
                                uint64_t seed, uint64_t n, uint32_t M) {
  const uint32_t m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  KppState S;
  uint64_t sm = seed + m;
  for (int q = 0; q < 4; ++q) S.s[q] = kpp_splitmix(&sm);
  S.chosen = (uint32_t)kpp_uint_less_than(S.s, n);
  S.r = 0.0;
  S.fallback = 0;
  S.err = 0;
  S.pad = 0;
  st[m] = S;
  bad[m] = 0;
}

}  // namespace tacgpu
