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

#include "cand_rules.hpp"
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
// Work-items of a kpp_update_kernel block: 8 rows each, so the kernel keeps
// four waves per SIMD at dsub 8 (16 rows each held it to two) and eight at
// dsub 4, for the rounds' dependent loads.
constexpr uint32_t kKppThreads = 512;

// Round c: write codeword c of every subspace from the row chosen last round,
// update the weights w = min(w, l2sq(x, c_new)) (the first round assigns),
// validate them, and emit f64 partial sums per block of kKppBlock rows.
//
// src[m][i] is the seed whose distance is w_i (w_i = l2sq(x_i, c_src)
// exactly: it is the minimum so far).  A seed c_new can lower w_i only if
// l2sq(x_i, c_new) < w_i, and by the candidate rule (cand_rules.hpp) it
// cannot when a rounded-down bound of ||c_src - c_new||^2 exceeds
// cand_radius(w_i): such weights are kept without reading the vector.
template <int D>
__global__ __launch_bounds__(kKppThreads) void kpp_update_kernel(
    const float* __restrict__ xs, float* __restrict__ w, uint16_t* __restrict__ src,
    double* __restrict__ bsum, uint32_t* __restrict__ bad, const KppState* __restrict__ st,
    float* __restrict__ cb, uint64_t n, uint32_t K, uint32_t c, uint32_t NB) {
  constexpr int DP = Pad<D>::value;
  constexpr float g = cand_gamma(D);
  __shared__ double part[kKppThreads / 64];
  __shared__ float lo_tab[1024];  // bound of ||c_j - c_new||^2 per earlier seed j
  const uint32_t m = blockIdx.y, b = blockIdx.x;
  const uint64_t lo = (uint64_t)b * kKppBlock;
  const uint64_t hi = lo + kKppBlock < n ? lo + kKppBlock : n;
  float* wm = w + (uint64_t)m * n;
  uint16_t* sm = src + (uint64_t)m * n;
  const float* xm = xs + (uint64_t)m * n * DP;
  // Each thread owns kPer rows: weights and sources are loaded first (they
  // do not depend on the draw, so they are in flight while the new seed and
  // its bounds are read), then only the rows the bound cannot settle load
  // their vectors.
  constexpr uint32_t kPer = kKppBlock / kKppThreads;
  float wv[kPer];
  uint32_t sv[kPer];
  bool need[kPer];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint64_t i = lo + j * kKppThreads + threadIdx.x;
    wv[j] = 0.0f;
    sv[j] = 0;
    if (c > 0 && i < hi) {
      wv[j] = wm[i];
      sv[j] = sm[i];
    }
  }
  if (st[m].err) return;
  const uint32_t chosen = st[m].chosen;
  float cv[D];
  load_padded<D>(xs + ((uint64_t)m * n + chosen) * DP, cv);
  if (b == 0 && threadIdx.x < (uint32_t)D) cb[((uint64_t)m * K + c) * D + threadIdx.x] = cv[threadIdx.x];
  for (uint32_t j = threadIdx.x; j < c; j += blockDim.x) {
    float cj[D];
#pragma unroll
    for (int k = 0; k < D; ++k) cj[k] = cb[((uint64_t)m * K + j) * D + k];
    lo_tab[j] = cand_lower_bound(exact_l2sq<D>(cj, cv), g);
  }
  __syncthreads();
  double acc = 0.0;
  bool invalid = false;
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint64_t i = lo + j * kKppThreads + threadIdx.x;
    need[j] = i < hi && (c == 0 || !cand_cannot_beat(lo_tab[sv[j]], wv[j], g));
  }
  float xv[kPer][D];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint64_t i = lo + j * kKppThreads + threadIdx.x;
    if (need[j]) load_padded<D>(xm + i * DP, xv[j]);
  }
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint64_t i = lo + j * kKppThreads + threadIdx.x;
    if (i >= hi) continue;
    float wi = wv[j];
    if (need[j]) {
      const float d = exact_l2sq<D>(xv[j], cv);
      if (c == 0) {
        wi = d;
        wm[i] = d;
        sm[i] = 0;
      } else if (d < wi) {  // kmeans.zig:134: replace on strict <
        wi = d;
        wm[i] = d;  // unchanged weights are not rewritten
        sm[i] = (uint16_t)c;
      }
    }
    invalid |= !(wi >= 0.0f && wi <= 3.402823466e38f);  // rng.zig:62 NonFinite
    acc += (double)wi;
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
  if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = acc;
  if (invalid) atomicOr(&bad[m], 1u);
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
#pragma unroll
    for (uint32_t q = 0; q < kKppThreads / 64; ++q) t += part[q];
    bsum[(uint64_t)m * NB + b] = t;
  }
}

// Round c draw: one block per subspace.  Checks the weights, draws u, finds
// the candidate with the partial sums and a block-local prefix, and either
// fixes `chosen` or raises `fallback` (always, with exact_only: every draw
// then takes the exact sequential evaluation).
__global__ __launch_bounds__(1024) void kpp_select_kernel(
    const float* __restrict__ w, const double* __restrict__ bsum, uint32_t* __restrict__ bad,
    KppState* __restrict__ st, uint64_t n, uint32_t NB, uint32_t exact_only) {
  __shared__ double s_before, s_total, s_u, s_r, carry;
  __shared__ uint32_t s_block, s_first, s_stop;
  __shared__ double wsum[1024 / 64];
  const uint32_t m = blockIdx.x;
  KppState& S = st[m];
  const double* bm = bsum + (uint64_t)m * NB;
  const uint32_t lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  // Thread 0 alone reads and writes the subspace state; every thread acts
  // on the shared verdicts.
  if (threadIdx.x == 0) {
    s_stop = 1;
    s_first = 0xFFFFFFFFu;
    s_block = NB;
    carry = 0.0;
    if (!S.err) {
      S.fallback = 0;
      if (bad[m])
        S.err = 9;  // NonFinite
      else
        s_stop = 0;
    }
  }
  __syncthreads();
  if (s_stop) return;
  // Total of the block sums, in any order: the bands cover every order.
  double part = 0.0;
  for (uint32_t b = threadIdx.x; b < NB; b += blockDim.x) part += bm[b];
  for (int off = 32; off > 0; off >>= 1) part += __shfl_down(part, off, 64);
  if (lane == 0) wsum[wv] = part;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
    for (uint32_t q = 0; q < 1024 / 64; ++q) tot += wsum[q];
    if (!(tot > 0.0)) {
      S.err = 10;  // AllZero
      s_stop = 1;
    } else {
      S.r = kpp_float64(S.s);
      s_r = S.r;
      s_total = tot;
      s_u = S.r * tot;
    }
  }
  __syncthreads();
  if (s_stop) return;
  // First block whose inclusive prefix exceeds u (a block-wide scan; any
  // rounding: the candidate found below is verified against the bands).
  const double ud = s_u;
  for (uint32_t b0 = 0; b0 < NB; b0 += blockDim.x) {
    const uint32_t b = b0 + threadIdx.x;
    const double x = b < NB ? bm[b] : 0.0;
    double incl = x;
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(incl, off, 64);
      if (lane >= (uint32_t)off) incl += o;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    double before = carry;
    for (uint32_t q = 0; q < wv; ++q) before += wsum[q];
    {
      // the first such block: a wave ballot and one LDS atomic per wave (an
      // atomic from every lane to one address serializes)
      const uint64_t bl = __ballot(b < NB && ud < before + incl);
      if (lane == 0 && bl) atomicMin(&s_block, b + (uint32_t)__ffsll((long long)bl) - 1u);
    }
    __syncthreads();
    if (b == s_block) s_before = before + (incl - x);
    if (threadIdx.x == blockDim.x - 1) carry = before + incl;
    __syncthreads();
    if (s_block != NB) break;
  }
  if (s_block == NB || exact_only) {
    if (threadIdx.x == 0) S.fallback = 1;  // u at or beyond the total: the tail rule decides
    return;
  }
  const double r = s_r;
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
  uint32_t cand = 0xFFFFFFFFu;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    p += v[q];
    const uint64_t i = lo + threadIdx.x * 4 + q;
    if (cand == 0xFFFFFFFFu && i < n && u < p) cand = (uint32_t)(i - lo);
  }
  {
    // indices grow with the lane, so the wave's first candidate is its least
    const uint64_t bl = __ballot(cand != 0xFFFFFFFFu);
    if (bl) {
      const uint32_t c0 = __shfl(cand, __ffsll((long long)bl) - 1, 64);
      if (lane == 0) atomicMin(&s_first, c0);
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

// Exact weightedSample (rng.zig:60-81) for subspaces whose parallel decision
// was inconclusive, one block per such subspace.  The reference folds the
// f64 weights sequentially twice (the total, then the running cum up to the
// first u < cum).  Here the first fold is evaluated exactly in chunks of
// kFoldChunk weights (fold_rules.hpp with an f64 accumulator): all waves
// form the chunk descriptors, then wave 0 applies them in order, recording
// the exact running value before every chunk.  Because the weights are
// non-negative the running value never decreases, so the first u < cum lies
// in the first chunk whose end value exceeds u; wave 0 finds that chunk and
// folds only it term by term from its exact start.
// pre, chunks: [M][nc] scratch (nc = ceil(n / kFoldChunk)).
constexpr uint32_t kKppFallbackThreads = 1024;

// The body, for one weight vector wm[0 .. n) and its state S, run by a whole
// block of kKppFallbackThreads threads (the caller has checked that S needs
// it).  pm, cm: nc = ceil(n / kFoldChunk) entries of scratch.
__device__ __forceinline__ void kpp_fallback_block(const float* __restrict__ wm, uint64_t n, KppState& S,
                                          double* __restrict__ pm, FoldChunk* __restrict__ cm,
                                          uint32_t nc) {
  constexpr uint32_t kWaves = kKppFallbackThreads / kWave;
  __shared__ double wsum[kWaves];
  __shared__ double carry;
  __shared__ __attribute__((aligned(16))) float buf[kFoldChunk];
  const uint32_t lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  // Chunk sums and descriptors, each wave kFallbackBatch chunks at a time
  // (all their loads in flight together).
  constexpr uint32_t kFallbackBatch = 4;
  for (uint32_t j0 = wv * kFallbackBatch; j0 < nc; j0 += kWaves * kFallbackBatch) {
    double cs[kFallbackBatch];
    fold_chunk_sums_wave<kFallbackBatch>(wm, n, j0, nc, cs);
    if (lane == 0)
#pragma unroll
      for (uint32_t b = 0; b < kFallbackBatch; ++b)
        if (j0 + b < nc) pm[j0 + b] = cs[b];
  }
  __syncthreads();
  block_prefix_f64<kKppFallbackThreads>(pm, nc, wsum, &carry);
  for (uint32_t j0 = wv * kFallbackBatch; j0 < nc; j0 += kWaves * kFallbackBatch) {
    double pre[kFallbackBatch];
#pragma unroll
    for (uint32_t b = 0; b < kFallbackBatch; ++b) pre[b] = j0 + b < nc ? pm[j0 + b] : 0.0;
    fold_quantize_chunks_wave<double, kFallbackBatch>(wm, n, j0, nc, pre, cm + j0);
  }
  __syncthreads();
  if (wv != 0) return;
  // Wave 0 only from here: pm[j] becomes the exact value before chunk j.
  const double total = fold_apply_wave<double>(wm, n, cm, nc, buf, pm);
  __threadfence_block();
  const double u = S.r * total;
  uint32_t jf = 0xFFFFFFFFu;
  for (uint32_t j0 = 0; j0 < nc && jf == 0xFFFFFFFFu; j0 += kWave) {
    const uint32_t j = j0 + lane;
    const bool hit = j < nc && u < (j + 1 < nc ? pm[j + 1] : total);
    const uint64_t ballot = __ballot(hit);
    if (ballot) jf = j0 + (uint32_t)__ffsll((long long)ballot) - 1;
  }
  uint64_t found = ~0ull;
  if (jf != 0xFFFFFFFFu) {
    const uint64_t lo = (uint64_t)jf * kFoldChunk;
    const uint32_t len = fold_chunk_len(n, jf);
    wave_lds_sync();
    for (uint32_t t = lane; t < len; t += kWave) buf[t] = wm[lo + t];
    wave_lds_sync();
    double cum = pm[jf];
    for (uint32_t t = 0; t < len; ++t) {
      cum += (double)buf[t];
      if (u < cum) {
        found = lo + t;
        break;
      }
    }
  } else {
    // rng.zig:79-81: no u < cum: the last positive weight (index 0 if none)
    found = 0;
    for (uint64_t b = n; b > 0;) {
      const uint64_t lo = b > kWave ? b - kWave : 0;
      const uint64_t i = lo + lane;
      const uint64_t ballot = __ballot(i < b && wm[i] != 0.0f);
      if (ballot) {
        found = lo + 63 - (uint64_t)__clzll((long long)ballot);
        break;
      }
      b = lo;
    }
  }
  if (lane == 0) {
    S.chosen = (uint32_t)found;
    S.fallback = 0;
  }
}

__global__ __launch_bounds__(kKppFallbackThreads) void kpp_fallback_kernel(
    const float* __restrict__ w, KppState* __restrict__ st, uint64_t n, double* __restrict__ pre,
    FoldChunk* __restrict__ chunks, uint32_t nc) {
  const uint32_t m = blockIdx.x;
  KppState& S = st[m];
  // Every thread reads the flags here; the body rewrites them only at the
  // end, after its block barriers.
  if (S.err || !S.fallback) return;
  kpp_fallback_block(w + (uint64_t)m * n, n, S, pre + (uint64_t)m * nc,
                     chunks + (uint64_t)m * nc, nc);
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
