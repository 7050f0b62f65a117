// tac_kernels.hpp — gfx950 kernels of token-aware clustering
// (src/tac/tac.zig): the per-token Welford spreads (:604-638) and the batch of
// per-token kmeans.fit calls (runOneTokenKmeans :458-513, kmeans.zig:67-242)
// as one ragged engine.  Included once, by tac_gpu.hip, after kmeanspp.hpp.
// Compiled with -ffp-contract=off: every operation rounds on its own.
//
// A problem is one token's fit: rows [off, off + n) of the token-grouped
// matrix G (each token's vectors in ascending input order, as the reference
// gathers them), centroids [goff, goff + k) of the global table.  Rows are
// cut into tiles of rt rows and wcss chunks of kFoldChunk rows that never
// cross a problem.  Problems are listed by k descending, so the problems (and
// tiles) still seeding in k-means++ round c form a prefix of the lists.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pq_kernels.hpp"

namespace tacgpu {

struct TacProblem {
  uint32_t off, n, k, goff;
  uint32_t tile0, ntiles;    // tiles [tile0, tile0 + ntiles) of the tile list
  uint32_t chunk0, nchunks;  // wcss chunks [chunk0, chunk0 + nchunks)
  uint64_t hist0;            // ntiles * k tile-histogram counters
  uint64_t seed;             // p.seed ^ token id
  uint32_t code_bits;        // bits that tell the k codes apart
  uint32_t degenerate;       // k >= n (kmeans.zig:88-104)
  uint32_t range0, nranges;  // scan ranges of kTacScanTiles tiles
  uint64_t rsum0;            // nranges * k range sums
};

struct TacTile {
  uint32_t prob, row0;  // row0: first row of the tile, relative to the problem
};

struct TacChunk {
  uint32_t prob, j;  // j: chunk index within the problem
};

struct TacRange {
  uint32_t prob, r;  // r: scan range index within the problem
};

constexpr uint32_t kTacScanTiles = 32;  // tiles per scan range

// k per problem up to which hist and scatter keep per-code counters in LDS;
// larger problems count and rank codes within the tile's rows instead.
constexpr uint32_t kTacMaxCodes = 12288;
constexpr uint32_t kTacLdsFloats = 12288;  // staged rows: rt * (dim + 1) <= this
// Rows of more than 191 floats: 64-row tiles whose staged rows (and, for the
// assignment, a chunk of centroids) take up to kTacLdsWideFloats of LDS, which
// holds a tile and one centroid up to kTacMaxDim floats a row (the rest of
// the 160 KB is left to the kernels' static LDS).
constexpr uint32_t kTacMaxDim = 512;
constexpr uint32_t kTacLdsWideFloats = 40704;
static_assert(64u * (kTacMaxDim + 1u) + kTacMaxDim <= kTacLdsWideFloats, "a wide tile fits");

// Rows per tile (= threads of the tile kernels) for a dimension; 0 beyond the
// supported range.
__host__ __device__ inline uint32_t tac_rows_per_tile(uint32_t dim) {
  for (uint32_t rt = 128; rt >= 64; rt /= 2)
    if (rt * (dim + 1) <= kTacLdsFloats) return rt;
  return dim <= kTacMaxDim ? 64u : 0u;
}

// LDS floats the tile kernels may take for a dimension: 64 KB up to 191
// floats a row, kTacLdsWideFloats beyond.
__host__ __device__ inline uint32_t tac_tile_lds_floats(uint32_t dim) {
  return 64u * (dim + 1u) <= kTacLdsFloats ? 16384u : kTacLdsWideFloats;
}

// vec.l2sq (src/util/vec.zig:109-175) in the reference's order: dim 2 and 4
// are left folds, dims 64 and 128 accumulate in 4 lanes chunk after chunk and
// reduce ((a0 + a1) + a2) + a3, other dims take the generic path at the
// device's lane count (generic_vec: lanes, lane-order reduce, tail).  DIMC
// fixes the dimension at compile time (0: runtime d).
template <int DIMC>
__device__ __forceinline__ float tac_l2sq(const float* a, const float* b, uint32_t d_rt) {
  const uint32_t d = DIMC ? (uint32_t)DIMC : d_rt;
  if (d == 2) {
    const float d0 = a[0] - b[0];
    const float d1 = a[1] - b[1];
    return d0 * d0 + d1 * d1;
  }
  if (d == 4) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t = a[i] - b[i];
      s = s + t * t;
    }
    return s;
  }
  if (d == 64 || d == 128) {
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < d; c += 4) {
      const float t0 = a[c] - b[c], t1 = a[c + 1] - b[c + 1];
      const float t2 = a[c + 2] - b[c + 2], t3 = a[c + 3] - b[c + 3];
      acc0 = acc0 + t0 * t0;
      acc1 = acc1 + t1 * t1;
      acc2 = acc2 + t2 * t2;
      acc3 = acc3 + t3 * t3;
    }
    return ((acc0 + acc1) + acc2) + acc3;
  }
  return generic_vec<false>(a, b, d);
}

// ---------------------------------------------------------------------------
// Gather: G[q] = vectors[idx[q]] (tac.zig:466-475), one thread per float.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tac_gather_kernel(const float* __restrict__ v,
                                                         const uint32_t* __restrict__ idx,
                                                         float* __restrict__ G, uint64_t rows,
                                                         uint32_t dim) {
  // grid-stride, so rows * dim may exceed what one dispatch's grid can cover
  const uint64_t total = rows * dim, stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; f < total; f += stride) {
    const uint64_t q = f / dim;
    G[f] = v[(uint64_t)idx[q] * dim + f % dim];
  }
}

// ---------------------------------------------------------------------------
// Per-token spread by Welford (tac.zig:611-632): one wave per token, lane =
// dimension (PER dimensions per lane); the trace folds the dimensions in
// order and is divided by the f32 row count.  The f32 count after i rows is
// min(i, 2^24) exactly (count + 1 stops growing at 2^24), so its reciprocal
// comes from a table inv[i - 1] = fl(1 / min(i, 2^24)).
//
// The largest token's serial chain is the whole kernel's time, and a lone
// wave issues about one instruction per four cycles, so the loop is written
// for the fewest instructions per row: rows and reciprocals are loaded
// kTacSpreadBatch at a time into two register buffers used in turn, with no
// bounds test on a full batch (G carries tac_spread_pad_floats of slack and
// the table one batch of extra entries, so a batch may run past the token's
// last row into memory it owns), and the six operations of each row's update
// run without branches.  Only the token's last, partial batch tests the row
// count.  Lanes past dim read neighbouring floats and never store them.
// ---------------------------------------------------------------------------
typedef float tac_floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 tac_bf16x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kTacSpreadBatch = 32;
// Rows per batch of tac_spread_kernel<PER>: two batches of B x PER floats
// stay in registers, so wider rows take shorter batches.
__host__ __device__ constexpr uint32_t tac_spread_batch(int per) {
  return per <= 3 ? kTacSpreadBatch : per <= 6 ? 16u : 8u;
}
constexpr uint32_t kTacSpread64Rows = 64;  // rows per batch of tac_spread64_kernel
constexpr uint32_t kTacInvMax = 1u << 24;

// Rows of slack G and the reciprocal table need past a token's last row: a
// spread kernel's batch may run that far.
constexpr uint32_t kTacSpreadSlackRows = kTacSpread64Rows;

// Floats of slack G needs past its last row for the spread kernels' loads.
__host__ __device__ constexpr size_t tac_spread_pad_floats(uint32_t dim) {
  return (size_t)kTacSpreadSlackRows * dim + 64u * ((dim + 63u) / 64u);
}

__global__ void tac_inv_table_kernel(float* __restrict__ inv, uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  // i + 1 <= 2^24 is exact in f32
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    inv[i] = 1.0f / (float)(i < kTacInvMax ? (uint32_t)i + 1u : kTacInvMax);
}

template <int PER>
__global__ __launch_bounds__(kWave) void tac_spread_kernel(const float* __restrict__ G,
                                                           const uint32_t* __restrict__ offs,
                                                           const float* __restrict__ inv,
                                                           uint32_t dim,
                                                           float* __restrict__ spreads,
                                                           uint64_t j0) {
  extern __shared__ float m2s[];  // [dim]
  const uint64_t j = j0 + blockIdx.x;  // launched in slices of tokens
  const uint32_t lane = threadIdx.x;
  const uint32_t lo = offs[j], hi = offs[j + 1];
  if (hi == lo) {
    if (lane == 0) spreads[j] = 0.0f;
    return;
  }
  float mean[PER], m2[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    mean[u] = 0.0f;
    m2[u] = 0.0f;
  }
  constexpr uint32_t B = tac_spread_batch(PER);
  const float* gp = G + (uint64_t)lo * dim + lane;  // this lane's float of the next batch's row 0
  const float* ip = inv;                            // reciprocal for the next batch's row 0
  auto load = [&](float (&x)[B][PER], float (&v)[B]) {
    const float* p = gp;
#pragma unroll
    for (uint32_t b = 0; b < B; ++b) {
      v[b] = ip[b];
#pragma unroll
      for (int u = 0; u < PER; ++u) x[b][u] = p[64u * u];
      p += dim;
    }
    gp += (uint64_t)B * dim;
    ip += B;
  };
  auto fold_row = [&](const float (&x)[PER], float iv) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const float old = mean[u];
      const float delta = x[u] - old;
      mean[u] = old + delta * iv;
      m2[u] = m2[u] + delta * (x[u] - mean[u]);
    }
  };
  // A full batch issues row b's mean update beside row b - 1's m2 update (the
  // same operations on the same operands as fold_row), so no operation waits
  // on the one issued just before it.
  auto fold = [&](const float (&x)[B][PER], const float (&v)[B]) {
    float dp[PER];  // row b - 1's delta
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      dp[u] = x[0][u] - mean[u];
      mean[u] = mean[u] + dp[u] * v[0];
    }
#pragma unroll
    for (uint32_t b = 1; b < B; ++b) {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        // the scheduling barriers keep each pair together (left to itself
        // the scheduler regroups the three mean operations back to back)
        const float d = x[b][u] - mean[u];
        const float e = x[b - 1][u] - mean[u];  // mean after row b - 1
        __builtin_amdgcn_sched_barrier(0);
        const float t = d * v[b];
        const float q = dp[u] * e;
        __builtin_amdgcn_sched_barrier(0);
        mean[u] = mean[u] + t;
        m2[u] = m2[u] + q;
        __builtin_amdgcn_sched_barrier(0);
        dp[u] = d;
      }
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) m2[u] = m2[u] + dp[u] * (x[B - 1][u] - mean[u]);
  };
  auto fold_tail = [&](const float (&x)[B][PER], const float (&v)[B], uint32_t nb) {
#pragma unroll
    for (uint32_t b = 0; b < B; ++b)
      if (b < nb) fold_row(x[b], v[b]);
  };
  // xa holds the batch at the fold position; the next batch goes to xb while
  // xa is folded, then the roles swap.  A batch is loaded only when the batch
  // before it is whole, so no load passes row hi - 1 + B.
  float xa[B][PER], va[B], xb[B][PER], vb[B];
  uint32_t left = hi - lo;
  load(xa, va);
  for (;;) {
    if (left < B) {
      fold_tail(xa, va, left);
      break;
    }
    load(xb, vb);
    fold(xa, va);
    left -= B;
    if (left < B) {
      fold_tail(xb, vb, left);
      break;
    }
    load(xa, va);
    fold(xb, vb);
    left -= B;
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const uint32_t d = lane + 64u * u;
    if (d < dim) m2s[d] = m2[u];
  }
  __syncthreads();
  if (lane == 0) {
    float trace = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) trace = trace + m2s[d];
    spreads[j] = trace / (float)(hi - lo);
  }
}

// The same spread for 64-float rows, built for memory latency.  A block of
// one folding wave and kTacSpread64Loaders loading waves serves one token:
// the loaders fetch batches of 64 rows (one 16-byte load per lane brings four
// rows, 1 KB per instruction), each a quarter of every batch, four batches
// ahead of the fold, and store a batch into one of two LDS buffers a step
// before it is folded; wave 0 folds the other buffer, one dimension per lane.  One block barrier per
// batch.  The fold is tac_spread_kernel's, operation for operation.  Loads
// past a token's last batch repeat that batch (the same lines, so no new
// memory traffic), which keeps every step's loads unconditional.
constexpr uint32_t kTacSpread64Loaders = 4;
constexpr uint32_t kTacSpread64Threads = (kTacSpread64Loaders + 1) * kWave;

// Spreads of the largest tokens ahead of the grouping (64-float rows).  Up to
// kTacPreSlots tokens with the most rows (at least a threshold) get a slot:
// while the rows reach the device (chunk by chunk, in input order), their
// rows are copied to their places in G, the grouped copy (in input order,
// which is their order in G), and their Welford chains advance over the rows
// copied so far (tac_spread64_kernel in resume mode).  The chain is the same
// chain in the same order, so the spread launch that follows the grouping
// only finishes these tokens from their slots.
constexpr uint32_t kTacPreSlots = 8;
constexpr uint32_t kTacPreNone = 0xFFFFFFFFu;
struct TacPreSlot {
  float mean[64], m2[64];  // the chain's state, one dimension per entry
  uint32_t tok;            // token id, or kTacPreNone for an empty slot
  uint32_t lo;             // the token's first row in G
  uint32_t rows;           // rows copied to G so far
  uint32_t folded;         // rows folded into mean and m2 so far
};

// Rows per token id (ids < nd).  Block (x, y) counts the ids of tile y
// (kTacHistTile ids) among its share of the rows in LDS, then adds its
// non-zero counters to cnt: a hot id takes one device atomic per block, not
// one per row.
constexpr uint32_t kTacHistTile = 16384;
__global__ __launch_bounds__(1024) void tac_id_hist_kernel(const uint32_t* __restrict__ ids,
                                                           uint64_t n, uint32_t nd,
                                                           uint32_t* __restrict__ cnt) {
  __shared__ uint32_t h[kTacHistTile];
  const uint32_t id0 = blockIdx.y * kTacHistTile;
  const uint32_t span = nd - id0 < kTacHistTile ? nd - id0 : kTacHistTile;
  for (uint32_t i = threadIdx.x; i < span; i += blockDim.x) h[i] = 0u;
  __syncthreads();
  const uint64_t per = (n + gridDim.x - 1) / gridDim.x;
  const uint64_t a = (uint64_t)blockIdx.x * per;
  const uint64_t b = a + per < n ? a + per : n;
  for (uint64_t i = a + threadIdx.x; i < b; i += blockDim.x) {
    const uint32_t d = ids[i] - id0;  // ids below id0 wrap past span
    if (d < span) atomicAdd(&h[d], 1u);
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < span; i += blockDim.x)
    if (h[i] != 0u) atomicAdd(&cnt[id0 + i], h[i]);
}

// One block of 1024: the kTacPreSlots tokens with the most rows (ties: the
// lower id), those with at least nmin rows, each with its first row in G
// (the rows of every lower id); the slots' chains start empty.
__global__ __launch_bounds__(1024) void tac_pre_select_kernel(const uint32_t* __restrict__ cnt,
                                                              uint32_t nd, uint32_t nmin,
                                                              TacPreSlot* __restrict__ slots) {
  __shared__ uint64_t s_red[1024 / kWave];
  __shared__ uint32_t s_tok[kTacPreSlots];
  const uint32_t t = threadIdx.x, lane = t % kWave, wv = t / kWave;
  constexpr uint32_t NW = 1024 / kWave;
  for (uint32_t q = 0; q < kTacPreSlots; ++q) {
    // key = rows << 32 | ~id: the largest key is the most rows, then the lowest id
    uint64_t best = 0;
    for (uint32_t j = t; j < nd; j += 1024) {
      bool taken = false;
      for (uint32_t r = 0; r < q; ++r) taken = taken || s_tok[r] == j;
      const uint64_t key = taken ? 0ull : ((uint64_t)cnt[j] << 32) | (uint32_t)~j;
      best = key > best ? key : best;
    }
    for (int o = kWave / 2; o > 0; o >>= 1) {
      const uint64_t v = __shfl_xor(best, o, kWave);
      best = v > best ? v : best;
    }
    if (lane == 0) s_red[wv] = best;
    __syncthreads();
    if (t == 0) {
      uint64_t b = 0;
      for (uint32_t r = 0; r < NW; ++r) b = s_red[r] > b ? s_red[r] : b;
      s_tok[q] = (uint32_t)(b >> 32) >= nmin && nmin > 0 ? ~(uint32_t)b : kTacPreNone;
    }
    __syncthreads();
  }
  for (uint32_t q = 0; q < kTacPreSlots; ++q) {
    const uint32_t tok = s_tok[q];  // block-uniform
    uint64_t part = 0;
    if (tok != kTacPreNone)
      for (uint32_t j = t; j < tok; j += 1024) part += cnt[j];
    for (int o = kWave / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, kWave);
    if (lane == 0) s_red[wv] = part;
    __syncthreads();
    if (t < 64) {
      slots[q].mean[t] = 0.0f;
      slots[q].m2[t] = 0.0f;
    }
    if (t == 0) {
      uint64_t lo = 0;
      for (uint32_t r = 0; r < NW; ++r) lo += s_red[r];
      slots[q].tok = tok;
      slots[q].lo = (uint32_t)lo;
      slots[q].rows = 0;
      slots[q].folded = 0;
    }
    __syncthreads();
  }
}

// The slots' rows among input rows [r0, r1) of V (64 floats each) go to G
// after the rows copied before, in input order, in two launches over
// segments of kTacPreSeg rows (at most kTacPreMaxSegs per range): a count of
// each slot's rows per segment, then each segment's copy at the count of the
// segments before it.  Rows in a segment are taken in four 256-row groups.
constexpr uint32_t kTacPreSeg = 1024;
constexpr uint32_t kTacPreMaxSegs = 128;

__global__ __launch_bounds__(256) void tac_pre_count_kernel(const uint32_t* __restrict__ ids,
                                                            uint32_t r0, uint32_t r1,
                                                            const TacPreSlot* __restrict__ slots,
                                                            uint32_t* __restrict__ segcnt) {
  __shared__ uint32_t s_wc[kTacPreSlots][4];
  const uint32_t seg0 = r0 + blockIdx.x * kTacPreSeg;
  const uint32_t lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  uint32_t id[4];
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    const uint32_t r = seg0 + q * 256u + threadIdx.x;
    id[q] = r < r1 ? ids[r] : kTacPreNone;
  }
#pragma unroll
  for (uint32_t sl = 0; sl < kTacPreSlots; ++sl) {
    const uint32_t tok = slots[sl].tok;
    uint32_t c = 0;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q)
      c += (uint32_t)__popcll(__ballot(tok != kTacPreNone && id[q] == tok));
    if (lane == 0) s_wc[sl][wv] = c;
  }
  __syncthreads();
  if (threadIdx.x < kTacPreSlots) {
    const uint32_t sl = threadIdx.x;
    segcnt[blockIdx.x * kTacPreSlots + sl] = s_wc[sl][0] + s_wc[sl][1] + s_wc[sl][2] + s_wc[sl][3];
  }
}

__global__ __launch_bounds__(256) void tac_pre_copy_kernel(const float* __restrict__ V,
                                                           const uint32_t* __restrict__ ids,
                                                           uint32_t r0, uint32_t r1,
                                                           const TacPreSlot* __restrict__ slots,
                                                           const uint32_t* __restrict__ segcnt,
                                                           float* __restrict__ G) {
  __shared__ uint32_t s_src[kTacPreSeg];
  __shared__ uint64_t s_dst[kTacPreSeg];
  __shared__ uint32_t s_wc[kTacPreSlots][4][4];  // hits per slot, 256-row group, wave
  __shared__ uint32_t s_hc[4][4];                // hits of any slot per group, wave
  __shared__ uint64_t s_at[kTacPreSlots];        // the segment's first place per slot
  const uint32_t seg0 = r0 + blockIdx.x * kTacPreSeg;
  const uint32_t t = threadIdx.x, lane = t % kWave, wv = t / kWave;
  const uint64_t below = (1ull << lane) - 1ull;
  if (t < kTacPreSlots) {
    uint64_t at = (uint64_t)slots[t].lo + slots[t].rows;
    for (uint32_t g = 0; g < blockIdx.x; ++g) at += segcnt[g * kTacPreSlots + t];
    s_at[t] = at;
  }
  // the slot of each of this thread's rows (each row has at most one), its
  // rank among the slot's rows in its wave, and its place among the hits
  int sl_of[4];
  uint32_t rk[4], hp[4];
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    const uint32_t r = seg0 + q * 256u + t;
    const uint32_t id = r < r1 ? ids[r] : kTacPreNone;
    sl_of[q] = -1;
#pragma unroll
    for (uint32_t sl = 0; sl < kTacPreSlots; ++sl) {
      const uint32_t tok = slots[sl].tok;
      if (tok != kTacPreNone && id == tok) sl_of[q] = (int)sl;
    }
  }
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    rk[q] = 0;
#pragma unroll
    for (uint32_t sl = 0; sl < kTacPreSlots; ++sl) {
      const uint64_t b = __ballot(sl_of[q] == (int)sl);
      if (sl_of[q] == (int)sl) rk[q] = (uint32_t)__popcll(b & below);
      if (lane == 0) s_wc[sl][q][wv] = (uint32_t)__popcll(b);
    }
    const uint64_t hb = __ballot(sl_of[q] >= 0);
    hp[q] = (uint32_t)__popcll(hb & below);
    if (lane == 0) s_hc[q][wv] = (uint32_t)__popcll(hb);
  }
  __syncthreads();
  uint32_t m = 0;
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    uint32_t hbefore = m;
    for (uint32_t w = 0; w < wv; ++w) hbefore += s_hc[q][w];
    if (sl_of[q] >= 0) {
      const uint32_t sl = (uint32_t)sl_of[q];
      uint64_t dst = s_at[sl] + rk[q];
      for (uint32_t qq = 0; qq < q; ++qq)
        dst += s_wc[sl][qq][0] + s_wc[sl][qq][1] + s_wc[sl][qq][2] + s_wc[sl][qq][3];
      for (uint32_t w = 0; w < wv; ++w) dst += s_wc[sl][q][w];
      s_src[hbefore + hp[q]] = seg0 + q * 256u + t;
      s_dst[hbefore + hp[q]] = dst;
    }
    m += s_hc[q][0] + s_hc[q][1] + s_hc[q][2] + s_hc[q][3];
  }
  __syncthreads();
  // 16 float4 per row, 16 rows per pass
  for (uint32_t f = t; f < m * 16u; f += 256u) {
    const uint32_t c4 = f % 16u;
    const tac_floatx4 v = reinterpret_cast<const tac_floatx4*>(V + (uint64_t)s_src[f / 16u] * 64u)[c4];
    reinterpret_cast<tac_floatx4*>(G + s_dst[f / 16u] * 64u)[c4] = v;
  }
}

// With resume set, block q advances slot q's chain over the rows the last
// copy added (segcnt: its nseg segment counts; offs, spreads and j0 unused);
// otherwise a token that holds a slot of pre (nullable) only takes its
// finished chain from it.
__global__ __launch_bounds__(kTacSpread64Threads) void tac_spread64_kernel(
    const float* __restrict__ G, const uint32_t* __restrict__ offs,
    const float* __restrict__ inv, float* __restrict__ spreads, uint64_t j0,
    TacPreSlot* __restrict__ pre, uint32_t resume, const uint32_t* __restrict__ segcnt = nullptr,
    uint32_t nseg = 0) {
  constexpr uint32_t R = kTacSpread64Rows;
  constexpr uint32_t GW = R / 4 / kTacSpread64Loaders;  // 16-byte groups per loader per batch
  constexpr int NR = 4;                               // batches in flight per loader
  constexpr uint32_t C = 16;                          // rows read from LDS ahead of the fold
  __shared__ __attribute__((aligned(16))) float xs[2][R * 64];  // row-major batches
  __shared__ __attribute__((aligned(16))) float is[2][R];
  __shared__ float m2s[64];
  const uint64_t j = j0 + blockIdx.x;  // launched in slices of tokens
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  // rows [lo, lo + n) of G fold, their reciprocals from inv[ib]; a finished
  // token skips the fold
  uint32_t lo, n, ib = 0, rows_end = 0;
  bool finished = false;
  float mean = 0.0f, m2 = 0.0f;
  TacPreSlot* ps = nullptr;
  if (resume) {
    ps = pre + blockIdx.x;
    if (ps->tok == kTacPreNone) return;  // block-uniform
    rows_end = ps->rows;
    for (uint32_t g = 0; g < nseg; ++g) rows_end += segcnt[g * kTacPreSlots + blockIdx.x];
    ib = ps->folded;
    lo = ps->lo + ib;
    n = rows_end - ib;
    if (n == 0) {
      if (threadIdx.x == 0) ps->rows = rows_end;  // (= folded)
      return;
    }
    mean = ps->mean[lane];
    m2 = ps->m2[lane];
  } else {
    lo = offs[j];
    const uint32_t hi = offs[j + 1];
    if (hi == lo) {
      if (threadIdx.x == 0) spreads[j] = 0.0f;
      return;
    }
    n = hi - lo;
    if (pre) {
#pragma unroll
      for (uint32_t q = 0; q < kTacPreSlots; ++q)
        if (pre[q].tok == (uint32_t)j && pre[q].folded == n) {  // its chain covered all n rows
          finished = true;
          m2 = pre[q].m2[lane];
        }
    }
  }
  const uint32_t nb = (n + R - 1) / R;
  const tac_floatx4* g4 = reinterpret_cast<const tac_floatx4*>(G + (uint64_t)lo * 64);
  tac_floatx4 buf[NR][GW];
  float ivb[NR];
  // batch k (at most the last) into register slot `slot`: group q of a batch
  // holds rows 4q .. 4q + 3 (lane l: row 4q + l / 16, dimensions 4 (l % 16)
  // ..); G and inv carry a batch of slack, so a partial last batch loads whole
  // loader index (wave 0 only folds); wave-uniform, so the batch and quarter
  // offsets stay scalar and every load and store is a fixed lane offset plus
  // an immediate
  const uint32_t lw = w - 1u;
  const char* gq = reinterpret_cast<const char*>(g4) + (uint64_t)lw * GW * 1024u;
  const uint32_t voff = lane * 16u;
  auto load = [&](int slot, uint32_t k) {
    k = k < nb ? k : nb - 1;
    const char* p = gq + (uint64_t)k * (R * 256u) + voff;
#pragma unroll
    for (uint32_t g = 0; g < GW; ++g)
      buf[slot][g] = *reinterpret_cast<const tac_floatx4*>(p + g * 1024u);
    ivb[slot] = inv[(uint64_t)ib + (uint64_t)k * R + lane];
  };
  auto store = [&](int slot, uint32_t k) {
    char* x = reinterpret_cast<char*>(xs[k & 1u]) + lw * GW * 1024u + voff;
#pragma unroll
    for (uint32_t g = 0; g < GW; ++g)
      *reinterpret_cast<tac_floatx4*>(x + g * 1024u) = buf[slot][g];
    is[k & 1u][lane] = ivb[slot];  // every loader writes the same values
  };
  auto fold = [&](uint32_t k) {
    const float* x = xs[k & 1u];
    const float* iv = is[k & 1u];
    const uint32_t m = n - k * R < R ? n - k * R : R;
    if (m == R) {
      // row b's mean update beside row b - 1's m2 update, as tac_spread_kernel;
      // the next C rows are read from LDS while C rows fold
      float xc[2][C], ic[2][C];
      auto read = [&](int h, uint32_t c0) {
#pragma unroll
        for (uint32_t b = 0; b < C; ++b) xc[h][b] = x[(c0 + b) * 64u + lane];
#pragma unroll
        for (uint32_t q = 0; q < C / 4; ++q) {
          const tac_floatx4 v4 = *reinterpret_cast<const tac_floatx4*>(iv + c0 + 4u * q);
          ic[h][4 * q] = v4.x;
          ic[h][4 * q + 1] = v4.y;
          ic[h][4 * q + 2] = v4.z;
          ic[h][4 * q + 3] = v4.w;
        }
      };
      float xp = 0.0f, dp = 0.0f;
      read(0, 0);
#pragma unroll
      for (uint32_t cc = 0; cc < R / C; ++cc) {
        const int h = (int)(cc & 1u);
        if (cc + 1 < R / C) read(h ^ 1, (cc + 1) * C);
#pragma unroll
        for (uint32_t b = 0; b < C; ++b) {
          const float xb = xc[h][b], ivv = ic[h][b];
          if (cc == 0 && b == 0) {
            dp = xb - mean;
            mean = mean + dp * ivv;
          } else {
            const float d = xb - mean;
            const float e = xp - mean;  // mean after the previous row
            __builtin_amdgcn_sched_barrier(0);
            const float t = d * ivv;
            const float q = dp * e;
            __builtin_amdgcn_sched_barrier(0);
            mean = mean + t;
            m2 = m2 + q;
            __builtin_amdgcn_sched_barrier(0);
            dp = d;
          }
          xp = xb;
        }
      }
      m2 = m2 + dp * (xp - mean);
    } else {
      for (uint32_t b = 0; b < m; ++b) {
        const float xb = x[b * 64u + lane];
        const float old = mean;
        const float delta = xb - old;
        mean = old + delta * iv[b];
        m2 = m2 + delta * (xb - mean);
      }
    }
  };
  // step k: batch k sits in LDS buffer k & 1 and is folded; batches k + 1 ..
  // k + NR - 1 wait in registers; batch k + NR is loaded into the register
  // slot of batch k; batch k + 1 goes to the other LDS buffer
  // The loaders and the folding wave run separate loops with the same
  // number of block barriers (one before step 0, one after each step).
  if (finished) {
    // nothing to fold
  } else if (w > 0) {
#pragma unroll
    for (int q = 0; q < NR; ++q) load(q, (uint32_t)q);
    store(0, 0);
    __syncthreads();
    uint32_t k = 0;
    for (;;) {
#pragma unroll
      for (int sl = 0; sl < NR; ++sl) {
        load(sl, k + NR);
        store((sl + 1) % NR, k + 1);
        __syncthreads();
        if (++k == nb) break;
      }
      if (k == nb) break;
    }
  } else {
    __syncthreads();
    for (uint32_t k = 0; k < nb; ++k) {
      fold(k);
      __syncthreads();
    }
  }
  if (resume) {
    if (w == 0) {
      ps->mean[lane] = mean;
      ps->m2[lane] = m2;
    }
    if (threadIdx.x == 0) {
      ps->rows = rows_end;
      ps->folded = rows_end;
    }
    return;
  }
  if (w == 0) m2s[lane] = m2;
  __syncthreads();
  if (threadIdx.x == 0) {
    float trace = 0.0f;
    for (uint32_t d = 0; d < 64; ++d) trace = trace + m2s[d];
    spreads[j] = trace / (float)n;
  }
}

// ---------------------------------------------------------------------------
// Degenerate problems (k >= n, kmeans.zig:88-104): centroid c = row
// min(c, n - 1), assignment i = i, wcss 0, no iterations.  One block each.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tac_degenerate_kernel(
    const float* __restrict__ G, const TacProblem* __restrict__ probs, uint32_t P,
    float* __restrict__ C, uint32_t* __restrict__ code, float* __restrict__ wcss,
    uint32_t dim) {
  const uint32_t p = blockIdx.x;
  if (p >= P || !probs[p].degenerate) return;
  const TacProblem pr = probs[p];
  for (uint64_t f = threadIdx.x; f < (uint64_t)pr.k * dim; f += blockDim.x) {
    const uint32_t c = (uint32_t)(f / dim), d = (uint32_t)(f % dim);
    const uint32_t src = c < pr.n ? c : pr.n - 1;
    C[((uint64_t)pr.goff + c) * dim + d] = G[((uint64_t)pr.off + src) * dim + d];
  }
  for (uint32_t i = threadIdx.x; i < pr.n; i += blockDim.x) code[pr.off + i] = i;
  if (threadIdx.x == 0) wcss[p] = 0.0f;
}

// Stage rows [row0, row0 + rt) of a problem (zeros past its end) into LDS
// with stride ld; every thread of the block takes part.
// Loads go out U at a time before their stores, so a step waits one round
// trip for U floats rather than one.
__device__ __forceinline__ void tac_stage_rows(const float* __restrict__ G, const TacProblem& pr,
                                               uint32_t row0, uint32_t rt, uint32_t dim,
                                               uint32_t ld, float* xr) {
  constexpr uint32_t U = 16;
  const uint32_t rows = pr.n - row0 < rt ? pr.n - row0 : rt;
  const uint32_t total = rows * dim;
  const float* src = G + ((uint64_t)pr.off + row0) * dim;
  for (uint32_t f0 = threadIdx.x; f0 < total; f0 += U * blockDim.x) {
    float v[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t f = f0 + u * blockDim.x;
      v[u] = f < total ? src[f] : 0.0f;
    }
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
      const uint32_t f = f0 + u * blockDim.x;
      if (f < total) xr[(f / dim) * ld + f % dim] = v[u];
    }
  }
}

// ---------------------------------------------------------------------------
// k-means++ (kmeans.zig:106-136) per problem, with the PRNG seeded from
// p.seed ^ token id.  One launch per round.
//
// Round c runs over the tiles of the problems with k > c (a prefix of the
// tile list).  For c >= 1 each block first draws centroid c from the weights
// the previous round left (weightedSample, rng.zig:57-82); then it writes
// centroid c, sets w = l2sq to it (round 0) or min(w, l2sq) on strict <
// (kmeans.zig:129-135), validates the weights (rng.zig:62) and leaves one f64
// sum per tile.  Every block of a problem makes the same draw from the same
// inputs in the same order, so no block waits for another: the weights, tile
// sums and states of round c - 1 are read from one half of two buffers while
// round c writes the other (KppRound).  The sums are order-free; a candidate
// is kept only when the draw clears the error bands (kpp_decides).  Otherwise
// (rare: the draw lands within rounding of a boundary) the problem stalls:
// its draw of round c stays pending (fallback raised, pad = c), its weights
// and tile sums stay as round c - 1 left them, and later rounds only forward
// its state.  After the last round the host replays the stalled problems from
// the earliest pending round: tac_kpp_exact_round_kernel resolves a pending
// draw exactly and makes that round's update, then this kernel runs the next
// round with `replay` set, where only replaying problems (pad ==
// kKppReplaying) act.  Non-finite weights of round c stamp bad[p] with c
// (atomicMin); a draw fails with NonFinite when a stamp of an earlier round
// is present, so a stamp made while a round runs never changes its draws.
// ---------------------------------------------------------------------------
constexpr uint32_t kKppNoBad = 0xFFFFFFFFu;
// KppState.pad of a problem: 0 in the first pass; the round of its pending
// draw while fallback is raised; kKppReplaying once the exact draw has
// resolved it, for the rest of its rounds.
constexpr uint32_t kKppReplaying = 0xFFFFFFFFu;


// What a round's block needs of its tile and problem, in one load.
struct KppTile {
  uint32_t prob, row0, off, n, goff, tile0, ntiles, pad;
};

struct KppRound {
  const float* w_in;      // weights after round c - 1
  float* w_out;           // weights after round c
  const double* tsum_in;  // tile sums after round c - 1 (one per tile of the list)
  double* tsum_out;
  const KppState* st_in;  // states after the draw of round c - 1 (one per problem)
  KppState* st_out;
};

__global__ void tac_kpp_init_kernel(const TacProblem* __restrict__ probs, uint32_t P,
                                    KppState* __restrict__ st, uint32_t* __restrict__ bad) {
  const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= P) return;
  KppState S;
  uint64_t sm = probs[p].seed;
  for (int q = 0; q < 4; ++q) S.s[q] = kpp_splitmix(&sm);
  S.chosen = probs[p].degenerate ? 0u : (uint32_t)kpp_uint_less_than(S.s, probs[p].n);
  S.r = 0.0;
  S.fallback = 0;
  S.err = 0;
  S.pad = 0;
  st[p] = S;
  bad[p] = kKppNoBad;
}

// Inclusive and exclusive prefix of one f64 per thread over a block of
// rt <= 128 threads, in a fixed order (the exclusive value of thread t + 1 is
// the inclusive value of thread t, bit for bit).  Returns the block total.
// Ends with the block barrier that makes ws reusable only after the caller's
// next barrier.
__device__ inline double kpp_block_scan(double x, uint32_t rt, double* ws, double* incl,
                                        double* excl) {
  const uint32_t lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  double in = x;
  for (int off = 1; off < kWave; off <<= 1) {
    const double o = __shfl_up(in, off, kWave);
    if (lane >= (uint32_t)off) in += o;
  }
  const double up = __shfl_up(in, 1, kWave);
  if (lane == kWave - 1 || threadIdx.x == rt - 1) ws[wv] = in;
  __syncthreads();
  double before = 0.0;
  for (uint32_t q = 0; q < wv; ++q) before += ws[q];
  double total = 0.0;
  for (uint32_t q = 0; q < (rt + kWave - 1) / kWave; ++q) total += ws[q];
  *incl = before + in;
  *excl = lane == 0 ? before : before + up;
  return total;
}

// Row staging for 64-float rows: coalesced 16-byte loads, stored in LDS
// without padding with the 16-byte chunks of row r permuted by r & 15, so
// that a thread reading its own row chunk by chunk hits distinct banks.
__device__ __forceinline__ uint32_t tac_swz64(uint32_t row, uint32_t chunk) {
  return row * 64u + ((chunk ^ (row & 15u)) << 2);
}

template <int DIMC>
__global__ __launch_bounds__(128) void tac_kpp_round_kernel(
    const float* __restrict__ G, KppRound b, uint32_t* __restrict__ bad,
    const KppTile* __restrict__ ktiles, float* __restrict__ C, uint32_t c, uint32_t dim_rt,
    uint32_t exact_every, uint32_t replay) {
  const uint32_t dim = DIMC ? (uint32_t)DIMC : dim_rt;
  extern __shared__ __attribute__((aligned(16))) float tlds[];
  const uint32_t rt = blockDim.x, t = threadIdx.x;
  const uint32_t ld = DIMC == 64 ? 64u : dim + 1;
  // 64-float rows pass through LDS 64 at a time (the block has 128 threads,
  // one row each); other dims stage the whole tile
  float* xr = tlds;
  float* crow = tlds + (DIMC == 64 ? 64u * 64u : rt * ld);  // [dim]
  __shared__ double ws_a[2], ws_b[2], wsum[2], s_before;
  __shared__ uint32_t s_thr, s_tile, s_first, s_chosen;
  const KppTile tl = ktiles[blockIdx.x];
  const uint32_t p = tl.prob;
  const KppTile& pr = tl;
  const uint32_t i = tl.row0 + t;
  const bool row_ok = i < pr.n;
  // Issue every load that does not wait on the draw first: the state, the
  // run of tile sums this thread adds up, the weights and the tile's rows.
  KppState S = b.st_in[p];
  const uint32_t badp = bad[p];
  const uint32_t NB = pr.ntiles;
  const double* tb = b.tsum_in + pr.tile0;
  const uint32_t per = (NB + rt - 1) / rt;
  const uint32_t b0 = t * per < NB ? t * per : NB;
  const uint32_t b1 = b0 + per < NB ? b0 + per : NB;
  constexpr uint32_t kRegTiles = 16;  // runs up to this long stay in registers
  const bool in_regs = per <= kRegTiles;
  double tv[kRegTiles];
  if (c > 0 && in_regs) {
#pragma unroll
    for (uint32_t j = 0; j < kRegTiles; ++j) tv[j] = b0 + j < b1 ? tb[b0 + j] : 0.0;
  }
  const float old = (c > 0 && row_ok) ? b.w_in[pr.off + i] : 0.0f;
  // 64-float rows: coalesced 16-byte loads (chunk t & 15 of rows (t >> 4) +
  // 8 j); rows 0-63 go to LDS at once, rows 64-127 wait in registers
  tac_floatx4 v[16];
  uint32_t nq = 0;
  if (DIMC == 64) {
    const uint32_t rows = pr.n - tl.row0 < 128u ? pr.n - tl.row0 : 128u;
    const tac_floatx4* src =
        reinterpret_cast<const tac_floatx4*>(G + ((uint64_t)pr.off + tl.row0) * 64);
    nq = rows * 16u;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t q = t + (uint32_t)j * 128u;
      v[j] = q < nq ? src[q] : tac_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t q = t + (uint32_t)j * 128u;
      if (q < nq) *reinterpret_cast<tac_floatx4*>(xr + tac_swz64(q >> 4, q & 15u)) = v[j];
    }
  } else {
    const uint32_t rows = pr.n - tl.row0 < rt ? pr.n - tl.row0 : rt;
    const float* src = G + ((uint64_t)pr.off + tl.row0) * dim;
    for (uint32_t f = t; f < rows * dim; f += rt) xr[(f / dim) * ld + f % dim] = src[f];
  }
  if (replay && S.pad != kKppReplaying) return;  // uniform; writes nothing
  if (t == 0) {
    s_thr = 0xFFFFFFFFu;
    s_first = 0xFFFFFFFFu;
    s_tile = pr.ntiles;
    s_chosen = S.chosen;
  }
  // a problem whose draw is pending (an earlier round's) only forwards its state
  const bool draws = c > 0 && !S.err && !S.fallback;
  if (draws) {
    if (badp < c) {
      S.err = 9;  // NonFinite
    } else {
      // total and the tile holding the draw: thread t adds up a contiguous
      // run of the problem's tile sums
      double part = 0.0;
      if (in_regs) {
#pragma unroll
        for (uint32_t j = 0; j < kRegTiles; ++j)
          if (b0 + j < b1) part += tv[j];
      } else {
        for (uint32_t q = b0; q < b1; ++q) part += tb[q];
      }
      double incl, excl;
      const double total = kpp_block_scan(part, rt, ws_a, &incl, &excl);
      if (!(total > 0.0)) {
        S.err = 10;  // AllZero
      } else {
        const double r = kpp_float64(S.s);
        S.r = r;
        const double u = r * total;
        {
          // the first such thread: one ballot per wave, one LDS atomic per wave
          // (an atomic from every lane to one address serializes)
          const uint64_t bl = __ballot(b0 < b1 && u < incl);
          if (t % kWave == 0 && bl) atomicMin(&s_thr, t + (uint32_t)__ffsll((long long)bl) - 1u);
        }
        __syncthreads();
        if (t == s_thr) {
          double run = excl;
          if (in_regs) {
            bool found = false;
#pragma unroll
            for (uint32_t j = 0; j < kRegTiles; ++j) {
              if (!found && b0 + j < b1) {
                const double nx = run + tv[j];
                if (u < nx) {
                  found = true;
                  s_tile = b0 + j;
                  s_before = run;
                }
                run = nx;
              }
            }
          } else {
            for (uint32_t q = b0; q < b1; ++q) {
              const double nx = run + tb[q];
              if (u < nx) {
                s_tile = q;
                s_before = run;
                break;
              }
              run = nx;
            }
          }
        }
        __syncthreads();
        if (s_tile == NB || (exact_every && (c + p) % exact_every == 0)) {
          S.fallback = 1;  // u at or beyond the total: the tail rule decides
        } else {
          // one weight per thread inside the candidate tile (tiles hold rt rows)
          const uint64_t ci = (uint64_t)s_tile * rt + t;
          const double wv = ci < pr.n ? (double)b.w_in[pr.off + ci] : 0.0;
          double wi, we;
          kpp_block_scan(wv, rt, ws_b, &wi, &we);
          const double pi = s_before + wi, pprev = s_before + we;
          {
            const uint64_t bl = __ballot(ci < pr.n && u < pi);
            if (t % kWave == 0 && bl)
              atomicMin(&s_first, t + (uint32_t)__ffsll((long long)bl) - 1u);
          }
          __syncthreads();
          if (s_first == 0xFFFFFFFFu) {
            S.fallback = 1;
          } else {
            if (t == s_first)
              s_chosen = kpp_decides(r, total, pr.n, ci, pprev, pi) ? (uint32_t)ci : 0xFFFFFFFFu;
            __syncthreads();
            if (s_chosen == 0xFFFFFFFFu)
              S.fallback = 1;
            else
              S.chosen = s_chosen;
          }
        }
      }
    }
  }
  if (draws && S.fallback) S.pad = c;  // the draw of round c is pending
  if (t == 0 && tl.row0 == 0) b.st_out[p] = S;  // every round forwards the state
  if (S.err || S.fallback) return;               // uniform over the block
  const float* cg = G + ((uint64_t)pr.off + S.chosen) * dim;
  for (uint32_t d = t; d < dim; d += rt) {
    const float v = cg[d];
    crow[d] = v;
    if (tl.row0 == 0) C[((uint64_t)pr.goff + c) * dim + d] = v;
  }
  __syncthreads();
  double acc = 0.0;
  bool invalid = false;
  float d = 0.0f;
  if (DIMC == 64) {
    // pass 0: rows 0-63, already in LDS; pass 1: rows 64-127 (v[8..15]); wave
    // h reads in pass h
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h) {
        __syncthreads();
#pragma unroll
        for (int j = 8; j < 16; ++j) {
          const uint32_t q = t + (uint32_t)j * 128u;
          if (q < nq)
            *reinterpret_cast<tac_floatx4*>(xr + tac_swz64((q >> 4) - 64u, q & 15u)) = v[j];
        }
        __syncthreads();
      }
      if (t / 64 == (uint32_t)h && row_ok) {
        const uint32_t r = t - 64u * h;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 16; ++j) {
          const tac_floatx4 x = *reinterpret_cast<const tac_floatx4*>(xr + tac_swz64(r, j));
          const tac_floatx4 y = *reinterpret_cast<const tac_floatx4*>(crow + 4 * j);
          const float t0 = x.x - y.x, t1 = x.y - y.y, t2 = x.z - y.z, t3 = x.w - y.w;
          a0 = a0 + t0 * t0;
          a1 = a1 + t1 * t1;
          a2 = a2 + t2 * t2;
          a3 = a3 + t3 * t3;
        }
        d = ((a0 + a1) + a2) + a3;  // tac_l2sq<64>'s order
      }
    }
  } else if (row_ok) {
    d = tac_l2sq<DIMC>(xr + t * ld, crow, dim);
  }
  if (row_ok) {
    const float v = c > 0 ? (d < old ? d : old) : d;
    b.w_out[pr.off + i] = v;
    invalid = !(v >= 0.0f && v <= 3.402823466e38f);
    acc = (double)v;
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
  if (t % 64 == 0) wsum[t / 64] = acc;
  if (__any(invalid) && t % 64 == 0) atomicMin(&bad[p], c);
  __syncthreads();
  if (t == 0) {
    double s = 0.0;
    for (uint32_t q = 0; q < (rt + 63) / 64; ++q) s += wsum[q];
    b.tsum_out[blockIdx.x] = s;
  }
}

// The exact sequential weightedSample for problems whose draw in round c is
// pending (kpp_fallback_block over the weights after round c - 1; the wcss
// chunk scratch of the problem serves as its chunk scratch), followed by
// round c's update of that problem by this one block, which marks the problem
// as replaying.  Only launched in the replay pass; blocks of problems without
// a draw pending in round c return at once.
template <int DIMC>
__global__ __launch_bounds__(kKppFallbackThreads) void tac_kpp_exact_round_kernel(
    const float* __restrict__ G, KppRound b, uint32_t* __restrict__ bad,
    const TacProblem* __restrict__ probs, float* __restrict__ C, double* __restrict__ pre,
    FoldChunk* __restrict__ fchunks, uint32_t c, uint32_t dim_rt, uint32_t rt) {
  const uint32_t dim = DIMC ? (uint32_t)DIMC : dim_rt;
  extern __shared__ __attribute__((aligned(16))) float crow[];  // [dim]
  __shared__ double wpart[kKppFallbackThreads / kWave];
  __shared__ KppState S;  // the draw works on this copy; thread 0 writes it back
  const uint32_t p = blockIdx.x, t = threadIdx.x, lane = t % kWave, wv = t / kWave;
  if (t == 0) S = b.st_out[p];
  __syncthreads();
  if (S.err || !S.fallback || S.pad != c) return;  // uniform over the block
  const TacProblem pr = probs[p];
  kpp_fallback_block(b.w_in + pr.off, pr.n, S, pre + pr.chunk0, fchunks + pr.chunk0,
                     pr.nchunks);
  __syncthreads();
  const uint32_t chosen = S.chosen;
  if (t == 0) {
    S.pad = kKppReplaying;
    b.st_out[p] = S;
  }
  const float* cg = G + ((uint64_t)pr.off + chosen) * dim;
  for (uint32_t d = t; d < dim; d += kKppFallbackThreads) {
    const float v = cg[d];
    crow[d] = v;
    C[((uint64_t)pr.goff + c) * dim + d] = v;
  }
  __syncthreads();
  const uint32_t per_pass = kKppFallbackThreads / rt;  // rt divides the block
  for (uint32_t i0 = 0; i0 < pr.n; i0 += kKppFallbackThreads) {
    const uint32_t i = i0 + t;
    double acc = 0.0;
    bool invalid = false;
    if (i < pr.n) {
      const float d = tac_l2sq<DIMC>(G + ((uint64_t)pr.off + i) * dim, crow, dim);
      const float old = b.w_in[pr.off + i];
      const float v = d < old ? d : old;  // rounds with a draw have c >= 1
      b.w_out[pr.off + i] = v;
      invalid = !(v >= 0.0f && v <= 3.402823466e38f);
      acc = (double)v;
    }
    if (__any(invalid) && lane == 0) atomicMin(&bad[p], c);
    const uint32_t seg = rt < kWave ? rt : kWave;
    for (uint32_t off = seg / 2; off > 0; off >>= 1) acc += __shfl_down(acc, off, kWave);
    const uint32_t tile0 = i0 / rt;
    if (rt < kWave) {
      const uint32_t tile = tile0 + t / rt;
      if (t % rt == 0 && tile < pr.ntiles) b.tsum_out[pr.tile0 + tile] = acc;
    } else {
      if (lane == 0) wpart[wv] = acc;
      __syncthreads();
      const uint32_t wpt = rt / kWave;
      if (t < per_pass && tile0 + t < pr.ntiles) {
        double s = 0.0;
        for (uint32_t q = 0; q < wpt; ++q) s += wpart[t * wpt + q];
        b.tsum_out[pr.tile0 + tile0 + t] = s;
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// Lloyd assignment (kmeans.zig:344-365): per row, vec.argmin over the
// problem's centroids (first index on ties, strict <), min_to_any = that
// distance.  One block per tile; the tile's rows sit in LDS (stride dim + 1),
// centroids pass through LDS in chunks and are read as broadcasts.
// ---------------------------------------------------------------------------
template <int DIMC>
__global__ void tac_assign_kernel(const float* __restrict__ G, const float* __restrict__ C,
                                  const TacProblem* __restrict__ probs,
                                  const TacTile* __restrict__ tiles,
                                  const uint32_t* __restrict__ done, uint32_t* __restrict__ code,
                                  float* __restrict__ e, uint32_t dim_rt, uint32_t chunk_c) {
  const uint32_t dim = DIMC ? (uint32_t)DIMC : dim_rt;
  extern __shared__ __attribute__((aligned(16))) float tlds[];
  const uint32_t rt = blockDim.x, ld = dim + 1;
  float* xr = tlds;             // [rt][ld]
  float* cs = tlds + rt * ld;  // [chunk_c][dim]
  const TacTile tl = tiles[blockIdx.x];
  if (done[tl.prob]) return;
  const TacProblem pr = probs[tl.prob];
  tac_stage_rows(G, pr, tl.row0, rt, dim, ld, xr);
  const float* xrow = xr + threadIdx.x * ld;
  float best = 0.0f;
  uint32_t bi = 0;
  for (uint32_t c0 = 0; c0 < pr.k; c0 += chunk_c) {
    const uint32_t cnt = pr.k - c0 < chunk_c ? pr.k - c0 : chunk_c;
    __syncthreads();
    const float* src = C + ((uint64_t)pr.goff + c0) * dim;
    {
      // up to U loads out before their stores
      constexpr uint32_t U = 8;
      const uint32_t total = cnt * dim;
      for (uint32_t f0 = threadIdx.x; f0 < total; f0 += U * rt) {
        float v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
          const uint32_t f = f0 + u * rt;
          v[u] = f < total ? src[f] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
          const uint32_t f = f0 + u * rt;
          if (f < total) cs[f] = v[u];
        }
      }
    }
    __syncthreads();
    for (uint32_t q = 0; q < cnt; ++q) {
      const float d = tac_l2sq<DIMC>(xrow, cs + q * dim, dim);
      if (c0 + q == 0) {
        best = d;  // vec.argmin starts from values[0]
      } else if (d < best) {
        best = d;
        bi = c0 + q;
      }
    }
  }
  const uint32_t i = tl.row0 + threadIdx.x;
  if (i < pr.n) {
    code[pr.off + i] = bi;
    e[pr.off + i] = best;
  }
}

// ---------------------------------------------------------------------------
// Lloyd assignment for 64-float rows on the matrix cores: the same result as
// tac_assign_kernel, with most of the arithmetic moved to MFMA.
//
// Screen.  s(x, c) = h_c - x.c with h_c = ||c||^2 / 2 (fp32, any order) and
// x.c from eight v_mfma_f32_16x16x32_bf16 per 16 rows x 16 centroids over
// bf16 hi/lo pieces (v_hi = bf16(v), v_lo = bf16(v - v_hi), round to nearest
// even): (x_hi + x_lo) . (c_hi + c_lo) as four exact bf16 products per
// dimension, 256 terms added in fp32 in some order.  For the tame components
// below, |v - v_hi - v_lo| <= 2^-16 |v| + 2^-125, so the products miss x.c by
// at most 2.0001 * 2^-16 ||x|| ||c|| plus underflow, the sum adds gamma_256
// (2^-16) of 1.016 ||x|| ||c||, and h carries gamma_64 of ||c||^2 / 2:
// altogether at most 2^-15 (0.76 ||x||^2 + 0.82 ||c||^2) plus terms below
// 2^-120 (||x|| + ||c||), inside E = Gm (||x||^2 + 2 cmax2) + 1e-35 with
// Gm = 512 u (u = 2^-24) = 2^-15, cmax2 >= ||c||^2 for every centroid of the
// problem, and the addend covering products in the subnormal range (the
// bound the fp32 matrix-core screen this replaced was given).
// Candidates.  The reference distance (tac_l2sq<64>: four 16-term lane sums
// and three adds, g = gamma_20 relative) of the winner c* is at most that of
// the screen's minimum c_m, so s(c*) <= s_min + 2E + 1.01 g ||x - c_m||^2
// and ||x - c_m||^2 <= ||x||^2 + 2 (s_min + E).  tac_screen_threshold
// bounds this with the factors doubled and 1e-30 added, which covers the
// rounding of its own arithmetic.  Every centroid whose screen value is at
// most the threshold gets the reference distance; the lexicographic minimum
// of (distance bits, index) over them is the reference's first-index argmin
// (non-negative finite distances).
// Lanes.  A 16-row group x 16 centroids: lane l feeds row l % 16 and
// centroid l % 16 at dimension 4 s + l / 16 and holds the dot products of
// rows 4 (l / 16) + i, i < 4, with centroid l % 16.  Each lane keeps the two
// smallest screen values of its centroids (those with c % 16 = l % 16) per
// row; when the second is at most the threshold the lane may hold more
// candidates, and every centroid of its class gets the reference distance
// (a row with a NaN screen value gets it for every centroid).  A block whose rows or
// centroids have non-finite, subnormal or huge components (where the bounds
// do not hold) takes tac_assign_kernel's exact search for all its rows.
// One block of 256 work-items per tile of 128 rows; wave w takes rows
// 32 w .. 32 w + 31 as two row groups, four accumulator chains at a time.
// Lane layout of v_mfma_f32_16x16x32_bf16: lane l supplies row (A) or
// centroid (B) l % 16 at k = 8 (l / 16) + i, i < 8, and holds the dot
// products of rows 4 (l / 16) + i, i < 4, with centroid l % 16; MFMA t of a
// tile takes dimensions 32 (t % 2) + k of the pieces (x_hi or x_lo) x (c_hi
// or c_lo) that t / 2 names.  The chunk's centroids sit in LDS as bf16 rows
// [c_hi x 64 | c_lo x 64 | 8 pad], 272 bytes, so the 16 centroids a
// half-wave reads fall in distinct banks.
// ---------------------------------------------------------------------------
// This lane's slot in a shared LDS list when `take` (every lane of the wave
// calls it): the wave's ballot, one atomic add by its first taking lane, and
// the rank among the taking lanes below.
__device__ __forceinline__ uint32_t tac_wave_append(bool take, uint32_t* counter) {
  const uint64_t bl = __ballot(take);
  const uint32_t lane = threadIdx.x % kWave;
  uint32_t base = 0;
  if (bl) {
    const int leader = __ffsll((long long)bl) - 1;
    if ((int)lane == leader) base = atomicAdd(counter, (uint32_t)__popcll(bl));
    base = __shfl(base, leader, kWave);
  }
  const uint64_t below = bl & ((1ull << lane) - 1ull);
  return base + (uint32_t)__popcll(below);
}

constexpr uint32_t kTacMfmaRows = 128;     // rows per tile (tac_rows_per_tile(64))
constexpr uint32_t kTacMfmaThreads = 256;
constexpr uint32_t kTacMfmaChunk = 128;    // centroids staged in LDS at a time
constexpr uint32_t kTacMfmaLd = 65;        // LDS row stride (floats)
constexpr uint32_t kTacMfmaLd16 = 136;     // LDS row stride of the bf16 centroid pieces

// Components for which the screen's bounds hold: finite, |v| < 1e18 and not
// subnormal.
__device__ __forceinline__ bool tac_screen_tame(float v) {
  const float a = fabsf(v);
  return a < 1e18f && (a == 0.0f || a >= 1.17549435e-38f);
}

__device__ __forceinline__ float tac_screen_threshold(float s_min, float x2, float cmax2) {
  constexpr float u = 5.9604644775390625e-8f;
  const float E = 512.0f * u * (x2 + 2.0f * cmax2) + 1e-35f;
  return s_min + 2.0f * E + 2.0f * (32.0f * u) * (x2 + 2.0f * fabsf(s_min) + 2.0f * E) + 1e-30f;
}

// Per Lloyd iteration, before the assignment: h[c] = ||c||^2 / 2 for every
// centroid of an unfinished problem, NaN when a component breaks
// tac_screen_tame (the assignment then takes the exact search).
__global__ __launch_bounds__(256) void tac_cnorm_kernel(const float* __restrict__ C,
                                                        const uint32_t* __restrict__ cprob,
                                                        const uint32_t* __restrict__ done,
                                                        uint32_t K, float* __restrict__ h) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= K) return;
  if (done[cprob[c]]) return;
  const float4* row = reinterpret_cast<const float4*>(C + (uint64_t)c * 64);
  float n = 0.0f;
  bool tame = true;
#pragma unroll 4
  for (int q = 0; q < 16; ++q) {
    const float4 v = row[q];
    tame = tame && tac_screen_tame(v.x) && tac_screen_tame(v.y) && tac_screen_tame(v.z) &&
           tac_screen_tame(v.w);
    n = n + v.x * v.x;
    n = n + v.y * v.y;
    n = n + v.z * v.z;
    n = n + v.w * v.w;
  }
  h[c] = tame ? 0.5f * n : __builtin_nanf("");
}


__global__ __launch_bounds__(kTacMfmaThreads) __attribute__((amdgpu_waves_per_eu(2))) void tac_assign_mfma_kernel(
    const float* __restrict__ G, const float* __restrict__ C, const float* __restrict__ h,
    const TacProblem* __restrict__ probs, const TacTile* __restrict__ tiles,
    const uint32_t* __restrict__ done, uint32_t* __restrict__ code, float* __restrict__ e) {
  constexpr uint32_t R = kTacMfmaRows, LD = kTacMfmaLd, CH = kTacMfmaChunk;
  __shared__ float xr[R * LD];
  // the chunk's centroids: bf16 pieces for the screen, fp32 rows for the
  // exact search (which restages them)
  constexpr uint32_t kCsBytes = CH * LD * 4 > CH * kTacMfmaLd16 * 2 ? CH * LD * 4
                                                                    : CH * kTacMfmaLd16 * 2;
  __shared__ __attribute__((aligned(16))) uint8_t cbuf[kCsBytes];
  float* cs = reinterpret_cast<float*>(cbuf);
  __bf16* cb16 = reinterpret_cast<__bf16*>(cbuf);
  __shared__ float hs[CH];
  __shared__ float x2s[R];
  __shared__ unsigned long long rowkey[R];
  // (row, centroid) candidates from the front; (row, column class) entries
  // from the back: a row's lane contributes at most one of the two
  __shared__ uint32_t queue[R * 16];
  __shared__ uint32_t full[R];  // rows whose screen values are not all numbers
  __shared__ uint32_t qn, cn, nfull, exact, hmax;
  const TacTile tl = tiles[blockIdx.x];
  if (done[tl.prob]) return;
  const TacProblem pr = probs[tl.prob];
  const uint32_t t = threadIdx.x, lane = t % 64, w = t / 64, li = lane % 16, lq = lane / 16;
  const uint32_t rows = pr.n - tl.row0 < R ? pr.n - tl.row0 : R;
  if (t == 0) {
    qn = 0;
    cn = 0;
    nfull = 0;
    exact = 0;
    hmax = 0;  // bits of the largest h of the problem (NaN: an untame centroid)
    // the candidate queue holds 16-bit centroid indices
    if (pr.k > 0xFFFFu) exact = 1;
  }
  {
    // the tile's rows: every 16-byte load issued before the first is used
    // (a load-store loop waited a round trip per step: 5-12 us per tile)
    constexpr uint32_t Q = R * 16 / kTacMfmaThreads;  // 16-byte pieces per work-item
    const tac_floatx4* src =
        reinterpret_cast<const tac_floatx4*>(G + ((uint64_t)pr.off + tl.row0) * 64);
    const uint32_t nq = rows * 16u;
    tac_floatx4 v4[Q];
#pragma unroll
    for (uint32_t j = 0; j < Q; ++j) {
      const uint32_t q = t + j * kTacMfmaThreads;
      v4[j] = q < nq ? src[q] : tac_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (uint32_t j = 0; j < Q; ++j) {
      const uint32_t q = t + j * kTacMfmaThreads;
      if (q < nq) {
        float* d = xr + (q >> 4) * LD + 4u * (q & 15u);
        d[0] = v4[j].x;
        d[1] = v4[j].y;
        d[2] = v4[j].z;
        d[3] = v4[j].w;
      }
    }
  }
  __syncthreads();
  if (t < R) {
    float x2 = 0.0f;
    bool tame = true;
    if (t < rows) {
      for (int d = 0; d < 64; ++d) {
        const float v = xr[t * LD + d];
        tame = tame && tac_screen_tame(v);
        x2 = x2 + v * v;
      }
      if (!tame) atomicOr(&exact, 1u);
    }
    x2s[t] = x2;
    rowkey[t] = ~0ull;
  }
  __syncthreads();
  const float* Cp = C + (uint64_t)pr.goff * 64;
  if (!exact) {
    // A operands of the wave's two row groups (rows past the tile read 0):
    // the hi and lo pieces of dimensions 32 dh + 8 lq + i.
    tac_bf16x8 xh[2][2], xl[2][2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const uint32_t r = 32 * w + 16 * g + li;
#pragma unroll
      for (int dh = 0; dh < 2; ++dh)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = r < rows ? xr[r * LD + 32 * dh + 8 * lq + i] : 0.0f;
          const __bf16 hi = (__bf16)v;
          xh[g][dh][i] = hi;
          xl[g][dh][i] = (__bf16)(v - (float)hi);
        }
    }
    float b1[2][4], b2[2][4];
    uint32_t i1[2][4], i2[2][4];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        b1[g][v] = __builtin_inff();
        b2[g][v] = __builtin_inff();
        i1[g][v] = 0;
        i2[g][v] = 0;
      }
    // Chunks of CH centroids pass through LDS; each work-item holds its
    // four runs of 8 floats (and h) of the next chunk in registers while the
    // current one is worked on, and stores them as bf16 pieces.
    constexpr uint32_t PF = CH * 64 / 8 / kTacMfmaThreads;  // runs of 8 floats
    tac_floatx4 pf[PF][2];
    float ph = __builtin_inff();
    auto fetch = [&](uint32_t c0) {
      const uint32_t cnt = pr.k - c0 < CH ? pr.k - c0 : CH;
#pragma unroll
      for (uint32_t j = 0; j < PF; ++j) {
        const uint32_t f = t + j * kTacMfmaThreads, cc = f / 8;
        const tac_floatx4* src =
            reinterpret_cast<const tac_floatx4*>(Cp + (uint64_t)c0 * 64 + 8ull * f);
        pf[j][0] = cc < cnt ? src[0] : tac_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        pf[j][1] = cc < cnt ? src[1] : tac_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      if (t < CH) ph = t < cnt ? h[pr.goff + c0 + t] : __builtin_inff();
    };
    fetch(0);
    for (uint32_t c0 = 0; c0 < pr.k; c0 += CH) {
      const uint32_t cnt = pr.k - c0 < CH ? pr.k - c0 : CH;
      __syncthreads();
#pragma unroll
      for (uint32_t j = 0; j < PF; ++j) {
        const uint32_t f = t + j * kTacMfmaThreads, cc = f / 8, d0 = 8 * (f % 8);
        tac_bf16x8 hi8, lo8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = pf[j][i / 4][i % 4];
          const __bf16 hi = (__bf16)v;
          hi8[i] = hi;
          lo8[i] = (__bf16)(v - (float)hi);
        }
        *reinterpret_cast<tac_bf16x8*>(cb16 + cc * kTacMfmaLd16 + d0) = hi8;
        *reinterpret_cast<tac_bf16x8*>(cb16 + cc * kTacMfmaLd16 + 64 + d0) = lo8;
      }
      if (t < CH) {
        hs[t] = ph;
        // NaN bits exceed every finite value's, so a NaN h shows in hmax.
        // hmax only grows, so a value at or below what it already holds
        // cannot change it: only the larger ones take the (serializing)
        // atomic, after the first chunk few do.
        const uint32_t hb = __float_as_uint(ph) & 0x7FFFFFFFu;
        if (t < cnt && hb > hmax) atomicMax(&hmax, hb);
      }
      __syncthreads();
      if (c0 + CH < pr.k) fetch(c0 + CH);
      // Two centroid groups at a time: four independent accumulator chains
      // (2 row groups x 2 centroid groups) keep the matrix core busy.  A
      // group past the chunk's centroids reads the padding (h = inf).
      for (uint32_t cg = 0; cg < CH / 16 && cg * 16 < cnt; cg += 2) {
        tac_bf16x8 ch[2][2], cl[2][2];
        float hv[2];
        uint32_t cidx[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t cc = (cg + j) * 16 + li;
#pragma unroll
          for (int dh = 0; dh < 2; ++dh) {
            const __bf16* row = cb16 + cc * kTacMfmaLd16 + 32 * dh + 8 * lq;
            ch[j][dh] = *reinterpret_cast<const tac_bf16x8*>(row);
            cl[j][dh] = *reinterpret_cast<const tac_bf16x8*>(row + 64);
          }
          hv[j] = hs[cc];
          cidx[j] = c0 + cc;
        }
        tac_floatx4 acc[2][2];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[g][j] = tac_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int dh = 0; dh < 2; ++dh)
#pragma unroll
          for (int pc = 0; pc < 4; ++pc)
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
              for (int j = 0; j < 2; ++j)
                acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    pc < 2 ? xh[g][dh] : xl[g][dh], pc % 2 == 0 ? ch[j][dh] : cl[j][dh],
                    acc[g][j], 0, 0, 0);
        // Two smallest screen values per (row group, row) without branches;
        // centroids arrive in ascending index order.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const float sv = hv[j] - acc[g][j][v];
              const bool lt1 = sv < b1[g][v], lt2 = sv < b2[g][v];
              b2[g][v] = lt1 ? b1[g][v] : (lt2 ? sv : b2[g][v]);
              i2[g][v] = lt1 ? i1[g][v] : (lt2 ? cidx[j] : i2[g][v]);
              b1[g][v] = lt1 ? sv : b1[g][v];
              i1[g][v] = lt1 ? cidx[j] : i1[g][v];
            }
      }
    }
    if (hmax >= 0x7F800000u) exact = 1;  // an untame centroid (uniform: read after a barrier)
    const float cmax2 = 2.0f * __uint_as_float(hmax);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float m = b1[g][v];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) m = fminf(m, __shfl_xor(m, off, 64));
        const uint32_t r = 32 * w + 16 * g + 4 * lq + v;
        const float thr = tac_screen_threshold(m, x2s[r], cmax2);
        // A NaN screen value (or threshold) cannot occur with tame inputs;
        // it sends the row to the full search all the same.  The row's 16
        // lanes agree through the reduction, and lane 16 q lists it.
        const bool over = !(m <= thr);
        // This lane sees the centroids of its column class li (c % 16 == li)
        // only, and keeps their two smallest screen values.  With the second
        // above the threshold, its only possible candidate is the first;
        // with the second at or below it the class may hold more, and every
        // centroid of the class gets the reference distance.  Other classes
        // are settled by their own lanes.  List slots by a wave ballot and
        // one LDS atomic per wave (lanes adding to one counter one by one
        // serialize).
        const bool cls = r < rows && !over && b2[g][v] <= thr;
        const bool cand = r < rows && !over && !cls && b1[g][v] <= thr;
        const uint32_t qs = tac_wave_append(cand, &qn);
        if (cand) queue[qs] = (r << 16) | i1[g][v];
        const uint32_t cs_ = tac_wave_append(cls, &cn);
        if (cls) queue[R * 16 - 1 - cs_] = (r << 16) | li;
        const bool fr = r < rows && li == 0 && over;
        const uint32_t fs = tac_wave_append(fr, &nfull);
        if (fr) full[fs] = r;
      }
    __syncthreads();
    if (!exact) {
      for (uint32_t q = t; q < qn; q += kTacMfmaThreads) {
        const uint32_t r = queue[q] >> 16, c = queue[q] & 0xFFFFu;
        const float d = tac_l2sq<64>(xr + r * LD, Cp + (uint64_t)c * 64, 64);
        atomicMin(&rowkey[r], ((unsigned long long)__float_as_uint(d) << 32) | c);
      }
      // Column classes: per = ceil(k / 16) centroids each, the work-items
      // over all (entry, centroid) pairs.
      const uint32_t per = (pr.k + 15) / 16;
      for (uint32_t q = t; q < cn * per; q += kTacMfmaThreads) {
        const uint32_t ent = queue[R * 16 - 1 - q / per];
        const uint32_t r = ent >> 16, c = (ent & 15u) + 16u * (q % per);
        if (c < pr.k) {
          const float d = tac_l2sq<64>(xr + r * LD, Cp + (uint64_t)c * 64, 64);
          atomicMin(&rowkey[r], ((unsigned long long)__float_as_uint(d) << 32) | c);
        }
      }
      // Rows with a NaN screen value: every centroid, the block's
      // work-items side by side.
      // (each work-item keeps its own minimum, the wave reduces it, and one
      // LDS atomic per wave and row merges them)
      for (uint32_t j = 0; j < nfull; ++j) {
        const uint32_t r = full[j];
        unsigned long long best = ~0ull;
        for (uint32_t c = t; c < pr.k; c += kTacMfmaThreads) {
          const float d = tac_l2sq<64>(xr + r * LD, Cp + (uint64_t)c * 64, 64);
          const unsigned long long key = ((unsigned long long)__float_as_uint(d) << 32) | c;
          best = key < best ? key : best;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const unsigned long long o = __shfl_xor(best, off, 64);
          best = o < best ? o : best;
        }
        if (lane == 0) atomicMin(&rowkey[r], best);
      }
      __syncthreads();
      if (t < rows) {
        const unsigned long long k = rowkey[t];
        code[pr.off + tl.row0 + t] = (uint32_t)k;
        e[pr.off + tl.row0 + t] = __uint_as_float((uint32_t)(k >> 32));
      }
      return;
    }
  }
  // The exact search of tac_assign_kernel: vec.argmin from values[0], strict <.
  float best = 0.0f;
  uint32_t bi = 0;
  for (uint32_t c0 = 0; c0 < pr.k; c0 += CH) {
    const uint32_t cnt = pr.k - c0 < CH ? pr.k - c0 : CH;
    __syncthreads();
    for (uint32_t f = t; f < cnt * 64; f += kTacMfmaThreads)
      cs[(f / 64) * LD + f % 64] = Cp[(uint64_t)c0 * 64 + f];
    __syncthreads();
    if (t < rows)
      for (uint32_t q = 0; q < cnt; ++q) {
        const float d = tac_l2sq<64>(xr + t * LD, cs + q * LD, 64);
        if (c0 + q == 0) {
          best = d;
        } else if (d < best) {
          best = d;
          bi = c0 + q;
        }
      }
  }
  if (t < rows) {
    code[pr.off + tl.row0 + t] = bi;
    e[pr.off + tl.row0 + t] = best;
  }
}

// ---------------------------------------------------------------------------
// Stable grouping of each problem's rows by code, so that every cluster's
// members are folded in ascending row order (kmeans.zig:177-184).
// Step 1: tile histograms hist[hist0 + t * k + c].
// ---------------------------------------------------------------------------
__global__ void tac_hist_kernel(const uint32_t* __restrict__ code,
                                const TacProblem* __restrict__ probs,
                                const TacTile* __restrict__ tiles,
                                const uint32_t* __restrict__ done, uint32_t* __restrict__ hist) {
  extern __shared__ uint32_t hcnt[];  // [k], or the tile's codes when k > kTacMaxCodes
  const TacTile tl = tiles[blockIdx.x];
  if (done[tl.prob]) return;
  const TacProblem pr = probs[tl.prob];
  if (pr.k > kTacMaxCodes) {
    // The tile's row of counters is cleared, then the first row of each code
    // in the tile writes that code's count.
    uint32_t* out = hist + pr.hist0 + (uint64_t)(blockIdx.x - pr.tile0) * pr.k;
    const uint32_t i = tl.row0 + threadIdx.x;
    hcnt[threadIdx.x] = i < pr.n ? code[pr.off + i] : 0xFFFFFFFFu;
    for (uint32_t c = threadIdx.x; c < pr.k; c += blockDim.x) out[c] = 0;
    __syncthreads();
    const uint32_t cd = hcnt[threadIdx.x];
    if (cd == 0xFFFFFFFFu) return;
    for (uint32_t j = 0; j < threadIdx.x; ++j)
      if (hcnt[j] == cd) return;
    uint32_t cnt = 0;
    for (uint32_t j = threadIdx.x; j < blockDim.x; ++j) cnt += hcnt[j] == cd ? 1u : 0u;
    out[cd] = cnt;
    return;
  }
  for (uint32_t c = threadIdx.x; c < pr.k; c += blockDim.x) hcnt[c] = 0;
  __syncthreads();
  const uint32_t i = tl.row0 + threadIdx.x;
  if (i < pr.n) atomicAdd(&hcnt[code[pr.off + i]], 1u);
  __syncthreads();
  uint32_t* out = hist + pr.hist0 + (uint64_t)(blockIdx.x - pr.tile0) * pr.k;
  for (uint32_t c = threadIdx.x; c < pr.k; c += blockDim.x) out[c] = hcnt[c];
}

// Step 2: every code's tile counts become exclusive offsets over the tiles
// (in place); cluster sizes go to counts and cluster starts (relative to the
// problem's first row) to start.  A problem's tiles split into ranges of
// kTacScanTiles: tac_scan_partial_kernel sums each range per code,
// tac_scan_apply_kernel adds the ranges before its own and rewrites its
// tiles; range 0 also writes counts and starts.  One block per range.
__global__ __launch_bounds__(256) void tac_scan_partial_kernel(
    const uint32_t* __restrict__ hist, const TacProblem* __restrict__ probs,
    const TacRange* __restrict__ ranges, const uint32_t* __restrict__ done,
    uint32_t* __restrict__ rsum) {
  const TacRange rg = ranges[blockIdx.x];
  if (done[rg.prob]) return;
  const TacProblem pr = probs[rg.prob];
  const uint32_t t0 = rg.r * kTacScanTiles;
  const uint32_t t1 = t0 + kTacScanTiles < pr.ntiles ? t0 + kTacScanTiles : pr.ntiles;
  for (uint32_t c = threadIdx.x; c < pr.k; c += blockDim.x) {
    const uint32_t* h = hist + pr.hist0 + c;
    uint32_t sum = 0;
    for (uint32_t t = t0; t < t1; ++t) sum += h[(uint64_t)t * pr.k];
    rsum[pr.rsum0 + (uint64_t)rg.r * pr.k + c] = sum;
  }
}

__global__ __launch_bounds__(256) void tac_scan_apply_kernel(
    uint32_t* __restrict__ hist, const TacProblem* __restrict__ probs,
    const TacRange* __restrict__ ranges, const uint32_t* __restrict__ done,
    const uint32_t* __restrict__ rsum, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ start) {
  __shared__ uint32_t wsum[256 / kWave];
  __shared__ uint32_t carry;
  const TacRange rg = ranges[blockIdx.x];
  if (done[rg.prob]) return;
  const TacProblem pr = probs[rg.prob];
  const uint32_t t0 = rg.r * kTacScanTiles;
  const uint32_t t1 = t0 + kTacScanTiles < pr.ntiles ? t0 + kTacScanTiles : pr.ntiles;
  const uint32_t* rs = rsum + pr.rsum0;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (uint32_t c0 = 0; c0 < pr.k; c0 += blockDim.x) {
    const uint32_t c = c0 + threadIdx.x;
    uint32_t total = 0;
    if (c < pr.k) {
      uint32_t run = 0;
      for (uint32_t r = 0; r < rg.r; ++r) run += rs[(uint64_t)r * pr.k + c];
      uint32_t* h = hist + pr.hist0 + c;
      for (uint32_t t = t0; t < t1; ++t) {
        const uint32_t v = h[(uint64_t)t * pr.k];
        h[(uint64_t)t * pr.k] = run;
        run += v;
      }
      if (rg.r == 0) {
        for (uint32_t r = 0; r < pr.nranges; ++r) total += rs[(uint64_t)r * pr.k + c];
        counts[pr.goff + c] = total;
      }
    }
    if (rg.r == 0) {  // uniform over the block
      const uint32_t ex = block_exclusive_scan(total, wsum);
      if (c < pr.k) start[pr.goff + c] = carry + ex;
      __syncthreads();
      if (threadIdx.x == blockDim.x - 1) carry += ex + total;
      __syncthreads();
    }
  }
}

// Step 3: stable scatter of row indices.  The tile's waves go in row order;
// inside a wave equal codes are ranked with ballots (a match on every code
// bit).  sorted[off + start[c] + tile offset + rank] = absolute row.
__global__ void tac_scatter_kernel(const uint32_t* __restrict__ code,
                                   const uint32_t* __restrict__ hist,
                                   const uint32_t* __restrict__ start,
                                   const TacProblem* __restrict__ probs,
                                   const TacTile* __restrict__ tiles,
                                   const uint32_t* __restrict__ done,
                                   uint32_t* __restrict__ sorted) {
  extern __shared__ uint32_t run[];  // [k], or the tile's codes when k > kTacMaxCodes
  const TacTile tl = tiles[blockIdx.x];
  if (done[tl.prob]) return;
  const TacProblem pr = probs[tl.prob];
  const uint32_t* hm = hist + pr.hist0 + (uint64_t)(blockIdx.x - pr.tile0) * pr.k;
  const uint32_t i = tl.row0 + threadIdx.x;
  const bool valid = i < pr.n;
  const uint32_t cd = valid ? code[pr.off + i] : 0u;
  if (pr.k > kTacMaxCodes) {
    // rank = earlier rows of the tile with the same code
    run[threadIdx.x] = valid ? cd : 0xFFFFFFFFu;
    __syncthreads();
    if (!valid) return;
    uint32_t rank = 0;
    for (uint32_t j = 0; j < threadIdx.x; ++j) rank += run[j] == cd ? 1u : 0u;
    sorted[pr.off + start[pr.goff + cd] + hm[cd] + rank] = pr.off + i;
    return;
  }
  for (uint32_t c = threadIdx.x; c < pr.k; c += blockDim.x) run[c] = start[pr.goff + c] + hm[c];
  const uint32_t lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const uint32_t nw = (blockDim.x + kWave - 1) / kWave;
  for (uint32_t r = 0; r < nw; ++r) {
    __syncthreads();
    if (wv == r) {
      uint64_t match = __ballot(valid);
      for (uint32_t b = 0; b < pr.code_bits; ++b) {
        const bool bit = (cd >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        match &= bit ? bal : ~bal;
      }
      const uint32_t rank = __popcll(match & lt_mask);
      const uint32_t total = __popcll(match);
      uint32_t pos = 0;
      if (valid) pos = run[cd] + rank;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      if (valid && rank == total - 1) run[cd] = pos + 1;
      if (valid) sorted[pr.off + pos] = pr.off + i;
    }
  }
}

// ---------------------------------------------------------------------------
// Cluster sums and update (kmeans.zig:177-198): one wave per global cluster,
// lane = dimension (PER dimensions per lane), members folded in ascending row
// order from 0; centroid = sum * fl(1 / fl(count)).  Empty clusters are left
// to the reseed kernel.  Member rows are loaded tac_fold_batch(PER) at a time
// (one member per lane for dim <= 64, so a large cluster's chain waits on one
// gather per 64 members), and the next batch's row indices are read while
// the current batch is added.  Only the last, partial batch tests members.
// ---------------------------------------------------------------------------
// Clusters of at least kTacFoldBig members (64-float rows) are folded by
// tac_fold_big_kernel from a list the wave kernel builds (big[0] = count).
constexpr uint32_t kTacFoldBig = 512;

__host__ __device__ constexpr uint32_t tac_fold_batch(int per) { return per == 1 ? 64u : per == 2 ? 32u : 16u; }

template <int PER>
__global__ __launch_bounds__(256) void tac_fold_kernel(
    const float* __restrict__ G, const uint32_t* __restrict__ sorted,
    const uint32_t* __restrict__ counts, const uint32_t* __restrict__ start,
    const uint32_t* __restrict__ cprob, const TacProblem* __restrict__ probs,
    const uint32_t* __restrict__ done, float* __restrict__ C, uint32_t kappa, uint32_t dim,
    uint32_t* __restrict__ big) {
  constexpr uint32_t kTacFoldBatch = tac_fold_batch(PER);
  const uint32_t g = blockIdx.x * (256 / kWave) + threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (g >= kappa) return;
  const uint32_t p = cprob[g];
  if (done[p]) return;
  const uint32_t cnt = counts[g];
  if (cnt == 0) return;
  if (big != nullptr && cnt >= kTacFoldBig) {  // left to tac_fold_big_kernel
    if (lane == 0) big[1 + atomicAdd(&big[0], 1u)] = g;
    return;
  }
  const uint32_t* mem = sorted + probs[p].off + start[g];
  float s[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) s[u] = 0.0f;
  // lane b < kTacFoldBatch holds member index b of the current batch
  uint32_t idx = lane < kTacFoldBatch && lane < cnt ? mem[lane] : 0u;
  const float* gl = G + lane;
  for (uint32_t q0 = 0; q0 < cnt; q0 += kTacFoldBatch) {
    const uint32_t nb = cnt - q0 < kTacFoldBatch ? cnt - q0 : kTacFoldBatch;
    float v[kTacFoldBatch][PER];
    if (nb == kTacFoldBatch) {
      // a whole batch: no per-member tests, the row index read into a scalar
      // register.  Lanes past dim read the next row's floats (G carries at
      // least 64 * PER floats of slack) and never store their sums.
#pragma unroll
      for (uint32_t b = 0; b < kTacFoldBatch; ++b) {
        const uint32_t row = __builtin_amdgcn_readlane(idx, (int)b);
        const float* rp = gl + (uint64_t)row * dim;
#pragma unroll
        for (int u = 0; u < PER; ++u) v[b][u] = rp[kWave * u];
      }
      const uint32_t nq = q0 + kTacFoldBatch + lane;
      idx = lane < kTacFoldBatch && nq < cnt ? mem[nq] : 0u;
#pragma unroll
      for (uint32_t b = 0; b < kTacFoldBatch; ++b)
#pragma unroll
        for (int u = 0; u < PER; ++u) s[u] = s[u] + v[b][u];
      continue;
    }
#pragma unroll
    for (uint32_t b = 0; b < kTacFoldBatch; ++b) {
      const uint32_t row = __shfl(idx, (int)b, kWave);
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const uint32_t d = lane + kWave * u;
        v[b][u] = (b < nb && d < dim) ? G[(uint64_t)row * dim + d] : 0.0f;
      }
    }
    const uint32_t nq = q0 + kTacFoldBatch + lane;
    idx = lane < kTacFoldBatch && nq < cnt ? mem[nq] : 0u;
#pragma unroll
    for (uint32_t b = 0; b < kTacFoldBatch; ++b)
      if (b < nb)
#pragma unroll
        for (int u = 0; u < PER; ++u) s[u] = s[u] + v[b][u];
  }
  const float inv = 1.0f / (float)cnt;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const uint32_t d = lane + kWave * u;
    if (d < dim) C[(uint64_t)g * dim + d] = s[u] * inv;
  }
}

// The same cluster sums for clusters of at least kTacFoldBig members, one
// block per listed cluster (blocks stride over the list): a wave folding 64
// members per gathered batch waits a full memory round trip per batch, so
// four loader waves gather the member rows instead (one 16-byte piece per
// lane, four rows per load instruction), four batches ahead, and store each
// batch into one of two LDS buffers a step before wave 0 folds it, lane =
// dimension, in member order from 0.0f.  Member indices are staged in LDS a
// segment of kTacFoldBigSeg at a time by the whole block, so the loaders'
// only global loads are rows.  One block barrier per batch; loader and folder
// loops count the same barriers.
constexpr uint32_t kTacFoldBigLoaders = 4;
constexpr uint32_t kTacFoldBigThreads = (kTacFoldBigLoaders + 1) * kWave;
constexpr uint32_t kTacFoldBigBlocks = 512;
constexpr uint32_t kTacFoldBigSeg = 4096;  // member indices staged at a time

__global__ __launch_bounds__(kTacFoldBigThreads) void tac_fold_big_kernel(
    const float* __restrict__ G, const uint32_t* __restrict__ sorted,
    const uint32_t* __restrict__ counts, const uint32_t* __restrict__ start,
    const uint32_t* __restrict__ cprob, const TacProblem* __restrict__ probs,
    float* __restrict__ C, const uint32_t* __restrict__ big) {
  constexpr uint32_t B = 64;                           // members per batch
  constexpr uint32_t RW = B / kTacFoldBigLoaders;      // members per loader per batch
  constexpr uint32_t GW = RW / 4;                      // load instructions per loader per batch
  constexpr int NR = 4;                                // batches in flight per loader
  constexpr uint32_t CR = 16;                          // rows read from LDS ahead of the fold
  __shared__ __attribute__((aligned(16))) float xs[2][B * 64];
  __shared__ uint32_t ids[kTacFoldBigSeg];
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const uint32_t nbig = big[0];
  for (uint32_t li = blockIdx.x; li < nbig; li += gridDim.x) {
    const uint32_t g = big[1 + li];
    const uint32_t cnt = counts[g];
    const uint32_t* mem = sorted + probs[cprob[g]].off + start[g];
    float sum = 0.0f;
    for (uint32_t s0 = 0; s0 < cnt; s0 += kTacFoldBigSeg) {
      const uint32_t sn = cnt - s0 < kTacFoldBigSeg ? cnt - s0 : kTacFoldBigSeg;
      for (uint32_t t = threadIdx.x; t < sn; t += kTacFoldBigThreads) ids[t] = mem[s0 + t];
      __syncthreads();
      const uint32_t nb = (sn + B - 1) / B;
      if (w > 0) {
        const uint32_t lw = w - 1u;
        tac_floatx4 buf[NR][GW];
        // batch k into register slot `slot`; lane l fetches piece l % 16 of
        // member RW lw + 4 q + l / 16 (past the segment: its last member again,
        // which the fold never reads, so every load is unconditional)
        auto load = [&](int slot, uint32_t k) {
#pragma unroll
          for (uint32_t q = 0; q < GW; ++q) {
            uint32_t m = k * B + RW * lw + 4u * q + lane / 16u;
            m = m < sn ? m : sn - 1u;
            buf[slot][q] = *reinterpret_cast<const tac_floatx4*>(G + (uint64_t)ids[m] * 64u +
                                                                  4u * (lane % 16u));
          }
        };
        auto store = [&](int slot, uint32_t k) {
          char* x = reinterpret_cast<char*>(xs[k & 1u]) + lw * RW * 256u + lane * 16u;
#pragma unroll
          for (uint32_t q = 0; q < GW; ++q)
            *reinterpret_cast<tac_floatx4*>(x + q * 1024u) = buf[slot][q];
        };
#pragma unroll
        for (int q = 0; q < NR; ++q) load(q, (uint32_t)q);
        store(0, 0);
        __syncthreads();
        uint32_t k = 0;
        for (;;) {
#pragma unroll
          for (int sl = 0; sl < NR; ++sl) {
            load(sl, k + NR);
            store((sl + 1) % NR, k + 1);
            __syncthreads();
            if (++k == nb) break;
          }
          if (k == nb) break;
        }
      } else {
        __syncthreads();
        for (uint32_t k = 0; k < nb; ++k) {
          const float* x = xs[k & 1u];
          const uint32_t m = sn - k * B < B ? sn - k * B : B;
          if (m == B) {
            float xc[2][CR];
#pragma unroll
            for (uint32_t b = 0; b < CR; ++b) xc[0][b] = x[b * 64u + lane];
#pragma unroll
            for (uint32_t cc = 0; cc < B / CR; ++cc) {
              const int h = (int)(cc & 1u);
              if (cc + 1 < B / CR) {
#pragma unroll
                for (uint32_t b = 0; b < CR; ++b)
                  xc[h ^ 1][b] = x[((cc + 1) * CR + b) * 64u + lane];
              }
#pragma unroll
              for (uint32_t b = 0; b < CR; ++b) sum = sum + xc[h][b];
            }
          } else {
            for (uint32_t b = 0; b < m; ++b) sum = sum + x[b * 64u + lane];
          }
          __syncthreads();
        }
      }
      __syncthreads();  // ids and the buffers are reused by the next segment or cluster
    }
    if (w == 0) C[(uint64_t)g * 64u + lane] = sum * (1.0f / (float)cnt);
  }
}

// ---------------------------------------------------------------------------
// wcss per problem: the serial fp32 fold of min_to_any over its rows
// (kmeans.zig:179), evaluated exactly in chunks (fold_rules.hpp).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tac_chunk_sums_kernel(
    const float* __restrict__ e, const TacProblem* __restrict__ probs,
    const TacChunk* __restrict__ chl, uint32_t nchl, const uint32_t* __restrict__ done,
    double* __restrict__ pre) {
  const uint32_t c = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (c >= nchl) return;
  const TacChunk ch = chl[c];
  if (done[ch.prob]) return;
  const TacProblem pr = probs[ch.prob];
  const double s = fold_chunk_sum_wave(e + pr.off, pr.n, ch.j);
  if (threadIdx.x % kWave == 0) pre[c] = s;
}

__global__ __launch_bounds__(256) void tac_chunk_prefix_kernel(
    double* __restrict__ pre, const TacProblem* __restrict__ probs,
    const uint32_t* __restrict__ done) {
  __shared__ double ws[256 / kWave];
  __shared__ double carry;
  const uint32_t p = blockIdx.x;
  if (done[p]) return;
  const TacProblem pr = probs[p];
  block_prefix_f64<256>(pre + pr.chunk0, pr.nchunks, ws, &carry);
}

__global__ __launch_bounds__(256) void tac_quantize_kernel(
    const float* __restrict__ e, const double* __restrict__ pre,
    const TacProblem* __restrict__ probs, const TacChunk* __restrict__ chl, uint32_t nchl,
    const uint32_t* __restrict__ done, FoldChunk* __restrict__ fchunks) {
  const uint32_t c = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (c >= nchl) return;
  const TacChunk ch = chl[c];
  if (done[ch.prob]) return;
  const TacProblem pr = probs[ch.prob];
  fold_quantize_chunk_wave<float>(e + pr.off, pr.n, ch.j, pre[c], fchunks + c);
}

__global__ __launch_bounds__(kWave) void tac_wcss_apply_kernel(
    const float* __restrict__ e, const FoldChunk* __restrict__ fchunks,
    const TacProblem* __restrict__ probs, const uint32_t* __restrict__ done,
    float* __restrict__ wcss) {
  __shared__ __attribute__((aligned(16))) float buf[kFoldChunk];
  const uint32_t p = blockIdx.x;
  if (done[p]) return;
  const TacProblem pr = probs[p];
  const float s = fold_apply_wave<float>(e + pr.off, pr.n, fchunks + pr.chunk0, pr.nchunks, buf,
                                         static_cast<float*>(nullptr));
  if (threadIdx.x == 0) wcss[p] = s;
}

// ---------------------------------------------------------------------------
// Empty-cluster reseed (kmeans.zig:199-211), one block per problem: empty
// clusters in ascending order each take the row of argmax(min_to_any)
// (first index on ties; index 0 when min_to_any[0] is NaN, as a strict >
// scan from values[0] gives) and mark it claimed with -inf.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tac_reseed_kernel(
    const float* __restrict__ G, float* __restrict__ e, const uint32_t* __restrict__ counts,
    const TacProblem* __restrict__ probs, const uint32_t* __restrict__ done,
    float* __restrict__ C, uint32_t* __restrict__ empties, uint32_t dim) {
  __shared__ uint32_t elist[256];
  __shared__ uint32_t ewsum[256 / kWave];
  __shared__ float rv[256 / kWave];
  __shared__ uint32_t ri[256 / kWave];
  __shared__ uint32_t s_far;
  const uint32_t p = blockIdx.x;
  if (done[p]) return;
  const TacProblem pr = probs[p];
  const uint32_t lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  float* em = e + pr.off;
  for (uint32_t c0 = 0; c0 < pr.k; c0 += blockDim.x) {
    const uint32_t c = c0 + threadIdx.x;
    const bool empty = c < pr.k && counts[pr.goff + c] == 0;
    const uint32_t pos = block_exclusive_scan(empty ? 1u : 0u, ewsum);
    if (empty) elist[pos] = c;
    uint32_t found = 0;
    for (uint32_t q = 0; q < blockDim.x / kWave; ++q) found += ewsum[q];
    __syncthreads();
    if (threadIdx.x == 0 && found) atomicAdd(&empties[p], found);
    for (uint32_t q = 0; q < found; ++q) {
      // argmax over em[0 .. n): first index of the largest value
      float bv = -__builtin_inff();
      uint32_t bidx = 0xFFFFFFFFu;
      for (uint32_t i = threadIdx.x; i < pr.n; i += blockDim.x) {
        const float v = em[i];
        if (bidx == 0xFFFFFFFFu || v > bv) {
          if (!(v != v)) {  // NaN never wins after index 0
            bv = v;
            bidx = i;
          }
        }
      }
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_down(bv, off, kWave);
        const uint32_t oi = __shfl_down(bidx, off, kWave);
        if (oi != 0xFFFFFFFFu && (bidx == 0xFFFFFFFFu || ov > bv || (ov == bv && oi < bidx))) {
          bv = ov;
          bidx = oi;
        }
      }
      if (lane == 0) {
        rv[wv] = bv;
        ri[wv] = bidx;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        float v = rv[0];
        uint32_t ix = ri[0];
        for (uint32_t ww = 1; ww < blockDim.x / kWave; ++ww)
          if (ri[ww] != 0xFFFFFFFFu &&
              (ix == 0xFFFFFFFFu || rv[ww] > v || (rv[ww] == v && ri[ww] < ix))) {
            v = rv[ww];
            ix = ri[ww];
          }
        const float e0 = em[0];
        if (e0 != e0 || ix == 0xFFFFFFFFu) ix = 0;  // values[0] NaN: the scan keeps 0
        // a value equal to values[0] never displaces index 0 (strict >)
        if (ix != 0 && !(v > e0)) ix = 0;
        s_far = ix;
      }
      __syncthreads();
      const uint32_t far = s_far;
      const uint32_t cc = elist[q];
      for (uint32_t d = threadIdx.x; d < dim; d += blockDim.x)
        C[((uint64_t)pr.goff + cc) * dim + d] = G[((uint64_t)pr.off + far) * dim + d];
      __syncthreads();
      if (threadIdx.x == 0) em[far] = -__builtin_inff();
      __syncthreads();
    }
    __syncthreads();
  }
}

// Convergence per problem (kmeans.zig:214-223): skipped at iteration 0;
// rel = (prev - wcss) / (prev > 0 ? prev : 1); stop when rel < tol.
__global__ void tac_converge_kernel(const float* __restrict__ wcss, float* __restrict__ prev,
                                    uint32_t* __restrict__ done, uint32_t* __restrict__ iters,
                                    uint32_t P, uint32_t t, float tol) {
  const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= P || done[p]) return;
  iters[p] = t + 1;
  const float w = wcss[p];
  if (t > 0) {
    const float pv = prev[p];
    const float denom = pv > 0.0f ? pv : 1.0f;
    const float rel = (pv - w) / denom;
    if (rel < tol) done[p] = 1;
  }
  prev[p] = w;
}

// Output: assignments[idx[off + i]] = goff + code[off + i] (tac.zig:504-510).
__global__ void tac_output_kernel(const uint32_t* __restrict__ code,
                                  const uint32_t* __restrict__ idx,
                                  const TacProblem* __restrict__ probs,
                                  const TacTile* __restrict__ tiles,
                                  uint32_t* __restrict__ assign) {
  const TacTile tl = tiles[blockIdx.x];
  const TacProblem pr = probs[tl.prob];
  const uint32_t i = tl.row0 + threadIdx.x;
  if (i < pr.n) assign[idx[pr.off + i]] = pr.goff + code[pr.off + i];
}

}  // namespace tacgpu
