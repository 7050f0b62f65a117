// cand_kernels.hpp — exact candidate-set assignment for the Lloyd iterations
// after the first (src/tac/kmeans.zig:344-365 semantics).  Included once, by
// tac_gpu.hip, after pq_kernels.hpp.
//
// Why the result equals the exhaustive first-index argmin.
//   Let a be the vector's code from the previous iteration (any valid index
//   works: a is only an anchor) and U2 = ref(x, c_a), the reference distance
//   to that codeword in the current codebook.  For every codeword c the
//   reference fold (D squares and D-1 adds, separately rounded) satisfies
//     |ref(x, c) - T(x, c)| <= g T(x, c) + eta,    g = gamma_{D+2},
//   where T is the exact squared distance and eta < 1e-43 covers underflow.
//   The reference's first-index argmin c* has ref(x, c*) <= U2, so T(x, c*)
//   and T(x, c_a) are both at most rho^2 = (U2 + eta) / (1 - g), and by the
//   triangle inequality ||c_a - c*||^2 <= 4 rho^2.  Hence c* lies in
//     S = {a} + {c : lo(a, c) <= R2},   R2 >= 4 rho^2 (rounded up),
//   for any lower bound lo(a, c) <= ||c_a - c||^2.  The kernel evaluates
//   ref() on S exactly as the reference does and keeps the lexicographic
//   minimum of (distance bits, index): c* has the global minimum and the
//   smallest index among its ties, so that minimum is c*.
//
// Anchors.  Lloyd iterations after the first anchor each vector at its
// previous code.  The first iteration and encode anchor it at the nearest of
// the codewords nearest the centre of its cell (cand_anchors of them) in a
// grid over the codebook's bounding box (grid_build_kernel); a vector
// outside the box takes the nearest cell.  The rule above holds for any
// anchor, so the anchor only decides how many candidates are evaluated.
//
// Neighbour tables.  After every update, nbr_build_kernel sorts, for each
// codeword a, the other codewords by lo(a, c) and keeps the first L of them
// as one u32 key each: the bits of lo with the low 12 bits replaced by c << 4
// (K <= 256).  Clearing low bits of a non-negative float lowers it, so the
// key's value part stays a lower bound, and sorted keys put S \ {a} in a
// prefix of the row.  If the whole kept row lies inside R2 while codewords
// are missing from it, S may be larger than the row: the vector goes to a
// deferred list that the pruned full search (pq_kernels.hpp) resolves, as
// do non-finite or huge distances and non-finite codebooks.
//
// Load balance.  Each wave assigns 64 vectors at a time.  A vector's
// candidates are cut into items of at most kCandItem; a wave scan of the
// item counts lays the items out over the wave's lanes, an item's result
// folds into its vector's 64-bit LDS key with an atomic minimum, and every
// lane then writes its own vector's result.  The work per lane follows the
// mean candidate count, not the largest in the wave, and the waves of a
// block never wait for one another.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cand_rules.hpp"
#include "pq_kernels.hpp"

namespace tacgpu {

constexpr int kCandThreads = 1024;      // threads per candidate block
// The neighbour rows stay in global memory (64 KB per subspace at K = 256,
// L2-resident) and are read as two 16-byte loads per item: staged in LDS they
// took 66 KB of it, held the kernel to one block per CU and added bank
// conflicts to the codeword gathers.  The row samples are staged in LDS.
constexpr int kCandWaves = kCandThreads / kWave;
constexpr uint32_t kCandLdsMax = 160 * 1024;

constexpr uint32_t kCandCells = 6561;  // grid cells per subspace (encode anchors), 9^4
// Anchor codewords per grid cell: three for encode, two for the first Lloyd
// iteration, whose block also holds the sort-tile counts (two blocks per CU
// either way).
template <bool TOKENS>
constexpr uint32_t cand_anchors() { return TOKENS ? 3u : 2u; }
constexpr uint32_t kCandAnchorsMax = 3;

// LDS layout of cand_kernel, shared by the host launcher:
//   lcb [K][DP] f32 | lsamp [K][8] u32: the top 16 bits of the value bits
//   of row entries 0, 7, 15, ..., 119 (the 16 samples, two per word; all-ones
//   past the row) | grid anchors only:
//   lanc [cells][na] anchors (na = cand_anchors; u8 up to K = 256, else u16),
//   lgrid [2][8] f32 (cell
//   origin, cells per unit) |
//   per wave: gx [64][DP] f32, gbest [64] u64, ga [64] u32 (the anchor's
//   row offset),
//   gitem [64 * 8] u16 (lane | item << 6) | lmax, lcnt u32 | training only:
//   lhist [tiles][(K + 1) / 2] u32, the block's sort-tile histograms of the
//   new codes as u16 pairs (at most kSortTile per bin)
struct CandLds {
  uint32_t samp_off, anc_off, grid_off, wave_off, wave_bytes, scal_off, hist_off, total;
};
__host__ __device__ inline uint32_t cand_up16(uint32_t b) { return (b + 15u) & ~15u; }
__host__ __device__ inline CandLds cand_lds(uint32_t K, uint32_t DP, uint32_t cells = 0,
                                            uint32_t hist_tiles = 0, uint32_t anchor_bytes = 0) {
  CandLds s;
  s.samp_off = cand_up16(K * DP * 4u);
  s.anc_off = s.samp_off + K * 8u * 4u;
  s.grid_off = cand_up16(s.anc_off + cells * anchor_bytes);
  s.wave_off = s.grid_off + (cells ? 64u : 0u);
  s.wave_bytes = 64u * (DP * 4u + 8u + 4u) + 64u * 8u * 2u;
  s.scal_off = s.wave_off + (uint32_t)kCandWaves * s.wave_bytes;
  s.hist_off = s.scal_off + 16u;
  s.total = s.hist_off + hist_tiles * ((K + 1u) / 2u) * 4u;
  return s;
}

// Sort tiles per training candidate block at most: the block's chunk is
// whole tiles, so its histograms are complete.
constexpr uint32_t kCandHistTiles = 16;

// Cells per dimension of the encode grid: the largest G with G^D <= kCandCells.
__host__ __device__ inline uint32_t cand_grid_side(uint32_t D) {
  uint32_t G = 1;
  for (;;) {
    uint64_t p = 1;
    for (uint32_t k = 0; k < D; ++k) p *= (G + 1);
    if (p > kCandCells) return G;
    ++G;
  }
}

// Exchange partner of lane ^ LX within a wave: DPP moves for 1, 2 and 8
// (quad permutes and a row rotation by 8), a swizzle for 4 and 16, a
// permute for 32.
template <uint32_t LX>
__device__ inline uint32_t lane_xor(uint32_t v) {
  if constexpr (LX == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false);  // quad_perm 1,0,3,2
  } else if constexpr (LX == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false);  // quad_perm 2,3,0,1
  } else if constexpr (LX == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);  // row_ror:8
  } else if constexpr (LX == 4 || LX == 16) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (int)(0x1Fu | (LX << 10)));  // xor mask
  } else {
    static_assert(LX == 32, "lane_xor: 1, 2, 4, 8, 16 or 32");
    return (uint32_t)__shfl_xor((int)v, 32, kWave);
  }
}

// Stage (2^KB, 2^JB) of a bitonic network over the 64 R keys of a wave, key
// e = lane R + r in v[r]: keys e and e ^ 2^JB end in ascending order when
// e & 2^KB is 0, in descending order otherwise.
template <int R, int KB, int JB>
__device__ inline void bitonic_stage(uint32_t (&v)[R], uint32_t lane) {
  constexpr uint32_t k = 1u << KB, j = 1u << JB;
  if constexpr (j >= (uint32_t)R) {
    const bool lower = (lane & (j / R)) == 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t o = lane_xor<j / R>(v[r]);
      const bool up = ((lane * R + r) & k) == 0;
      v[r] = up == lower ? min(v[r], o) : max(v[r], o);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if ((r & j) == 0) {
        const bool up = ((lane * R + r) & k) == 0;
        const uint32_t lo = min(v[r], v[r | j]), hi = max(v[r], v[r | j]);
        v[r] = up ? lo : hi;
        v[r | j] = up ? hi : lo;
      }
    }
  }
}
template <int R, int KB, int JB>
__device__ inline void bitonic_stages(uint32_t (&v)[R], uint32_t lane) {
  bitonic_stage<R, KB, JB>(v, lane);
  if constexpr (JB > 0) bitonic_stages<R, KB, JB - 1>(v, lane);
}
template <int R>
constexpr int wave_log_keys() { return R == 4 ? 8 : R == 2 ? 7 : 6; }
// Sorts the wave's 64 R keys ascending (key e = lane R + r).
template <int R, int KB = 1>
__device__ inline void wave_bitonic_sort(uint32_t (&v)[R], uint32_t lane) {
  bitonic_stages<R, KB, KB - 1>(v, lane);
  if constexpr (KB < wave_log_keys<R>()) wave_bitonic_sort<R, KB + 1>(v, lane);
}
// Sorts a bitonic sequence of the wave's 64 R keys ascending.
template <int R>
__device__ inline void wave_bitonic_merge(uint32_t (&v)[R], uint32_t lane) {
  constexpr int LOG = wave_log_keys<R>();
  bitonic_stages<R, LOG, LOG - 1>(v, lane);  // e & 2^LOG is 0: ascending everywhere
}

// One block per (codeword a, subspace m), one wave up to K = 256, four
// beyond: lo(a, c) for every c != a as a key (all-ones for a and past K),
// and the first L <= 128 keys in ascending order written to nbr[m][a][0 ..
// L), cand_pad_key(a) to the rest of the stored row nbr[m][a][L ..
// cand_row_len(L)).  Keys are distinct (the codeword id is part of the key),
// so the row is the unique sorted prefix.  Each wave sorts its 256 keys in
// registers (bitonic network, lane exchanges without LDS); with four waves
// the four sorted runs meet in LDS, where the 128 smallest of two runs are
// the element-wise minimum of the first 128 of one and the first 128 of the
// other reversed (a bitonic sequence, merged in registers), twice.
// Block (0, m) also clears the subspace's deferred count for the assignment
// that follows on the same stream.
__host__ __device__ inline uint32_t nbr_lds_bytes(uint32_t K) { return K > 256 ? 4096u : 0u; }

template <int D>
__global__ __launch_bounds__(256) void nbr_build_kernel(const float* __restrict__ cb,
                                                        uint32_t* __restrict__ nbr,
                                                        uint32_t* __restrict__ defer_count,
                                                        const uint32_t* __restrict__ done,
                                                        uint32_t K, uint32_t L) {
  extern __shared__ uint32_t runs[];  // [4][256], four waves only
  const uint32_t a = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const uint32_t lane = t % kWave, w = t / kWave;
  if (a == 0 && t == 0) defer_count[m] = 0;
  if (done && done[m]) return;
  constexpr float g = cand_gamma(D);
  const float* cbm = cb + (uint64_t)m * K * D;
  float ca[D];
#pragma unroll
  for (int k = 0; k < D; ++k) ca[k] = cbm[(uint64_t)a * D + k];
  uint32_t v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t c = w * 256u + (uint32_t)r * kWave + lane;
    uint32_t key = kCandNoKey;
    if (c < K && c != a) {
      float cv[D];
#pragma unroll
      for (int k = 0; k < D; ++k) cv[k] = cbm[(uint64_t)c * D + k];
      key = cand_key(cand_lower_bound(exact_l2sq<D>(ca, cv), g), c);
    }
    v[r] = key;
  }
  wave_bitonic_sort<4>(v, lane);
  const uint32_t Lr = cand_row_len(L);  // <= 128
  uint32_t* row = nbr + ((uint64_t)m * K + a) * Lr;
  if (blockDim.x == kWave) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t e = lane * 4u + (uint32_t)r;
      if (e < Lr) row[e] = e < L ? v[r] : cand_pad_key(a);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) runs[w * 256u + lane * 4u + (uint32_t)r] = v[r];
  __syncthreads();
  uint32_t h[2];
  if (w < 2) {  // runs 2w and 2w + 1 -> their 128 smallest, into run 2w's first half
    const uint32_t* A = runs + 2u * w * 256u;
    const uint32_t* B = A + 256u;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t e = lane * 2u + (uint32_t)r;
      h[r] = min(A[e], B[127u - e]);
    }
    wave_bitonic_merge<2>(h, lane);
#pragma unroll
    for (int r = 0; r < 2; ++r) runs[2u * w * 256u + lane * 2u + (uint32_t)r] = h[r];
  }
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t e = lane * 2u + (uint32_t)r;
      h[r] = min(runs[e], runs[512u + 127u - e]);
    }
    wave_bitonic_merge<2>(h, lane);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t e = lane * 2u + (uint32_t)r;
      if (e < Lr) row[e] = e < L ? h[r] : cand_pad_key(a);
    }
  }
}

// Grid anchors of subspace m = blockIdx.y: the bounding box of the
// codewords (lo, hi per dimension), G cells per dimension, and for each cell
// the NA codewords nearest its centre (any choice is valid; nearness only
// keeps the candidate sets small; with K < NA the nearest repeats).
// grid[m] = {lo[8], G / (hi - lo)[8]}, anchors[m][cell][0 .. NA).
template <int D, uint32_t NA, typename AnchorT>
__global__ __launch_bounds__(kBlock) void grid_build_kernel(const float* __restrict__ cb,
                                                            AnchorT* __restrict__ anchors,
                                                            float* __restrict__ grid,
                                                            uint32_t K, uint32_t G,
                                                            uint32_t cells,
                                                            const uint32_t* __restrict__ skip) {
  __shared__ float lcb[kCandMaxK * D];
  __shared__ float box[2 * D];
  const uint32_t m = blockIdx.y;
  if (skip && skip[m]) return;  // a subspace another encode pass serves
  const float* cbm = cb + (uint64_t)m * K * D;
  for (uint32_t j = threadIdx.x; j < K * D; j += blockDim.x) lcb[j] = cbm[j];
  __syncthreads();
  if (threadIdx.x < D) {
    float lo = lcb[threadIdx.x], hi = lcb[threadIdx.x];
    for (uint32_t c = 1; c < K; ++c) {
      lo = fminf(lo, lcb[c * D + threadIdx.x]);
      hi = fmaxf(hi, lcb[c * D + threadIdx.x]);
    }
    const float inv = hi > lo ? (float)G / (hi - lo) : 0.0f;
    box[threadIdx.x] = lo;
    box[D + threadIdx.x] = inv;
    if (blockIdx.x == 0) {
      grid[m * 16 + threadIdx.x] = lo;
      grid[m * 16 + 8 + threadIdx.x] = inv;
    }
  }
  __syncthreads();
  const uint32_t cell = blockIdx.x * blockDim.x + threadIdx.x;
  if (cell >= cells) return;
  float ctr[D];
  uint32_t r = cell;
#pragma unroll
  for (int k = 0; k < D; ++k) {
    const uint32_t ck = r % G;
    r /= G;
    ctr[k] = box[k] + ((float)ck + 0.5f) / (box[D + k] > 0.0f ? box[D + k] : 1.0f);
  }
  float bd[NA];
  uint32_t bc[NA];
#pragma unroll
  for (uint32_t q = 0; q < NA; ++q) {
    bd[q] = __builtin_inff();
    bc[q] = 0;
  }
  for (uint32_t c = 0; c < K; ++c) {
    float d = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const float u = ctr[k] - lcb[c * D + k];
      d = d + u * u;
    }
    // Insert into the ascending list of the NA nearest (strict <: the
    // earlier index stays ahead on ties).
#pragma unroll
    for (int q = (int)NA - 1; q >= 0; --q) {
      if (d < bd[q]) {
        if (q + 1 < (int)NA) {
          bd[q + 1] = bd[q];
          bc[q + 1] = bc[q];
        }
        bd[q] = d;
        bc[q] = c;
      }
    }
  }
#pragma unroll
  for (uint32_t q = 0; q < NA; ++q)
    anchors[((uint64_t)m * cells + cell) * NA + q] = (AnchorT)(q < K ? bc[q] : bc[0]);
}

// Inclusive sum over the 64 lanes of a wave with DPP moves: shifts of 1, 2,
// 4, 8 within each row of 16 lanes, then the row totals carried forward
// with the row broadcasts of lanes 15 and 31.
__device__ inline uint32_t wave_inclusive_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// The exact candidate-set assignment.  GRID picks the anchor: the nearer of
// the vector's grid cell's two codewords (true), or codes[m][i], the
// previous Lloyd iteration's code (false).  TOKENS picks the layout.
// Training (TOKENS false): block (chunk b, subspace m) of a 2-D grid;
// x = xs[m][i][DP]; the result goes to codes[m][i] with e[m][i], the
// reference distance; iteration 0 runs with grid anchors, later iterations
// from the previous codes.  Encode (TOKENS true, GRID true): a 1-D grid
// whose blocks run XCD-contiguously as (chunk, subspace) so that the M
// blocks of a chunk share one L2; x = x[i][m*D ..] (token-major) and the code
// goes to out[i][m].  Vectors the rule cannot settle are first listed in the
// block's own slice slice[m][b*chunk ..] (an LDS counter), then appended to
// the subspace's dense list defer[m][0 .. defer_count[m]) with one global
// atomic per block.  Training also counts the new codes per sort tile of
// kSortTile vectors (the chunk is whole tiles) and writes
// hist[m][tile][code] for the update's counting sort; the deferred vectors'
// codes are added there by assign_list_kernel.
// Up to dsub 4 the kernel is held to 64 VGPRs (8 waves per SIMD): two
// 16-wave blocks then share a CU, as the LDS allows; past 64 only one fits.
template <int D, bool GRID, bool TOKENS, typename CodeT, typename AnchorT>
__global__ __launch_bounds__(kCandThreads, D <= 4 ? 8 : 4) void cand_kernel(
    const float* __restrict__ xin, const float* __restrict__ cb,
    const uint32_t* __restrict__ nbr, const AnchorT* __restrict__ anchors,
    const float* __restrict__ grid, uint16_t* __restrict__ codes, float* __restrict__ e,
    CodeT* __restrict__ out, uint32_t* __restrict__ slice, uint32_t* __restrict__ defer,
    uint32_t* __restrict__ defer_count, const uint32_t* __restrict__ done, uint64_t n,
    uint32_t dim, uint32_t M, uint32_t K, uint32_t L, uint32_t chunk, uint32_t nchunks,
    uint32_t G, uint32_t cells, uint32_t* __restrict__ hist, uint32_t T) {
  constexpr int DP = Pad<D>::value;
  constexpr float g = cand_gamma(D);
  extern __shared__ __attribute__((aligned(16))) float lds[];
  static_assert(GRID || !TOKENS, "token-major input takes grid anchors");
  uint32_t m, b;
  if constexpr (TOKENS) {
    const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
    if (logical >= nchunks * M) return;  // grid padding to a multiple of 8
    b = logical / M;
    m = logical % M;
    if (done && done[m]) return;  // a subspace another encode pass serves
  } else {
    b = blockIdx.x;
    m = blockIdx.y;
    if (done[m]) return;
  }
  const uint32_t tiles = TOKENS ? 0u : chunk / kSortTile;  // the chunk is whole tiles
  const uint32_t Kw = (K + 1u) / 2u;                       // u16 pairs per tile
  constexpr uint32_t NA = cand_anchors<TOKENS>();
  const CandLds lay = cand_lds(K, DP, GRID ? cells : 0u, tiles, GRID ? NA * (uint32_t)sizeof(AnchorT) : 0u);
  uint8_t* base = reinterpret_cast<uint8_t*>(lds);
  float* lcb = lds;
  uint32_t* lsamp = reinterpret_cast<uint32_t*>(base + lay.samp_off);
  AnchorT* lanc = reinterpret_cast<AnchorT*>(base + lay.anc_off);
  float* lgrid = reinterpret_cast<float*>(base + lay.grid_off);
  const uint32_t t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  uint8_t* wb = base + lay.wave_off + wave * lay.wave_bytes;
  float* gx = reinterpret_cast<float*>(wb);
  unsigned long long* gbest = reinterpret_cast<unsigned long long*>(gx + 64 * DP);
  uint32_t* ga = reinterpret_cast<uint32_t*>(gbest + 64);
  uint16_t* gitem = reinterpret_cast<uint16_t*>(ga + 64);
  uint32_t* lmax = reinterpret_cast<uint32_t*>(base + lay.scal_off);
  uint32_t* lcnt = lmax + 1;
  uint32_t* lhist = reinterpret_cast<uint32_t*>(base + lay.hist_off);
  for (uint32_t j = threadIdx.x; j < tiles * Kw; j += blockDim.x) lhist[j] = 0;

  if (t == 0) {
    *lmax = 0;
    *lcnt = 0;
  }
  __syncthreads();
  const float* cbm = cb + (uint64_t)m * K * D;
  for (uint32_t c = t; c < K; c += blockDim.x) {
    float v[DP];
#pragma unroll
    for (int k = 0; k < DP; ++k) v[k] = k < D ? cbm[(uint64_t)c * D + k] : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) s = s + v[k] * v[k];
#pragma unroll
    for (int k = 0; k < DP; ++k) lcb[c * DP + k] = v[k];
    atomicMax(lmax, __float_as_uint(s));  // >= 0x7f800000: a non-finite codeword
  }
  const uint32_t Lr = cand_row_len(L);  // stored row length
  const uint32_t* nbm = nbr + (uint64_t)m * K * Lr;
  const uint32_t* rows = nbm;  // row a at rows + a * rs
  const uint32_t rs = Lr;
  // The 16 truncated samples of a row as 8 words, sample 2w in the low half of word w.
  for (uint32_t j = t; j < K * 8; j += blockDim.x) {
    const uint32_t* row = nbm + (j / 8) * Lr;
    const uint32_t q = 2u * (j % 8u);
    lsamp[j] = (uint32_t)cand_sample16(row, L, q) | ((uint32_t)cand_sample16(row, L, q + 1u) << 16);
  }
  if constexpr (GRID) {
    const AnchorT* am = anchors + (uint64_t)m * cells * NA;
    for (uint32_t j = t; j < cells * NA; j += blockDim.x) lanc[j] = am[j];
    if (t < 16) lgrid[t] = grid[m * 16 + t];
  }
  __syncthreads();
  const bool all_deferred = *lmax >= 0x7f800000u;
  const bool row_complete = L + 1 >= K;  // every other codeword is in the row

  const uint64_t lo_i = (uint64_t)b * chunk;
  const uint64_t hi_i = lo_i + chunk < n ? lo_i + chunk : n;
  uint16_t* cm = codes + (uint64_t)m * n;
  float* em = e + (uint64_t)m * n;
  auto load_x = [&](uint64_t i, float (&v)[D]) {
    if constexpr (TOKENS) {
      const float* src = xin + i * dim + (uint64_t)m * D;
#pragma unroll
      for (int k = 0; k < D; ++k) v[k] = src[k];
    } else {
      load_padded<D>(xin + ((uint64_t)m * n + i) * DP, v);
    }
  };
  // Wave w takes the 64-vector groups w, w + kCandWaves, ... of the chunk;
  // each group's vectors (and previous codes) are loaded one group ahead.
  float xq[D];
  uint32_t aq = 0;
#pragma unroll
  for (int k = 0; k < D; ++k) xq[k] = 0.0f;
  const uint64_t first_i = lo_i + (uint64_t)wave * kWave + lane;
  if (first_i < hi_i) {
    load_x(first_i, xq);
    if constexpr (!GRID) aq = cm[first_i];
  }
  constexpr uint64_t kStride = (uint64_t)kCandWaves * kWave;
  for (uint64_t g0 = lo_i + (uint64_t)wave * kWave; g0 < hi_i; g0 += kStride) {
    // Phase 1: anchor distance, R2 and the number of items of this lane's vector.
    const uint64_t i = g0 + lane;
    const bool valid = i < hi_i;
    float x[D];
#pragma unroll
    for (int k = 0; k < D; ++k) x[k] = xq[k];
    uint32_t a = valid ? aq : 0u;
    if (i + kStride < hi_i) {
      load_x(i + kStride, xq);
      if constexpr (!GRID) aq = cm[i + kStride];
    }
    uint32_t cell = 0;  // grid anchors: NaN coordinates land in cell 0 (fmaxf)
    if constexpr (GRID) {
#pragma unroll
      for (int k = D - 1; k >= 0; --k) {
        const float f = fminf(fmaxf((x[k] - lgrid[k]) * lgrid[8 + k], 0.0f), (float)(G - 1));
        cell = cell * G + (uint32_t)f;
      }
      cell = cell < cells ? cell : 0u;
      a = lanc[cell * NA];
    }
    bool deferred = valid && (all_deferred || a >= K);
    uint32_t nit = 0;
    float U2 = 0.0f, R2 = 0.0f;
    if (valid && !deferred) {
      float ca[D];
      load_padded<D>(lcb + a * DP, ca);
      U2 = exact_l2sq<D>(x, ca);
      if constexpr (GRID) {  // the nearest of the cell's anchors
#pragma unroll
        for (uint32_t q = 1; q < NA; ++q) {
          const uint32_t a2 = lanc[cell * NA + q];
          float cb2[D];
          load_padded<D>(lcb + a2 * DP, cb2);
          const float V2 = exact_l2sq<D>(x, cb2);
          if (V2 < U2) {
            U2 = V2;
            a = a2;
          }
        }
      }
      if (!cand_tame(U2)) {  // NaN, inf or too large for the bound arithmetic
        deferred = true;
      } else {
        R2 = cand_radius(U2, g);
        const uint4 s0 = *reinterpret_cast<const uint4*>(lsamp + a * 8);
        const uint4 s1 = *reinterpret_cast<const uint4*>(lsamp + a * 8 + 4);
        const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        nit = cand_items_words(sw, R2, L, row_complete, &deferred);
        if constexpr (GRID) {
          // A grid anchor sits farther from its vector than a previous code:
          // the long rows' items 8-15 cost more there than the full search
          // they would save, so such a vector is deferred past 8 items.
          if (nit > 8u && !row_complete) {
            nit = 0;
            deferred = true;
          }
        }
      }
    }
    // Phase 2: the wave's items, laid out by an exclusive scan of the counts.
    // The wave's scratch holds 64 * 8 items; a vector may take up to 16, so
    // in the rare wave whose total passes 512 the vectors above 8 items go
    // to the deferred list (the full search) instead.
    uint32_t incl = wave_inclusive_sum(nit);
    uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
    if (total > 64u * 8u) {
      if (nit > 8u) {
        nit = 0;
        deferred = true;
      }
      incl = wave_inclusive_sum(nit);
      total = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
    }
    // The bound also keeps a corrupted count inside the scratch.
    total = min(total, 64u * 8u);
    const bool live = valid && !deferred;
    const uint64_t dm = __ballot(valid && deferred);
    if (dm) {
      uint32_t at = 0;
      if (lane == 0) at = atomicAdd(lcnt, (uint32_t)__popcll(dm));
      at = __shfl(at, 0, kWave);
      if (valid && deferred)
        slice[(uint64_t)m * n + lo_i + at + (uint32_t)__popcll(dm & ((1ull << lane) - 1ull))] =
            (uint32_t)i;
    }
    if (live) {
#pragma unroll
      for (int k = 0; k < DP; ++k) gx[lane * DP + k] = k < D ? x[k] : 0.0f;
      gbest[lane] = cand_best_key(U2, a);
      ga[lane] = a * rs;  // the anchor's row offset
    }
    {
      uint16_t* gi = gitem + (incl - nit);
#pragma unroll
      for (uint32_t q = 0; q < kCandSamples; ++q)
        if (q < nit) gi[q] = (uint16_t)(lane | (q << 6));
    }
    wave_lds_sync();
    // Phase 3: items, 64 at a time.  All 8 entries of an item are evaluated
    // without branches and folded into the vector's key: the items cover the
    // candidate set, and every entry (a kept neighbour or the anchor as
    // padding) names a real codeword, so the extra (distance, index) keys
    // leave the minimum unchanged.
    for (uint32_t w = lane; w < total; w += kWave) {
      const uint32_t it = gitem[w];
      const uint32_t u = it & 63u, j0 = ((it >> 6) & 15u) * kCandItem;
      const uint32_t* row = rows + ga[u] + j0;
      uint32_t keys[kCandItem];
      {  // rows of whole items, 32-byte aligned: two 16-byte loads
        const uint4 k0 = *reinterpret_cast<const uint4*>(row);
        const uint4 k1 = *reinterpret_cast<const uint4*>(row + 4);
        keys[0] = k0.x; keys[1] = k0.y; keys[2] = k0.z; keys[3] = k0.w;
        keys[4] = k1.x; keys[5] = k1.y; keys[6] = k1.z; keys[7] = k1.w;
      }
      float xv[D];
      load_padded<D>(gx + u * DP, xv);
      unsigned long long best = ~0ull;
#pragma unroll
      for (uint32_t k = 0; k < kCandItem; ++k) {
        const uint32_t c16 = keys[k] & kCandIdField;  // c << 4
        float cv[D];
        load_padded<D>(lcb + (c16 >> 4) * DP, cv);
        const unsigned long long key =
            ((unsigned long long)cand_f2u(exact_l2sq<D>(xv, cv)) << 32) | c16;
        best = key < best ? key : best;
      }
      atomicMin(&gbest[u], best);
    }
    wave_lds_sync();
    if (live) {
      const unsigned long long k = gbest[lane];
      if constexpr (TOKENS) {
        out[i * M + m] = (CodeT)cand_best_code(k);
      } else {
        const uint32_t code = cand_best_code(k);
        cm[i] = (uint16_t)code;
        em[i] = __uint_as_float((uint32_t)(k >> 32));
        atomicAdd(&lhist[(uint32_t)((i - lo_i) / kSortTile) * Kw + code / 2u], 1u << (16u * (code & 1u)));
      }
    }
    wave_lds_sync();  // the scratch is rewritten by the next group
  }
  __syncthreads();  // the slice's global writes, lcnt and lhist
  if constexpr (!TOKENS) {
    const uint32_t tile0 = (uint32_t)(lo_i / kSortTile);
    for (uint32_t j = t; j < tiles * K; j += blockDim.x) {
      const uint32_t tt = j / K, c = j % K;
      if (tile0 + tt < T)
        hist[((uint64_t)m * T + tile0 + tt) * K + c] = (lhist[tt * Kw + c / 2u] >> (16u * (c & 1u))) & 0xFFFFu;
    }
  }
  const uint32_t nd = *lcnt;
  if (nd == 0) return;
  __syncthreads();  // every thread has read lcnt before it is reused
  if (t == 0) *lcnt = atomicAdd(&defer_count[m], nd);
  __syncthreads();
  const uint32_t at = *lcnt;
  for (uint32_t q = t; q < nd; q += kCandThreads)
    defer[(uint64_t)m * n + at + q] = slice[(uint64_t)m * n + lo_i + q];
}

// pruned_argmin (pq_kernels.hpp) for one vector x held by the S consecutive
// lanes of a group (sub = lane % S; every lane of the group passes the same
// x), with Kp / kPruneBlock a multiple of S.  Lane sub takes blocks [sub nb /
// S, (sub + 1) nb / S) of the first pass, walking each block from entry sub
// (mod kPruneBlock) so that the group's lanes read distinct LDS banks; a
// block's minimum does not depend on that order (fminf over the entries).
// The group's block minima then meet in a top-2 merge: the smaller best1
// wins, best2 is the smaller of the loser's best1 and the winner's best2,
// and equal best1 values make best2 equal best1 (no gap, so a rescan), as
// one lane's top-2 over all blocks makes them.  The winning block's entries
// and a rescan's codewords are spread over the lanes and their (distance,
// index) minima merged lexicographically, which keeps the first index of
// the reference scan's minimum; with SEED_FIRST a NaN distance to codeword
// 0 is the result (vec.argmin keeps dists[0] when nothing compares below
// it).  Every lane returns the result; rescans counts on lane sub 0.
template <int S>
__device__ inline float group_xor_f(float v, uint32_t o) {
  if constexpr (S >= 2) {
    if (o == 1) return __uint_as_float(lane_xor<1>(__float_as_uint(v)));
  }
  if constexpr (S >= 4) {
    if (o == 2) return __uint_as_float(lane_xor<2>(__float_as_uint(v)));
  }
  return v;
}
template <int S>
__device__ inline uint32_t group_xor_u(uint32_t v, uint32_t o) {
  if constexpr (S >= 2) {
    if (o == 1) return lane_xor<1>(v);
  }
  if constexpr (S >= 4) {
    if (o == 2) return lane_xor<2>(v);
  }
  return v;
}
// (d, c) <- the lexicographic minimum of the group's (distance, index) pairs
// (distances non-negative or +inf; NaN never wins).
template <int S>
__device__ inline void group_lex_min(float& d, uint32_t& c) {
#pragma unroll
  for (uint32_t o = 1; o < (uint32_t)S; o <<= 1) {
    const float od = group_xor_f<S>(d, o);
    const uint32_t oc = group_xor_u<S>(c, o);
    if (od < d || (od == d && oc < c)) {
      d = od;
      c = oc;
    }
  }
}

template <int D, int S, bool SEED_FIRST>
__device__ __forceinline__ void pruned_argmin_lanes(const float (&x)[D], const float* lcb,
                                                    const float* lnc, uint32_t K, uint32_t Kp,
                                                    uint32_t maxbits, uint32_t sub,
                                                    uint32_t& bidx, float& bdist,
                                                    uint32_t& rescans) {
  static_assert(S == 2 || S == 4, "lanes per vector: 2 or 4");
  constexpr int DP = Pad<D>::value;
  constexpr int B = kPruneBlock;
  bool rescan = maxbits >= 0x7f800000u;  // a non-finite codeword: reference scan
  if (!rescan) {
    float xp[D];
#pragma unroll
    for (int k = 0; k < D; ++k) xp[k] = -2.0f * x[k];
    const uint32_t per = Kp / B / S, b0 = sub * per;
    float best1 = __builtin_inff(), best2 = __builtin_inff();
    uint32_t bblk = b0;
    for (uint32_t b = b0; b < b0 + per; ++b) {
      float mb = __builtin_inff();
#pragma unroll
      for (int t = 0; t < B; ++t) {
        const uint32_t c = b * B + (((uint32_t)t + sub) & (B - 1));
        float cv[D];
        load_padded<D>(lcb + c * DP, cv);
        float acc = lnc[c];
#pragma unroll
        for (int k = 0; k < D; ++k) acc = __builtin_fmaf(xp[k], cv[k], acc);
        mb = fminf(mb, acc);
      }
      const bool lt1 = mb < best1;
      const bool lt2 = mb < best2;
      best2 = lt1 ? best1 : (lt2 ? mb : best2);
      best1 = lt1 ? mb : best1;
      bblk = lt1 ? b : bblk;
    }
#pragma unroll
    for (uint32_t o = 1; o < (uint32_t)S; o <<= 1) {
      const float o1 = group_xor_f<S>(best1, o), o2 = group_xor_f<S>(best2, o);
      const uint32_t ob = group_xor_u<S>(bblk, o);
      if (o1 < best1) {
        best2 = best1 < o2 ? best1 : o2;
        best1 = o1;
        bblk = ob;
      } else if (best1 < o1) {
        best2 = best2 < o1 ? best2 : o1;
      } else {
        best2 = best1;
        bblk = ob < bblk ? ob : bblk;
      }
    }
    constexpr float u = 5.9604644775390625e-8f;  // 2^-24
    constexpr float gD = (float)D * u / (1.0f - (float)D * u);
    constexpr float gR = (float)(D + 2) * u / (1.0f - (float)(D + 2) * u);
    const float cmax2 = __uint_as_float(maxbits);
    const float cmax = sqrtf(cmax2);
    float x2 = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) x2 = x2 + x[k] * x[k];
    const float nx = sqrtf(x2);
    const float ea = 2.0f * gD * (1.0f + gD) * (cmax2 + 2.0f * nx * cmax);
    float thr = 2.0f * ea * (1.0f + gR) + gR * (fabsf(best2 + x2) + fabsf(best1 + x2));
    thr = 2.0f * thr + 1e-30f;
    const bool tame = (cmax2 + 2.0f * nx * cmax) < 1e38f;
    if (tame && (best2 - best1) > thr) {  // false on NaN
      float best = __builtin_inff();
      uint32_t idx = bblk * B;
#pragma unroll
      for (int t = 0; t < B / S; ++t) {
        const uint32_t c = bblk * B + (uint32_t)t * S + sub;
        if (c < K) {
          float cv[D];
          load_padded<D>(lcb + c * DP, cv);
          const float d = exact_l2sq<D>(x, cv);
          if (d < best) {
            best = d;
            idx = c;
          }
        }
      }
      group_lex_min<S>(best, idx);
      bidx = idx;
      bdist = best;
      return;
    }
    rescan = true;
  }
  // Reference scan: lane sub takes codewords sub, sub + S, ...
  if (sub == 0) ++rescans;
  float d0 = 0.0f;
  if (SEED_FIRST) {
    float c0[D];
    load_padded<D>(lcb, c0);
    d0 = exact_l2sq<D>(x, c0);
  }
  float best = __builtin_inff();
  uint32_t idx = 0xFFFFFFFFu;
  for (uint32_t c = sub; c < K; c += S) {
    float cv[D];
    load_padded<D>(lcb + c * DP, cv);
    const float d = exact_l2sq<D>(x, cv);
    if (d < best) {
      best = d;
      idx = c;
    }
  }
  group_lex_min<S>(best, idx);
  if (idx == 0xFFFFFFFFu) idx = 0;  // nothing below +inf: index 0, +inf
  if (SEED_FIRST && d0 != d0) {     // NaN at codeword 0 stays the minimum
    idx = 0;
    best = d0;
  }
  bidx = idx;
  bdist = best;
}

// The deferred vectors: the pruned exact search over all K codewords
// (pq_kernels.hpp), vectors gathered through the dense list defer[m][..];
// a persistent grid of gridDim.x blocks per subspace walks tiles of
// kBlock * VPT / S entries; each new code is added to its sort tile's count
// in hist[m][tile][code].  S > 1 (with VPT 1): S lanes share a vector's
// search (pruned_argmin_lanes), for K with Kp / kPruneBlock a multiple of
// S: a search is a serial chain over its codewords, and few deferred
// vectors leave few waves per SIMD to hide it; many deferred vectors keep
// the SIMDs busy anyway, and there one lane per vector costs less, so a
// subspace with `split` deferred vectors or more takes one lane per vector
// (the grid is sized for the S-lane tiles, which are smaller).  With stats
// (profiling): stats[0] += deferred vectors, stats[1] += n per subspace.
template <int D, int VPT, int S = 1>
__global__ __launch_bounds__(kBlock) void assign_list_kernel(
    const float* __restrict__ xs, const float* __restrict__ cb, uint16_t* __restrict__ codes,
    float* __restrict__ e, const uint32_t* __restrict__ defer,
    const uint32_t* __restrict__ defer_count, const uint32_t* __restrict__ done, uint64_t n,
    uint32_t K, unsigned long long* __restrict__ rescans, unsigned long long* __restrict__ stats,
    uint32_t* __restrict__ hist, uint32_t T, uint32_t split) {
  static_assert(S == 1 || VPT == 1, "lane groups take one vector each");
  constexpr int DP = Pad<D>::value;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t m = blockIdx.y;
  if (done[m]) return;
  const uint32_t cnt = defer_count[m];
  const bool lanes = S > 1 && cnt < split;  // uniform over the grid's subspace
  const uint32_t kTile = lanes ? kBlock * VPT / S : kBlock * VPT;
  if (stats && blockIdx.x == 0 && threadIdx.x == 0) {
    atomicAdd(&stats[0], (unsigned long long)cnt);
    atomicAdd(&stats[1], (unsigned long long)n);
  }
  if ((uint64_t)blockIdx.x * kTile >= cnt) return;
  const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
  float* lcb = lds;
  float* lnc = lds + Kp * DP;
  uint32_t& lmax = *reinterpret_cast<uint32_t*>(lnc + Kp);
  uint32_t& lcount = *(&lmax + 1);
  if (threadIdx.x == 0) {
    lmax = 0;
    lcount = 0;
  }
  __syncthreads();
  stage_pruned<D>(lcb, lnc, &lmax, cb + (uint64_t)m * K * D, K, Kp);
  __syncthreads();
  const float* xm = xs + (uint64_t)m * n * DP;
  const uint32_t* lst = defer + (uint64_t)m * n;
  uint32_t mine = 0;
  if constexpr (S > 1) {
    if (lanes) {
      const uint32_t sub = threadIdx.x % S;
      for (uint64_t t0 = (uint64_t)blockIdx.x * kTile; t0 < cnt; t0 += (uint64_t)gridDim.x * kTile) {
        const uint64_t q = t0 + threadIdx.x / S;
        const uint32_t idx = q < cnt ? lst[q] : 0xFFFFFFFFu;
        float x[D];
        if (idx != 0xFFFFFFFFu) {
          load_padded<D>(xm + (uint64_t)idx * DP, x);
        } else {
#pragma unroll
          for (int k = 0; k < D; ++k) x[k] = 0.0f;
        }
        uint32_t bidx;
        float best;
        pruned_argmin_lanes<D, S, true>(x, lcb, lnc, K, Kp, lmax, sub, bidx, best, mine);
        if (sub == 0 && idx != 0xFFFFFFFFu) {
          codes[(uint64_t)m * n + idx] = (uint16_t)bidx;
          e[(uint64_t)m * n + idx] = best;
          atomicAdd(&hist[((uint64_t)m * T + idx / kSortTile) * K + bidx], 1u);
        }
      }
      flush_rescans(mine, &lcount, rescans);
      return;
    }
  }
  for (uint64_t t0 = (uint64_t)blockIdx.x * kTile; t0 < cnt; t0 += (uint64_t)gridDim.x * kTile) {
    float x[VPT][D];
    uint32_t idx[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const uint64_t q = t0 + threadIdx.x + (uint64_t)j * kBlock;
      idx[j] = q < cnt ? lst[q] : 0xFFFFFFFFu;
      if (idx[j] != 0xFFFFFFFFu) {
        load_padded<D>(xm + (uint64_t)idx[j] * DP, x[j]);
      } else {
#pragma unroll
        for (int k = 0; k < D; ++k) x[j][k] = 0.0f;
      }
    }
    uint32_t bidx[VPT];
    float best[VPT];
    pruned_argmin<D, VPT, true>(x, lcb, lnc, K, Kp, lmax, bidx, best, mine);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (idx[j] != 0xFFFFFFFFu) {
        codes[(uint64_t)m * n + idx[j]] = (uint16_t)bidx[j];
        e[(uint64_t)m * n + idx[j]] = best[j];
        atomicAdd(&hist[((uint64_t)m * T + idx[j] / kSortTile) * K + bidx[j]], 1u);
      }
    }
  }
  flush_rescans(mine, &lcount, rescans);
}

// The deferred vectors of an encode: PQ.encode's scan semantics (best from
// +inf, strict <; src/index/pq.zig:64-73) through the pruned exact search,
// vectors gathered through defer[m][..] from the token-major input; codes
// to out[i][m].  Each thread takes VPT deferred vectors (their searches
// interleave), a persistent grid of gridDim.x blocks per subspace walks
// tiles of kBlock * VPT / S entries.  Two widths are launched back to back
// and a subspace's deferred count picks one: VPT 1 below a quarter of the
// rows, VPT 8 (the full search's interleave) above; the other launch returns
// at once.  S > 1 (with VPT 1): S lanes share a vector's search below
// `split` deferred vectors, one lane from there, as in assign_list_kernel.
template <int D, int VPT, typename CodeT, int S = 1>
__global__ __launch_bounds__(kBlock) void encode_list_kernel(
    const float* __restrict__ x, const float* __restrict__ cb, CodeT* __restrict__ out,
    const uint32_t* __restrict__ defer, const uint32_t* __restrict__ defer_count, uint64_t n,
    uint32_t dim, uint32_t M, uint32_t K, unsigned long long* __restrict__ rescans,
    unsigned long long* __restrict__ stats, uint32_t split) {
  static_assert(S == 1 || VPT == 1, "lane groups take one vector each");
  constexpr int DP = Pad<D>::value;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t m = blockIdx.y;
  const uint32_t cnt = defer_count[m];
  const bool wide = 4ull * cnt > n;
  if ((VPT > 1) != wide) return;  // the other width serves this subspace
  const bool lanes = S > 1 && cnt < split;
  const uint32_t kTile = lanes ? kBlock * VPT / S : kBlock * VPT;
  if (stats && blockIdx.x == 0 && threadIdx.x == 0) {
    atomicAdd(&stats[0], (unsigned long long)cnt);
    atomicAdd(&stats[1], (unsigned long long)n);
  }
  if ((uint64_t)blockIdx.x * kTile >= cnt) return;
  const uint32_t Kp = (K + kPruneBlock - 1) / kPruneBlock * kPruneBlock;
  float* lcb = lds;
  float* lnc = lds + Kp * DP;
  uint32_t& lmax = *reinterpret_cast<uint32_t*>(lnc + Kp);
  uint32_t& lcount = *(&lmax + 1);
  if (threadIdx.x == 0) {
    lmax = 0;
    lcount = 0;
  }
  __syncthreads();
  stage_pruned<D>(lcb, lnc, &lmax, cb + (uint64_t)m * K * D, K, Kp);
  __syncthreads();
  const uint32_t* lst = defer + (uint64_t)m * n;
  uint32_t mine = 0;
  if constexpr (S > 1) {
    if (lanes) {
      const uint32_t sub = threadIdx.x % S;
      for (uint64_t t0 = (uint64_t)blockIdx.x * kTile; t0 < cnt; t0 += (uint64_t)gridDim.x * kTile) {
        const uint64_t q = t0 + threadIdx.x / S;
        const uint32_t idx = q < cnt ? lst[q] : 0xFFFFFFFFu;
        const float* src = x + (uint64_t)(idx != 0xFFFFFFFFu ? idx : 0u) * dim + (uint64_t)m * D;
        float xv[D];
#pragma unroll
        for (int k = 0; k < D; ++k) xv[k] = src[k];
        uint32_t bidx;
        float best;
        pruned_argmin_lanes<D, S, false>(xv, lcb, lnc, K, Kp, lmax, sub, bidx, best, mine);
        if (sub == 0 && idx != 0xFFFFFFFFu) out[(uint64_t)idx * M + m] = (CodeT)bidx;
      }
      flush_rescans(mine, &lcount, rescans);
      return;
    }
  }
  for (uint64_t t0 = (uint64_t)blockIdx.x * kTile; t0 < cnt; t0 += (uint64_t)gridDim.x * kTile) {
    float xv[VPT][D];
    uint32_t idx[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const uint64_t q = t0 + threadIdx.x + (uint64_t)j * kBlock;
      idx[j] = q < cnt ? lst[q] : 0xFFFFFFFFu;
      const float* src = x + (uint64_t)(idx[j] != 0xFFFFFFFFu ? idx[j] : 0u) * dim +
                         (uint64_t)m * D;
#pragma unroll
      for (int k = 0; k < D; ++k) xv[j][k] = src[k];
    }
    uint32_t bidx[VPT];
    float best[VPT];
    pruned_argmin<D, VPT, false>(xv, lcb, lnc, K, Kp, lmax, bidx, best, mine);
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      if (idx[j] != 0xFFFFFFFFu) out[(uint64_t)idx[j] * M + m] = (CodeT)bidx[j];
  }
  flush_rescans(mine, &lcount, rescans);
}

}  // namespace tacgpu
