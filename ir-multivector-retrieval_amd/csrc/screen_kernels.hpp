// screen_kernels.hpp — the full search for sub-dimensions 5-8 (records of 8
// floats) and K <= 256 with its first pass on the matrix cores, for the Lloyd
// assignment and for encode.  Included once, by tac_gpu.hip, after
// cand_kernels.hpp.
//
// Screen.  For a vector x and codeword c (dimensions past D are 0), the
// search ranks codewords by s(c) = ||c||^2 - 2 x.c.  Here s comes from two
// chained v_mfma_f32_32x32x16_bf16 per 32 codewords x 32 vectors, 32
// products added to the accumulator input n = fl(sum_d c_d^2):
//   A = [a_hi | a_lo] with B = [x_hi | x_hi], then A with B = [x_lo | x_lo]
// (8 slots each half) with a = -2 c (exact), v_hi = bf16(v), v_lo =
// bf16(v - v_hi) (round to nearest even), so the products sum to
// (a_hi + a_lo) . (x_hi + x_lo).  For a finite v, |v - v_hi - v_lo| <=
// 2^-16 |v| + 2^-125 (the absolute term covers subnormal or flushed pieces),
// so per dimension the products miss a x_d by at most
// 2.0001 * 2^-16 |a| |x_d| + 2^-124.9 (|a| + |x_d|); n is within gamma_8 ||c||^2
// of ||c||^2; the bf16 products are exact in fp32 but for underflow (2^-126
// each); and the matrix core adds the 33 terms in fp32 in some order
// (gamma_32 of their absolute sum, at most 2^-19 (2.032 ||x|| ||c|| + ||c||^2),
// plus 2^-126 per addition if partial sums flush).  Altogether
//   |s~ - s| <= 2^-14 (1.07 ||x|| ||c|| + 0.04 ||c||^2) + 2^-123 (2 ||c|| + ||x||) + 2^-120,
// and the kernel uses twice that with cmax^2 = max_c fl(||c||^2) in place of
// ||c||^2.  It needs fl(||x||^2) <= 2^120 and cmax^2 <= 2^120
// (false for a NaN or infinite component): every component is then below
// 2^60 (times 1 + 4u), so no product or partial sum overflows.  A codebook
// past that sends every vector to the deferred list below, a vector past it
// goes there alone.
//
// Layout and the exact result.  The codeword pieces are the A operand
// (lane l: codeword 32 g + l % 32, piece l / 32) and the vector pieces the B
// operand (lane l: vector l % 32 of a 32-vector group), so lane l holds the
// screen values of its vector against codewords 32 g + 8 j + 4 (l / 32) + i,
// j, i < 4, of codeword group g.  It folds them into the minima of blocks of
// 8 (j 0-1 and j 2-3) and keeps the two smallest block minima; the blocks of
// the vector's two lanes partition the codewords.  After the two lanes merge
// their top-2 (a permlane swap: both lanes end with the same result), the
// argument of pruned_argmin (pq_kernels.hpp) applies unchanged: when the gap
// between the two smallest block minima exceeds the threshold built from the
// screen bound and the reference distance's gamma_{D+2}, the reference's
// first-index argmin lies in the winning block, whose codewords then get the
// reference distance (four per lane, merged by (distance, index)).  Equal
// block minima leave no gap.  A vector without the gap joins the subspace's
// deferred list, whose pruned exact search (assign_list_kernel or
// encode_list_kernel, cand_kernels.hpp) follows: about 0.5% of the corpus
// rows at m8/d8, far fewer than the waves that would stall on an in-wave
// scan of all K codewords.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cand_kernels.hpp"
#include "screen_rules.hpp"

namespace tacgpu {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kScreenMaxK = 256;     // codewords in the kernel's LDS table
constexpr uint32_t kScreenVecGroups = 2;  // 32-vector groups per wave pass

// Minimum and maximum in the IEEE 754-2019 sense (v_minimum3_f32 /
// v_maximum3_f32: no canonicalising moves, which fminf / fmaxf add in IEEE
// mode); the screen's operands are never NaN where the results count (tame
// vectors and codebooks, +inf padding).
__device__ __forceinline__ float min2f(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float min3f(float a, float b, float c) { return min2f(min2f(a, b), c); }

// The values of lanes l and l ^ 16 (R = 16) or l and l ^ 32 (R = 32), as a
// pair that is the same in both lanes (v_permlane16_swap / v_permlane32_swap
// of v with itself); reductions over the pair are symmetric in it.
template <int R>
__device__ __forceinline__ void pair_of(uint32_t v, uint32_t& a, uint32_t& b) {
  static_assert(R == 16 || R == 32, "row pairs");
  if constexpr (R == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = s[0];
    b = s[1];
  } else {
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = s[0];
    b = s[1];
  }
}

// Merge the top-2 block minima (b1 <= b2, block bb of b1) of lanes l and l ^ R.
template <int R>
__device__ __forceinline__ void screen_merge(float& b1, float& b2, uint32_t& bb) {
  uint32_t d1, s1, d2, s2, db, sb;
  pair_of<R>(__float_as_uint(b1), d1, s1);
  pair_of<R>(__float_as_uint(b2), d2, s2);
  pair_of<R>(bb, db, sb);
  const float D1 = __uint_as_float(d1), S1 = __uint_as_float(s1);
  // second smallest of {D1, D2, S1, S2} with D1 <= D2, S1 <= S2
  b2 = min3f(max2f(D1, S1), __uint_as_float(d2), __uint_as_float(s2));
  bb = S1 < D1 ? sb : db;  // ties leave b2 == b1: no gap
  b1 = min2f(D1, S1);
}

// (d, c) <- the smaller of the (distance, index) pairs of lanes l and l ^ R.
template <int R>
__device__ __forceinline__ void screen_lex_min(float& d, uint32_t& c) {
  uint32_t dd, sd, dc, sc;
  pair_of<R>(__float_as_uint(d), dd, sd);
  pair_of<R>(c, dc, sc);
  const float Dv = __uint_as_float(dd), Sv = __uint_as_float(sd);
  const bool s_wins = Sv < Dv || (Sv == Dv && sc < dc);
  d = s_wins ? Sv : Dv;
  c = s_wins ? sc : dc;
}

// The full search for D in 5..8 and K <= kScreenMaxK = blockDim.x, one
// block of 4 waves per (tile of kSortTile rows, subspace m), 64 vectors per
// wave pass.  The vectors the screen settles get their code (the first index
// of the minimum: vec.argmin's and PQ.encode's scan agree on finite
// distances); the others go to defer[m][..] (defer_count[m] must be zero at
// the launch, and the deferred-list kernel of the same semantics must
// follow).
//  - Lloyd assignment (ENCODE false; CodeT uint16_t): x = xs [M][n][8]
//    records, blockIdx.x = tile, blockIdx.y = m; codes[m][i], e[m][i] =
//    reference distance; hist[m][tile][c] = the settled vectors of the tile
//    with code c (assign_list_kernel adds the deferred ones).
//  - Encode (ENCODE true): x = token-major rows [n][dim], sub-vector m at
//    m * D; the M blocks of a tile are adjacent in an XCD's share of the
//    grid (xcd_contiguous), so a row crosses HBM once; codes[i * M + m];
//    encode_list_kernel follows.
template <int D, bool ENCODE, typename CodeT>
__global__ __launch_bounds__(256) void screen_kernel(
    const float* __restrict__ x_in, const float* __restrict__ cb, CodeT* __restrict__ codes,
    float* __restrict__ e, uint32_t* __restrict__ defer, uint32_t* __restrict__ defer_count,
    const uint32_t* __restrict__ done, uint64_t n, uint32_t dim, uint32_t M, uint32_t K,
    uint32_t* __restrict__ hist, uint32_t T) {
  static_assert(D >= 5 && D <= 8, "records of 8 floats");
  static_assert(kSortTile % (4 * 32 * kScreenVecGroups) == 0, "whole wave passes per tile");
  constexpr uint32_t VG = kScreenVecGroups;
  // [g][h][c % 32]: the pieces a_hi (h 0), a_lo (h 1) of codeword c in group g
  // (each half-wave reads 32 consecutive entries)
  __shared__ bf16x8 lA[kScreenMaxK * 2];
  // norms in accumulator order: codeword 32 g + 8 j + 4 h + i at 32 g + 16 h + 4 j + i,
  // +inf past K
  __shared__ __attribute__((aligned(16))) float lnorm[kScreenMaxK];
  __shared__ __attribute__((aligned(16))) float lcb[kScreenMaxK * 8];  // fp32 codewords
  __shared__ uint32_t s_hist[kScreenMaxK];
  __shared__ uint32_t s_list[kSortTile];  // the tile's deferred rows
  __shared__ uint32_t s_max, s_cnt, s_base;
  uint32_t m, tile;
  if constexpr (ENCODE) {
    const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
    if (logical >= T * M) return;  // grid padding to a multiple of 8
    tile = logical / M;
    m = logical % M;
  } else {
    tile = blockIdx.x;
    m = blockIdx.y;
    if (done[m]) return;
  }
  const uint32_t t = threadIdx.x, lane = t % kWave, w = t / kWave;
  const uint32_t col = lane % 32, h = lane / 32;
  const uint32_t ngroups = (K + 31u) / 32u;  // codeword groups of 32 (padding past K)
  if (t == 0) {
    s_max = 0;
    s_cnt = 0;
  }
  if (!ENCODE && t < K) s_hist[t] = 0;
  {
    // The pieces of codeword c = t, padding past K.
    const uint32_t c = t;
    const float* cbm = cb + (uint64_t)m * K * D;
    float v[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) v[d] = (c < K && d < D) ? cbm[(uint64_t)c * D + d] : 0.0f;
    float n2 = v[0] * v[0];
#pragma unroll
    for (int d = 1; d < D; ++d) n2 = n2 + v[d] * v[d];
    bf16x8 ch, cl;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const float a = -2.0f * v[d];  // exact
      const __bf16 hi = (__bf16)a;
      ch[d] = hi;
      cl[d] = (__bf16)(a - (float)hi);
      lcb[c * 8 + d] = v[d];
    }
    const uint32_t r = c % 32;
    lnorm[(c - r) + 16 * ((r / 4) % 2) + 4 * (r / 8) + r % 4] = c < K ? n2 : __builtin_inff();
    lA[(c - r) * 2 + r] = ch;
    lA[(c - r) * 2 + 32 + r] = cl;
    // the largest norm's bits (norms are non-negative or NaN, and a NaN's
    // bits sort above +inf's)
    uint32_t mx = c < K ? __float_as_uint(n2) : 0u;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const uint32_t other = (uint32_t)__shfl_xor((int)mx, o, kWave);
      mx = other > mx ? other : mx;
    }
    __syncthreads();  // s_max cleared
    if (lane == 0) atomicMax(&s_max, mx);
  }
  __syncthreads();
  const float cmax2 = __uint_as_float(s_max);
  const bool cb_ok = cmax2 <= kScreenTame;  // false on NaN
  const float cmax = sqrtf(cmax2);
  const float* xm = ENCODE ? x_in + (uint64_t)m * D : x_in + (uint64_t)m * n * 8;
  const bool vec4 = !ENCODE || (D == 8 && dim % 4 == 0 &&
                                 ((uintptr_t)x_in & 15u) == 0);  // 16-byte aligned rows
  const uint64_t tile0 = (uint64_t)tile * kSortTile;
  const uint64_t tile1 = tile0 + kSortTile < n ? tile0 + kSortTile : n;
  const bf16x8* arow = lA + h * 32 + col;                              // + 64 per group
  const floatx4* nrow = reinterpret_cast<const floatx4*>(lnorm) + h * 4;  // + 8 per group
  for (uint64_t row0 = tile0 + w * (32 * VG); row0 < tile1; row0 += 4 * 32 * VG) {
    // B operands of vector row0 + 32 vg + col: [x_hi | x_hi] and [x_lo | x_lo];
    // rows past the tile repeat its last row and are not written.
    bf16x8 Xh[VG], Xl[VG];
    float x[VG][D], x2[VG];
#pragma unroll
    for (uint32_t vg = 0; vg < VG; ++vg) {
      const uint64_t r = row0 + 32 * vg + col;
      const uint64_t rr = r < tile1 ? r : tile1 - 1;
      const float* src = xm + rr * (ENCODE ? (uint64_t)dim : 8u);
      float xv[8];
      if (vec4) {
        const float4 a0 = *reinterpret_cast<const float4*>(src);
        const float4 a1 = *reinterpret_cast<const float4*>(src + 4);
        xv[0] = a0.x; xv[1] = a0.y; xv[2] = a0.z; xv[3] = a0.w;
        xv[4] = a1.x; xv[5] = a1.y; xv[6] = a1.z; xv[7] = a1.w;
      } else {
#pragma unroll
        for (int d = 0; d < 8; ++d) xv[d] = d < D ? src[d] : 0.0f;
      }
#pragma unroll
      for (int d = 0; d < D; ++d) x[vg][d] = xv[d];
      // ||x||^2 for the bound and the tameness test (any rounding order does)
      float s2 = xv[0] * xv[0];
#pragma unroll
      for (int d = 1; d < D; ++d) s2 = __builtin_fmaf(xv[d], xv[d], s2);
      x2[vg] = s2;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const float xd = d < D ? xv[d] : 0.0f;
        Xh[vg][d] = (__bf16)xd;
        Xl[vg][d] = (__bf16)(xd - (float)Xh[vg][d]);
      }
    }
    // First pass: this lane holds codewords 32 g + 8 j + 4 h + i (j, i < 4) of
    // its vector; blocks of 8 (j 0-1 and j 2-3) numbered (2 g + s) 2 + h, the
    // two smallest block minima per vector.
    float b1[VG], b2[VG];
    uint32_t bb[VG];
#pragma unroll
    for (uint32_t vg = 0; vg < VG; ++vg) {
      b1[vg] = __builtin_inff();
      b2[vg] = __builtin_inff();
      bb[vg] = h;
    }
    for (uint32_t g = 0; g < ngroups; ++g) {
      const bf16x8 A = arow[g * 64];
      const floatx4 n0 = nrow[g * 8 + 0], n1 = nrow[g * 8 + 1];
      const floatx4 n2 = nrow[g * 8 + 2], n3 = nrow[g * 8 + 3];
      const floatx16 N = {n0[0], n0[1], n0[2], n0[3], n1[0], n1[1], n1[2], n1[3],
                          n2[0], n2[1], n2[2], n2[3], n3[0], n3[1], n3[2], n3[3]};
#pragma unroll
      for (uint32_t vg = 0; vg < VG; ++vg) {
        floatx16 c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Xh[vg], N, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Xl[vg], c, 0, 0, 0);
#pragma unroll
        for (uint32_t sb = 0; sb < 2; ++sb) {
          const float v = min2f(min3f(min3f(c[8 * sb], c[8 * sb + 1], c[8 * sb + 2]),
                                      min2f(c[8 * sb + 3], c[8 * sb + 4]),
                                      min2f(c[8 * sb + 5], c[8 * sb + 6])),
                                c[8 * sb + 7]);
          const uint32_t blk = (2 * g + sb) * 2 + h;
          b2[vg] = min2f(b2[vg], max2f(b1[vg], v));  // second smallest (b1 <= b2)
          bb[vg] = v < b1[vg] ? blk : bb[vg];
          b1[vg] = min2f(b1[vg], v);
        }
      }
    }
#pragma unroll
    for (uint32_t vg = 0; vg < VG; ++vg) screen_merge<32>(b1[vg], b2[vg], bb[vg]);
    // The threshold test, then the reference distance to the winning block
    // (lane h takes its codewords 32 g + 8 (2 s + h) + 4 hw + i), or the
    // deferred list.
#pragma unroll
    for (uint32_t vg = 0; vg < VG; ++vg) {
      const uint64_t r = row0 + 32 * vg + col;
      // an upper bound of ||x|| from the raw square root (1 ulp, so the
      // factor), floored at 2^-50: the bound needs no more precision
      const float nx = __builtin_amdgcn_sqrtf(max2f(x2[vg], 7.888609052210118e-31f)) * 1.000001f;
      // b2 = +inf: every other block holds padding only (a tame codeword's
      // screen value is finite), so the winning block holds every codeword.
      const bool ok = cb_ok && x2[vg] <= kScreenTame &&
                      screen_separates<D>(b1[vg], b2[vg], x2[vg], screen_err(nx, cmax, cmax2));
      if (ok) {
        float best = __builtin_inff();
        uint32_t idx = 0xFFFFFFFFu;
        const uint32_t g = bb[vg] / 4, sb = (bb[vg] / 2) % 2, hw = bb[vg] % 2;
        const uint32_t c0 = 32 * g + 8 * (2 * sb + h) + 4 * hw;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
          const uint32_t c = c0 + i;
          if (c < K) {
            float cv[D];
            load_padded<D>(lcb + c * 8, cv);
            const float d2 = exact_l2sq<D>(x[vg], cv);
            if (d2 < best) {  // c rises with i: the first of this lane's ties stays
              best = d2;
              idx = c;
            }
          }
        }
        screen_lex_min<32>(best, idx);
        if (h == 0 && r < tile1) {
          if constexpr (ENCODE) {
            codes[r * M + m] = (CodeT)idx;
          } else {
            codes[(uint64_t)m * n + r] = (CodeT)idx;
            e[(uint64_t)m * n + r] = best;
            atomicAdd(&s_hist[idx], 1u);
          }
        }
      } else if (h == 0 && r < tile1) {
        s_list[atomicAdd(&s_cnt, 1u)] = (uint32_t)r;  // at most kSortTile rows
      }
    }
  }
  __syncthreads();
  if constexpr (!ENCODE) {
    uint32_t* out = hist + ((uint64_t)m * T + tile) * K;
    if (t < K) out[t] = s_hist[t];
  }
  const uint32_t cnt = s_cnt;
  if (cnt == 0) return;
  if (t == 0) s_base = atomicAdd(&defer_count[m], cnt);
  __syncthreads();
  uint32_t* lst = defer + (uint64_t)m * n + s_base;
  for (uint32_t i = t; i < cnt; i += blockDim.x) lst[i] = s_list[i];
}

}  // namespace tacgpu
