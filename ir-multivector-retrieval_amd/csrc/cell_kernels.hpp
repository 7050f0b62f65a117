// cell_kernels.hpp — cell-list encode (PQ.encode, src/index/pq.zig:59-76, over
// token-major rows as storage.build encodes them, src/index/storage.zig:384-401)
// for sub-dimensions 1-4 and K <= 256.  Included once, by tac_gpu.hip, after
// cand_kernels.hpp.
//
// Per subspace, a uniform grid (cell_rules.hpp) covers the codebook's
// bounding box joined with mean +- 3 sigma of a strided sample of the rows
// being encoded.  Every fine cell lists the codewords that can be the
// reference's first-index argmin anywhere in the cell (cell_rules.hpp gives
// the exclusion test and why it is exact); lists are built coarse to fine:
// a coarse cell tests all K codewords against the codeword nearest its
// centre, each of its fine cells tests the coarse list against the coarse
// list's codeword nearest the fine centre.  The encode pass then evaluates,
// for every vector inside the grid, all entries of its cell's list with the
// reference distance and keeps the lexicographic (distance bits, index)
// minimum, which is the reference's code.  Lists are padded with the fine
// anchor to whole items of kCellItem (4) entries, and a wave's vectors have
// their items laid out over its lanes by a scan of their counts.  Vectors
// outside the grid (and NaN) and cells whose list passes kCellMaxItems items
// take the pruned full search through the deferred list.  A subspace takes
// this pass when many of its rows lie outside the codebook's box and its
// codebook and grid are tame (cell_box_kernel); the others take the anchored
// candidate encode (cand_kernels.hpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cand_kernels.hpp"
#include "cell_rules.hpp"

namespace tacgpu {

// Grid parameters per subspace, 16 words: lo[0..3] and s[4..7] as f32 bits,
// [8] 1 when the grid is usable, [9] the list items handed out so far.
constexpr uint32_t kCellParWords = 16;
constexpr uint32_t kCellSample = 4096;      // rows sampled for the grid box
constexpr uint32_t kCellItemsPerCell = 8;   // list space per subspace: items per cell
constexpr uint32_t kCellWaveItems = 1024;   // items a wave lays out per 64 vectors
// Share of a subspace's sampled rows outside the codebook's bounding box past
// which the cell lists serve it: the anchored encode leaves such rows to the
// full search.
constexpr double kCellOutside = 0.15;
// Rows per encode call from which the choice is made at all (below it every
// subspace takes the anchored pass: the choice costs the box kernel and the
// other pass's launches, about 0.1 ms).
constexpr uint64_t kCellMinRows = 1ull << 22;

// One block per subspace: the codebook's bounding box and finiteness, then
// over a strided sample of the rows the share outside that box and the
// per-dimension mean and standard deviation (finite values only), the grid
// origin and scale (cell_grid_params), and the pass the subspace takes:
// par[m][8] = sel[m] = 1 for the cell lists (mode 1, or mode -1 with more
// than kCellOutside of the sample outside the box), 0 for the anchored
// encode.  Also clears the item counter and the subspace's deferred count.
template <int D>
__global__ __launch_bounds__(256) void cell_box_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ cb,
                                                       uint32_t* __restrict__ par,
                                                       uint32_t* __restrict__ sel,
                                                       uint32_t* __restrict__ defer_count,
                                                       uint64_t n, uint32_t dim, uint32_t K,
                                                       int mode,
                                                       unsigned long long* __restrict__ cells_stat) {
  constexpr int kRows = kCellSample / 256;  // sample rows per thread
  const uint32_t m = blockIdx.x, t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const uint32_t nw = blockDim.x / kWave;
  __shared__ double red[4][5 * D];
  __shared__ double cbox[2 * D];
  __shared__ uint32_t wbad[4], wout[4];
  // the sample's rows, loaded first
  const uint64_t S = n < kCellSample ? n : kCellSample;
  const uint64_t stride = S ? n / S : 1;
  float v[kRows][D];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const uint64_t q = t + (uint64_t)r * 256u;
    const float* row = x + (q < S ? q : 0) * stride * dim + (uint64_t)m * D;
#pragma unroll
    for (int j = 0; j < D; ++j) v[r][j] = q < S ? row[j] : __builtin_nanf("");
  }
  // the codebook's box
  double mn[D], mx[D];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    mn[j] = __builtin_inf();
    mx[j] = -__builtin_inf();
  }
  const float* cbm = cb + (uint64_t)m * K * D;
  for (uint32_t c = t; c < K; c += blockDim.x)
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const float f = cbm[(uint64_t)c * D + j];
      if (!(f - f == 0.0f)) bad = true;  // inf or NaN
      mn[j] = fmin(mn[j], (double)f);
      mx[j] = fmax(mx[j], (double)f);
    }
  for (int off = kWave / 2; off > 0; off >>= 1)
#pragma unroll
    for (int j = 0; j < D; ++j) {
      mn[j] = fmin(mn[j], __shfl_xor(mn[j], off, kWave));
      mx[j] = fmax(mx[j], __shfl_xor(mx[j], off, kWave));
    }
  const bool any_bad = __ballot(bad) != 0;
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      red[wave][j] = mn[j];
      red[wave][D + j] = mx[j];
    }
    wbad[wave] = any_bad ? 1u : 0u;
  }
  __syncthreads();
  if (t < (uint32_t)D) {
    double lo = red[0][t], hi = red[0][D + t];
    for (uint32_t w = 1; w < nw; ++w) {
      lo = fmin(lo, red[w][t]);
      hi = fmax(hi, red[w][D + t]);
    }
    cbox[t] = lo;
    cbox[D + t] = hi;
  }
  __syncthreads();
  // the sample against the box: rows outside it, moments of the finite values
  double sm[D], sq[D], ct[D];
#pragma unroll
  for (int j = 0; j < D; ++j) sm[j] = sq[j] = ct[j] = 0.0;
  uint32_t out = 0;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const uint64_t q = t + (uint64_t)r * 256u;
    bool outside = false;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const double d = (double)v[r][j];
      outside = outside || !(d >= cbox[j] && d <= cbox[D + j]);
      if (d > -1e30 && d < 1e30) {
        sm[j] += d;
        sq[j] += d * d;
        ct[j] += 1.0;
      }
    }
    out += (q < S && outside) ? 1u : 0u;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      sm[j] += __shfl_xor(sm[j], off, kWave);
      sq[j] += __shfl_xor(sq[j], off, kWave);
      ct[j] += __shfl_xor(ct[j], off, kWave);
    }
    out += (uint32_t)__shfl_xor((int)out, off, kWave);
  }
  __syncthreads();  // red is reused
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      red[wave][2 * D + j] = sm[j];
      red[wave][3 * D + j] = sq[j];
      red[wave][4 * D + j] = ct[j];
    }
    wout[wave] = out;
  }
  __syncthreads();
  if (t != 0) return;
  bool ok = K > 0;
  uint32_t outside_rows = 0;
  for (uint32_t w = 0; w < nw; ++w) {
    ok = ok && wbad[w] == 0;
    outside_rows += wout[w];
  }
  uint32_t* pm = par + (uint64_t)m * kCellParWords;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    double lo = cbox[j], hi = cbox[D + j], s1 = 0, s2 = 0, c = 0;
    for (uint32_t w = 0; w < nw; ++w) {
      s1 += red[w][2 * D + j];
      s2 += red[w][3 * D + j];
      c += red[w][4 * D + j];
    }
    if (c > 0) {
      const double mu = s1 / c;
      const double var = fmax(s2 / c - mu * mu, 0.0);
      const double sd = sqrt(var);
      lo = fmin(lo, mu - 3.0 * sd);
      hi = fmax(hi, mu + 3.0 * sd);
    }
    float lf = 0.0f, sf = 0.0f;
    if (!ok || !cell_grid_params(lo, hi, cell_side(D), &lf, &sf)) ok = false;
    pm[j] = __float_as_uint(lf);
    pm[4 + j] = __float_as_uint(sf);
  }
  const bool wide = (double)outside_rows > kCellOutside * (double)S;
  const bool use = ok && (mode == 1 || (mode < 0 && wide));
  pm[8] = use ? 1u : 0u;
  pm[9] = 0u;
  sel[m] = use ? 1u : 0u;
  defer_count[m] = 0;
  if (use && cells_stat) atomicAdd(cells_stat, 1ull);
}

template <int D>
__device__ inline void cell_params(const uint32_t* __restrict__ pm, float (&lo)[D],
                                   float (&s)[D]) {
#pragma unroll
  for (int j = 0; j < D; ++j) {
    lo[j] = __uint_as_float(pm[j]);
    s[j] = __uint_as_float(pm[4 + j]);
  }
}

// The subspace's codewords as doubles and its grid axes, staged in LDS by a
// whole block (K <= 256).
template <int D>
__device__ inline void cell_stage(const float* __restrict__ cbm, const uint32_t* __restrict__ pm,
                                  uint32_t K, double* lcb, CellAxis* lax) {
  for (uint32_t i = threadIdx.x; i < K * D; i += blockDim.x) lcb[i] = (double)cbm[i];
  if (threadIdx.x < (uint32_t)D)
    lax[threadIdx.x] = cell_axis(__uint_as_float(pm[threadIdx.x]), __uint_as_float(pm[4 + threadIdx.x]));
}

// The nearest of the codewords ids[0 .. cnt) (all K when ids is null) to
// the point p, exact double distances, the first on ties; returns its
// position in the list.
template <int D>
__device__ inline uint32_t cell_nearest(const double* lcb, const uint8_t* ids, uint32_t cnt,
                                        const double (&p)[D]) {
  double bd = __builtin_inf();
  uint32_t be = 0;
#pragma unroll 4
  for (uint32_t e = 0; e < cnt; ++e) {
    const double* v = lcb + (ids ? (uint32_t)ids[e] : e) * D;
    double dist = 0.0;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const double d = p[j] - v[j];
      dist += d * d;
    }
    if (dist < bd) {
      bd = dist;
      be = e;
    }
  }
  return be;
}

// One wave per coarse cell, four per block, lanes over the codewords
// (K <= 256): the anchor is the codeword nearest the coarse box's centre
// (first index on ties), and the codewords the exclusion test keeps are
// listed in index order: cids[m][q][0 .. ccnt[m][q]).
template <int D>
__global__ __launch_bounds__(256) void cell_coarse_kernel(const float* __restrict__ cb,
                                                          const uint32_t* __restrict__ par,
                                                          uint8_t* __restrict__ cids,
                                                          uint32_t* __restrict__ ccnt,
                                                          uint32_t K) {
  constexpr uint32_t Gc = cell_coarse_side(D), Gs = cell_sub_side(D), Cc = cell_coarse_count(D);
  const uint32_t m = blockIdx.y, t = threadIdx.x, lane = t % kWave;
  const uint32_t q = blockIdx.x * (blockDim.x / kWave) + t / kWave;
  const uint32_t* pm = par + (uint64_t)m * kCellParWords;
  if (pm[8] == 0) return;  // the anchored pass serves this subspace
  __shared__ double lcb[256 * D];
  __shared__ CellAxis lax[D];
  cell_stage<D>(cb + (uint64_t)m * K * D, pm, K, lcb, lax);
  __syncthreads();
  if (q >= Cc) return;
  double a[D], b[D], mid[D];
  uint32_t r = q;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const uint32_t kc = r % Gc;
    r /= Gc;
    cell_interval_axis(lax[j], kc * Gs, kc * Gs + Gs, &a[j], &b[j]);
    mid[j] = 0.5 * (a[j] + b[j]);
  }
  // lane l holds codewords l, l + 64, l + 128, l + 192
  double bd = __builtin_inf();
  uint32_t bc = 0xFFFFFFFFu;
#pragma unroll
  for (uint32_t h = 0; h < 4; ++h) {
    const uint32_t c = lane + h * kWave;
    if (c < K) {
      double dist = 0.0;
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const double d = mid[j] - lcb[c * D + j];
        dist += d * d;
      }
      if (dist < bd) {  // c rises with h: the first of a lane's ties stays
        bd = dist;
        bc = c;
      }
    }
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const double od = __shfl_xor(bd, off, kWave);
    const uint32_t oc = (uint32_t)__shfl_xor((int)bc, off, kWave);
    if (od < bd || (od == bd && oc < bc)) {
      bd = od;
      bc = oc;
    }
  }
  const uint32_t c0 = bc < K ? bc : 0u;
  double v0[D];
#pragma unroll
  for (int j = 0; j < D; ++j) v0[j] = lcb[c0 * D + j];
  const double mt0 = cell_max_t<D>(v0, a, b);
  const double g = cell_gamma(D);
  uint8_t* dst = cids + ((uint64_t)m * Cc + q) * K;
  uint32_t cnt = 0;
#pragma unroll
  for (uint32_t h = 0; h < 4; ++h) {
    const uint32_t c = lane + h * kWave;
    bool keep = false;
    if (c < K) {
      double v[D];
#pragma unroll
      for (int j = 0; j < D; ++j) v[j] = lcb[c * D + j];
      keep = c == c0 || !cell_excluded<D>(v, v0, mt0, a, b, g);
    }
    const uint64_t bal = __ballot(keep);
    if (keep) dst[cnt + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull))] = (uint8_t)c;
    cnt += (uint32_t)__popcll(bal);
  }
  if (lane == 0) ccnt[(uint64_t)m * Cc + q] = cnt;
}

// One block per 256 / F coarse cells of a subspace, one thread per fine cell
// (F fine cells per coarse cell): the fine anchor is the coarse-list
// codeword nearest the fine box's centre, the list keeps the coarse-list
// codewords the exclusion test keeps (coarse-list order), padded with the
// anchor to whole items of kCellItem.  The block's lists take one run of the
// subspace's item space (an atomic on its counter); a cell past
// kCellMaxItems items, or every cell of a block whose run would overflow the
// space, gets record 0 (deferred).  rec[m][cell] = first item | items << 24.
template <int D>
__global__ __launch_bounds__(256) void cell_fine_kernel(const float* __restrict__ cb,
                                                        uint32_t* __restrict__ par,
                                                        const uint8_t* __restrict__ cids,
                                                        const uint32_t* __restrict__ ccnt,
                                                        uint32_t* __restrict__ rec,
                                                        uint8_t* __restrict__ lists, uint32_t K,
                                                        uint32_t cap_items) {
  constexpr uint32_t Gc = cell_coarse_side(D), Gs = cell_sub_side(D), Cc = cell_coarse_count(D);
  constexpr uint32_t F = cell_fine_per_coarse(D), CPB = 256 / F, cells = cell_count(D);
  const uint32_t m = blockIdx.y, t = threadIdx.x;
  const uint32_t r = t / F, f = t % F;
  const uint32_t q = blockIdx.x * CPB + r;
  const bool live = r < CPB && q < Cc;
  uint32_t* pm = par + (uint64_t)m * kCellParWords;
  uint32_t* recm = rec + (uint64_t)m * cells;
  if (pm[8] == 0) return;  // the anchored pass serves this subspace
  __shared__ double lcb[256 * D];
  __shared__ CellAxis lax[D];
  __shared__ __attribute__((aligned(4))) uint8_t lids[CPB][256];
  __shared__ uint32_t lcnt[CPB], scan[256], sbase;
  cell_stage<D>(cb + (uint64_t)m * K * D, pm, K, lcb, lax);
  // Entries past a coarse list's count are read (and ignored) by the
  // four-entry steps: they stay valid ids.
  for (uint32_t i = t; i < CPB * 256u; i += blockDim.x) {
    const uint32_t r2 = i / 256u, e = i % 256u, q2 = blockIdx.x * CPB + r2;
    lids[r2][e] = (q2 < Cc && e < K) ? cids[((uint64_t)m * Cc + q2) * K + e] : 0u;
  }
  if (t < CPB) {
    const uint32_t q2 = blockIdx.x * CPB + t;
    lcnt[t] = q2 < Cc ? ccnt[(uint64_t)m * Cc + q2] : 0u;
  }
  __syncthreads();
  uint32_t nit = 0, c0 = 0, cnt = 0;
  uint32_t mask[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) mask[w] = 0u;
  if (live) {
    cnt = lcnt[r];
    double a[D], b[D], mid[D];
    uint32_t rq = q, rf = f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const uint32_t k = (rq % Gc) * Gs + rf % Gs;
      rq /= Gc;
      rf /= Gs;
      cell_interval_axis(lax[j], k, k + 1, &a[j], &b[j]);
      mid[j] = 0.5 * (a[j] + b[j]);
    }
    const uint8_t* ids = lids[r];
    const uint32_t be = cnt ? cell_nearest<D>(lcb, ids, cnt, mid) : 0u;
    c0 = cnt ? ids[be] : 0u;
    double v0[D];
#pragma unroll
    for (int j = 0; j < D; ++j) v0[j] = lcb[c0 * D + j];
    const double mt0 = cell_max_t<D>(v0, a, b);
    const double g = cell_gamma(D);
    uint32_t L = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t bits = 0;
      const uint32_t e1 = cnt < 32u * (w + 1) ? cnt : 32u * (w + 1);
      // four entries a step: one 4-byte id load, four independent tests
      for (uint32_t e = 32u * w; e < e1; e += 4u) {
        const uint32_t quad = *reinterpret_cast<const uint32_t*>(ids + e);
        double v[4][D];
#pragma unroll
        for (uint32_t h = 0; h < 4; ++h) {
          const double* p = lcb + ((quad >> (8u * h)) & 0xFFu) * D;
#pragma unroll
          for (int j = 0; j < D; ++j) v[h][j] = p[j];
        }
#pragma unroll
        for (uint32_t h = 0; h < 4; ++h) {
          const uint32_t eh = e + h;
          const bool keep = eh < e1 && (eh == be || !cell_excluded<D>(v[h], v0, mt0, a, b, g));
          bits |= keep ? 1u << (eh - 32u * w) : 0u;
        }
      }
      mask[w] = bits;
      L += (uint32_t)__popc(bits);
    }
    nit = (L + kCellItem - 1u) / kCellItem;
    if (cnt == 0 || nit > kCellMaxItems) nit = 0;
  }
  scan[t] = nit;
  __syncthreads();
  if (t == 0) {
    uint32_t sum = 0;
    for (uint32_t i = 0; i < blockDim.x; ++i) {
      const uint32_t v = scan[i];
      scan[i] = sum;
      sum += v;
    }
    uint32_t base = sum ? atomicAdd(&pm[9], sum) : 0u;
    if (sum && (base > cap_items || cap_items - base < sum)) base = 0xFFFFFFFFu;
    sbase = base;
  }
  __syncthreads();
  if (!live) return;
  uint32_t out = 0;
  if (nit && sbase != 0xFFFFFFFFu) {
    const uint32_t item0 = sbase + scan[t];
    uint8_t* dst = lists + ((uint64_t)m * cap_items + item0) * kCellItem;
    uint32_t wpos = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      uint32_t bits = mask[w];
      while (bits) {
        const uint32_t e = 32u * w + (uint32_t)__builtin_ctz(bits);
        bits &= bits - 1u;
        dst[wpos++] = lids[r][e];
      }
    }
    for (; wpos < nit * kCellItem; ++wpos) dst[wpos] = (uint8_t)c0;
    out = item0 | (nit << 24);
  }
  recm[q * F + f] = out;
}

// LDS layout of cell_encode_kernel, shared by the host launcher:
//   lcb [K][DP] f32 | per wave: gx [64][DP] f32, gbest [64] u64, ga [64] u32
//   (the vector's first list item), gitem [kCellWaveItems] u16
//   (lane | item << 6) | lmax, lcnt u32
struct CellLds {
  uint32_t wave_off, wave_bytes, scal_off, total;
};
__host__ __device__ inline CellLds cell_lds(uint32_t K, uint32_t DP) {
  CellLds s;
  s.wave_off = cand_up16(K * DP * 4u);
  s.wave_bytes = 64u * (DP * 4u + 8u + 4u) + kCellWaveItems * 2u;
  s.scal_off = s.wave_off + (uint32_t)kCandWaves * s.wave_bytes;
  s.total = s.scal_off + 16u;
  return s;
}

// The record of a row's cell (0 outside the grid or on NaN).
template <int D>
__device__ inline uint32_t cell_record(const float (&x)[D], const float (&lo)[D],
                                       const float (&s)[D], const uint32_t* __restrict__ recm) {
  bool in = true;
  uint32_t k[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    bool ij;
    k[j] = cell_coord(x[j], lo[j], s[j], cell_side(D), &ij);
    in = in && ij;
  }
  return in ? recm[cell_id<D>(k)] : 0u;
}

// The encode pass: blocks run XCD-contiguously as (chunk, subspace) so the
// M blocks of a chunk share one L2.  Each wave takes 64 vectors at a time
// (their rows loaded two groups ahead, their cell records one group ahead);
// a vector's items are laid out over the wave's lanes by a scan, every
// entry of every item is evaluated with the reference distance and folded
// into the vector's 64-bit LDS key, and every lane writes its vector's code
// to out[i][m].  Deferred vectors go to the block's slice of slice[m][..],
// then to the subspace's dense list defer[m][0 .. defer_count[m]) (one
// global atomic per block), for encode_list_kernel.
template <int D, typename CodeT>
__global__ __launch_bounds__(kCandThreads, 8) void cell_encode_kernel(
    const float* __restrict__ xin, const float* __restrict__ cb, const uint32_t* __restrict__ par,
    const uint32_t* __restrict__ rec, const uint8_t* __restrict__ lists, CodeT* __restrict__ out,
    uint32_t* __restrict__ slice, uint32_t* __restrict__ defer, uint32_t* __restrict__ defer_count,
    uint64_t n, uint32_t dim, uint32_t M, uint32_t K, uint32_t chunk, uint32_t nchunks,
    uint32_t cap_items) {
  constexpr int DP = Pad<D>::value;
  constexpr uint32_t cells = cell_count(D);
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  if (logical >= nchunks * M) return;  // grid padding to a multiple of 8
  const uint32_t b = logical / M, m = logical % M;
  const uint32_t* pm = par + (uint64_t)m * kCellParWords;
  if (pm[8] == 0) return;  // the anchored pass serves this subspace
  const CellLds lay = cell_lds(K, DP);
  uint8_t* base = reinterpret_cast<uint8_t*>(lds);
  float* lcb = lds;
  const uint32_t t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  uint8_t* wb = base + lay.wave_off + wave * lay.wave_bytes;
  float* gx = reinterpret_cast<float*>(wb);
  unsigned long long* gbest = reinterpret_cast<unsigned long long*>(gx + 64 * DP);
  uint32_t* ga = reinterpret_cast<uint32_t*>(gbest + 64);
  uint16_t* gitem = reinterpret_cast<uint16_t*>(ga + 64);
  uint32_t* lmax = reinterpret_cast<uint32_t*>(base + lay.scal_off);
  uint32_t* lcnt = lmax + 1;
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
  float glo[D], gs[D];
  cell_params<D>(pm, glo, gs);
  __syncthreads();
  const bool all_deferred = *lmax >= 0x7f800000u;
  const uint32_t* recm = rec + (uint64_t)m * cells;
  const uint32_t* lm = reinterpret_cast<const uint32_t*>(lists + (uint64_t)m * cap_items * kCellItem);

  const uint64_t lo_i = (uint64_t)b * chunk;
  const uint64_t hi_i = lo_i + chunk < n ? lo_i + chunk : n;
  auto load_x = [&](uint64_t i, float (&v)[D]) {
    if (i < hi_i) {
      const float* src = xin + i * dim + (uint64_t)m * D;
#pragma unroll
      for (int k = 0; k < D; ++k) v[k] = src[k];
    } else {
#pragma unroll
      for (int k = 0; k < D; ++k) v[k] = 0.0f;
    }
  };
  constexpr uint64_t kStride = (uint64_t)kCandWaves * kWave;
  const uint64_t first_i = lo_i + (uint64_t)wave * kWave + lane;
  // rows of this group and the next, the cell record of this group
  float x0[D], x1[D];
  load_x(first_i, x0);
  load_x(first_i + kStride, x1);
  uint32_t r0 = (first_i < hi_i && !all_deferred) ? cell_record<D>(x0, glo, gs, recm) : 0u;
  for (uint64_t g0 = lo_i + (uint64_t)wave * kWave; g0 < hi_i; g0 += kStride) {
    const uint64_t i = g0 + lane;
    const bool valid = i < hi_i;
    float x[D];
#pragma unroll
    for (int k = 0; k < D; ++k) x[k] = x0[k];
    const uint32_t r = r0;
    // next group's record from its rows, the group after's rows
#pragma unroll
    for (int k = 0; k < D; ++k) x0[k] = x1[k];
    r0 = (i + kStride < hi_i && !all_deferred) ? cell_record<D>(x0, glo, gs, recm) : 0u;
    load_x(i + 2 * kStride, x1);
    // Phase 1: the vector's items.
    uint32_t nit = valid && !all_deferred ? r >> 24 : 0u;
    const uint32_t first = r & 0xFFFFFFu;
    bool deferred = valid && nit == 0;
    // Phase 2: the wave's items, laid out by an inclusive scan of the
    // counts; past kCellWaveItems items in a wave, vectors above 16 items
    // defer.
    uint32_t incl = wave_inclusive_sum(nit);
    uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
    if (total > kCellWaveItems) {
      if (nit > kCellWaveItems / kWave) {
        nit = 0;
        deferred = true;
      }
      incl = wave_inclusive_sum(nit);
      total = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
    }
    total = min(total, kCellWaveItems);
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
      gbest[lane] = ~0ull;
      ga[lane] = first;
    }
    {
      uint32_t most = nit;  // the wave's largest count bounds the loop
      for (int off = kWave / 2; off > 0; off >>= 1) most = max(most, (uint32_t)__shfl_xor((int)most, off, kWave));
      uint16_t* gi = gitem + (incl - nit);
      for (uint32_t q = 0; q < most; ++q)
        if (q < nit) gi[q] = (uint16_t)(lane | (q << 6));
    }
    wave_lds_sync();
    // Phase 3: items, 64 at a time; the entries of an item are evaluated
    // without branches (padding repeats the cell's anchor, a real codeword).
    for (uint32_t w = lane; w < total; w += kWave) {
      const uint32_t it = gitem[w];
      const uint32_t u = it & 63u, j = (it >> 6) & 31u;
      const uint32_t ids = lm[ga[u] + j];
      float xv[D];
      load_padded<D>(gx + u * DP, xv);
      unsigned long long best = ~0ull;
#pragma unroll
      for (uint32_t k = 0; k < kCellItem; ++k) {
        const uint32_t c = (ids >> (8u * k)) & 0xFFu;
        float cv[D];
        load_padded<D>(lcb + c * DP, cv);
        const unsigned long long key =
            ((unsigned long long)cand_f2u(exact_l2sq<D>(xv, cv)) << 32) | (c << 4);
        best = key < best ? key : best;
      }
      atomicMin(&gbest[u], best);
    }
    wave_lds_sync();
    if (live) out[i * M + m] = (CodeT)cand_best_code(gbest[lane]);
    wave_lds_sync();  // the scratch is rewritten by the next group
  }
  __syncthreads();  // the slice's global writes and lcnt
  const uint32_t nd = *lcnt;
  if (nd == 0) return;
  __syncthreads();  // every thread has read lcnt before it is reused
  if (t == 0) *lcnt = atomicAdd(&defer_count[m], nd);
  __syncthreads();
  const uint32_t at = *lcnt;
  for (uint32_t q = t; q < nd; q += kCandThreads)
    defer[(uint64_t)m * n + at + q] = slice[(uint64_t)m * n + lo_i + q];
}

}  // namespace tacgpu
