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

namespace tacgpu {

// ---------------------------------------------------------------------------
// .tac per-document layouts (src/index/storage.zig:674-686, :705-749).
// Each doc d occupies align8(4 + 4 n_d + n_d m cb) payload bytes:
//   u32 n_d | u32 centroid id x n_d | codes (n_d x m x cb bytes) | zeros.
// doc_index[d] is the payload offset of doc d; doc_index[n_docs] the total.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t doc_bytes(uint64_t n_d, uint32_t m, uint32_t cb) {
  return (4 + 4 * n_d + n_d * m * cb + 7) & ~7ull;
}

constexpr int kScanBlock = 256;
constexpr int kScanPer = 4;  // elements per thread in the u64 scan

// Phase 1: per-block exclusive scan of doc sizes into doc_index, block totals
// into `sums`.
// Offsets that decrease or pass n_tokens raise `status` (the writer then
// does not run) and count as empty documents.
__global__ __launch_bounds__(kScanBlock) void doc_sizes_scan_kernel(
    const uint64_t* __restrict__ doc_offsets, uint64_t n_docs, uint64_t n_tokens, uint32_t m,
    uint32_t cb, uint64_t* __restrict__ doc_index, uint64_t* __restrict__ sums,
    uint32_t* __restrict__ status) {
  __shared__ uint64_t warp_tot[kScanBlock / 64];
  const uint64_t base = (uint64_t)blockIdx.x * kScanBlock * kScanPer + threadIdx.x * kScanPer;
  uint64_t v[kScanPer];
  uint64_t local = 0;
#pragma unroll
  for (int q = 0; q < kScanPer; ++q) {
    const uint64_t d = base + q;
    v[q] = 0;
    if (d < n_docs) {
      const uint64_t a = doc_offsets[d], b = doc_offsets[d + 1];
      if (b < a || b > n_tokens)
        atomicOr(status, 1u);
      else
        v[q] = doc_bytes(b - a, m, cb);
    }
    local += v[q];
  }
  const uint32_t lane = threadIdx.x % 64, w = threadIdx.x / 64;
  uint64_t incl = local;
  for (int off = 1; off < 64; off <<= 1) {
    const uint64_t o = __shfl_up(incl, off, 64);
    if (lane >= (uint32_t)off) incl += o;
  }
  if (lane == 63) warp_tot[w] = incl;
  __syncthreads();
  uint64_t before = 0;
  for (uint32_t q = 0; q < w; ++q) before += warp_tot[q];
  uint64_t run = before + incl - local;
#pragma unroll
  for (int q = 0; q < kScanPer; ++q) {
    const uint64_t d = base + q;
    if (d < n_docs) doc_index[d] = run;
    run += v[q];
  }
  if (threadIdx.x == kScanBlock - 1) sums[blockIdx.x] = before + incl;
}

// Phase 2 (one block): exclusive scan of the block totals in place; the
// grand total lands in doc_index[n_docs].
__global__ __launch_bounds__(kScanBlock) void doc_sums_scan_kernel(
    uint64_t* __restrict__ sums, uint32_t nb, uint64_t* __restrict__ doc_index, uint64_t n_docs) {
  __shared__ uint64_t warp_tot[kScanBlock / 64];
  __shared__ uint64_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  const uint32_t lane = threadIdx.x % 64, w = threadIdx.x / 64;
  for (uint32_t b0 = 0; b0 < nb; b0 += kScanBlock) {
    const uint32_t b = b0 + threadIdx.x;
    const uint64_t x = b < nb ? sums[b] : 0;
    uint64_t incl = x;
    for (int off = 1; off < 64; off <<= 1) {
      const uint64_t o = __shfl_up(incl, off, 64);
      if (lane >= (uint32_t)off) incl += o;
    }
    if (lane == 63) warp_tot[w] = incl;
    __syncthreads();
    uint64_t before = carry;
    for (uint32_t q = 0; q < w; ++q) before += warp_tot[q];
    if (b < nb) sums[b] = before + incl - x;
    __syncthreads();
    if (threadIdx.x == kScanBlock - 1) carry = before + incl;
    __syncthreads();
  }
  if (threadIdx.x == 0) doc_index[n_docs] = carry;
}

// Phase 3: add each block's carry-in.
__global__ __launch_bounds__(kScanBlock) void doc_scan_add_kernel(
    uint64_t* __restrict__ doc_index, const uint64_t* __restrict__ sums, uint64_t n_docs) {
  const uint64_t base = (uint64_t)blockIdx.x * kScanBlock * kScanPer + threadIdx.x * kScanPer;
  const uint64_t add = sums[blockIdx.x];
#pragma unroll
  for (int q = 0; q < kScanPer; ++q)
    if (base + q < n_docs) doc_index[base + q] += add;
}

// One wave per document (grid-stride): n_d, the centroid ids and the codes,
// then zero padding.  Doc starts are 8-aligned, so the id array is 4-aligned;
// codes are copied as 32-bit words when source and destination allow.
__global__ __launch_bounds__(256) void doc_write_kernel(
    const uint64_t* __restrict__ doc_offsets, uint64_t n_docs, const uint32_t* __restrict__ assign,
    const uint8_t* __restrict__ codes, uint32_t m, uint32_t cb,
    const uint64_t* __restrict__ doc_index, uint8_t* __restrict__ payload) {
  const uint32_t lane = threadIdx.x % 64;
  const uint64_t waves = (uint64_t)gridDim.x * (blockDim.x / 64);
  for (uint64_t d = (uint64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64; d < n_docs;
       d += waves) {
    const uint64_t lo = doc_offsets[d], n_d = doc_offsets[d + 1] - lo;
    uint8_t* p = payload + doc_index[d];
    uint32_t* ids = reinterpret_cast<uint32_t*>(p + 4);
    if (lane == 0) *reinterpret_cast<uint32_t*>(p) = (uint32_t)n_d;
    for (uint64_t k = lane; k < n_d; k += 64) ids[k] = assign[lo + k];
    const uint64_t nbytes = n_d * m * cb;
    const uint8_t* src = codes + lo * m * cb;
    uint8_t* dst = p + 4 + 4 * n_d;
    if (((uintptr_t)src & 3) == 0 && (nbytes & 3) == 0) {
      const uint32_t* s4 = reinterpret_cast<const uint32_t*>(src);
      uint32_t* d4 = reinterpret_cast<uint32_t*>(dst);
      for (uint64_t q = lane; q < nbytes / 4; q += 64) d4[q] = s4[q];
    } else {
      for (uint64_t q = lane; q < nbytes; q += 64) dst[q] = src[q];
    }
    const uint64_t used = 4 + 4 * n_d + nbytes;
    const uint64_t total = doc_bytes(n_d, m, cb);
    for (uint64_t q = used + lane; q < total; q += 64) p[q] = 0;
  }
}

// ---------------------------------------------------------------------------
// CRC-32/ISO-HDLC of a device buffer (std.hash.Crc32, as storage.zig applies
// it to the whole image before the footer, :612-617, :782-786).
//
// Reflected representation: bit 31 holds the coefficient of x^0.  The
// register after bytes B starting from register r is
//   crc(r, B) = crc(0, B) ^ (r * x^(8|B|) mod P),
// so zero-seeded CRCs of consecutive pieces combine left to right by one
// modular multiplication each.  The buffer splits into an unaligned head
// (< 16 bytes), a body of whole kCrcLeaf-byte leaves and a tail
// (< kCrcLeaf bytes).  A thread owns one leaf and runs kCrcWays interleaved
// slicing-by-8 chains over its consecutive sub-leaves (independent LDS
// lookups in flight), joins them, the 256 leaves of a block combine in an
// LDS tree, one block combines the block results, and one thread adds head,
// tail and the all-ones preset.
// ---------------------------------------------------------------------------
constexpr uint32_t kCrcPoly = 0xEDB88320u;
constexpr uint32_t kCrcLeaf = 256;       // bytes per thread (power of two)
constexpr uint32_t kCrcLeafLog2 = 8;
constexpr uint32_t kCrcWays = 4;         // interleaved chains per thread
constexpr uint32_t kCrcSub = kCrcLeaf / kCrcWays;  // 64 bytes per chain
constexpr uint32_t kCrcSubLog2 = 6;
constexpr int kCrcBlock = 256;

__host__ __device__ inline uint32_t crc_mulmod(uint32_t a, uint32_t b) {
  uint32_t p = 0;
  for (int i = 0; i < 32; ++i) {
    if ((a >> (31 - i)) & 1u) p ^= b;
    b = (b & 1u) ? (b >> 1) ^ kCrcPoly : b >> 1;
  }
  return p;
}

// Multiplication tables for the shifts: tx[j][i] = x^(8 * 2^j) * x^i mod P
// (j = 0..63, i = 0..31), so r * x^(8 * 2^j) is the XOR of tx[j][i] over the
// coefficients i that r holds: 32 independent selects instead of a 32-step
// serial chain.
constexpr uint32_t kCrcTxRows = 64;

inline void crc_tx_host(uint32_t* tx) {  // [kCrcTxRows][32]
  uint32_t t = 0x40000000u;  // x^1
  for (int j = 0; j < 3; ++j) t = crc_mulmod(t, t);  // x^8
  for (uint32_t j = 0; j < kCrcTxRows; ++j) {
    uint32_t v = t;  // x^(8 * 2^j) * x^0
    for (int i = 0; i < 32; ++i) {
      tx[j * 32 + i] = v;
      v = (v & 1u) ? (v >> 1) ^ kCrcPoly : v >> 1;  // times x
    }
    t = crc_mulmod(t, t);
  }
}

// Branch-free: every row entry is loaded (eight 16-byte LDS reads) and
// masked by its coefficient bit.
__device__ __forceinline__ uint32_t crc_mul_row(uint32_t r, const uint32_t* row) {
  const uint4* row4 = reinterpret_cast<const uint4*>(row);
  uint32_t p0 = 0, p1 = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint4 v = row4[q];
    const int i = 4 * q;
    p0 ^= v.x & (0u - ((r >> (31 - i)) & 1u));
    p1 ^= v.y & (0u - ((r >> (30 - i)) & 1u));
    p0 ^= v.z & (0u - ((r >> (29 - i)) & 1u));
    p1 ^= v.w & (0u - ((r >> (28 - i)) & 1u));
  }
  return p0 ^ p1;
}

// r * x^(8 * count * 2^shift) mod P with tx rows in LDS (one row per set bit).
__device__ __forceinline__ uint32_t crc_shift_tx(uint32_t r, uint64_t count, uint32_t shift,
                                                 const uint32_t* tx) {
  while (count) {
    const uint32_t j = (uint32_t)__builtin_ctzll(count);
    r = crc_mul_row(r, tx + (j + shift) * 32);
    count &= count - 1;
  }
  return r;
}

// Slicing-by-8 tables in LDS: T[k][i] = CRC contribution of byte value i
// followed by k zero bytes, from a zero register.
__device__ inline void crc_tables(uint32_t (*T)[256]) {
  for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
    uint32_t r = i;
    for (int k = 0; k < 8; ++k) r = (r & 1u) ? (r >> 1) ^ kCrcPoly : r >> 1;
    T[0][i] = r;
  }
  __syncthreads();
  for (int k = 1; k < 8; ++k) {
    for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
      const uint32_t v = T[k - 1][i];
      T[k][i] = (v >> 8) ^ T[0][v & 0xFFu];
    }
    __syncthreads();
  }
}

// Eight bytes (lo = bytes 0-3, hi = bytes 4-7, little-endian): byte j needs
// the table with 7 - j trailing zero bytes.
__device__ __forceinline__ uint32_t crc_step8(uint32_t r, uint32_t lo, uint32_t hi,
                                              const uint32_t (*T)[256]) {
  r ^= lo;
  return T[7][r & 0xFFu] ^ T[6][(r >> 8) & 0xFFu] ^ T[5][(r >> 16) & 0xFFu] ^ T[4][r >> 24] ^
         T[3][hi & 0xFFu] ^ T[2][(hi >> 8) & 0xFFu] ^ T[1][(hi >> 16) & 0xFFu] ^ T[0][hi >> 24];
}

struct CrcNode {
  uint32_t crc;
  uint32_t leaves;
};

__device__ __forceinline__ CrcNode crc_join(CrcNode a, CrcNode b, const uint32_t* tx) {
  if (!b.leaves) return a;
  return CrcNode{crc_shift_tx(a.crc, b.leaves, kCrcLeafLog2, tx) ^ b.crc, a.leaves + b.leaves};
}

// Combines the block's 256 nodes in order (one per thread, `mine`): a
// shuffle tree inside each wave, then one thread joins the four wave results.
// Every thread returns the block's combination.
__device__ inline CrcNode crc_block_combine(CrcNode mine, CrcNode* wave_res, const uint32_t* tx) {
  const uint32_t lane = threadIdx.x % 64, w = threadIdx.x / 64;
  for (uint32_t span = 1; span < 64; span <<= 1) {
    const CrcNode other{__shfl_down(mine.crc, span, 64), __shfl_down(mine.leaves, span, 64)};
    if (lane % (2 * span) == 0 && lane + span < 64) mine = crc_join(mine, other, tx);
  }
  if (lane == 0) wave_res[w] = mine;
  __syncthreads();
  if (threadIdx.x == 0) {
    CrcNode acc = wave_res[0];
    for (uint32_t q = 1; q < kCrcBlock / 64; ++q) acc = crc_join(acc, wave_res[q], tx);
    wave_res[0] = acc;
  }
  __syncthreads();
  const CrcNode out = wave_res[0];
  __syncthreads();
  return out;
}

// Leaves of the 16-byte aligned body: every block reduces its 256 leaves to
// one CrcNode.  g_tx is the [64][32] shift table in global memory.
__global__ __launch_bounds__(kCrcBlock) void crc_leaf_kernel(const uint8_t* __restrict__ body,
                                                             uint64_t n_leaves,
                                                             const uint32_t* __restrict__ g_tx,
                                                             CrcNode* __restrict__ nodes) {
  __shared__ uint32_t T[8][256];
  __shared__ __attribute__((aligned(16))) uint32_t tx[kCrcTxRows * 32];
  __shared__ CrcNode node[kCrcBlock / 64];
  for (uint32_t f = threadIdx.x; f < kCrcTxRows * 32; f += kCrcBlock) tx[f] = g_tx[f];
  crc_tables(T);  // synchronises
  const uint64_t leaf = (uint64_t)blockIdx.x * kCrcBlock + threadIdx.x;
  uint32_t r = 0;
  uint32_t have = 0;
  if (leaf < n_leaves) {
    const uint4* p = reinterpret_cast<const uint4*>(body + leaf * kCrcLeaf);
    uint4 v[kCrcWays][kCrcSub / 16];
#pragma unroll
    for (uint32_t w = 0; w < kCrcWays; ++w)
#pragma unroll
      for (uint32_t q = 0; q < kCrcSub / 16; ++q) v[w][q] = p[w * (kCrcSub / 16) + q];
    uint32_t rw[kCrcWays];
#pragma unroll
    for (uint32_t w = 0; w < kCrcWays; ++w) rw[w] = 0;
#pragma unroll
    for (uint32_t q = 0; q < kCrcSub / 16; ++q)
#pragma unroll
      for (uint32_t w = 0; w < kCrcWays; ++w) {
        rw[w] = crc_step8(rw[w], v[w][q].x, v[w][q].y, T);
        rw[w] = crc_step8(rw[w], v[w][q].z, v[w][q].w, T);
      }
    r = rw[0];
#pragma unroll
    for (uint32_t w = 1; w < kCrcWays; ++w) r = crc_mul_row(r, tx + kCrcSubLog2 * 32) ^ rw[w];
    have = 1;
  }
  const CrcNode blk = crc_block_combine(CrcNode{r, have}, node, tx);
  if (threadIdx.x == 0) nodes[blockIdx.x] = blk;
}

// One block: folds the block nodes in order, then head, body and tail.
__global__ __launch_bounds__(kCrcBlock) void crc_final_kernel(
    const uint8_t* __restrict__ buf, uint64_t head, uint64_t n_leaves, uint64_t tail,
    const CrcNode* __restrict__ nodes, uint32_t n_nodes, const uint32_t* __restrict__ g_tx,
    uint32_t* __restrict__ crc_out) {
  __shared__ uint32_t T[8][256];
  __shared__ __attribute__((aligned(16))) uint32_t tx[kCrcTxRows * 32];
  __shared__ CrcNode node[kCrcBlock / 64];
  for (uint32_t f = threadIdx.x; f < kCrcTxRows * 32; f += kCrcBlock) tx[f] = g_tx[f];
  crc_tables(T);  // synchronises
  CrcNode acc{0, 0};
  for (uint32_t b0 = 0; b0 < n_nodes; b0 += kCrcBlock) {
    const uint32_t b = b0 + threadIdx.x;
    const CrcNode part = crc_block_combine(b < n_nodes ? nodes[b] : CrcNode{0, 0}, node, tx);
    acc = crc_join(acc, part, tx);
  }
  if (threadIdx.x != 0) return;
  uint32_t rr = 0xFFFFFFFFu;
  for (uint64_t i = 0; i < head; ++i) rr = T[0][(rr ^ buf[i]) & 0xFFu] ^ (rr >> 8);
  rr = crc_shift_tx(rr, n_leaves, kCrcLeafLog2, tx) ^ acc.crc;
  // The tail starts 16-byte aligned (or at byte 0 when the head took all).
  const uint8_t* t = buf + head + n_leaves * kCrcLeaf;
  uint64_t i = 0;
  if (((uintptr_t)t & 7) == 0) {
    const uint2* t8 = reinterpret_cast<const uint2*>(t);
    for (; i + 8 <= tail; i += 8) {
      const uint2 v = t8[i / 8];
      rr = crc_step8(rr, v.x, v.y, T);
    }
  }
  for (; i < tail; ++i) rr = T[0][(rr ^ t[i]) & 0xFFu] ^ (rr >> 8);
  *crc_out = rr ^ 0xFFFFFFFFu;
}

}  // namespace tacgpu
