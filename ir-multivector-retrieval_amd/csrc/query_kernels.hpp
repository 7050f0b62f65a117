// query_kernels.hpp — gfx950 kernels of the query side that consumes PQ
// codes: the per-query distance table (src/index/pq.zig:92-123) and refine's
// exact MaxSim over candidate documents (src/retrieval/refine.zig:83-145).
// Included once, by tac_gpu.hip.  Compiled with -ffp-contract=off: every
// multiply and add is rounded separately, in the reference's order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pq_kernels.hpp"

namespace tacgpu {

// vec.dot (src/util/vec.zig:37-103): dims 2 and 4 are left folds from 0,
// dims 64 and 128 accumulate in 4 lanes chunk after chunk and reduce
// ((a0 + a1) + a2) + a3, other dims take the generic path at the device's
// lane count (generic_vec: lanes, lane-order reduce, tail).
// `a` and `b` may live in LDS or global memory.
__device__ inline float ref_dot(const float* a, const float* b, uint32_t d) {
  if (d == 2) return a[0] * b[0] + a[1] * b[1];
  if (d == 4) {
    float s = 0.0f;
    for (int i = 0; i < 4; ++i) s = s + a[i] * b[i];
    return s;
  }
  if (d == 64 || d == 128) {
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
    for (uint32_t c = 0; c < d; c += 4) {
      acc0 = acc0 + a[c] * b[c];
      acc1 = acc1 + a[c + 1] * b[c + 1];
      acc2 = acc2 + a[c + 2] * b[c + 2];
      acc3 = acc3 + a[c + 3] * b[c + 3];
    }
    return ((acc0 + acc1) + acc2) + acc3;
  }
  return generic_vec<true>(a, b, d);
}

// PQ.buildDistanceTable: table[((mm * K) + c) * n_q + i] =
// dot(query_i[mm * D .. +D], codebook[mm][c]); one thread per entry, so
// consecutive threads write consecutive i.
__global__ __launch_bounds__(256) void distance_table_kernel(
    const float* __restrict__ q, const float* __restrict__ cb, float* __restrict__ table,
    uint32_t n_q, uint32_t dim, uint32_t M, uint32_t K, uint32_t D) {
  const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t total = (uint64_t)M * K * n_q;
  if (g >= total) return;
  const uint32_t i = (uint32_t)(g % n_q);
  const uint64_t mc = g / n_q;
  const uint32_t mm = (uint32_t)(mc / K);
  table[g] = ref_dot(q + (uint64_t)i * dim + (uint64_t)mm * D, cb + mc * D, D);
}

// Refine status codes per candidate (tac_status values).
constexpr uint32_t kRefineOk = 0;
constexpr uint32_t kRefineDocOutOfRange = 18;
constexpr uint32_t kRefineLayoutCorrupt = 19;

struct RefineIndex {
  const float* centroids;            // [kappa][dim]
  const uint64_t* doc_index;         // [n_docs + 1]
  const uint8_t* payload;            // per-doc layouts
  const uint64_t* doc_token_offsets; // [n_docs + 1]
  const float* norms;                // [n_tokens]
  uint64_t n_docs, n_tokens, payload_len;
  uint32_t dim, kappa, M, K;
};

__device__ __forceinline__ uint32_t load_u32_le(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

// One wave per candidate document (grid-stride over candidates).  The wave
// covers QP = n_q rounded up to a power of two (at most 64) query tokens and
// S = 64 / QP document tokens at a time: lane (s, i) takes query token i0 + i
// against document token k0 + s, for every k
//   cent  = dot(q_i, centroid[c_k])            (centroid rows staged in LDS)
//   res   = sum over m of table[m][code_km][i]  (in m order, from 0)
//   score = cent + norm_k * res
// and keeps the first k of its running maximum (strict >, from -inf).  The S
// slots of a query token then merge (larger value; on equal values the
// earlier k, which keeps the sign of a zero maximum the reference would
// keep), and lane 0 folds best_0 + best_1 + ... in i order (0 for an empty
// document).  Layout checks follow refine.zig:51-65,107-114; a failing
// candidate writes its status and score 0, and `first_bad` keeps the lowest
// such index.
constexpr int kRefineWaves = 4;
constexpr uint32_t kRefineRowFloats = 640;  // per-wave LDS for centroid rows

__host__ __device__ inline uint32_t refine_qp(uint32_t n_q) {
  uint32_t qp = 1;
  while (qp < n_q && qp < 64) qp <<= 1;
  return qp;
}

__host__ __device__ inline uint32_t refine_slots(uint32_t n_q, uint32_t dim) {
  uint32_t s = 64 / refine_qp(n_q);
  while (s > 1 && s * (dim + 1) > kRefineRowFloats) s >>= 1;
  return s;
}

// Per-block dynamic LDS floats: queries [n_q][dim + 1], then per wave the
// centroid rows [S][dim + 1], 64 best values and 64 best token indices.
__host__ __device__ inline uint32_t refine_lds_floats(uint32_t n_q, uint32_t dim) {
  const uint32_t S = refine_slots(n_q, dim);
  return n_q * (dim + 1) + kRefineWaves * (S * (dim + 1) + 128);
}

__global__ __launch_bounds__(64 * kRefineWaves) void refine_kernel(
    RefineIndex ix, const float* __restrict__ q, uint32_t n_q, const float* __restrict__ table,
    const uint32_t* __restrict__ doc_ids, uint32_t n_cand, float* __restrict__ scores,
    uint32_t* __restrict__ status, uint32_t* __restrict__ first_bad) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
  const uint32_t ld = ix.dim + 1;  // odd stride: distinct rows hit distinct banks
  const uint32_t QP = refine_qp(n_q), S = refine_slots(n_q, ix.dim);
  const uint32_t slot = lane / QP, qi = lane % QP;
  float* qs = lds;                                                  // [n_q][dim + 1]
  float* crow = lds + (size_t)n_q * ld + (size_t)w * (S * ld + 128);  // [S][dim + 1]
  float* bestv = crow + (size_t)S * ld;                             // [64]
  uint32_t* bestk = reinterpret_cast<uint32_t*>(bestv + 64);        // [64]
  for (uint32_t f = threadIdx.x; f < n_q * ix.dim; f += blockDim.x)
    qs[(f / ix.dim) * ld + f % ix.dim] = q[f];
  __syncthreads();
  const uint32_t cb = ix.K <= 256 ? 1u : 2u;
  const uint32_t stride = gridDim.x * kRefineWaves;
  for (uint32_t cand = blockIdx.x * kRefineWaves + w; cand < n_cand; cand += stride) {
    const uint64_t doc = doc_ids[cand];
    uint32_t st = kRefineOk;
    uint32_t n_d = 0;
    uint64_t lo = 0, t_lo = 0;
    if (doc >= ix.n_docs) {
      st = kRefineDocOutOfRange;
    } else {
      lo = ix.doc_index[doc];
      const uint64_t hi = ix.doc_index[doc + 1];
      if (hi < lo || hi > ix.payload_len || hi - lo < 4) {
        st = kRefineLayoutCorrupt;
      } else {
        n_d = load_u32_le(ix.payload + lo);
        t_lo = ix.doc_token_offsets[doc];
        const uint64_t t_hi = ix.doc_token_offsets[doc + 1];
        if (hi - lo < 4 + 4ull * n_d + (uint64_t)n_d * ix.M * cb || t_hi - t_lo != n_d ||
            t_hi > ix.n_tokens)
          st = kRefineLayoutCorrupt;
      }
    }
    const uint8_t* lay = ix.payload + lo;
    float total = 0.0f;
    for (uint32_t i0 = 0; st == kRefineOk && i0 < n_q; i0 += QP) {
      const uint32_t i = i0 + qi;
      float b = -__builtin_inff();
      uint32_t bk = 0xFFFFFFFFu;
      for (uint32_t k0 = 0; k0 < n_d; k0 += S) {
        // centroid rows of tokens k0 .. k0 + S - 1
        bool bad_id = false;
        for (uint32_t f = lane; f < S * ix.dim; f += 64) {
          const uint32_t s = f / ix.dim, d = f % ix.dim;
          if (k0 + s < n_d) {
            const uint32_t cid = load_u32_le(lay + 4 + 4ull * (k0 + s));
            if (cid >= ix.kappa)
              bad_id = true;
            else
              crow[s * ld + d] = ix.centroids[(uint64_t)cid * ix.dim + d];
          }
        }
        if (__any(bad_id)) {
          st = kRefineLayoutCorrupt;
          break;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const uint32_t k = k0 + slot;
        bool bad = false;
        if (slot < S && i < n_q && k < n_d) {  // S may be below 64 / QP
          const float cent = ref_dot(qs + (size_t)i * ld, crow + (size_t)slot * ld, ix.dim);
          const uint8_t* codes = lay + 4 + 4ull * n_d + (uint64_t)k * ix.M * cb;
          float res = 0.0f;
          for (uint32_t mm = 0; mm < ix.M; ++mm) {
            const uint32_t code =
                cb == 1 ? codes[mm] : (uint32_t)codes[2 * mm] | (uint32_t)codes[2 * mm + 1] << 8;
            if (code >= ix.K) {
              bad = true;
              break;
            }
            res = res + table[((uint64_t)mm * ix.K + code) * n_q + i];
          }
          const float scaled = ix.norms[t_lo + k] * res;
          const float score = cent + scaled;
          if (!bad && score > b) {
            b = score;
            bk = k;
          }
        }
        __builtin_amdgcn_wave_barrier();
        if (__any(bad)) {
          st = kRefineLayoutCorrupt;
          break;
        }
      }
      if (st != kRefineOk) break;
      bestv[lane] = b;
      bestk[lane] = bk;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      if (lane == 0 && n_d > 0) {
        const uint32_t cnt = n_q - i0 < QP ? n_q - i0 : QP;
        for (uint32_t j = 0; j < cnt; ++j) {
          float v = bestv[j];
          uint32_t vk = bestk[j];
          for (uint32_t s = 1; s < S; ++s) {
            const float o = bestv[s * QP + j];
            const uint32_t ok = bestk[s * QP + j];
            if (o > v || (o == v && ok < vk)) {
              v = o;
              vk = ok;
            }
          }
          total = total + v;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) {
      scores[cand] = st == kRefineOk ? total : 0.0f;
      status[cand] = st;
      if (st != kRefineOk) atomicMin(first_bad, cand);
    }
  }
}

}  // namespace tacgpu
