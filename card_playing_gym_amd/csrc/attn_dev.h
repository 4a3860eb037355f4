// Device helpers of the decode-attention kernels (gfx950): element loads and stores of any
// supported dtype, the 16-bit MFMA operand types, lane reductions across the 16-lane
// groups of a wave, and the K / V stream loads (buffer descriptors over one (row, head)
// segment of the pool, non-temporal cache policy).  Used by attention.hip and by the
// fused layer-step kernel (layer.hip).
#pragma once

#include "attention.h"
#include "common.h"

namespace cg {
namespace {

__device__ __forceinline__ float load_any(const void *p, int dtype, int64_t i) {
  switch (dtype) {
    case CG_BF16:
      return to_f32(static_cast<const bf16 *>(p)[i]);
    case CG_F16:
      return to_f32(static_cast<const f16 *>(p)[i]);
    default:
      return static_cast<const float *>(p)[i];
  }
}

__device__ __forceinline__ void store_any(void *p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case CG_BF16:
      static_cast<bf16 *>(p)[i] = from_f32<bf16>(v);
      break;
    case CG_F16:
      static_cast<f16 *>(p)[i] = from_f32<f16>(v);
      break;
    default:
      static_cast<float *>(p)[i] = v;
  }
}


constexpr float NEG_BIG = -1.0e30f;

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(8))) float f32x8;

template <typename TKV>
struct Mfma16;  // 16-bit operand helpers

template <>
struct Mfma16<bf16> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ vec from(const f32x8 &f) { return __builtin_convertvector(f, bf16x8); }
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16<f16> {
  typedef f16x8 vec;
  static __device__ __forceinline__ vec from(const f32x8 &f) { return __builtin_convertvector(f, f16x8); }
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

__device__ __forceinline__ Rsrc kv_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, int(bytes), 0x00020000);
}
// Cache policy of the K / V stream loads (buffer instruction bits: 1 sc0, 2 nt, 16 sc1).
#ifndef CG_KV_CPOL
#define CG_KV_CPOL 2
#endif
__device__ __forceinline__ uint4 kv_load16(Rsrc r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CG_KV_CPOL);
  return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// Max / min of an int over the 16 lanes of a DPP row.
__device__ __forceinline__ int row16_max(int v) {
  v = max(v, dpp_i<0xB1>(v));
  v = max(v, dpp_i<0x4E>(v));
  v = max(v, dpp_i<0x124>(v));
  v = max(v, dpp_i<0x128>(v));
  return v;
}
__device__ __forceinline__ int row16_min(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x124>(v));
  v = min(v, dpp_i<0x128>(v));
  return v;
}

// ---- the unit order of the persistent decode-attention kernel (and of packed chunks) -----
constexpr int STREAM_KT = 64;       // keys per tile of the persistent kernel
constexpr int ORDER_BUCKETS = 256;  // tile counts >= 255 share the last bucket

// Work of a (row, KV head) unit: its widest query's visible keys in 64-key tiles, times its
// 16-query tiles (one for the decode runs of the persistent kernel; a packed chunk of c
// tokens has G c queries).
__device__ __forceinline__ int unit_tiles(const AttnArgs &a, int u) {
  const int b = u / a.kv_heads;
  const int64_t row = a.rows ? a.rows[b] : int64_t(b);
  int64_t count = a.T;
  if (a.seq_start) {
    int64_t lo = a.seq_start[b], hi = a.seq_start[b + 1];
    lo = lo < 0 ? 0 : (lo > a.n_tokens ? a.n_tokens : lo);
    hi = hi < lo ? lo : (hi > a.n_tokens ? a.n_tokens : hi);
    count = hi - lo;
  }
  int64_t kend = a.key_lengths[b] + a.kl_add + (count - 1);
  if (kend > a.span) kend = a.span;
  if (row < 0 || row >= a.capacity || kend < 0) kend = 0;
  const int64_t qtiles = (int64_t(a.n_heads / a.kv_heads) * count + 15) / 16;
  return int(min<int64_t>(ORDER_BUCKETS - 1, (kend + STREAM_KT - 1) / STREAM_KT * qtiles));
}

// Units whose bucket the first pass keeps in LDS for the second (one byte each); units
// past it are measured again from their lengths.
constexpr int ORDER_CACHE = 32768;
// Up to this many units the order is assembled in LDS and written out in unit order
// (coalesced) instead of one scattered store per unit.
constexpr int ORDER_STAGE = 8192;

// order = the units sorted by descending work: a counting sort by one whole block
// (any size; ties land in any order, which changes only which wave computes a unit, not its
// result).  Called by every thread of the block.
__device__ __forceinline__ void order_units(const AttnArgs &a, int32_t *__restrict__ order) {
  static_assert(ORDER_BUCKETS <= 256, "buckets are kept as bytes");
  __shared__ int hist[ORDER_BUCKETS], scan[2][ORDER_BUCKETS];
  __shared__ uint8_t bucket[ORDER_CACHE];
  __shared__ int32_t staged[ORDER_STAGE];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int U = a.n_seqs * a.kv_heads;
  for (int i = tid; i < ORDER_BUCKETS; i += nt) hist[i] = 0;
  __syncthreads();
  // Each pass takes eight units per thread at a time, so their loads (lengths, rows, chunk
  // bounds) are in flight together instead of one round trip per unit.
  constexpr int PER = 8;
  for (int base = 0; base < U; base += PER * nt) {
    int w[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int u = base + tid + k * nt;
      w[k] = u < U ? unit_tiles(a, u) : -1;
      if (u < U && u < ORDER_CACHE) bucket[u] = uint8_t(w[k]);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (w[k] >= 0) atomicAdd(&hist[w[k]], 1);
  }
  __syncthreads();
  // Exclusive suffix sums (bucket k starts after every larger bucket): Hillis-Steele over
  // the reversed histogram.
  int src = 0;
  for (int i = tid; i < ORDER_BUCKETS; i += nt) scan[0][i] = hist[ORDER_BUCKETS - 1 - i];
  __syncthreads();
  for (int off = 1; off < ORDER_BUCKETS; off <<= 1) {
    for (int i = tid; i < ORDER_BUCKETS; i += nt) scan[src ^ 1][i] = scan[src][i] + (i >= off ? scan[src][i - off] : 0);
    __syncthreads();
    src ^= 1;
  }
  // scan[src][i]: inclusive sum of reversed buckets 0..i, i.e. of buckets K - 1 - i .. K - 1.
  for (int k = tid; k < ORDER_BUCKETS; k += nt) hist[k] = scan[src][ORDER_BUCKETS - 1 - k] - hist[k];
  __syncthreads();
  for (int base = 0; base < U; base += PER * nt) {
    int w[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int u = base + tid + k * nt;
      w[k] = u >= U ? -1 : u < ORDER_CACHE ? int(bucket[u]) : unit_tiles(a, u);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)
      if (w[k] >= 0) {
        const int slot = atomicAdd(&hist[w[k]], 1);
        if (U <= ORDER_STAGE) staged[slot] = base + tid + k * nt;
        else order[slot] = base + tid + k * nt;
      }
  }
  if (U <= ORDER_STAGE) {
    __syncthreads();
    for (int i = tid; i < U; i += nt) order[i] = staged[i];
  }
}

}  // namespace
}  // namespace cg
