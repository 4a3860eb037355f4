// Device helpers of the decode-attention kernels (gfx950): element loads and stores of any
// supported dtype, the 16-bit MFMA operand types, lane reductions across the 16-lane
// groups of a wave, and the K / V stream loads (buffer descriptors over one (row, head)
// segment of the pool, non-temporal cache policy).  Used by attention.hip and by the
// fused layer-step kernel (layer.hip).
#pragma once

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


}  // namespace
}  // namespace cg
