// Shared device helpers and host-side error plumbing for libcardgym_hip.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

#include "../../include/cardgym_hip.h"

namespace cg {

// ---- element conversion ---------------------------------------------------------
// bf16 and fp16 values travel as raw 16-bit patterns; conversions are explicit so the
// rounding is the one Tensor.to uses: round to nearest even, NaN -> 0x7FC0 for bf16.

struct bf16 {
  uint16_t bits;
};
struct f16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return __uint_as_float(uint32_t(v.bits) << 16); }
__device__ __forceinline__ float to_f32(f16 v) {
  _Float16 h;
  __builtin_memcpy(&h, &v.bits, 2);
  return float(h);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);

template <>
__device__ __forceinline__ float from_f32<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  // v_cvt_pk_bf16_f32 rounds to nearest even (denormals kept); NaN is canonicalised to
  // 0x7fc0, the quiet NaN torch's conversion produces.
  const __bf16 h = __bf16(v);
  bf16 r;
  r.bits = v != v ? uint16_t(0x7fc0) : __builtin_bit_cast(uint16_t, h);
  return r;
}
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) {
  // v_cvt_f16_f32 rounds to nearest even in the default mode and keeps denormals.
  _Float16 h = _Float16(v);
  f16 r;
  __builtin_memcpy(&r.bits, &h, 2);
  return r;
}

// Four values at once, the one conversion every 16-bit store of K / V into the pool and of
// stored queries goes through (the trunk step's fused append and cg_kv_write_step /
// cg_kv_write_range): 8 bytes, element 0 in the low half.  bf16: NaN inputs are first
// replaced by the quiet NaN 0x7fc00000, then two v_cvt_pk_bf16_f32 round to nearest even
// (subnormals kept), so the bits are from_f32<bf16>'s, NaN -> 0x7fc0 included; f16: nearest
// even per element (v_cvt_f16_f32), as from_f32<f16>.
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;

__device__ __forceinline__ f32x4 canonical_nan(f32x4 v) {
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = v[r] != v[r] ? __uint_as_float(0x7fc00000u) : v[r];
  return v;
}

template <typename T>
__device__ __forceinline__ u32x2 cvt4(f32x4 v);
template <>
__device__ __forceinline__ u32x2 cvt4<bf16>(f32x4 v) {
  return __builtin_bit_cast(u32x2, __builtin_convertvector(canonical_nan(v), bf16x4));
}
template <>
__device__ __forceinline__ u32x2 cvt4<f16>(f32x4 v) {
  const f16 e0 = from_f32<f16>(v[0]), e1 = from_f32<f16>(v[1]), e2 = from_f32<f16>(v[2]), e3 = from_f32<f16>(v[3]);
  return u32x2{uint32_t(e0.bits) | uint32_t(e1.bits) << 16, uint32_t(e2.bits) | uint32_t(e3.bits) << 16};
}

// Bit-preserving conversion between storage types (same type: copy).
template <typename TO, typename TI>
__device__ __forceinline__ TO convert(TI v) {
  return from_f32<TO>(to_f32(v));
}
template <>
__device__ __forceinline__ float convert<float, float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ bf16 convert<bf16, bf16>(bf16 v) {
  return v;
}
template <>
__device__ __forceinline__ f16 convert<f16, f16>(f16 v) {
  return v;
}

// ---- wave helpers ----------------------------------------------------------------
constexpr int WAVE = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
  return v;
}

// Exact-erf GELU (torch.nn.GELU default): 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

// ---- host error plumbing ------------------------------------------------------------
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string &message);

#define CG_REQUIRE(cond, code, msg)                                   \
  do {                                                                \
    if (!(cond)) throw ::cg::Error((code), std::string(msg));         \
  } while (0)

#define CG_HIP(call)                                                                   \
  do {                                                                                 \
    hipError_t _e = (call);                                                            \
    if (_e != hipSuccess)                                                              \
      throw ::cg::Error(CG_ERR_HIP, std::string(#call) + ": " + hipGetErrorString(_e)); \
  } while (0)

#define CG_LAUNCHED()                                                                     \
  do {                                                                                    \
    hipError_t _e = hipGetLastError();                                                    \
    if (_e != hipSuccess)                                                                 \
      throw ::cg::Error(CG_ERR_HIP, std::string("kernel launch: ") + hipGetErrorString(_e)); \
  } while (0)

// Runs `body` and converts any exception into a status code + thread-local message.
template <typename F>
int guarded(F &&body) {
  try {
    body();
    return CG_OK;
  } catch (const Error &e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return CG_ERR_HIP;
  } catch (...) {
    set_last_error("unknown error");
    return CG_ERR_HIP;
  }
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_size(int32_t dtype) {
  switch (dtype) {
    case CG_F32:
      return 4;
    case CG_BF16:
    case CG_F16:
      return 2;
    default:
      throw Error(CG_ERR_INVALID, "unknown dtype " + std::to_string(dtype));
  }
}

inline void check_layer(const cg_kv_layer *layer) {
  CG_REQUIRE(layer != nullptr, CG_ERR_INVALID, "cache layer is NULL");
  CG_REQUIRE(layer->k != nullptr && layer->v != nullptr, CG_ERR_INVALID, "cache k/v is NULL");
  CG_REQUIRE(layer->capacity > 0 && layer->kv_heads > 0 && layer->max_len > 0 && layer->head_dim > 0,
             CG_ERR_INVALID, "cache dimensions must be positive");
  dtype_size(layer->dtype);
}

}  // namespace cg
