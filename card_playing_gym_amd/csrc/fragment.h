// Device building blocks of the fused bf16 kernels (gfx950): 16-row blocks of eight waves
// whose stages multiply an LDS panel (the A operand, bf16) by weights streamed from L2 in
// MFMA fragment order straight into registers (the B operand), with buffer-descriptor
// loads, non-temporal result stores and DPP row reductions.  Used by the per-layer kernel
// (layer.hip) and the policy / value heads (heads.hip).
#pragma once

#include "common.h"

namespace cg {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;

constexpr int PANEL = 256;            // widest K of a stage (d_model, and the chunk width)
constexpr int ROWB = PANEL * 2 + 16;  // LDS bytes per panel row: bf16 + 16 B pad
constexpr int WAVES = 8;              // waves per block; each owns 32 columns of a stage
constexpr int FN = 2;                 // 16-column fragments per wave and stage
constexpr int THREADS = 64 * WAVES;
constexpr int KS = PANEL / 32;        // 32-wide k-steps per stage

// Global reads go through buffer descriptors (base and size in scalar registers, 32-bit
// per-lane byte offsets): an offset past the end returns 0 instead of faulting, so no
// load needs a branch, and a fragment loads straight into the registers it is used from.
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

__device__ __forceinline__ Rsrc rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, int(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 bload16(Rsrc r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ float bloadf(Rsrc r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ int bloadi(Rsrc r, uint32_t off) {
  return int(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
// Results (residual rows, queries, appended keys / values, hidden rows) are written with
// the non-temporal policy: left dirty in L2 they are written back while the next layer's
// attention streams the pool, which slowed it by ~10 %.
#ifndef CG_NT_STORE
#define CG_NT_STORE 1
#endif
template <typename T>
__device__ __forceinline__ void gst(T *p, T v) {
  if constexpr (CG_NT_STORE && sizeof(T) == 4) {
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, v), reinterpret_cast<uint32_t *>(p));
  } else if constexpr (CG_NT_STORE && sizeof(T) == 2) {
    __builtin_nontemporal_store(__builtin_bit_cast(uint16_t, v), reinterpret_cast<uint16_t *>(p));
  } else {
    *p = v;
  }
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations, not for
// its global loads (the next stage's weights stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// Returns v unchanged but opaque to the optimiser: a kernel short of registers passes row
// and lane indices through it so per-lane offsets are formed where they are used instead of
// being hoisted out of its stage loop.
__device__ __forceinline__ int opaque(int v) {
  __asm__ volatile("" : "+s"(v));
  return v;
}
template <typename T>
__device__ __forceinline__ const T *opaque_ptr(const T *p) {
  __asm__ volatile("" : "+s"(p));
  return p;
}
__device__ __forceinline__ int opaque_lane(int v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ f32x4 mma(const uint4 &a, const uint4 &b, f32x4 c) {
  bf16x8 av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
}

// Weights are stored in MFMA fragment order (pack_fragments below): matrix W [N, K] as
// blocks of 16 rows x 32 k, block (nb, kb) at ((nb * kblocks + kb) * 64 + lane) * 16 bytes,
// lane (li, lg) holding W[16 nb + li][32 kb + 8 lg .. +7] -- exactly the B fragment of
// v_mfma_f32_16x16x32_bf16, so every fragment load is one contiguous 1 KB wave access.
// A stage's slice for one wave: row blocks nb0 + j (j < FN), k blocks kb0 + ks (ks < KS).
// Row blocks past the matrix read as 0 (their output columns are discarded by the
// epilogue); k blocks past the stage's width meet zero A-panel columns.
struct Slice {
  Rsrc w;
  uint32_t kblocks;
  int nb0, kb0;
};

__device__ __forceinline__ uint32_t kblocks_of(int k) { return uint32_t(k + 31) / 32; }

__device__ __forceinline__ uint32_t slice_base(const Slice &s, int j, int lane) {
  return ((uint32_t(s.nb0 + j) * s.kblocks + uint32_t(s.kb0)) * 64 + uint32_t(lane)) * 16;
}

__device__ __forceinline__ void load_slice(uint4 (&buf)[KS][FN], const Slice &s, int lane) {
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const uint32_t base = slice_base(s, j, lane);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) buf[ks][j] = bload16(s.w, base + 1024 * ks);
  }
}

// Keeps k-step ks's refill loads where they are written, right after the MFMAs that read
// the registers.  Left to itself the scheduler sinks a stage's refills below most of its
// MFMAs (the wave waited down to 3 loads in flight before issuing the next 16), so every
// wave's weight stream nearly drained once per stage, all waves at about the same time.
#ifndef CG_PIN_REFILL
#define CG_PIN_REFILL 1
#endif
__device__ __forceinline__ void pin_refill() {
  if (CG_PIN_REFILL) __builtin_amdgcn_sched_barrier(0);
}

// acc[i][j] += panel rows (16 i + l % 16) x W fragment j over all 256 k (panel columns
// past a stage's width are zero, and output columns past the matrix are discarded by the
// epilogue, so no step needs a guard).  Each fragment register is refilled with the next
// stage's fragment as soon as its MFMAs are issued, so the next stage's weights stream in
// during this stage; the code is branch-free so the loads land in the registers the
// MFMAs read.
template <int FM>
__device__ __forceinline__ void stage_mma(f32x4 (&acc)[FM][FN], const unsigned char *lds,
                                          uint4 (&w)[KS][FN], const Slice &next, bool refill, int lane) {
  const int li = lane & 15, lg = lane >> 4;
  uint32_t base[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) base[j] = slice_base(next, j, lane);
  auto a_frag = [&](int ks, int i) {
    return *reinterpret_cast<const uint4 *>(lds + (16 * i + li) * ROWB + (32 * ks + 8 * lg) * 2);
  };
  if constexpr (FM == 1) {
    // One row tile: the stage's A fragments are read up front, one LDS round trip instead
    // of one per k-step.
    uint4 af[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) af[ks] = a_frag(ks, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[0][j] = mma(af[ks], w[ks][j], acc[0][j]);
      if (refill) {
#pragma unroll
        for (int j = 0; j < FN; ++j) w[ks][j] = bload16(next.w, base[j] + 1024 * ks);
      }
      pin_refill();
    }
  } else {
    // Taller blocks: the A fragments of k-step ks + 1 are read while ks multiplies (all of
    // them up front would take 4 FM x KS registers); every weight fragment feeds FM MFMAs.
    uint4 af[2][FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[0][i] = a_frag(0, i);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) {
#pragma unroll
        for (int i = 0; i < FM; ++i) af[(ks + 1) & 1][i] = a_frag(ks + 1, i);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mma(af[ks & 1][i], w[ks][j], acc[i][j]);
      if (refill) {
#pragma unroll
        for (int j = 0; j < FN; ++j) w[ks][j] = bload16(next.w, base[j] + 1024 * ks);
      }
      pin_refill();
    }
  }
}

template <int FM>
__device__ __forceinline__ void zero(f32x4 (&acc)[FM][FN]) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Sum over the 16 lanes of a DPP row (the 16 columns of one MFMA fragment row): quad
// butterflies, then rotations by 4 and 8 within the row; every lane ends with the sum.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum16(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x128>(v);  // row_ror:8
  return v;
}

// GELU with erf (torch.nn.GELU()): 0.5 x (1 + erf(x / sqrt 2)), erf from the rational
// approximation of Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7, far below the bf16
// rounding the result gets): erfc(z) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^{-z^2},
// t = 1 / (1 + p z) for z = |x| / sqrt 2 >= 0.  With q = erfc(z) / 2 (the halves folded into
// the coefficients), Phi(x) = 1 - q for x >= 0 and q for x < 0, so with h = 0.5 - q (one FMA)
// GELU(x) = x / 2 + |x| h for either sign: one more FMA, no compare, select or sign insert.
// Computing h adds at most ~1.5e-8 to Phi, below the approximation's own 7.5e-8.  GELU(+inf)
// = +inf and GELU(-inf) = NaN, as torch's formula gives; GELU(-0) is +0 (torch: -0, the same
// value).  Thirteen VALU instructions, two of them transcendental.
__device__ __forceinline__ float gelu_fast(float x) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752f, fabsf(x), 1.0f));
  float poly = fmaf(0.5f * 1.061405429f, t, 0.5f * -1.453152027f);
  poly = fmaf(poly, t, 0.5f * 1.421413741f);
  poly = fmaf(poly, t, 0.5f * -0.284496736f);
  poly = fmaf(poly, t, 0.5f * 0.254829592f);
  const float e = __builtin_amdgcn_exp2f((x * (-0.5f * 1.4426950408889634f)) * x);
  const float h = fmaf(-(poly * t), e, 0.5f);  // 0.5 - q
  return fmaf(fabsf(x), h, 0.5f * x);
}

// GELU of four bf16 values (packed two per word, low half first) -> four bf16 values: the
// MLP's GELU under autocast, whose input is the bf16 output of mlp[0] (trunk.py:135).
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
__device__ __forceinline__ u32x2_t gelu_bf16x4(u32x2_t x) {
  f32x4 y;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    y[2 * r] = gelu_fast(__uint_as_float(x[r] << 16));
    y[2 * r + 1] = gelu_fast(__uint_as_float(x[r] & 0xffff0000u));
  }
  return __builtin_bit_cast(u32x2_t, __builtin_convertvector(y, bf16x4_t));
}


}  // namespace
}  // namespace cg
