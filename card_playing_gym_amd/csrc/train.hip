// Training side of the trunk (gfx950, fp32): the pieces of a packed-row forward that keeps
// what its backward needs, and that backward (cardgym/nn/trunk.py:124-181, 285-374 under
// autograd; packed rows as in cardgym/nn/packing.py:36-40).
//
//   * gemm_strided_kernel   C = alpha op(A) op(B) + beta C for any strides: the weight
//                           gradients (dW = dY^T X) and input gradients (dX = dY W) of
//                           every projection, on v_mfma_f32_16x16x4_f32;
//   * layernorm_fwd / _bwd  LayerNorm keeping (mean, rstd) per row; the backward's input
//                           gradient per row and per-block partial sums of dw / db;
//   * rmsnorm_bwd           the input RMSNorm's backward (gain only);
//   * gelu_fwd / _bwd       erf GELU and its derivative;
//   * attn_fwd              causal attention inside each packed sequence (GQA), keeping
//                           the log-sum-exp of every (token, head);
//   * attn_bwd_dq / _dkv    its backward: dQ (and D = rowsum(dO * O)) per (token, head),
//                           dK / dV per (token, KV head) summed over the head group.
// The attention kernels give each (token, head) one wave whose lanes take 64 keys (or
// queries) at a time; head_dim is a template parameter (8 to 64).
#include <algorithm>
#include <cmath>
#include <string>

#include "common.h"

namespace cg {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

// bf16 (autocast) precision: values are kept in fp32 storage holding bf16 numbers.  A pair of
// fp32 values to packed bf16, round to nearest even (v_cvt_pk_bf16_f32): a in the low half.
__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
// Four consecutive k of an MFMA fragment as the bf16 operand of v_mfma_f32_16x16x16_bf16.
__device__ __forceinline__ s16x4 bf16x4_of(f32x4 v) {
  const u32x2 p = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
  return __builtin_bit_cast(s16x4, p);
}
// The bf16 value nearest x, as fp32.
__device__ __forceinline__ float round_bf16(float x) { return __builtin_bit_cast(float, pack_bf16(0.f, x) & 0xffff0000u); }

// erf by Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26:
// erf(x) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) e^(-x^2), t = 1 / (1 + p x) for x >= 0
// (odd in x), |error| <= 1.5e-7.  `gauss` receives e^(-x^2), which GELU's derivative reuses.
__device__ __forceinline__ float erf_as(float x, float &gauss) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, ax, 1.0f));
  const float poly =
      t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f), 0.254829592f);
  gauss = __expf(-ax * ax);
  return copysignf(1.0f - poly * gauss, x);
}

// erf GELU, u Phi(u), and its derivative Phi(u) + u phi(u) (phi(u) = e^(-u^2 / 2) / sqrt(2 pi)).
__device__ __forceinline__ float gelu_exact(float u) {
  float gauss;
  return 0.5f * u * (1.0f + erf_as(u * 0.70710678118654752f, gauss));
}
__device__ __forceinline__ float gelu_grad(float u) {
  float gauss;
  const float cdf = 0.5f * (1.0f + erf_as(u * 0.70710678118654752f, gauss));
  return fmaf(u * 0.3989422804014327f, gauss, cdf);
}

// What a GEMM does with each result v = alpha (A B)[m, n] on its way out: add bias[n], round
// to bf16 when `round` (autocast: a bf16 product's output), add beta times the prior value
// (read from `cin` when set, else from C itself: the fp32 residual), then either multiply by
// gelu'(aux_in[m, n]) (GELU_GRAD: the MLP's backward; rounded again under `round`) or also
// write gelu(v) to aux_out[m, n] (GELU: the MLP's forward; rounded under `round`).
// aux_in / aux_out / cin share C's row stride.
enum EpiMode : int32_t { EPI_PLAIN = 0, EPI_GELU = 1, EPI_GELU_GRAD = 2 };
struct Epi {
  const float *bias = nullptr;
  const float *cin = nullptr;
  const float *aux_in = nullptr;
  float *aux_out = nullptr;
  int32_t mode = EPI_PLAIN;
  int32_t round = 0;  // bf16 operands (the GEMM rounds them as it stages) and bf16 outputs
};

__device__ __forceinline__ float epi_value(const Epi &e, float v, float beta, float prior, float bias, float aux) {
  v += bias;
  if (e.round) v = round_bf16(v);
  if (beta != 0.f) v += beta * prior;
  if (e.mode == EPI_GELU_GRAD) {
    v *= gelu_grad(aux);
    if (e.round) v = round_bf16(v);
  }
  return v;
}

__device__ __forceinline__ void epilogue(const Epi &e, float v, float beta, float *__restrict__ C, int64_t ldc,
                                         int64_t m, int64_t n) {
  const int64_t i = m * ldc + n;
  v = epi_value(e, v, beta, beta != 0.f ? (e.cin ? e.cin[i] : C[i]) : 0.f, e.bias ? e.bias[n] : 0.f,
                e.mode == EPI_GELU_GRAD ? e.aux_in[i] : 0.f);
  C[i] = v;
  if (e.mode == EPI_GELU) e.aux_out[i] = e.round ? round_bf16(gelu_exact(v)) : gelu_exact(v);
}

// ---- strided GEMM ---------------------------------------------------------------------
// Tile 128 x 128, four waves (2 x 2, each 64 x 64 = 4 x 4 MFMA tiles), 16 k per LDS stage,
// double-buffered.  A(m, k) = A[m * sam + k * sak], B(k, n) = B[k * sbk + n * sbn]; tiles are
// staged through LDS with 16-byte loads along whichever index has stride 1, and sit there as
// [row][16 k] (row pitch GT_LDK).  MFMA 16x16x4 f32: lane (li, lg) gives A(row li, k) and
// B(k, col li) for the instruction's k index lg; the result sits in lane (li, lg) as rows
// 4 lg + r, column li.  The four MFMAs s = 0..3 of a stage give lane group lg the stage's k
// = 4 lg + s (the sum over k does not depend on which instruction adds which term), so a
// lane's fragments for a whole stage are one 16-byte LDS read per 16-row block.  Split K
// (grid.z > 1): slice z covers k in [z kc, (z + 1) kc) and writes its partial product to
// part[z] ([m, n]); a second pass sums them.
constexpr int GT_M = 128, GT_N = 128, GT_K = 16;
constexpr int GT_LDK = GT_K + 4;  // LDS row pitch, floats: 16-lane groups of 16-byte reads hit 64 banks once

// A ROWS x 16 (rows x k) operand tile (ROWS 64 or 128) with element (r, k) at p[r * sr + k *
// sk], ROWS / 64 float4 per thread.  MODE 1: k contiguous (float4 = 4 k of a row; k extent a multiple of 4); MODE 2:
// rows contiguous (float4 = 4 rows at one k; row extent a multiple of 4); MODE 0: any strides.
// Loads go to clamped, always valid addresses with no branches (so the next stage's loads all
// fly at once during this stage's MFMAs); rows >= rows_left or k >= k_left are zeroed when the
// tile is written to LDS, after the MFMAs.
template <int ROWS>
struct TileRegs {
  float4 v[ROWS / 64];
};

// Row of float4 slot idx in the k-contiguous layouts (MODE 1 and 0): four 4-k blocks of 16 rows
// per 64 slots, the four rows of each 16-slot group 4 apart, so that their LDS rows (pitch 20
// floats) start 0, 16, 32, 48 banks apart and a 16-lane write covers the 64 banks once.
__device__ __forceinline__ int slot_row(int idx) { return (idx >> 6) * 16 + ((idx >> 2) & 3) * 4 + ((idx >> 4) & 3); }

template <int MODE, int ROWS>
__device__ __forceinline__ TileRegs<ROWS> load_tile(const float *__restrict__ p, int64_t sr, int64_t sk, int rows_left,
                                                    int k_left, int tid) {
  TileRegs<ROWS> t;
#pragma unroll
  for (int e = 0; e < ROWS / 64; ++e) {
    const int idx = tid + e * 256;  // ROWS x 16 floats = ROWS * 4 float4
    if constexpr (MODE == 2) {      // 32 groups of 4 rows x 16 k (k fastest across lanes)
      const int k = idx & 15, r = (idx >> 4) * 4;
      const int rc = max(0, min(r, rows_left - 4)), kc = min(k, k_left - 1);
      t.v[e] = *reinterpret_cast<const float4 *>(p + int64_t(kc) * sk + rc);
    } else if constexpr (MODE == 1) {  // 128 rows x 4 groups of 4 k
      const int r = slot_row(idx), k = (idx & 3) * 4;
      const int rc = min(r, rows_left - 1), kc = max(0, min(k, k_left - 4));
      t.v[e] = *reinterpret_cast<const float4 *>(p + int64_t(rc) * sr + kc);
    } else {  // same slots as MODE 1, element by element
      const int r = slot_row(idx), k = (idx & 3) * 4;
      const int64_t base = int64_t(min(r, rows_left - 1)) * sr;
      t.v[e] = float4{p[base + int64_t(min(k, k_left - 1)) * sk], p[base + int64_t(min(k + 1, k_left - 1)) * sk],
                      p[base + int64_t(min(k + 2, k_left - 1)) * sk], p[base + int64_t(min(k + 3, k_left - 1)) * sk]};
    }
  }
  return t;
}

template <int MODE, int ROWS>
__device__ __forceinline__ void store_tile(float *lds, const TileRegs<ROWS> &t, int tid, int rows_left, int k_left) {
#pragma unroll
  for (int e = 0; e < ROWS / 64; ++e) {
    const int idx = tid + e * 256;
    const float4 v = t.v[e];
    if constexpr (MODE == 2) {
      const int k = idx & 15, r = (idx >> 4) * 4;
      const bool ok = k < k_left && r < rows_left;  // row extent a multiple of 4: all four rows or none
      lds[(r + 0) * GT_LDK + k] = ok ? v.x : 0.f;
      lds[(r + 1) * GT_LDK + k] = ok ? v.y : 0.f;
      lds[(r + 2) * GT_LDK + k] = ok ? v.z : 0.f;
      lds[(r + 3) * GT_LDK + k] = ok ? v.w : 0.f;
    } else {
      const int r = slot_row(idx), k = (idx & 3) * 4;
      const bool row = r < rows_left;
      float4 o;
      if constexpr (MODE == 1) {
        const bool ok = row && k < k_left;  // k extent a multiple of 4
        o = ok ? v : float4{0.f, 0.f, 0.f, 0.f};
      } else {
        o = float4{row && k < k_left ? v.x : 0.f, row && k + 1 < k_left ? v.y : 0.f, row && k + 2 < k_left ? v.z : 0.f,
                   row && k + 3 < k_left ? v.w : 0.f};
      }
      *reinterpret_cast<float4 *>(lds + r * GT_LDK + k) = o;
    }
  }
}

// bf16 operands: the same tile converted once as it is written to LDS, [row][16 k] bf16 at a
// 40-byte row pitch (16-lane groups of 8-byte fragment reads hit distinct banks).
constexpr int GT_LDKB = GT_K + 4;  // row pitch in bf16 elements

template <int MODE, int ROWS>
__device__ __forceinline__ void store_tile_bf16(unsigned short *lds, const TileRegs<ROWS> &t, int tid, int rows_left,
                                                int k_left) {
#pragma unroll
  for (int e = 0; e < ROWS / 64; ++e) {
    const int idx = tid + e * 256;
    const float4 v = t.v[e];
    if constexpr (MODE == 2) {
      const int k = idx & 15, r = (idx >> 4) * 4;
      const bool ok = k < k_left && r < rows_left;
      const unsigned lo = pack_bf16(ok ? v.x : 0.f, ok ? v.y : 0.f), hi = pack_bf16(ok ? v.z : 0.f, ok ? v.w : 0.f);
      lds[(r + 0) * GT_LDKB + k] = static_cast<unsigned short>(lo);
      lds[(r + 1) * GT_LDKB + k] = static_cast<unsigned short>(lo >> 16);
      lds[(r + 2) * GT_LDKB + k] = static_cast<unsigned short>(hi);
      lds[(r + 3) * GT_LDKB + k] = static_cast<unsigned short>(hi >> 16);
    } else {
      const int r = slot_row(idx), k = (idx & 3) * 4;
      const bool row = r < rows_left;
      float4 o;
      if constexpr (MODE == 1) {
        o = (row && k < k_left) ? v : float4{0.f, 0.f, 0.f, 0.f};
      } else {
        o = float4{row && k < k_left ? v.x : 0.f, row && k + 1 < k_left ? v.y : 0.f, row && k + 2 < k_left ? v.z : 0.f,
                   row && k + 3 < k_left ? v.w : 0.f};
      }
      *reinterpret_cast<u32x2 *>(lds + r * GT_LDKB + k) = u32x2{pack_bf16(o.x, o.y), pack_bf16(o.z, o.w)};
    }
  }
}

template <int AM, int BM, int TM, bool BF>
__global__ __launch_bounds__(256, 3) void gemm_strided_kernel(int32_t M, int32_t N, int32_t K, int32_t kc, float alpha,
                                                           const float *__restrict__ A, int64_t sam, int64_t sak,
                                                           const float *__restrict__ B, int64_t sbk, int64_t sbn,
                                                           float beta, float *__restrict__ C, int64_t ldc,
                                                           float *__restrict__ part, const Epi epi) {
  constexpr int FM = TM / 32;  // 16-row MFMA blocks per wave: a wave takes TM / 2 rows x 64 columns
  // fp32 tiles [row][GT_LDK floats]; bf16 tiles [row][GT_LDKB halves] (half the storage)
  constexpr int PITCH = BF ? GT_LDKB / 2 : GT_LDK;  // row pitch in 4-byte words
  __shared__ __align__(16) float as[2][TM * PITCH];
  __shared__ __align__(16) float bs[2][GT_N * PITCH];
  auto as16 = [&](int b) { return reinterpret_cast<unsigned short *>(as[b]); };
  auto bs16 = [&](int b) { return reinterpret_cast<unsigned short *>(bs[b]); };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lg = lane >> 4;
  int mt = blockIdx.y, nt = blockIdx.x;
  if (gridDim.z == 1) {  // XCD-aware order: XCD k (block ids = k mod 8) takes a contiguous run of
                         // tiles, N fastest, so the rows of A it reads stay in its own L2
    const int tiles = gridDim.x * gridDim.y, b = blockIdx.x + gridDim.x * blockIdx.y;
    const int xcd = b & 7, per = tiles >> 3, extra = tiles & 7;
    const int t = xcd * per + min(xcd, extra) + (b >> 3);
    mt = t / gridDim.x;
    nt = t % gridDim.x;
  }
  const int m0 = mt * TM, n0 = nt * GT_N;
  const int kbeg = blockIdx.z * kc, kend = min(K, kbeg + kc);
  const float *a0 = A + int64_t(m0) * sam, *b0 = B + int64_t(n0) * sbn;
  f32x4 acc[FM][4];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  int buf = 0;
  const int ma = M - m0, nb_ = N - n0;
  if (kbeg < kend) {
    const auto ta0 = load_tile<AM, TM>(a0 + int64_t(kbeg) * sak, sam, sak, ma, kend - kbeg, tid);
    const auto tb0 = load_tile<BM, GT_N>(b0 + int64_t(kbeg) * sbk, sbn, sbk, nb_, kend - kbeg, tid);
    if constexpr (BF) {
      store_tile_bf16<AM, TM>(as16(0), ta0, tid, ma, kend - kbeg);
      store_tile_bf16<BM, GT_N>(bs16(0), tb0, tid, nb_, kend - kbeg);
    } else {
      store_tile<AM, TM>(as[0], ta0, tid, ma, kend - kbeg);
      store_tile<BM, GT_N>(bs[0], tb0, tid, nb_, kend - kbeg);
    }
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += GT_K) {
    const bool more = k0 + GT_K < kend;
    const int kl = kend - k0 - GT_K;  // k left after this stage
    TileRegs<TM> na;
    TileRegs<GT_N> nb;
    if (more) {  // the next stage's loads fly during this stage's MFMAs
      na = load_tile<AM, TM>(a0 + int64_t(k0 + GT_K) * sak, sam, sak, ma, kl, tid);
      nb = load_tile<BM, GT_N>(b0 + int64_t(k0 + GT_K) * sbk, sbn, sbk, nb_, kl, tid);
    }
    const float *ta = as[buf], *tb = bs[buf];
    if constexpr (BF) {  // bf16 operands: the stage's 16 k in one v_mfma_f32_16x16x16_bf16 per tile,
                         // lane group lg holding k = 4 lg .. 4 lg + 3 as the fp32 path does
      const unsigned short *ta16 = as16(buf), *tb16 = bs16(buf);
      s16x4 bb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bb[j] = *reinterpret_cast<const s16x4 *>(tb16 + (wn * 64 + j * 16 + li) * GT_LDKB + 4 * lg);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const s16x4 ab = *reinterpret_cast<const s16x4 *>(ta16 + (wm * (TM / 2) + i * 16 + li) * GT_LDKB + 4 * lg);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ab, bb[j], acc[i][j], 0, 0, 0);
      }
    } else {
      f32x4 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const f32x4 *>(tb + (wn * 64 + j * 16 + li) * GT_LDK + 4 * lg);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const f32x4 af = *reinterpret_cast<const f32x4 *>(ta + (wm * (TM / 2) + i * 16 + li) * GT_LDK + 4 * lg);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[s], bf[j][s], acc[i][j], 0, 0, 0);
      }
    }
    if (more) {
      if constexpr (BF) {
        store_tile_bf16<AM, TM>(as16(buf ^ 1), na, tid, ma, kl);
        store_tile_bf16<BM, GT_N>(bs16(buf ^ 1), nb, tid, nb_, kl);
      } else {
        store_tile<AM, TM>(as[buf ^ 1], na, tid, ma, kl);
        store_tile<BM, GT_N>(bs[buf ^ 1], nb, tid, nb_, kl);
      }
    }
    __syncthreads();
    buf ^= 1;
  }
  if (part) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * (TM / 2) + i * 16 + 4 * lg + r, n = n0 + wn * 64 + j * 16 + li;
          if (m < M && n < N) part[(int64_t(blockIdx.z) * M + m) * N + n] = acc[i][j][r];
        }
    return;
  }
  // Epilogue: every operand it reads (prior C or cin, bias, aux_in) is loaded for a whole
  // 16-row block at once from clamped, always valid addresses, and unused values are dropped by
  // selects, so the loads overlap instead of waiting one by one behind per-element branches.
  const bool prior = beta != 0.f, fwd_gelu = epi.mode == EPI_GELU;
  const float *pin = epi.cin ? epi.cin : C, *ain = epi.mode == EPI_GELU_GRAD ? epi.aux_in : C;
  float bj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = min(n0 + wn * 64 + j * 16 + li, N - 1);
    bj[j] = epi.bias ? epi.bias[n] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    float pv[4][4], av[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = min(m0 + wm * (TM / 2) + i * 16 + 4 * lg + r, M - 1), n = min(n0 + wn * 64 + j * 16 + li, N - 1);
        pv[j][r] = pin[m * ldc + n];
        av[j][r] = ain[m * ldc + n];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * (TM / 2) + i * 16 + 4 * lg + r, n = n0 + wn * 64 + j * 16 + li;
        const float v = epi_value(epi, alpha * acc[i][j][r], beta, prior ? pv[j][r] : 0.f, bj[j], av[j][r]);
        if (m < M && n < N) {
          const int64_t o = int64_t(m) * ldc + n;
          C[o] = v;
          if (fwd_gelu) epi.aux_out[o] = epi.round ? round_bf16(gelu_exact(v)) : gelu_exact(v);
        }
      }
  }
}

// C[m, n] = epilogue(alpha * sum_z part[z][m, n]).  A thread takes four consecutive entries
// (float4 loads when N is a multiple of 4) and keeps four slices in flight.
__global__ void gemm_reduce_kernel(int32_t M, int32_t N, int32_t slices, float alpha, const float *__restrict__ part,
                                   float beta, float *__restrict__ C, int64_t ldc, const Epi epi) {
  const int64_t total = int64_t(M) * N, quads = (total + 3) / 4;
  const bool vec = (N & 3) == 0;
  for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; q < quads; q += int64_t(gridDim.x) * blockDim.x) {
    const int64_t i0 = 4 * q;
    f32x4 s[4] = {};
    if (vec) {
      int z = 0;
      for (; z + 3 < slices; z += 4)
#pragma unroll
        for (int u = 0; u < 4; ++u) s[u] += *reinterpret_cast<const f32x4 *>(part + int64_t(z + u) * total + i0);
      for (; z < slices; ++z) s[0] += *reinterpret_cast<const f32x4 *>(part + int64_t(z) * total + i0);
    } else {
      for (int z = 0; z < slices; ++z)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (i0 + e < total) s[0][e] += part[int64_t(z) * total + i0 + e];
    }
    const f32x4 t = (s[0] + s[1]) + (s[2] + s[3]);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i0 + e < total) epilogue(epi, alpha * t[e], beta, C, ldc, (i0 + e) / N, (i0 + e) % N);
  }
}

// Launch plan: row tile TM and split K.  A short reduction over few 128-row tiles takes
// 64-row tiles (twice the blocks, no second pass); a long reduction into a small output (the
// weight gradients reduce over every token) is split over k into enough (tile, slice) blocks
// to fill the chip, and a second pass sums the slices.
struct GemmPlan {
  int tm, slices, kc;
};
GemmPlan gemm_plan(int32_t m, int32_t n, int32_t k, bool generic) {
  const int64_t nt = (n + GT_N - 1) / GT_N, tiles128 = int64_t((m + GT_M - 1) / GT_M) * nt;
  int tm = GT_M;
  if (!generic && m > 64 && tiles128 < 512 && !(k >= 1024 && tiles128 < 128)) tm = 64;
  const int64_t tiles = int64_t((m + tm - 1) / tm) * nt;
  // Split K toward 512 blocks, but never past the 768 the chip holds at once (256 CUs x 3
  // blocks): 408 tiles split in two would run as a full wave plus a 48-block tail, slower
  // than the unsplit 408 tiles (13041-token packed batches hit this).
  int slices = 1;
  if (tiles < 512 && k >= 4 * GT_K * 16) {
    slices = int(std::min<int64_t>({(512 + tiles - 1) / tiles, 768 / tiles, k / (GT_K * 16)}));
    slices = std::max(1, std::min(slices, 64));
  }
  const int kc = ((k + slices - 1) / slices + GT_K - 1) / GT_K * GT_K;
  slices = (k + kc - 1) / kc;
  return {tm, slices, kc};
}

// ---- LayerNorm / RMSNorm -----------------------------------------------------------------
// One wave per row.
__global__ void layernorm_fwd_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                     const float *__restrict__ b, float eps, float *__restrict__ y,
                                     float *__restrict__ mean, float *__restrict__ rstd, int32_t n, int32_t d) {
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n) return;
  const float *xr = x + int64_t(row) * d;
  float s = 0.f;
  for (int k = lane; k < d; k += 64) s += xr[k];
  const float mu = wave_sum(s) / float(d);
  float v = 0.f;
  for (int k = lane; k < d; k += 64) {
    const float c = xr[k] - mu;
    v = fmaf(c, c, v);
  }
  const float r = 1.0f / sqrtf(wave_sum(v) / float(d) + eps);
  float *yr = y + int64_t(row) * d;
  for (int k = lane; k < d; k += 64) yr[k] = (xr[k] - mu) * r * w[k] + b[k];
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = r;
  }
}

// The same for d <= 256 NV, d a multiple of 4, 16-byte aligned rows: lane l owns the float4
// columns 4 l + 256 v of a row (two-pass mean and variance from registers), wave w takes rows
// r0 + w, r0 + w + 4, ... of its block's 16, loading the next row while it reduces this one.
template <int NV>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                             const float *__restrict__ b, float eps,
                                                             float *__restrict__ y, float *__restrict__ mean,
                                                             float *__restrict__ rstd, int32_t n, int32_t d) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r0 = blockIdx.x * 16, r1 = min(n, r0 + 16);
  const float4 zero = {0.f, 0.f, 0.f, 0.f};
  float4 wv[NV], bv[NV], xa[NV];
  bool in[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = 4 * lane + 256 * v;
    in[v] = c < d;
    wv[v] = in[v] ? *reinterpret_cast<const float4 *>(w + c) : zero;
    bv[v] = in[v] ? *reinterpret_cast<const float4 *>(b + c) : zero;
  }
  auto load = [&](int row, float4 (&xs)[NV]) {
#pragma unroll
    for (int v = 0; v < NV; ++v)
      xs[v] = in[v] ? *reinterpret_cast<const float4 *>(x + int64_t(row) * d + 4 * lane + 256 * v) : zero;
  };
  int row = r0 + wave;
  if (row < r1) load(row, xa);
  for (; row < r1; row += 4) {
    float4 xc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) xc[v] = xa[v];
    if (row + 4 < r1) load(row + 4, xa);
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) s += (xc[v].x + xc[v].y) + (xc[v].z + xc[v].w);
    const float mu = wave_sum(s) / float(d);
    float q = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (!in[v]) continue;
      const float a0 = xc[v].x - mu, a1 = xc[v].y - mu, a2 = xc[v].z - mu, a3 = xc[v].w - mu;
      q += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
    }
    const float r = 1.0f / sqrtf(wave_sum(q) / float(d) + eps);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (!in[v]) continue;
      *reinterpret_cast<float4 *>(y + int64_t(row) * d + 4 * lane + 256 * v) =
          float4{(xc[v].x - mu) * r * wv[v].x + bv[v].x, (xc[v].y - mu) * r * wv[v].y + bv[v].y,
                 (xc[v].z - mu) * r * wv[v].z + bv[v].z, (xc[v].w - mu) * r * wv[v].w + bv[v].w};
    }
    if (lane == 0) {
      mean[row] = mu;
      rstd[row] = r;
    }
  }
}

// dx = rstd (g - mean(g) - xhat mean(g xhat)) (+ residual), g = dy * w; per block of
// `rows_per_block` rows, partial dw = sum dy xhat and db = sum dy into part[blockIdx][0 / 1][d].
// A NULL mean selects RMSNorm (no centring, no bias).  Any d (norm_bwd_rows_kernel takes the
// common shapes).
__global__ void norm_bwd_kernel(const float *__restrict__ x, const float *__restrict__ dy,
                                const float *__restrict__ w, const float *__restrict__ mean,
                                const float *__restrict__ rstd, const float *__restrict__ residual,
                                float *__restrict__ dx, float *__restrict__ part, int32_t n, int32_t d,
                                int32_t rows_per_block) {
  extern __shared__ float acc_lds[];  // [2][d]
  const int waves = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int k = threadIdx.x; k < 2 * d; k += blockDim.x) acc_lds[k] = 0.f;
  __syncthreads();
  const int r0 = blockIdx.x * rows_per_block;
  for (int row = r0 + wave; row < min(n, r0 + rows_per_block); row += waves) {
    const float *xr = x + int64_t(row) * d, *gr = dy + int64_t(row) * d;
    const float mu = mean ? mean[row] : 0.f, r = rstd[row];
    float sg = 0.f, sgx = 0.f;
    for (int k = lane; k < d; k += 64) {
      const float xh = (xr[k] - mu) * r, g = gr[k] * w[k];
      sg += g;
      sgx = fmaf(g, xh, sgx);
    }
    const float mg = mean ? wave_sum(sg) / float(d) : 0.f, mgx = wave_sum(sgx) / float(d);
    float *dxr = dx + int64_t(row) * d;
    for (int k = lane; k < d; k += 64) {
      const float xh = (xr[k] - mu) * r;
      dxr[k] = r * (gr[k] * w[k] - mg - xh * mgx) + (residual ? residual[int64_t(row) * d + k] : 0.f);
      atomicAdd(&acc_lds[k], gr[k] * xh);  // LDS atomics: order within a block only
      atomicAdd(&acc_lds[d + k], gr[k]);
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < 2 * d; k += blockDim.x) part[int64_t(blockIdx.x) * 2 * d + k] = acc_lds[k];
}

// The same for d <= 256 NV, d a multiple of 4, 16-byte aligned rows: lane l owns the float4
// columns 4 l + 256 v (v < NV) and keeps them, the gain and its dw / db partials in registers;
// wave w of a block takes rows r0 + w, r0 + w + 4, ... of its NORM_ROWS, loading the next row
// while it reduces the current one.
constexpr int NORM_ROWS = 16;

__device__ __forceinline__ float4 f4_fma(float4 a, float4 b, float4 c) {
  return float4{fmaf(a.x, b.x, c.x), fmaf(a.y, b.y, c.y), fmaf(a.z, b.z, c.z), fmaf(a.w, b.w, c.w)};
}

template <int NV>
__global__ __launch_bounds__(256) void norm_bwd_rows_kernel(const float *__restrict__ x, const float *__restrict__ dy,
                                                            const float *__restrict__ w, const float *__restrict__ mean,
                                                            const float *__restrict__ rstd,
                                                            const float *__restrict__ residual, float *__restrict__ dx,
                                                            float *__restrict__ part, int32_t n, int32_t d) {
  __shared__ float4 red[4][2 * 64 * NV];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r0 = blockIdx.x * NORM_ROWS, r1 = min(n, r0 + NORM_ROWS);
  const float4 zero = {0.f, 0.f, 0.f, 0.f};
  float4 wv[NV], pw[NV], pb[NV], xa[NV], ga[NV];
  bool in[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = 4 * lane + 256 * v;
    in[v] = c < d;
    wv[v] = in[v] ? *reinterpret_cast<const float4 *>(w + c) : zero;
    pw[v] = zero;
    pb[v] = zero;
  }
  auto load = [&](int row, float4 (&xs)[NV], float4 (&gs)[NV]) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int64_t i = int64_t(row) * d + 4 * lane + 256 * v;
      xs[v] = in[v] ? *reinterpret_cast<const float4 *>(x + i) : zero;
      gs[v] = in[v] ? *reinterpret_cast<const float4 *>(dy + i) : zero;
    }
  };
  int row = r0 + wave;
  float mu_n = 0.f, r_n = 0.f;
  if (row < r1) {
    load(row, xa, ga);
    mu_n = mean ? mean[row] : 0.f;
    r_n = rstd[row];
  }
  for (; row < r1; row += 4) {
    float4 xc[NV], gc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      xc[v] = xa[v];
      gc[v] = ga[v];
    }
    const float mu = mu_n, r = r_n;
    if (row + 4 < r1) {
      load(row + 4, xa, ga);
      mu_n = mean ? mean[row + 4] : 0.f;
      r_n = rstd[row + 4];
    }
    float4 xh[NV], g[NV];
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      xh[v] = float4{(xc[v].x - mu) * r, (xc[v].y - mu) * r, (xc[v].z - mu) * r, (xc[v].w - mu) * r};
      g[v] = float4{gc[v].x * wv[v].x, gc[v].y * wv[v].y, gc[v].z * wv[v].z, gc[v].w * wv[v].w};
      sg += (g[v].x + g[v].y) + (g[v].z + g[v].w);
      sgx += (g[v].x * xh[v].x + g[v].y * xh[v].y) + (g[v].z * xh[v].z + g[v].w * xh[v].w);
    }
    const float mg = mean ? wave_sum(sg) / float(d) : 0.f, mgx = wave_sum(sgx) / float(d);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (!in[v]) continue;
      const int64_t i = int64_t(row) * d + 4 * lane + 256 * v;
      float4 o = {r * (g[v].x - mg - xh[v].x * mgx), r * (g[v].y - mg - xh[v].y * mgx),
                  r * (g[v].z - mg - xh[v].z * mgx), r * (g[v].w - mg - xh[v].w * mgx)};
      if (residual) {
        const float4 a = *reinterpret_cast<const float4 *>(residual + i);
        o = float4{o.x + a.x, o.y + a.y, o.z + a.z, o.w + a.w};
      }
      *reinterpret_cast<float4 *>(dx + i) = o;
      pw[v] = f4_fma(gc[v], xh[v], pw[v]);
      pb[v] = float4{pb[v].x + gc[v].x, pb[v].y + gc[v].y, pb[v].z + gc[v].z, pb[v].w + gc[v].w};
    }
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    red[wave][v * 64 + lane] = pw[v];
    red[wave][(NV + v) * 64 + lane] = pb[v];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * 64 * NV; i += 256) {
    const int which = i / (64 * NV), v = (i / 64) % NV, c = 4 * (i % 64) + 256 * v;
    if (c >= d) continue;
    const float4 a = red[0][i], b = red[1][i], e = red[2][i], f = red[3][i];
    *reinterpret_cast<float4 *>(part + int64_t(blockIdx.x) * 2 * d + which * d + c) =
        float4{(a.x + b.x) + (e.x + f.x), (a.y + b.y) + (e.y + f.y), (a.z + b.z) + (e.z + f.z),
               (a.w + b.w) + (e.w + f.w)};
  }
}

// dw[c] (+)= sum_p part[p][0][c] and db[c] (+)= sum_p part[p][1][c] (db NULL: RMSNorm): 64 of
// the 2 d columns per block, its 16 waves splitting the partial rows.
__global__ __launch_bounds__(1024) void norm_params_kernel(const float *__restrict__ part, int32_t parts, int32_t d,
                                                           float *__restrict__ dw, float *__restrict__ db,
                                                           int32_t accumulate) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < 2 * d) {
    int p = wave;
    for (; p + 48 < parts; p += 64) {
      s0 += part[int64_t(p) * 2 * d + c];
      s1 += part[int64_t(p + 16) * 2 * d + c];
      s2 += part[int64_t(p + 32) * 2 * d + c];
      s3 += part[int64_t(p + 48) * 2 * d + c];
    }
    for (; p < parts; p += 16) s0 += part[int64_t(p) * 2 * d + c];
  }
  red[wave][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (wave != 0 || c >= 2 * d) return;
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) s += red[q][lane];
  float *o = c < d ? dw + c : (db ? db + (c - d) : nullptr);
  if (o) *o = accumulate ? *o + s : s;
}

// out[c] = sum_r in[r * ld + c] (+ out[c] when accumulate): column sums of per-block
// partials and bias gradients.  A block takes 64 columns x `chunk` rows: its four waves
// split the rows, each lane one column (coalesced rows), and meet in LDS; blockIdx.y's
// chunk lands in out[y][c] (a second pass sums the chunks).
__global__ __launch_bounds__(256) void column_sum_kernel(const float *__restrict__ in, int32_t rows, int32_t cols,
                                                         int64_t ld, float *__restrict__ out, int32_t accumulate,
                                                         int32_t chunk, int32_t round_in, int32_t round_out) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int r0 = blockIdx.y * chunk, r1 = min(rows, r0 + chunk);
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < cols) {
    int r = r0 + wave;
    auto at = [&](int rr) {
      const float v = in[int64_t(rr) * ld + c];
      return round_in ? round_bf16(v) : v;
    };
    for (; r + 12 < r1; r += 16) {
      s0 += at(r);
      s1 += at(r + 4);
      s2 += at(r + 8);
      s3 += at(r + 12);
    }
    for (; r < r1; r += 4) s0 += at(r);
  }
  red[wave][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (wave == 0 && c < cols) {
    float s = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    if (round_out) s = round_bf16(s);
    float *o = out + int64_t(blockIdx.y) * cols + c;
    *o = accumulate ? *o + s : s;
  }
}

// ---- GELU -------------------------------------------------------------------------------

__global__ void gelu_fwd_kernel(const float *__restrict__ u, float *__restrict__ g, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    g[i] = gelu_exact(u[i]);
}

// du = dg * (Phi(u) + u phi(u)).
__global__ void gelu_bwd_kernel(const float *__restrict__ u, const float *__restrict__ dg, float *__restrict__ du,
                                int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    du[i] = dg[i] * gelu_grad(u[i]);
  }
}

// ---- attention ------------------------------------------------------------------------------
// Packed rows: token t belongs to sequence s with seq_start[s] <= t < seq_start[s + 1];
// seq_of[t] = s.  q [N, H, D], k / v [N, KVH, D] (row strides ldq / ldk / ldv floats; the
// gradients dq / dk / dv use the same strides, so they land in a [q | k | v] row buffer
// like their inputs), o and do [N, H, D] dense, lse / dsum [N, H].  Query t of a sequence
// sees its keys start .. t.
struct AttnTrain {
  int32_t n, H, KVH;
  float scale;
  const int64_t *seq_start;
  const int32_t *seq_of;
  const float *q, *k, *v;
  int64_t ldq, ldk, ldv;
  const float *o, *dout, *lse;
  float *out, *lse_out, *dsum, *dq, *dk, *dv;
  int32_t round;  // bf16 outputs (o, dq, dk, dv), as SDPA on bf16 operands returns them
};

__device__ __forceinline__ float attn_out(const AttnTrain &a, float v) { return a.round ? round_bf16(v) : v; }

// The three kernels work on 16 x 16 tiles of (query, key) pairs with v_mfma_f32_16x16x4_f32.
// A contraction over head_dim gives lane (li, lg) the d slice [lg DC, (lg + 1) DC) (DC =
// D / 4), one MFMA per d of the slice (the sum over d is the same whichever lane adds which
// term).  A score tile leaves its MFMA with lane (li, lg) holding rows 4 lg + r, column li;
// a contraction over those rows (keys or queries) is the four MFMAs r = 0..3, MFMA r taking
// rows {4 lg + r} from the lane's own registers, so scores never leave the lane.  Outputs
// over d come out transposed ([d][row]) so that each lane stores four consecutive d.
constexpr int KT = 64;  // keys per staged K / V tile (forward and dQ)

template <int D>
struct AttnDims {
  static constexpr int DC = D / 4;                      // d per lane in a contraction over d
  static constexpr int DT = (D + 15) / 16;              // 16-wide d tiles of an output
  static constexpr int LD = DT * 16 + 4;                // LDS row, floats; d in [D, 16 DT) hold 0
  static constexpr int C4 = D / 4;                      // float4 per row
  static constexpr int PER_KV = (2 * KT * C4 + 255) / 256;  // float4 per thread, one K + V tile
  static constexpr int QR = D <= 32 ? 64 : 32;             // query tokens per dK / dV unit (VGPRs bound it at 64)
  static constexpr int QH = QR / 16;                        // its 16-query sub-tiles
  static constexpr int PER_Q = (2 * QR * C4 + 255) / 256;   // float4 per thread, one Q + dO unit
};

template <int DC>
__device__ __forceinline__ void lds_slice(const float *p, float (&out)[DC]) {
  if constexpr (DC % 4 == 0) {
#pragma unroll
    for (int i = 0; i < DC; i += 4) {
      const float4 v = *reinterpret_cast<const float4 *>(p + i);
      out[i] = v.x;
      out[i + 1] = v.y;
      out[i + 2] = v.z;
      out[i + 3] = v.w;
    }
  } else {
    static_assert(DC % 2 == 0, "head_dim a multiple of 8");
#pragma unroll
    for (int i = 0; i < DC; i += 2) {
      const float2 v = *reinterpret_cast<const float2 *>(p + i);
      out[i] = v.x;
      out[i + 1] = v.y;
    }
  }
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float max_over_rows(float x) {  // over lanes li, li + 16, li + 32, li + 48
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float sum_over_rows(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Zeroes the d >= D columns of `rows` LDS rows (they feed output rows that are never stored).
template <int D>
__device__ __forceinline__ void zero_pad(float *t, int rows) {
  using S = AttnDims<D>;
  constexpr int W = S::DT * 16 - D;
  if constexpr (W > 0)
    for (int i = threadIdx.x; i < rows * W; i += blockDim.x) t[(i / W) * S::LD + D + i % W] = 0.f;
}

// K / V tile of keys [j0, j0 + KT) of KV head hk (rows past n read 0), global -> registers -> LDS.
template <int D>
__device__ __forceinline__ void kv_load(const AttnTrain &a, int hk, int64_t j0, float4 (&r)[AttnDims<D>::PER_KV]) {
  using S = AttnDims<D>;
#pragma unroll
  for (int e = 0; e < S::PER_KV; ++e) {
    const int i = threadIdx.x + 256 * e;
    float4 x = {0.f, 0.f, 0.f, 0.f};
    if (i < 2 * KT * S::C4) {
      const bool isv = i >= KT * S::C4;
      const int ii = isv ? i - KT * S::C4 : i, row = ii / S::C4, c = (ii % S::C4) * 4;
      const int64_t j = j0 + row;
      if (j < a.n) x = *reinterpret_cast<const float4 *>((isv ? a.v + j * a.ldv : a.k + j * a.ldk) + hk * D + c);
    }
    r[e] = x;
  }
}

template <int D>
__device__ __forceinline__ void kv_store(float *kt, float *vt, const float4 (&r)[AttnDims<D>::PER_KV]) {
  using S = AttnDims<D>;
#pragma unroll
  for (int e = 0; e < S::PER_KV; ++e) {
    const int i = threadIdx.x + 256 * e;
    if (i < 2 * KT * S::C4) {
      const bool isv = i >= KT * S::C4;
      const int ii = isv ? i - KT * S::C4 : i, row = ii / S::C4, c = (ii % S::C4) * 4;
      *reinterpret_cast<float4 *>((isv ? vt : kt) + row * S::LD + c) = r[e];
    }
  }
}

// Block of the forward and dQ kernels: 256 threads; wave w takes a strip of 16 tokens
// (strip w / gpb) of head g = gpb blockIdx.z + w % gpb of KV head blockIdx.y, gpb =
// min(G, 4) heads and 4 / gpb strips per block, so all waves share every staged K / V tile.
struct QueryStrip {
  int h;
  bool active;     // the wave has a head and tokens
  int64_t t0;      // first token of the wave's strip
  int64_t base;    // first token of the block
  int64_t b_last;  // last token of the block
};

__device__ __forceinline__ QueryStrip query_strip(const AttnTrain &a) {
  const int G = a.H / a.KVH, gpb = min(G, 4), tpb = 4 / gpb, wave = threadIdx.x >> 6;
  const int strip = wave / gpb, g = blockIdx.z * gpb + wave % gpb;
  QueryStrip q;
  q.base = int64_t(blockIdx.x) * 16 * tpb;
  q.b_last = min<int64_t>(a.n - 1, q.base + 16 * tpb - 1);
  q.t0 = q.base + 16 * strip;
  q.active = strip < tpb && g < G && q.t0 < a.n;
  q.h = blockIdx.y * G + min(g, G - 1);
  return q;
}

// Forward: online softmax over K / V tiles staged KT keys at a time.  S^T = K Q^T (keys on
// the rows, the lane's query li on the column), row statistics per query across the four
// lanes li + 16 lg, O^T += V^T P^T.
template <int D>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const AttnTrain a) {
  using S = AttnDims<D>;
  __shared__ __align__(16) float kt[2][KT * S::LD], vt[2][KT * S::LD];
  const int hk = blockIdx.y, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const QueryStrip w = query_strip(a);
  const int64_t t = w.t0 + li, w_last = min<int64_t>(a.n - 1, w.t0 + 15);
  const bool live = w.active && t < a.n;
  const int64_t start = live ? a.seq_start[a.seq_of[t]] : 0;
  const int64_t w_first = w.active ? a.seq_start[a.seq_of[w.t0]] : 0;  // first key any query of the strip sees
  const int64_t k_lo = a.seq_start[a.seq_of[w.base]];
  zero_pad<D>(kt[0], 2 * KT);
  zero_pad<D>(vt[0], 2 * KT);
  float qf[S::DC];
#pragma unroll
  for (int kk = 0; kk < S::DC; ++kk) qf[kk] = live ? a.q[t * a.ldq + w.h * D + lg * S::DC + kk] * a.scale : 0.f;
  f32x4 acc[S::DT];
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, l = 0.f;
  float4 pre[S::PER_KV];
  kv_load<D>(a, hk, k_lo, pre);
  kv_store<D>(kt[0], vt[0], pre);
  __syncthreads();
  int buf = 0;
  for (int64_t j0 = k_lo; j0 <= w.b_last; j0 += KT) {
    const bool more = j0 + KT <= w.b_last;
    if (more) kv_load<D>(a, hk, j0 + KT, pre);  // the next tile's loads fly during this one's MFMAs
    if (w.active && j0 <= w_last && j0 + KT - 1 >= w_first) {
      const float *K = kt[buf], *V = vt[buf];
      f32x4 s[4];
      bool any[4];
      float mt = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const int64_t jb = j0 + 16 * sub;
        any[sub] = jb <= w_last && jb + 15 >= w_first;
        s[sub] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (any[sub]) {
          float kf[S::DC];
          lds_slice<S::DC>(K + (16 * sub + li) * S::LD + lg * S::DC, kf);
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < S::DC; ++kk) c = mfma4(kf[kk], qf[kk], c);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t j = jb + 4 * lg + r;
            s[sub][r] = (live && j >= start && j <= t) ? c[r] : -INFINITY;
            mt = fmaxf(mt, s[sub][r]);
          }
        }
      }
      mt = max_over_rows(mt);
      const float mn = fmaxf(m, mt);
      const float corr = __expf(m - mn);
      m = mn;
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < S::DT; ++dt) acc[dt] *= corr;
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        if (!any[sub]) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[sub][r] = __expf(s[sub][r] - mn);
          l += s[sub][r];
        }
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[dt] = mfma4(V[(16 * sub + 4 * lg + r) * S::LD + dt * 16 + li], s[sub][r], acc[dt]);
      }
    }
    if (more) kv_store<D>(kt[buf ^ 1], vt[buf ^ 1], pre);
    __syncthreads();
    buf ^= 1;
  }
  l = sum_over_rows(l);
  if (!live) return;
  const float inv = 1.0f / l;
  float *orow = a.out + (t * a.H + w.h) * D;
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = dt * 16 + 4 * lg + r;
      if (d < D) orow[d] = attn_out(a, acc[dt][r] * inv);
    }
  if (lg == 0) a.lse_out[t * a.H + w.h] = m + logf(l);
}

// dQ (and D = rowsum(dO * O)) with the forward's blocks: S^T = K Q^T and dP^T = V dO^T per
// 16-key tile, P from the saved log-sum-exp, dS = P (dP - D), dQ^T += K^T dS^T.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const AttnTrain a) {
  using S = AttnDims<D>;
  __shared__ __align__(16) float kt[2][KT * S::LD], vt[2][KT * S::LD];
  const int hk = blockIdx.y, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const QueryStrip w = query_strip(a);
  const int64_t t = w.t0 + li, w_last = min<int64_t>(a.n - 1, w.t0 + 15);
  const bool live = w.active && t < a.n;
  const int64_t row = t * a.H + w.h;
  const int64_t start = live ? a.seq_start[a.seq_of[t]] : 0;
  const int64_t w_first = w.active ? a.seq_start[a.seq_of[w.t0]] : 0;
  const int64_t k_lo = a.seq_start[a.seq_of[w.base]];
  zero_pad<D>(kt[0], 2 * KT);
  zero_pad<D>(vt[0], 2 * KT);
  float qf[S::DC], gf[S::DC];
  float part = 0.f;
#pragma unroll
  for (int kk = 0; kk < S::DC; ++kk) {
    const int d = lg * S::DC + kk;
    qf[kk] = live ? a.q[t * a.ldq + w.h * D + d] * a.scale : 0.f;
    gf[kk] = live ? a.dout[row * D + d] : 0.f;
    part = fmaf(gf[kk], live ? a.o[row * D + d] : 0.f, part);
  }
  const float dsum = sum_over_rows(part);
  const float lse = live ? a.lse[row] : 0.f;
  f32x4 acc[S::DT];
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float4 pre[S::PER_KV];
  kv_load<D>(a, hk, k_lo, pre);
  kv_store<D>(kt[0], vt[0], pre);
  __syncthreads();
  int buf = 0;
  for (int64_t j0 = k_lo; j0 <= w.b_last; j0 += KT) {
    const bool more = j0 + KT <= w.b_last;
    if (more) kv_load<D>(a, hk, j0 + KT, pre);
    if (w.active && j0 <= w_last && j0 + KT - 1 >= w_first) {
      const float *K = kt[buf], *V = vt[buf];
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const int64_t jb = j0 + 16 * sub;
        if (!(jb <= w_last && jb + 15 >= w_first)) continue;
        float kf[S::DC], vf[S::DC];
        lds_slice<S::DC>(K + (16 * sub + li) * S::LD + lg * S::DC, kf);
        lds_slice<S::DC>(V + (16 * sub + li) * S::LD + lg * S::DC, vf);
        f32x4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < S::DC; ++kk) {
          st = mfma4(kf[kk], qf[kk], st);
          dp = mfma4(vf[kk], gf[kk], dp);
        }
        f32x4 ds;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t j = jb + 4 * lg + r;
          const float p = (live && j >= start && j <= t) ? __expf(st[r] - lse) : 0.f;
          ds[r] = p * (dp[r] - dsum);
        }
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[dt] = mfma4(K[(16 * sub + 4 * lg + r) * S::LD + dt * 16 + li], ds[r], acc[dt]);
      }
    }
    if (more) kv_store<D>(kt[buf ^ 1], vt[buf ^ 1], pre);
    __syncthreads();
    buf ^= 1;
  }
  if (!live) return;
  float *dqrow = a.dq + t * a.ldq + w.h * D;
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = dt * 16 + 4 * lg + r;
      if (d < D) dqrow[d] = attn_out(a, acc[dt][r] * a.scale);
    }
  if (lg == 0) a.dsum[row] = dsum;
}

// One staged query unit of the dK / dV kernel: QR tokens of one head (q scaled, dO, lse, D).
template <int D>
struct QueryUnit {
  float4 v[AttnDims<D>::PER_Q];
  float s;
};

template <int D>
__device__ __forceinline__ QueryUnit<D> unit_load(const AttnTrain &a, int h, int64_t t0) {
  using S = AttnDims<D>;
  QueryUnit<D> u;
#pragma unroll
  for (int e = 0; e < S::PER_Q; ++e) {
    const int i = threadIdx.x + 256 * e;
    float4 x = {0.f, 0.f, 0.f, 0.f};
    if (i < 2 * S::QR * S::C4) {
      const bool isg = i >= S::QR * S::C4;
      const int ii = isg ? i - S::QR * S::C4 : i, row = ii / S::C4, c = (ii % S::C4) * 4;
      const int64_t t = t0 + row;
      if (t < a.n) {
        if (isg) {
          x = *reinterpret_cast<const float4 *>(a.dout + (t * a.H + h) * D + c);
        } else {
          x = *reinterpret_cast<const float4 *>(a.q + t * a.ldq + h * D + c);
          x.x *= a.scale;
          x.y *= a.scale;
          x.z *= a.scale;
          x.w *= a.scale;
        }
      }
    }
    u.v[e] = x;
  }
  u.s = 0.f;
  const int64_t t = t0 + (threadIdx.x % S::QR);
  if (threadIdx.x < 2 * S::QR && t < a.n) u.s = threadIdx.x < S::QR ? a.lse[t * a.H + h] : a.dsum[t * a.H + h];
  return u;
}

template <int D>
__device__ __forceinline__ void unit_store(float *qs, float *gs, float *ls, const QueryUnit<D> &u) {
  using S = AttnDims<D>;
#pragma unroll
  for (int e = 0; e < S::PER_Q; ++e) {
    const int i = threadIdx.x + 256 * e;
    if (i < 2 * S::QR * S::C4) {
      const bool isg = i >= S::QR * S::C4;
      const int ii = isg ? i - S::QR * S::C4 : i, row = ii / S::C4, c = (ii % S::C4) * 4;
      *reinterpret_cast<float4 *>((isg ? gs : qs) + row * S::LD + c) = u.v[e];
    }
  }
  if (threadIdx.x < 2 * S::QR) ls[threadIdx.x] = u.s;  // [0, S::QR) lse, [S::QR, 2 S::QR) D
}

// dK / dV: a block holds 64 keys of KV head blockIdx.y, wave w keys j0 + 16 w + li in
// registers, and walks the units (16-token tile, head of the group) that can see them,
// staged through LDS.  S = Q K^T and dP = dO V^T (queries on the rows), P and dS per lane,
// dV^T += dO^T P and dK^T += Q^T dS (q staged scaled, so dK needs no further scale).
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dkv_kernel(const AttnTrain a) {
  using S = AttnDims<D>;
  __shared__ __align__(16) float qs[2][S::QR * S::LD], gs[2][S::QR * S::LD], ls[2][2 * S::QR];
  const int G = a.H / a.KVH, hk = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int64_t j0 = int64_t(blockIdx.x) * 64, jw = j0 + 16 * wave, j = jw + li;
  const bool live = j < a.n, wave_live = jw < a.n;
  const int64_t end = live ? a.seq_start[a.seq_of[j] + 1] : 0;
  const int64_t w_hi = wave_live ? a.seq_start[a.seq_of[min<int64_t>(a.n - 1, jw + 15)] + 1] : 0;
  const int64_t q_hi = a.seq_start[a.seq_of[min<int64_t>(a.n - 1, j0 + 63)] + 1];
  const int units = int((q_hi - j0 + S::QR - 1) / S::QR) * G;
  zero_pad<D>(qs[0], 2 * S::QR);
  zero_pad<D>(gs[0], 2 * S::QR);
  float kf[S::DC], vf[S::DC];
#pragma unroll
  for (int kk = 0; kk < S::DC; ++kk) {
    const int d = lg * S::DC + kk;
    kf[kk] = live ? a.k[j * a.ldk + hk * D + d] : 0.f;
    vf[kk] = live ? a.v[j * a.ldv + hk * D + d] : 0.f;
  }
  f32x4 dk[S::DT], dv[S::DT];
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt) {
    dk[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  unit_store<D>(qs[0], gs[0], ls[0], unit_load<D>(a, hk * G, j0));
  __syncthreads();
  int buf = 0;
  for (int u = 0; u < units; ++u) {
    const bool more = u + 1 < units;
    QueryUnit<D> next;
    if (more) next = unit_load<D>(a, hk * G + (u + 1) % G, j0 + S::QR * ((u + 1) / G));
    const int64_t t0 = j0 + S::QR * (u / G);
    // The unit's 16-query sub-tiles: independent S / dP chains, then the dV / dK updates.
    bool act[S::QH];
#pragma unroll
    for (int hf = 0; hf < S::QH; ++hf) act[hf] = wave_live && t0 + 16 * hf + 15 >= jw && t0 + 16 * hf < w_hi;
    bool any = false;
#pragma unroll
    for (int hf = 0; hf < S::QH; ++hf) any = any || act[hf];
    if (any) {
      const float *Q = qs[buf], *GO = gs[buf], *L = ls[buf];
      f32x4 sc[S::QH], dp[S::QH], p[S::QH], ds[S::QH];
#pragma unroll
      for (int hf = 0; hf < S::QH; ++hf) {
        sc[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (!act[hf]) continue;
        float qa[S::DC], ga[S::DC];
        lds_slice<S::DC>(Q + (16 * hf + li) * S::LD + lg * S::DC, qa);
        lds_slice<S::DC>(GO + (16 * hf + li) * S::LD + lg * S::DC, ga);
#pragma unroll
        for (int kk = 0; kk < S::DC; ++kk) {
          sc[hf] = mfma4(qa[kk], kf[kk], sc[hf]);
          dp[hf] = mfma4(ga[kk], vf[kk], dp[hf]);
        }
      }
#pragma unroll
      for (int hf = 0; hf < S::QH; ++hf) {
        const float4 lse4 = *reinterpret_cast<const float4 *>(L + 16 * hf + 4 * lg);
        const float4 dsum4 = *reinterpret_cast<const float4 *>(L + S::QR + 16 * hf + 4 * lg);
        const float lse[4] = {lse4.x, lse4.y, lse4.z, lse4.w}, dsm[4] = {dsum4.x, dsum4.y, dsum4.z, dsum4.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t t = t0 + 16 * hf + 4 * lg + r;
          p[hf][r] = (act[hf] && live && t >= j && t < end) ? __expf(sc[hf][r] - lse[r]) : 0.f;
          ds[hf][r] = p[hf][r] * (dp[hf][r] - dsm[r]);
        }
      }
#pragma unroll
      for (int hf = 0; hf < S::QH; ++hf) {
        if (!act[hf]) continue;
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            dv[dt] = mfma4(GO[(16 * hf + 4 * lg + r) * S::LD + dt * 16 + li], p[hf][r], dv[dt]);
            dk[dt] = mfma4(Q[(16 * hf + 4 * lg + r) * S::LD + dt * 16 + li], ds[hf][r], dk[dt]);
          }
      }
    }
    if (more) unit_store<D>(qs[buf ^ 1], gs[buf ^ 1], ls[buf ^ 1], next);
    __syncthreads();
    buf ^= 1;
  }
  if (!live) return;
  float *dkrow = a.dk + j * a.ldk + hk * D, *dvrow = a.dv + j * a.ldv + hk * D;
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = dt * 16 + 4 * lg + r;
      if (d < D) {
        dkrow[d] = attn_out(a, dk[dt][r]);
        dvrow[d] = attn_out(a, dv[dt][r]);
      }
    }
}

// dst[i] = 0: clears the accumulated gradients (a kernel rather than a memset node, so a
// captured backward replays it like any other launch).
__global__ void zero_fill_kernel(float *__restrict__ dst, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = 0.0f;
}

// dst[r, c] += alpha * src[r * ld_src + c] (ld_src 0 broadcasts one row: bias adds).
__global__ void add_strided_kernel(int32_t rows, int32_t cols, float alpha, const float *__restrict__ src,
                                   int64_t ld_src, float *__restrict__ dst, int64_t ld_dst) {
  const int64_t total = int64_t(rows) * cols;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / cols;
    const int c = int(i % cols);
    dst[r * ld_dst + c] += alpha * src[r * ld_src + c];
  }
}

// Gain-only RMSNorm keeping rstd per row (one wave per row).
__global__ void rmsnorm_fwd_kernel(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                   float *__restrict__ y, float *__restrict__ rstd, int32_t n, int32_t d) {
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n) return;
  const float *xr = x + int64_t(row) * d;
  float s = 0.f;
  for (int k = lane; k < d; k += 64) s = fmaf(xr[k], xr[k], s);
  const float r = 1.0f / sqrtf(wave_sum(s) / float(d) + eps);
  float *yr = y + int64_t(row) * d;
  for (int k = lane; k < d; k += 64) yr[k] = xr[k] * r * w[k];
  if (lane == 0) rstd[row] = r;
}

// seq_of[t] for packed rows.
__global__ void seq_of_kernel(const int64_t *__restrict__ seq_start, int32_t n_seqs, int32_t *__restrict__ seq_of) {
  const int s = blockIdx.x;
  if (s >= n_seqs) return;
  for (int64_t t = seq_start[s] + threadIdx.x; t < seq_start[s + 1]; t += blockDim.x) seq_of[t] = s;
}

unsigned blocks_of(int64_t items, int per_block) { return unsigned((items + per_block - 1) / per_block); }
unsigned grid_1d(int64_t n) { return unsigned(std::min<int64_t>((n + 255) / 256, 8192)); }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Operand checks shared by the attention launchers: the kernels load rows of q / k / v as
// float4, so rows start 16-byte aligned.
void check_attn_train(const cg_attn_train *p) {
  CG_REQUIRE(p && p->H > 0 && p->KVH > 0 && p->H % p->KVH == 0 && p->H / p->KVH <= 16, CG_ERR_INVALID,
             "training attention: H a multiple of KVH, at most 16 heads per KV head");
  CG_REQUIRE(p->q && p->k && p->v && p->seq_start && p->seq_of, CG_ERR_INVALID,
             "attention q, k, v, seq_start and seq_of are required");
  CG_REQUIRE(aligned16(p->q) && aligned16(p->k) && aligned16(p->v) && p->ldq % 4 == 0 && p->ldk % 4 == 0 &&
                 p->ldv % 4 == 0,
             CG_ERR_INVALID, "attention q / k / v: 16-byte aligned rows (pointers and row strides)");
}

// Operand mode (rows, k) of a GEMM input: 1 k contiguous, 2 rows contiguous, 0 any strides.
int operand_mode(const float *p, int64_t sr, int64_t sk, int32_t rows, int32_t kk) {
  if (!aligned16(p)) return 0;
  if (sk == 1 && sr % 4 == 0 && kk % 4 == 0) return 1;
  if (sr == 1 && sk % 4 == 0 && rows % 4 == 0) return 2;
  return 0;
}

GemmPlan plan_of(int32_t m, int32_t n, int32_t k, const float *a, int64_t sam, int64_t sak, const float *b,
                 int64_t sbk, int64_t sbn, int *am, int *bm) {
  *am = operand_mode(a, sam, sak, m, k);
  *bm = operand_mode(b, sbn, sbk, n, k);
  if (*am == 0 || *bm == 0) *am = *bm = 0;
  return gemm_plan(m, n, k, *am == 0);
}

void gemm_launch(int32_t m, int32_t n, int32_t k, float alpha, const float *a, int64_t sam, int64_t sak,
                 const float *b, int64_t sbk, int64_t sbn, float beta, float *c, int64_t ldc, void *workspace,
                 size_t workspace_size, const Epi &epi, void *stream) {
  CG_REQUIRE(m >= 0 && n >= 0 && k >= 0, CG_ERR_INVALID, "negative GEMM size");
  if (m == 0 || n == 0) return;
  CG_REQUIRE(a && b && c, CG_ERR_INVALID, "a, b and c are required");
  CG_REQUIRE((epi.mode != EPI_GELU || epi.aux_out) && (epi.mode != EPI_GELU_GRAD || epi.aux_in), CG_ERR_INVALID,
             "GEMM epilogue: GELU needs its second output, GELU' its pre-activation");
  int am, bm;
  const GemmPlan pl = plan_of(m, n, k, a, sam, sak, b, sbk, sbn, &am, &bm);
  const size_t need = pl.slices > 1 ? size_t(pl.slices) * size_t(m) * size_t(n) * 4 : 0;
  CG_REQUIRE(need == 0 || (workspace && workspace_size >= need), CG_ERR_INVALID,
             "GEMM: workspace too small, need " + std::to_string(need) + " bytes");
  const dim3 grid(unsigned((n + GT_N - 1) / GT_N), unsigned((m + pl.tm - 1) / pl.tm), unsigned(pl.slices));
  CG_REQUIRE(grid.y <= 65535, CG_ERR_UNSUPPORTED, "GEMM: too many row tiles");
  hipStream_t s = as_stream(stream);
  float *part = pl.slices > 1 ? static_cast<float *>(workspace) : nullptr;
  const int32_t kc = pl.kc;
  const bool bf = epi.round != 0;
#define CG_GEMM_CASE(A_, B_, T_)                                                                                 \
  if (am == A_ && bm == B_ && pl.tm == T_) {                                                                     \
    if (bf)                                                                                                      \
      gemm_strided_kernel<A_, B_, T_, true><<<grid, 256, 0, s>>>(m, n, k, kc, alpha, a, sam, sak, b, sbk, sbn, beta, \
                                                                 c, ldc, part, epi);                             \
    else                                                                                                         \
      gemm_strided_kernel<A_, B_, T_, false><<<grid, 256, 0, s>>>(m, n, k, kc, alpha, a, sam, sak, b, sbk, sbn,    \
                                                                  beta, c, ldc, part, epi);                      \
  }
  CG_GEMM_CASE(1, 1, 128)
  CG_GEMM_CASE(1, 2, 128)
  CG_GEMM_CASE(2, 1, 128)
  CG_GEMM_CASE(2, 2, 128)
  CG_GEMM_CASE(1, 1, 64)
  CG_GEMM_CASE(1, 2, 64)
  CG_GEMM_CASE(2, 1, 64)
  CG_GEMM_CASE(2, 2, 64)
  CG_GEMM_CASE(0, 0, 128)
#undef CG_GEMM_CASE
  CG_LAUNCHED();
  if (part) {
    gemm_reduce_kernel<<<grid_1d((int64_t(m) * n + 3) / 4), 256, 0, s>>>(m, n, pl.slices, alpha, part, beta, c, ldc,
                                                                        epi);
    CG_LAUNCHED();
  }
}

// Split-K partials of a GEMM (an upper bound over the operand layouts: the generic layout
// never splits more than the others).
size_t gemm_workspace_bytes(int32_t m, int32_t n, int32_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  size_t most = 0;
  for (bool generic : {false, true}) {
    const GemmPlan pl = gemm_plan(m, n, k, generic);
    if (pl.slices > 1) most = std::max(most, size_t(pl.slices) * size_t(m) * size_t(n) * 4);
  }
  return most;
}

size_t column_sum_ws(int32_t rows, int32_t cols) {
  return rows > 2048 ? size_t((rows + 255) / 256) * size_t(std::max(cols, 0)) * 4 : 0;
}

// out[c] (+)= sum_r x[r * ld + c]; with `bf16`, the sum of the bf16-rounded entries, rounded to
// bf16 (a bias gradient under autocast: the sum of a bf16 gradient, returned in bf16).
void column_sum_launch(const float *x, int32_t rows, int32_t cols, int64_t ld, float *out, int32_t accumulate,
                       void *workspace, size_t workspace_size, bool bf16, void *stream) {
  if (cols == 0) return;
  CG_REQUIRE(x && out && rows >= 0, CG_ERR_INVALID, "column sum operands are required");
  hipStream_t s = as_stream(stream);
  const int32_t r = bf16 ? 1 : 0;
  if (rows <= 2048) {
    column_sum_kernel<<<dim3(blocks_of(cols, 64), 1), 256, 0, s>>>(x, rows, cols, ld, out, accumulate, rows, r, r);
    CG_LAUNCHED();
    return;
  }
  const size_t need = column_sum_ws(rows, cols);
  CG_REQUIRE(workspace && workspace_size >= need, CG_ERR_INVALID, "column sum: workspace too small");
  const int chunks = (rows + 255) / 256;
  float *part = static_cast<float *>(workspace);
  column_sum_kernel<<<dim3(blocks_of(cols, 64), unsigned(chunks)), 256, 0, s>>>(x, rows, cols, ld, part, 0, 256, r, 0);
  CG_LAUNCHED();
  column_sum_kernel<<<dim3(blocks_of(cols, 64), 1), 256, 0, s>>>(part, chunks, cols, cols, out, accumulate, chunks, 0,
                                                                 r);
  CG_LAUNCHED();
}

// dst[r, c] = bf16(dst[r, c] + src[r * ld_src + c]): the value embedding added to v in fp32 and
// rounded once (the attention reads bf16 v).
__global__ void add_round_kernel(int32_t rows, int32_t cols, const float *__restrict__ src, int64_t ld_src,
                                 float *__restrict__ dst, int64_t ld_dst) {
  const int64_t total = int64_t(rows) * cols;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / cols;
    const int c = int(i % cols);
    float *d = dst + r * ld_dst + c;
    *d = round_bf16(*d + src[r * ld_src + c]);
  }
}

// Grid of the forward and dQ kernels: blocks of 16 tokens x four heads of a group, or more
// tokens per block when the group has fewer heads.
dim3 query_grid(const cg_attn_train &p) {
  const int G = p.H / p.KVH, gpb = std::min(G, 4), tpb = 4 / gpb;
  return dim3(blocks_of(p.n, 16 * tpb), unsigned(p.KVH), unsigned((G + gpb - 1) / gpb));
}


}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

size_t cg_gemm_workspace_size(int32_t m, int32_t n, int32_t k) { return gemm_workspace_bytes(m, n, k); }

int cg_gemm_strided(int32_t m, int32_t n, int32_t k, float alpha, const float *a, int64_t sam, int64_t sak,
                    const float *b, int64_t sbk, int64_t sbn, float beta, float *c, int64_t ldc,
                    int32_t compute_dtype, void *workspace, size_t workspace_size, void *stream) {
  return guarded([&] {
    CG_REQUIRE(compute_dtype == CG_F32 || compute_dtype == CG_BF16, CG_ERR_UNSUPPORTED,
               "GEMM compute dtype: CG_F32 or CG_BF16");
    Epi e;
    e.round = compute_dtype == CG_BF16;
    gemm_launch(m, n, k, alpha, a, sam, sak, b, sbk, sbn, beta, c, ldc, workspace, workspace_size, e, stream);
  });
}

int cg_layernorm_fwd(const float *x, const float *w, const float *b, float eps, float *y, float *mean, float *rstd,
                     int32_t n, int32_t d, void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(x && w && b && y && mean && rstd && d > 0, CG_ERR_INVALID, "LayerNorm operands are required");
    hipStream_t s = as_stream(stream);
    if (d % 4 == 0 && d <= 1024 && aligned16(x) && aligned16(w) && aligned16(b) && aligned16(y)) {
      switch ((d + 255) / 256) {
#define CG_LN_CASE(NV)                                                                                        \
  case NV:                                                                                                    \
    layernorm_rows_kernel<NV><<<blocks_of(n, 16), 256, 0, s>>>(x, w, b, eps, y, mean, rstd, n, d); \
    break;
        CG_LN_CASE(1)
        CG_LN_CASE(2)
        CG_LN_CASE(3)
        CG_LN_CASE(4)
#undef CG_LN_CASE
      }
    } else {
      layernorm_fwd_kernel<<<blocks_of(n, 4), 256, 0, s>>>(x, w, b, eps, y, mean, rstd, n, d);
    }
    CG_LAUNCHED();
  });
}

size_t cg_norm_bwd_workspace_size(int32_t n, int32_t d) {
  return n > 0 && d > 0 ? size_t((int64_t(n) + NORM_ROWS - 1) / NORM_ROWS) * 2 * size_t(d) * 4 : 0;
}

int cg_norm_bwd(const float *x, const float *dy, const float *w, const float *mean, const float *rstd, float *dx,
                const float *residual, float *dw, float *db, int32_t n, int32_t d, void *workspace,
                size_t workspace_size, int32_t accumulate, void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(x && dy && w && rstd && dx && dw && d > 0, CG_ERR_INVALID, "norm backward operands are required");
    CG_REQUIRE(mean == nullptr || db != nullptr, CG_ERR_INVALID, "LayerNorm backward needs db");
    CG_REQUIRE(workspace && workspace_size >= cg_norm_bwd_workspace_size(n, d), CG_ERR_INVALID,
               "norm backward: workspace too small");
    hipStream_t s = as_stream(stream);
    float *part = static_cast<float *>(workspace);
    const bool vec = d % 4 == 0 && d <= 1024 && aligned16(x) && aligned16(dy) && aligned16(w) && aligned16(dx) &&
                     (residual == nullptr || aligned16(residual)) && aligned16(part);
    const int32_t parts = int32_t((int64_t(n) + NORM_ROWS - 1) / NORM_ROWS);
    if (vec) {
      switch ((d + 255) / 256) {
#define CG_NORM_CASE(NV)                                                                                        \
  case NV:                                                                                                      \
    norm_bwd_rows_kernel<NV><<<unsigned(parts), 256, 0, s>>>(x, dy, w, mean, rstd, residual, dx, part, n, d); \
    break;
        CG_NORM_CASE(1)
        CG_NORM_CASE(2)
        CG_NORM_CASE(3)
        CG_NORM_CASE(4)
#undef CG_NORM_CASE
      }
    } else {
      norm_bwd_kernel<<<unsigned(parts), 256, 2 * d * sizeof(float), s>>>(x, dy, w, mean, rstd, residual, dx, part, n,
                                                                         d, NORM_ROWS);
    }
    CG_LAUNCHED();
    norm_params_kernel<<<blocks_of(2 * int64_t(d), 64), 1024, 0, s>>>(part, parts, d, dw, db, accumulate);
    CG_LAUNCHED();
  });
}

size_t cg_column_sum_workspace_size(int32_t rows, int32_t cols) { return column_sum_ws(rows, cols); }

int cg_column_sum(const float *x, int32_t rows, int32_t cols, int64_t ld, float *out, int32_t accumulate,
                  void *workspace, size_t workspace_size, void *stream) {
  return guarded([&] { column_sum_launch(x, rows, cols, ld, out, accumulate, workspace, workspace_size, false, stream); });
}

int cg_gelu_fwd(const float *u, float *g, int64_t n, void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(u && g, CG_ERR_INVALID, "GELU operands are required");
    gelu_fwd_kernel<<<grid_1d(n), 256, 0, as_stream(stream)>>>(u, g, n);
    CG_LAUNCHED();
  });
}

int cg_gelu_bwd(const float *u, const float *dg, float *du, int64_t n, void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(u && dg && du, CG_ERR_INVALID, "GELU backward operands are required");
    gelu_bwd_kernel<<<grid_1d(n), 256, 0, as_stream(stream)>>>(u, dg, du, n);
    CG_LAUNCHED();
  });
}

int cg_add_strided(int32_t rows, int32_t cols, float alpha, const float *src, int64_t ld_src, float *dst,
                   int64_t ld_dst, void *stream) {
  return guarded([&] {
    if (int64_t(rows) * cols == 0) return;
    CG_REQUIRE(src && dst && rows > 0 && cols > 0, CG_ERR_INVALID, "add operands are required");
    add_strided_kernel<<<grid_1d(int64_t(rows) * cols), 256, 0, as_stream(stream)>>>(rows, cols, alpha, src, ld_src,
                                                                                     dst, ld_dst);
    CG_LAUNCHED();
  });
}

int cg_rmsnorm_fwd(const float *x, const float *w, float eps, float *y, float *rstd, int32_t n, int32_t d,
                   void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(x && w && y && rstd && d > 0, CG_ERR_INVALID, "RMSNorm operands are required");
    rmsnorm_fwd_kernel<<<blocks_of(n, 4), 256, 0, as_stream(stream)>>>(x, w, eps, y, rstd, n, d);
    CG_LAUNCHED();
  });
}

int cg_seq_of(const int64_t *seq_start, int32_t n_seqs, int32_t *seq_of, void *stream) {
  return guarded([&] {
    if (n_seqs == 0) return;
    CG_REQUIRE(seq_start && seq_of, CG_ERR_INVALID, "seq_start and seq_of are required");
    seq_of_kernel<<<unsigned(n_seqs), 256, 0, as_stream(stream)>>>(seq_start, n_seqs, seq_of);
    CG_LAUNCHED();
  });
}

int cg_attn_train_fwd(const cg_attn_train *p, void *stream) {
  return guarded([&] {
    check_attn_train(p);
    if (p->n == 0) return;
    AttnTrain a{p->n, p->H, p->KVH, p->scale, p->seq_start, p->seq_of, p->q, p->k, p->v, p->ldq, p->ldk, p->ldv,
                nullptr, nullptr, nullptr, p->o, p->lse, nullptr, nullptr, nullptr, nullptr, p->round_bf16};
    CG_REQUIRE(a.out && a.lse_out, CG_ERR_INVALID, "attention forward outputs are required");
    CG_REQUIRE(aligned16(a.out), CG_ERR_INVALID, "attention output: 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const dim3 grid = query_grid(*p);
    switch (p->head_dim) {
      case 8: attn_fwd_kernel<8><<<grid, 256, 0, s>>>(a); break;
      case 16: attn_fwd_kernel<16><<<grid, 256, 0, s>>>(a); break;
      case 24: attn_fwd_kernel<24><<<grid, 256, 0, s>>>(a); break;
      case 32: attn_fwd_kernel<32><<<grid, 256, 0, s>>>(a); break;
      case 64: attn_fwd_kernel<64><<<grid, 256, 0, s>>>(a); break;
      default: throw Error(CG_ERR_UNSUPPORTED, "training attention: head_dim 8, 16, 24, 32 or 64");
    }
    CG_LAUNCHED();
  });
}

int cg_attn_train_bwd(const cg_attn_train *p, const float *dout, float *dsum, float *dq, float *dk, float *dv,
                      void *stream) {
  return guarded([&] {
    check_attn_train(p);
    if (p->n == 0) return;
    AttnTrain a{p->n, p->H, p->KVH, p->scale, p->seq_start, p->seq_of, p->q, p->k, p->v, p->ldq, p->ldk, p->ldv,
                p->o, dout, p->lse, nullptr, nullptr, dsum, dq, dk, dv, p->round_bf16};
    CG_REQUIRE(a.o && a.dout && a.lse && dsum && dq && dk && dv, CG_ERR_INVALID,
               "attention backward operands are required");
    CG_REQUIRE(aligned16(dout), CG_ERR_INVALID, "attention dO: 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const dim3 grid = query_grid(*p), grid_kv(blocks_of(p->n, 64), unsigned(p->KVH));
    switch (p->head_dim) {
#define CG_BWD_CASE(DD)                                  \
  case DD:                                               \
    attn_bwd_dq_kernel<DD><<<grid, 256, 0, s>>>(a);      \
    CG_LAUNCHED();                                       \
    attn_bwd_dkv_kernel<DD><<<grid_kv, 256, 0, s>>>(a);  \
    break;
      CG_BWD_CASE(8)
      CG_BWD_CASE(16)
      CG_BWD_CASE(24)
      CG_BWD_CASE(32)
      CG_BWD_CASE(64)
#undef CG_BWD_CASE
      default: throw Error(CG_ERR_UNSUPPORTED, "training attention: head_dim 8, 16, 24, 32 or 64");
    }
    CG_LAUNCHED();
  });
}

}  // extern "C"

// ---- the whole trunk: forward keeping activations, and backward -------------------------------
namespace {

void ok(int status) {
  if (status == CG_OK) return;
  char buf[512];
  cg_last_error(buf, sizeof(buf));
  throw Error(status, "training step: " + std::string(buf));
}

struct TrainDims {
  int64_t n, d, F, H, KVH, D, Q, KVW, QKV, L, P, V, pd;
  bool bf;  // bf16 autocast precision
};

TrainDims dims_of(const cg_train_config &c, int32_t n) {
  TrainDims t{};
  t.n = n;
  t.bf = c.bf16 != 0;
  t.d = c.d_model;
  t.F = c.d_ff;
  t.H = c.n_heads;
  t.KVH = c.n_kv_heads;
  t.D = c.d_model / c.n_heads;
  t.Q = t.H * t.D;
  t.KVW = t.KVH * t.D;
  t.QKV = t.Q + 2 * t.KVW;
  t.L = c.n_layers;
  t.P = c.ple_width;
  t.V = c.value_width;
  t.pd = c.per_layer_dim;
  return t;
}

// Per layer, in floats of n rows: xl, h1 (d), m1, r1 (1), qkv (QKV), o (Q), lse (H), x1, h2 (d),
// m2, r2 (1), u, g (F: the MLP's pre-activation and its GELU); then x_last (d), mf, rf (1) and
// seq_of (n int32).  Every array starts on a
// 256-byte boundary (the attention kernels load rows of qkv as float4).
struct SavedLayer {
  float *xl, *h1, *m1, *r1, *qkv, *o, *lse, *x1, *h2, *m2, *r2, *u, *g;
};

int64_t span_of(const TrainDims &t, int64_t cols) { return (t.n * cols + 63) / 64 * 64; }

int64_t layer_floats(const TrainDims &t) {
  return 4 * span_of(t, t.d) + 4 * span_of(t, 1) + span_of(t, t.QKV) + span_of(t, t.Q) + span_of(t, t.H) +
         2 * span_of(t, t.F);
}

SavedLayer saved_layer(const TrainDims &t, void *saved, int64_t l) {
  float *p = static_cast<float *>(saved) + l * layer_floats(t);
  SavedLayer s{};
  auto take = [&](int64_t cols) {
    float *q = p;
    p += span_of(t, cols);
    return q;
  };
  s.xl = take(t.d);
  s.h1 = take(t.d);
  s.m1 = take(1);
  s.r1 = take(1);
  s.qkv = take(t.QKV);
  s.o = take(t.Q);
  s.lse = take(t.H);
  s.x1 = take(t.d);
  s.h2 = take(t.d);
  s.m2 = take(1);
  s.r2 = take(1);
  s.u = take(t.F);
  s.g = take(t.F);
  return s;
}

struct SavedTail {
  float *x_last, *mf, *rf;
  int32_t *seq_of;
};
SavedTail saved_tail(const TrainDims &t, void *saved) {
  float *p = static_cast<float *>(saved) + t.L * layer_floats(t);
  float *mf = p + span_of(t, t.d), *rf = mf + span_of(t, 1);
  return {p, mf, rf, reinterpret_cast<int32_t *>(rf + span_of(t, 1))};
}

size_t max_gemm_ws(const TrainDims &t) {
  size_t m = 0;
  const int64_t shapes[][3] = {{t.n, t.QKV, t.d}, {t.n, t.d, t.Q}, {t.n, t.F, t.d}, {t.n, t.d, t.F},
                               {t.QKV, t.d, t.n}, {t.d, t.Q, t.n}, {t.F, t.d, t.n}, {t.d, t.F, t.n},
                               {t.n, t.d, t.QKV}, {t.n, t.Q, t.d}, {t.n, t.d, t.F}};
  for (auto &sh : shapes) m = std::max(m, cg_gemm_workspace_size(int32_t(sh[0]), int32_t(sh[1]), int32_t(sh[2])));
  return m;
}

// Scratch of one call: GEMM split-K partials, then (backward) dx, dx1, dh (d each), du (F), do (Q),
// dqkv (QKV), dsum (H), norm / column-sum partials.
struct Scratch {
  float *gemm_ws;
  size_t gemm_bytes;
  float *dx, *dx1, *dh, *du, *dout, *dqkv, *dsum, *red;
  size_t red_bytes;
};

size_t red_bytes_of(const TrainDims &t) {
  const int64_t cols = std::max({t.d, t.F, t.QKV});
  return std::max(cg_norm_bwd_workspace_size(int32_t(t.n), int32_t(t.d)),
                  cg_column_sum_workspace_size(int32_t(t.n), int32_t(cols)));
}

Scratch scratch_of(const TrainDims &t, void *base) {
  Scratch s{};
  char *p = static_cast<char *>(base);
  s.gemm_bytes = (max_gemm_ws(t) + 255) / 256 * 256;
  s.gemm_ws = reinterpret_cast<float *>(p);
  p += s.gemm_bytes;
  float *f = reinterpret_cast<float *>(p);
  auto take = [&](int64_t cols) {
    float *q = f;
    f += (t.n * cols + 63) / 64 * 64;
    return q;
  };
  s.dx = take(t.d);
  s.dx1 = take(t.d);
  s.dh = take(t.d);
  s.du = take(t.F);
  s.dout = take(t.Q);
  s.dqkv = take(t.QKV);
  s.dsum = take(t.H);
  s.red = f;
  s.red_bytes = red_bytes_of(t);
  return s;
}

size_t scratch_bytes(const TrainDims &t) {
  const int64_t cols = 3 * t.d + t.F + t.Q + t.QKV + t.H;
  return (max_gemm_ws(t) + 255) / 256 * 256 + size_t(t.n * cols + 64 * 7) * 4 + red_bytes_of(t) + 256;
}

struct Gemm {
  const Scratch &s;
  hipStream_t st;
  bool bf;  // bf16 operands and outputs (autocast), else fp32
  Epi with(Epi e) const {
    e.round = bf ? 1 : 0;
    return e;
  }
  // out[M, N] = alpha x[M, K] W[N, K]^T (+ the epilogue's terms)
  void nt(int64_t M, int64_t N, int64_t K, const float *x, const float *w, float *out, float beta = 0.f,
          const Epi &e = Epi{}) const {
    gemm_launch(int32_t(M), int32_t(N), int32_t(K), 1.f, x, K, 1, w, 1, K, beta, out, N, s.gemm_ws, s.gemm_bytes,
                with(e), st);
  }
  // out[M, K] = dy[M, N] W[N, K]
  void nn(int64_t M, int64_t N, int64_t K, const float *dy, const float *w, float *out, const Epi &e = Epi{}) const {
    gemm_launch(int32_t(M), int32_t(K), int32_t(N), 1.f, dy, N, 1, w, K, 1, 0.f, out, K, s.gemm_ws, s.gemm_bytes,
                with(e), st);
  }
  // out[N, K] = dy[M, N]^T x[M, K]
  void tn(int64_t M, int64_t N, int64_t K, const float *dy, const float *x, float *out) const {
    gemm_launch(int32_t(N), int32_t(K), int32_t(M), 1.f, dy, 1, N, x, K, 1, 0.f, out, K, s.gemm_ws, s.gemm_bytes,
                with(Epi{}), st);
  }
};

// (column offset, width, scale) of each repeat of a per-layer embedding (trunk.py:318-333).
template <typename F>
void ple_slices(int64_t d, int64_t pd, F &&f) {
  if (pd == d) {
    f(int64_t(0), d, 1.0f);
    return;
  }
  const int64_t reps = d % pd == 0 ? d / pd : (d + pd - 1) / pd;
  const float scale = 1.0f / std::sqrt(float(reps));
  for (int64_t r = 0; r < reps; ++r) f(r * pd, std::min(pd, d - r * pd), scale);
}

cg_attn_train attn_args(const TrainDims &t, const int64_t *seq_start, const int32_t *seq_of, const float *qkv,
                        float *o, float *lse) {
  cg_attn_train a{};
  a.n = int32_t(t.n);
  a.H = int32_t(t.H);
  a.KVH = int32_t(t.KVH);
  a.head_dim = int32_t(t.D);
  a.scale = 1.0f / std::sqrt(float(t.D));
  a.seq_start = seq_start;
  a.seq_of = seq_of;
  a.q = qkv;
  a.k = qkv + t.Q;
  a.v = qkv + t.Q + t.KVW;
  a.ldq = a.ldk = a.ldv = t.QKV;
  a.o = o;
  a.lse = lse;
  a.round_bf16 = t.bf ? 1 : 0;
  return a;
}

}  // namespace

extern "C" {

size_t cg_train_saved_size(const cg_train_config *c, int32_t n) {
  if (!c || n <= 0) return 0;
  const TrainDims t = dims_of(*c, n);
  return size_t(t.L * layer_floats(t) + span_of(t, t.d) + 2 * span_of(t, 1)) * 4 + size_t(t.n) * 4 + 256;
}

size_t cg_train_scratch_size(const cg_train_config *c, int32_t n) {
  if (!c || n <= 0) return 0;
  return scratch_bytes(dims_of(*c, n));
}

int cg_trunk_train_forward(const cg_train_config *c, const cg_train_block *blocks, const float *final_w,
                           const float *final_b, const float *x, const float *ple, const float *values,
                           const int64_t *seq_start, int32_t n_seqs, int32_t n, float *hidden, void *saved,
                           size_t saved_size, void *scratch, size_t scratch_size, void *stream) {
  return guarded([&] {
    CG_REQUIRE(c && blocks && final_w && final_b && x && seq_start && hidden && saved && scratch, CG_ERR_INVALID,
               "training forward: missing operand");
    CG_REQUIRE(n > 0 && n_seqs > 0, CG_ERR_INVALID, "training forward: empty batch");
    CG_REQUIRE(saved_size >= cg_train_saved_size(c, n) && scratch_size >= cg_train_scratch_size(c, n),
               CG_ERR_INVALID, "training forward: buffers too small");
    CG_REQUIRE(aligned16(saved) && aligned16(scratch), CG_ERR_INVALID, "training forward: saved / scratch 16-byte aligned");
    CG_REQUIRE((c->ple_width == 0 || ple) && (c->value_width == 0 || values), CG_ERR_INVALID,
               "training forward: ple / values lookups are required");
    const TrainDims t = dims_of(*c, n);
    hipStream_t st = as_stream(stream);
    const Scratch s = scratch_of(t, scratch);
    const Gemm gm{s, st, t.bf};
    const SavedTail tail = saved_tail(t, saved);
    ok(cg_seq_of(seq_start, n_seqs, tail.seq_of, st));
    CG_HIP(hipMemcpyAsync(saved_layer(t, saved, 0).xl, x, size_t(t.n * t.d) * 4, hipMemcpyDeviceToDevice, st));
    for (int64_t l = 0; l < t.L; ++l) {
      const cg_train_block &w = blocks[l];
      const SavedLayer a = saved_layer(t, saved, l);
      float *x_next = l + 1 < t.L ? saved_layer(t, saved, l + 1).xl : tail.x_last;
      ok(cg_layernorm_fwd(a.xl, w.ln_attn_w, w.ln_attn_b, c->eps, a.h1, a.m1, a.r1, int32_t(t.n), int32_t(t.d), st));
      gm.nt(t.n, t.QKV, t.d, a.h1, w.qkv_w, a.qkv);
      const int32_t vi = c->value_index ? c->value_index[l] : -1;
      if (vi >= 0) {
        if (t.bf) {  // v = bf16(v + value embedding): the attention reads bf16 v
          add_round_kernel<<<grid_1d(t.n * t.KVW), 256, 0, st>>>(int32_t(t.n), int32_t(t.KVW), values + vi * t.KVW,
                                                                 t.V, a.qkv + t.Q + t.KVW, t.QKV);
          CG_LAUNCHED();
        } else {
          ok(cg_add_strided(int32_t(t.n), int32_t(t.KVW), 1.f, values + vi * t.KVW, t.V, a.qkv + t.Q + t.KVW, t.QKV,
                            st));
        }
      }
      const cg_attn_train at = attn_args(t, seq_start, tail.seq_of, a.qkv, a.o, a.lse);
      ok(cg_attn_train_fwd(&at, st));
      Epi res;  // x1 = xl + o W_out^T
      res.cin = a.xl;
      gm.nt(t.n, t.d, t.Q, a.o, w.out_w, a.x1, 1.f, res);
      ok(cg_layernorm_fwd(a.x1, w.ln_mlp_w, w.ln_mlp_b, c->eps, a.h2, a.m2, a.r2, int32_t(t.n), int32_t(t.d), st));
      Epi up;  // u = h2 W_up^T + b_up, g = gelu(u)
      up.bias = w.up_b;
      up.aux_out = a.g;
      up.mode = EPI_GELU;
      gm.nt(t.n, t.F, t.d, a.h2, w.up_w, a.u, 0.f, up);
      Epi down;  // x_next = x1 + g W_down^T + b_down
      down.cin = a.x1;
      down.bias = w.down_b;
      gm.nt(t.n, t.d, t.F, a.g, w.down_w, x_next, 1.f, down);
      if (ple)
        ple_slices(t.d, t.pd, [&](int64_t off, int64_t width, float scale) {
          ok(cg_add_strided(int32_t(t.n), int32_t(width), scale, ple + l * t.pd, t.P, x_next + off, t.d, st));
        });
    }
    ok(cg_layernorm_fwd(tail.x_last, final_w, final_b, c->eps, hidden, tail.mf, tail.rf, int32_t(t.n),
                        int32_t(t.d), st));
  });
}

int cg_trunk_train_backward(const cg_train_config *c, const cg_train_block *blocks, const float *final_w,
                            const int64_t *seq_start, int32_t n, const float *dhidden, void *saved,
                            size_t saved_size, void *scratch, size_t scratch_size, const cg_train_grads *grads,
                            float *dx, float *dple, float *dvalues, void *stream) {
  return guarded([&] {
    CG_REQUIRE(c && blocks && final_w && seq_start && dhidden && saved && scratch && grads && dx, CG_ERR_INVALID,
               "training backward: missing operand");
    CG_REQUIRE(n > 0, CG_ERR_INVALID, "training backward: empty batch");
    CG_REQUIRE(saved_size >= cg_train_saved_size(c, n) && scratch_size >= cg_train_scratch_size(c, n),
               CG_ERR_INVALID, "training backward: buffers too small");
    CG_REQUIRE(aligned16(saved) && aligned16(scratch), CG_ERR_INVALID, "training backward: saved / scratch 16-byte aligned");
    const TrainDims t = dims_of(*c, n);
    hipStream_t st = as_stream(stream);
    const Scratch s = scratch_of(t, scratch);
    const Gemm gm{s, st, t.bf};
    const SavedTail tail = saved_tail(t, saved);
    const int32_t N = int32_t(t.n);
    ok(cg_norm_bwd(tail.x_last, dhidden, final_w, tail.mf, tail.rf, s.dx, nullptr, grads->final_dw,
                   grads->final_db, N, int32_t(t.d), s.red, s.red_bytes, 0, st));
    if (dple) {
      zero_fill_kernel<<<grid_1d(t.n * t.P), 256, 0, st>>>(dple, t.n * t.P);
      CG_LAUNCHED();
    }
    if (dvalues) {
      zero_fill_kernel<<<grid_1d(t.n * t.V), 256, 0, st>>>(dvalues, t.n * t.V);
      CG_LAUNCHED();
    }
    for (int64_t l = t.L - 1; l >= 0; --l) {
      const cg_train_block &w = blocks[l];
      const cg_train_block_grads &gw = grads->blocks[l];
      const SavedLayer a = saved_layer(t, saved, l);
      if (dple)
        ple_slices(t.d, t.pd, [&](int64_t off, int64_t width, float scale) {
          ok(cg_add_strided(N, int32_t(width), scale, s.dx + off, t.d, dple + l * t.pd, t.P, st));
        });
      gm.tn(t.n, t.d, t.F, s.dx, a.g, gw.down_w);
      column_sum_launch(s.dx, N, int32_t(t.d), t.d, gw.down_b, 0, s.red, s.red_bytes, t.bf, st);
      Epi dgelu;  // du = (dx W_down) gelu'(u)
      dgelu.aux_in = a.u;
      dgelu.mode = EPI_GELU_GRAD;
      gm.nn(t.n, t.d, t.F, s.dx, w.down_w, s.du, dgelu);
      gm.tn(t.n, t.F, t.d, s.du, a.h2, gw.up_w);
      column_sum_launch(s.du, N, int32_t(t.F), t.F, gw.up_b, 0, s.red, s.red_bytes, t.bf, st);
      gm.nn(t.n, t.F, t.d, s.du, w.up_w, s.dh);
      ok(cg_norm_bwd(a.x1, s.dh, w.ln_mlp_w, a.m2, a.r2, s.dx1, s.dx, gw.ln_mlp_w, gw.ln_mlp_b, N, int32_t(t.d),
                     s.red, s.red_bytes, 0, st));
      gm.tn(t.n, t.d, t.Q, s.dx1, a.o, gw.out_w);
      gm.nn(t.n, t.d, t.Q, s.dx1, w.out_w, s.dout);
      const cg_attn_train at = attn_args(t, seq_start, tail.seq_of, a.qkv, a.o, a.lse);
      ok(cg_attn_train_bwd(&at, s.dout, s.dsum, s.dqkv, s.dqkv + t.Q, s.dqkv + t.Q + t.KVW, st));
      const int32_t vi = c->value_index ? c->value_index[l] : -1;
      if (vi >= 0 && dvalues)
        ok(cg_add_strided(N, int32_t(t.KVW), 1.f, s.dqkv + t.Q + t.KVW, t.QKV, dvalues + vi * t.KVW, t.V, st));
      gm.tn(t.n, t.QKV, t.d, s.dqkv, a.h1, gw.qkv_w);
      gm.nn(t.n, t.QKV, t.d, s.dqkv, w.qkv_w, s.dh);
      ok(cg_norm_bwd(a.xl, s.dh, w.ln_attn_w, a.m1, a.r1, s.dx, s.dx1, gw.ln_attn_w, gw.ln_attn_b, N, int32_t(t.d),
                     s.red, s.red_bytes, 0, st));
    }
    CG_HIP(hipMemcpyAsync(dx, s.dx, size_t(t.n * t.d) * 4, hipMemcpyDeviceToDevice, st));
  });
}

}  // extern "C"
