// MFMA projections of the trunk with fused prologues and epilogues (gfx950).
//
// C[M, N] = A[M, K] . W[N, K]^T with fp32 accumulation, where
//   * A is the LayerNorm of fp32 rows computed on the fly (ln_attn / ln_mlp feeding
//     qkv_proj / mlp[0], cardgym/nn/trunk.py:143, 157), or a stored fp32 / bf16 matrix
//     (attention output into out_proj, GELU output into mlp[2]);
//   * the epilogue is one of: plain store (+bias), GELU(+bias) store, residual add into
//     the fp32 stream (+bias, + the per-layer embedding of Trunk._add_ple, trunk.py:318-333),
//     or the QKV split that writes q and appends k / v (+ value embedding) straight into
//     the KV pool at each token's slot (trunk.py:141-152 followed by
//     KVCache.write_step, kv_cache.py:84-105).
//
// Operands: CG_BF16 compute uses v_mfma_f32_16x16x32_bf16 (8 bf16 per lane per operand);
// CG_F32 uses v_mfma_f32_16x16x4_f32 eight times per 32-wide k chunk.  Lane l of a wave
// supplies row (l % 16) of its 16-row A tile and column (l % 16) of its 16-column W tile,
// eight consecutive k values starting at k0 + 8 (l / 16); A and W use the same lane -> k
// assignment, so the product sums every k exactly once.  The 16x16 fp32 result sits in
// lane l as rows 4 (l / 16) + r, r < 4, column l % 16.
//
// Workgroup: 4 waves in a 2 x 2 arrangement, each wave a 32 x 32 tile (2 x 2 MFMA tiles),
// so a workgroup covers 64 x 64 of C.  K must be a multiple of 8 (a partial last chunk is
// zero-filled).
#include "common.h"
#include "gemm.h"

namespace cg {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) unsigned short u16x8;

constexpr int WM = 2, WN = 2, FM = 2, FN = 2;
constexpr int BM = WM * FM * 16, BN = WN * FN * 16;
constexpr int THREADS = 64 * WM * WN;
constexpr int KC = 32;

struct Frag {
  float f[8];
};

__device__ __forceinline__ void load8_f32(const float *p, float (&o)[8]) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0];
  const float4 b = reinterpret_cast<const float4 *>(p)[1];
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

__device__ __forceinline__ void load8_bf16(const bf16 *p, float (&o)[8]) {
  const uint4 r = reinterpret_cast<const uint4 *>(p)[0];
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ bf16x8 to_bf16x8(const float (&f)[8]) {
  u16x8 u;
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = from_f32<bf16>(f[i]).bits;
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ float4 f4(const float *p) { return reinterpret_cast<const float4 *>(p)[0]; }

template <int AM, typename TW, typename TC, int EPI>
__global__ __launch_bounds__(THREADS) void gemm_kernel(GemmArgs g) {
  __shared__ float row_mean[BM], row_rstd[BM];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int li = lane & 15, lg = lane >> 4;

  if constexpr (AM == A_LN) {
    // Row statistics for the workgroup's BM rows: one wave per row, two passes in fp32.
    const float *A = static_cast<const float *>(g.A);
    for (int r = wave; r < BM; r += WM * WN) {
      const int m = m0 + r;
      float mean = 0.f, rstd = 0.f;
      if (m < g.M) {
        const float *x = A + int64_t(m) * g.lda;
        float s = 0.f;
        for (int k = lane; k < g.K; k += 64) s += x[k];
        mean = wave_sum(s) / float(g.K);
        float v = 0.f;
        for (int k = lane; k < g.K; k += 64) {
          const float d = x[k] - mean;
          v = fmaf(d, d, v);
        }
        rstd = rsqrtf(wave_sum(v) / float(g.K) + g.eps);
      }
      if (lane == 0) {
        row_mean[r] = mean;
        row_rstd[r] = rstd;
      }
    }
    __syncthreads();
  }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  int a_row[FM];
  bool a_ok[FM];
  float a_mean[FM], a_rstd[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int r = wm * FM * 16 + i * 16 + li;
    a_row[i] = m0 + r;
    a_ok[i] = a_row[i] < g.M;
    if constexpr (AM == A_LN) {
      a_mean[i] = row_mean[r];
      a_rstd[i] = row_rstd[r];
    }
  }
  int w_col[FN];
  bool w_ok[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    w_col[j] = n0 + wn * FN * 16 + j * 16 + li;
    w_ok[j] = w_col[j] < g.N;
  }

  for (int k0 = 0; k0 < g.K; k0 += KC) {
    const int k = k0 + 8 * lg;
    const bool k_ok = k < g.K;
    float af[FM][8], wf[FN][8];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (a_ok[i] && k_ok) {
        if constexpr (AM == A_BF16) {
          load8_bf16(static_cast<const bf16 *>(g.A) + int64_t(a_row[i]) * g.lda + k, af[i]);
        } else {
          load8_f32(static_cast<const float *>(g.A) + int64_t(a_row[i]) * g.lda + k, af[i]);
        }
        if constexpr (AM == A_LN) {
          float w[8], b[8];
          load8_f32(g.ln_w + k, w);
          load8_f32(g.ln_b + k, b);
#pragma unroll
          for (int e = 0; e < 8; ++e) af[i][e] = fmaf((af[i][e] - a_mean[i]) * a_rstd[i], w[e], b[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) af[i][e] = 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if (w_ok[j] && k_ok) {
        if constexpr (sizeof(TW) == 2) {
          load8_bf16(static_cast<const bf16 *>(g.W) + int64_t(w_col[j]) * g.K + k, wf[j]);
        } else {
          load8_f32(static_cast<const float *>(g.W) + int64_t(w_col[j]) * g.K + k, wf[j]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) wf[j][e] = 0.f;
      }
    }
    if constexpr (sizeof(TC) == 2) {
      bf16x8 av[FM], wv[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) av[i] = to_bf16x8(af[i]);
#pragma unroll
      for (int j = 0; j < FN; ++j) wv[j] = to_bf16x8(wf[j]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], wv[j], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], wf[j][e], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue: lane holds C[m][n] for m = tile row 4 lg + r, n = tile column li.
  const int kvw = g.kv_heads * g.head_dim;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = w_col[j];
    if (!w_ok[j]) continue;
    const float bias = g.bias ? g.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * FM * 16 + i * 16 + 4 * lg + r;
        if (m >= g.M) continue;
        const float c = acc[i][j][r] + bias;
        if constexpr (EPI == EPI_STORE || EPI == EPI_GELU || EPI == EPI_SCALE_ADD) {
          float v = c;
          if constexpr (EPI == EPI_GELU) v = gelu_erf(c);
          if constexpr (EPI == EPI_SCALE_ADD) v = (c + g.addend[int64_t(m) * g.ld_add + n]) * g.scale;
          const int64_t o = int64_t(m) * g.ldo + n;
          if (g.out_dtype == CG_BF16) static_cast<bf16 *>(g.out)[o] = from_f32<bf16>(v);
          else static_cast<float *>(g.out)[o] = v;
        } else if constexpr (EPI == EPI_RESID) {
          float v = c;
          if (g.ple) v = fmaf(g.ple[int64_t(m) * g.ld_ple + g.ple_off + n % g.ple_dim], g.ple_scale, v);
          g.resid[int64_t(m) * g.ldr + n] += v;
        } else {  // EPI_QKV
          if (n < g.q_cols) {
            static_cast<float *>(g.out)[int64_t(m) * g.ldo + n] = c;
          } else {
            const int row = g.tok_row[m];
            if (row < 0) continue;
            const bool is_v = n >= g.q_cols + kvw;
            const int kv = n - g.q_cols - (is_v ? kvw : 0);
            const int h = kv / g.head_dim, d = kv % g.head_dim;
            float v = c;
            if (is_v && g.vemb_off >= 0) v += g.vemb[int64_t(m) * g.ld_vemb + g.vemb_off + kv];
            const int64_t dst =
                ((int64_t(row) * g.kv_heads + h) * g.max_len + g.tok_pos[m]) * g.head_dim + d;
            void *base = is_v ? g.vc : g.kc;
            if (g.kv_dtype == CG_BF16) static_cast<bf16 *>(base)[dst] = from_f32<bf16>(v);
            else if (g.kv_dtype == CG_F16) static_cast<f16 *>(base)[dst] = from_f32<f16>(v);
            else static_cast<float *>(base)[dst] = v;
          }
        }
      }
    }
  }
}

template <int AM, typename TW, typename TC>
void launch_epi(const GemmArgs &g, dim3 grid, hipStream_t s) {
  switch (g.epi) {
    case EPI_STORE:
      gemm_kernel<AM, TW, TC, EPI_STORE><<<grid, THREADS, 0, s>>>(g);
      break;
    case EPI_GELU:
      gemm_kernel<AM, TW, TC, EPI_GELU><<<grid, THREADS, 0, s>>>(g);
      break;
    case EPI_RESID:
      gemm_kernel<AM, TW, TC, EPI_RESID><<<grid, THREADS, 0, s>>>(g);
      break;
    case EPI_QKV:
      gemm_kernel<AM, TW, TC, EPI_QKV><<<grid, THREADS, 0, s>>>(g);
      break;
    case EPI_SCALE_ADD:
      gemm_kernel<AM, TW, TC, EPI_SCALE_ADD><<<grid, THREADS, 0, s>>>(g);
      break;
    default:
      throw Error(CG_ERR_INVALID, "unknown epilogue");
  }
  CG_LAUNCHED();
}

template <typename TW, typename TC>
void launch_a(const GemmArgs &g, dim3 grid, hipStream_t s) {
  switch (g.a_mode) {
    case A_LN:
      return launch_epi<A_LN, TW, TC>(g, grid, s);
    case A_F32:
      return launch_epi<A_F32, TW, TC>(g, grid, s);
    case A_BF16:
      return launch_epi<A_BF16, TW, TC>(g, grid, s);
  }
  throw Error(CG_ERR_INVALID, "unknown A operand mode");
}

}  // namespace

void launch_gemm(const GemmArgs &g, hipStream_t s) {
  CG_REQUIRE(g.M >= 0 && g.N > 0 && g.K > 0, CG_ERR_INVALID, "GEMM sizes must be positive");
  CG_REQUIRE(g.K % 8 == 0, CG_ERR_UNSUPPORTED, "GEMM inner size must be a multiple of 8");
  CG_REQUIRE(g.a_mode != A_LN || g.K <= 4096, CG_ERR_UNSUPPORTED, "LayerNorm width above 4096");
  if (g.M == 0) return;
  dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM);
  CG_REQUIRE(grid.y <= 65535u, CG_ERR_UNSUPPORTED, "too many rows for one launch");
  const bool w_bf16 = g.w_dtype == CG_BF16;
  if (g.compute == CG_BF16) {
    if (w_bf16) return launch_a<bf16, bf16>(g, grid, s);
    return launch_a<float, bf16>(g, grid, s);
  }
  CG_REQUIRE(g.compute == CG_F32, CG_ERR_INVALID, "compute dtype must be CG_F32 or CG_BF16");
  CG_REQUIRE(!w_bf16, CG_ERR_INVALID, "fp32 compute needs fp32 weights");
  return launch_a<float, float>(g, grid, s);
}

}  // namespace cg

using namespace cg;

extern "C" int cg_linear(const float *x, const float *w, const float *bias, float *y, int32_t m,
                         int32_t n, int32_t k, int32_t act, int32_t compute_dtype, void *stream) {
  return guarded([&] {
    CG_REQUIRE(x && w && y, CG_ERR_INVALID, "x, w and y are required");
    CG_REQUIRE(act == CG_ACT_NONE || act == CG_ACT_GELU, CG_ERR_INVALID, "unknown activation");
    GemmArgs g{};
    g.M = m;
    g.N = n;
    g.K = k;
    g.compute = compute_dtype;
    g.a_mode = A_F32;
    g.A = x;
    g.lda = k;
    g.W = w;
    g.w_dtype = CG_F32;
    g.bias = bias;
    g.epi = act == CG_ACT_GELU ? EPI_GELU : EPI_STORE;
    g.out = y;
    g.out_dtype = CG_F32;
    g.ldo = n;
    launch_gemm(g, as_stream(stream));
  });
}

extern "C" int cg_linear_add_scale(const float *x, const float *w, const float *addend, float *y,
                                   int32_t m, int32_t n, int32_t k, float scale,
                                   int32_t compute_dtype, void *stream) {
  return guarded([&] {
    CG_REQUIRE(x && w && addend && y, CG_ERR_INVALID, "x, w, addend and y are required");
    GemmArgs g{};
    g.M = m;
    g.N = n;
    g.K = k;
    g.compute = compute_dtype;
    g.a_mode = A_F32;
    g.A = x;
    g.lda = k;
    g.W = w;
    g.w_dtype = CG_F32;
    g.epi = EPI_SCALE_ADD;
    g.addend = addend;
    g.ld_add = n;
    g.scale = scale;
    g.out = y;
    g.out_dtype = CG_F32;
    g.ldo = n;
    launch_gemm(g, as_stream(stream));
  });
}
