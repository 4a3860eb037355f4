// MFMA projections of the trunk with fused epilogues (gfx950).
//
// C[M, N] = A[M, K] . W[N, K]^T with fp32 accumulation; A and W are stored in the compute
// type (bf16 for the autocast path, fp32 otherwise).  The epilogue is one of:
//   * plain store (+bias) or GELU(+bias) store (mlp[0] + nn.GELU, trunk.py:139);
//   * the QKV split that writes q and appends k / v (+ value embedding) straight into the
//     KV pool at each token's slot (trunk.py:141-152 followed by KVCache.write_step,
//     kv_cache.py:84-105) -- the append costs no separate pass over K/V;
//   * residual add into the fp32 stream (+bias, + the per-layer embedding of
//     Trunk._add_ple, trunk.py:318-333), optionally followed by the LayerNorm of the
//     updated row (the next ln_mlp / ln_attn, trunk.py:154-160): with full-row tiles the
//     epilogue owns whole rows, so the norm costs no extra launch or re-read.
//
// Main loop: the workgroup stages 128-byte-wide K chunks of its A rows and W rows in LDS
// (16-byte coalesced global loads, double-buffered: chunk k+1 is in flight while chunk k
// feeds the MFMAs).  Fragments: lane l supplies row (l % 16) of a 16-row A tile and column
// (l % 16) of a 16-column W tile, eight consecutive k values from 8 (l / 16); A and W use
// the same lane -> k assignment, so every k is summed once.  bf16 uses
// v_mfma_f32_16x16x32_bf16 (one per 32 k), fp32 uses v_mfma_f32_16x16x4_f32 eight times.
// The 16x16 fp32 result sits in lane l as rows 4 (l / 16) + r, r < 4, column l % 16.
#include "common.h"
#include "gemm.h"

namespace cg {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;

constexpr int CHUNK_BYTES = 128;                // K bytes per row per staged chunk
constexpr int LDS_ROW = CHUNK_BYTES + 16;        // padded LDS row (bytes)
constexpr int VPR = CHUNK_BYTES / 16;            // 16-byte vectors per row chunk

template <typename TC, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmArgs g) {
  constexpr int THREADS = 64 * WM * WN;
  constexpr int ES = int(sizeof(TC));
  constexpr int KC = CHUNK_BYTES / ES;  // elements per chunk
  constexpr int VA = (BM * VPR + THREADS - 1) / THREADS;
  constexpr int VW = (BN * VPR + THREADS - 1) / THREADS;
  constexpr int FM = BM / WM / 16, FN = BN / WN / 16;
  static_assert(FM >= 1 && FN >= 1, "tile too small for the wave layout");
  __shared__ __align__(16) unsigned char smem[2 * (BM + BN) * LDS_ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int li = lane & 15, lg = lane >> 4;
  const char *A = static_cast<const char *>(g.A);
  const char *W = static_cast<const char *>(g.W);
  const int64_t lda_b = g.lda * ES, ldw_b = int64_t(g.K) * ES;
  const int k_bytes = g.K * ES;
  const int nchunks = (g.K + KC - 1) / KC;

  uint4 ra[VA], rw[VW];
  auto gload = [&](int kc) {
    const int kb0 = kc * CHUNK_BYTES;
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      const int v = tid + i * THREADS;
      uint4 val = {0u, 0u, 0u, 0u};
      const int r = v / VPR, kb = kb0 + (v % VPR) * 16;
      if (v < BM * VPR && m0 + r < g.M && kb < k_bytes)
        val = *reinterpret_cast<const uint4 *>(A + int64_t(m0 + r) * lda_b + kb);
      ra[i] = val;
    }
#pragma unroll
    for (int i = 0; i < VW; ++i) {
      const int v = tid + i * THREADS;
      uint4 val = {0u, 0u, 0u, 0u};
      const int r = v / VPR, kb = kb0 + (v % VPR) * 16;
      if (v < BN * VPR && n0 + r < g.N && kb < k_bytes)
        val = *reinterpret_cast<const uint4 *>(W + int64_t(n0 + r) * ldw_b + kb);
      rw[i] = val;
    }
  };
  auto sstore = [&](int buf) {
    unsigned char *base = smem + buf * (BM + BN) * LDS_ROW;
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      const int v = tid + i * THREADS;
      if (v < BM * VPR) *reinterpret_cast<uint4 *>(base + (v / VPR) * LDS_ROW + (v % VPR) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < VW; ++i) {
      const int v = tid + i * THREADS;
      if (v < BN * VPR)
        *reinterpret_cast<uint4 *>(base + (BM + v / VPR) * LDS_ROW + (v % VPR) * 16) = rw[i];
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf) {
    const unsigned char *base = smem + buf * (BM + BN) * LDS_ROW;
#pragma unroll
    for (int ks = 0; ks < KC / 32; ++ks) {
      const int kb = (ks * 32 + 8 * lg) * ES;
      if constexpr (ES == 2) {
        bf16x8 af[FM], wf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const bf16x8 *>(base + (wm * FM * 16 + i * 16 + li) * LDS_ROW + kb);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          wf[j] = *reinterpret_cast<const bf16x8 *>(base + (BM + wn * FN * 16 + j * 16 + li) * LDS_ROW + kb);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], wf[j], acc[i][j], 0, 0, 0);
      } else {
        float af[FM][8], wf[FN][8];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const float4 *p = reinterpret_cast<const float4 *>(base + (wm * FM * 16 + i * 16 + li) * LDS_ROW + kb);
          const float4 x = p[0], y = p[1];
          af[i][0] = x.x; af[i][1] = x.y; af[i][2] = x.z; af[i][3] = x.w;
          af[i][4] = y.x; af[i][5] = y.y; af[i][6] = y.z; af[i][7] = y.w;
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const float4 *p = reinterpret_cast<const float4 *>(base + (BM + wn * FN * 16 + j * 16 + li) * LDS_ROW + kb);
          const float4 x = p[0], y = p[1];
          wf[j][0] = x.x; wf[j][1] = x.y; wf[j][2] = x.z; wf[j][3] = x.w;
          wf[j][4] = y.x; wf[j][5] = y.y; wf[j][6] = y.z; wf[j][7] = y.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], wf[j][e], acc[i][j], 0, 0, 0);
      }
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kc = 0; kc < nchunks; ++kc) {
    const bool more = kc + 1 < nchunks;
    if (more) gload(kc + 1);
    compute(kc & 1);
    if (more) sstore((kc + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue ------------------------------------------------------------------------
  if constexpr (EPI == EPI_RESID || EPI == EPI_RESID_LN) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * FN * 16 + j * 16 + li;
      const bool n_ok = n < g.N;
      const float bias = (n_ok && g.bias) ? g.bias[n] : 0.f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * FM * 16 + i * 16 + 4 * lg + r;
          float x = 0.f;
          if (n_ok && m < g.M) {
            x = acc[i][j][r] + bias;
            if (g.ple) x = fmaf(g.ple[int64_t(m) * g.ld_ple + g.ple_off + n % g.ple_dim], g.ple_scale, x);
            float *dst = g.resid + int64_t(m) * g.ldr + n;
            x += *dst;
            *dst = x;
          }
          acc[i][j][r] = x;
        }
    }
    if constexpr (EPI == EPI_RESID_LN) {
      // Row statistics: lanes with the same (l / 16) hold the same 4 rows of a tile; their
      // 16 columns reduce by shuffles, then the WN column slices meet in LDS.
      float *red = reinterpret_cast<float *>(smem);  // [2][WN][BM]
      float mean[FM][4], rstd[FM][4];
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
              const int n = n0 + wn * FN * 16 + j * 16 + li;
              const float v = acc[i][j][r];
              const float d = pass == 0 ? v : v - mean[i][r];
              s += n < g.N ? (pass == 0 ? d : d * d) : 0.f;
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o, 64);
            if (li == 0) red[(pass * WN + wn) * BM + wm * FM * 16 + i * 16 + 4 * lg + r] = s;
          }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = wm * FM * 16 + i * 16 + 4 * lg + r;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < WN; ++w) s += red[(pass * WN + w) * BM + row];
            if (pass == 0) mean[i][r] = s / float(g.N);
            else rstd[i][r] = rsqrtf(s / float(g.N) + g.eps);
          }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * FN * 16 + j * 16 + li;
        if (n >= g.N) continue;
        const float w = g.ln_w[n], b = g.ln_b[n];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * FM * 16 + i * 16 + 4 * lg + r;
            if (m >= g.M) continue;
            const float y = fmaf((acc[i][j][r] - mean[i][r]) * rstd[i][r], w, b);
            const int64_t o = int64_t(m) * g.ldo + n;
            if (g.out_dtype == CG_BF16) static_cast<bf16 *>(g.out)[o] = from_f32<bf16>(y);
            else static_cast<float *>(g.out)[o] = y;
          }
      }
    }
    return;
  }

  const int kvw = g.kv_heads * g.head_dim;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * FN * 16 + j * 16 + li;
    if (n >= g.N) continue;
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
          if constexpr (EPI == EPI_SCALE_ADD) {
            const float cc = g.round_c ? to_f32(from_f32<bf16>(c)) : c;
            const int64_t ai = int64_t(m) * g.ld_add + n;
            if (g.add_dtype == CG_BF16) {
              const float sum = to_f32(from_f32<bf16>(cc + to_f32(static_cast<const bf16 *>(g.addend)[ai])));
              v = to_f32(from_f32<bf16>(sum * g.scale));
            } else {
              v = (cc + static_cast<const float *>(g.addend)[ai]) * g.scale;
            }
          }
          const int64_t o = int64_t(m) * g.ldo + n;
          if (g.out_dtype == CG_BF16) static_cast<bf16 *>(g.out)[o] = from_f32<bf16>(v);
          else static_cast<float *>(g.out)[o] = v;
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

// Tile shapes: 64x64 (2x2 waves of 32x32) for the wide projections, 16 rows x 256
// columns (4 waves side by side) when the epilogue needs whole rows.
template <typename TC, int EPI>
void launch_tile(const GemmArgs &g, hipStream_t s) {
  dim3 grid((g.N + 63) / 64, (g.M + 63) / 64);
  CG_REQUIRE(grid.y <= 65535u, CG_ERR_UNSUPPORTED, "too many rows for one launch");
  gemm_kernel<TC, 64, 64, 2, 2, EPI><<<grid, 256, 0, s>>>(g);
  CG_LAUNCHED();
}

template <typename TC, int EPI>
void launch_rows(const GemmArgs &g, hipStream_t s) {
  dim3 grid(1, (g.M + 15) / 16);
  CG_REQUIRE(grid.y <= 65535u, CG_ERR_UNSUPPORTED, "too many rows for one launch");
  gemm_kernel<TC, 16, 256, 1, 4, EPI><<<grid, 256, 0, s>>>(g);
  CG_LAUNCHED();
}

template <typename TC>
void launch_typed(const GemmArgs &g, hipStream_t s) {
  switch (g.epi) {
    case EPI_STORE:
      return launch_tile<TC, EPI_STORE>(g, s);
    case EPI_GELU:
      return launch_tile<TC, EPI_GELU>(g, s);
    case EPI_RESID:
      if (g.N <= 256) return launch_rows<TC, EPI_RESID>(g, s);
      return launch_tile<TC, EPI_RESID>(g, s);
    case EPI_QKV:
      return launch_tile<TC, EPI_QKV>(g, s);
    case EPI_SCALE_ADD:
      return launch_tile<TC, EPI_SCALE_ADD>(g, s);
    case EPI_RESID_LN:
      CG_REQUIRE(g.N <= 256, CG_ERR_UNSUPPORTED, "fused residual LayerNorm needs d_model <= 256");
      return launch_rows<TC, EPI_RESID_LN>(g, s);
  }
  throw Error(CG_ERR_INVALID, "unknown epilogue");
}

// One wave per row; every lane's loads are issued before the reductions.
template <int PER_LANE>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const float *__restrict__ x,
                                                             const int32_t *__restrict__ index,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ b, float eps,
                                                             void *__restrict__ y, int32_t y_dtype,
                                                             int32_t n, int32_t d) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const int src = index ? index[row] : row;
  float v[PER_LANE];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int k = lane + 64 * i;
    v[i] = (src >= 0 && k < d) ? x[int64_t(src) * d + k] : 0.f;
    s += v[i];
  }
  const float mean = wave_sum(s) / float(d);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int k = lane + 64 * i;
    const float t = k < d ? v[i] - mean : 0.f;
    q = fmaf(t, t, q);
  }
  const float rstd = rsqrtf(wave_sum(q) / float(d) + eps);
#pragma unroll
  for (int i = 0; i < PER_LANE; ++i) {
    const int k = lane + 64 * i;
    if (k >= d) continue;
    const float out = src >= 0 ? fmaf((v[i] - mean) * rstd, w[k], b[k]) : 0.f;
    const int64_t o = int64_t(row) * d + k;
    if (y_dtype == CG_BF16) static_cast<bf16 *>(y)[o] = from_f32<bf16>(out);
    else static_cast<float *>(y)[o] = out;
  }
}

__global__ void convert_kernel(const float *__restrict__ x, void *__restrict__ y, int32_t dtype, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    if (dtype == CG_BF16) static_cast<bf16 *>(y)[i] = from_f32<bf16>(x[i]);
    else static_cast<float *>(y)[i] = x[i];
  }
}

}  // namespace

void launch_gemm(const GemmArgs &g, hipStream_t s) {
  CG_REQUIRE(g.M >= 0 && g.N > 0 && g.K > 0, CG_ERR_INVALID, "GEMM sizes must be positive");
  CG_REQUIRE(g.K % 8 == 0, CG_ERR_UNSUPPORTED, "GEMM inner size must be a multiple of 8");
  CG_REQUIRE(g.lda % 8 == 0, CG_ERR_UNSUPPORTED, "GEMM row stride must be a multiple of 8");
  CG_REQUIRE((reinterpret_cast<uintptr_t>(g.A) | reinterpret_cast<uintptr_t>(g.W)) % 16 == 0,
             CG_ERR_INVALID, "GEMM operands must be 16-byte aligned");
  if (g.M == 0) return;
  if (g.compute == CG_BF16) return launch_typed<bf16>(g, s);
  CG_REQUIRE(g.compute == CG_F32, CG_ERR_INVALID, "compute dtype must be CG_F32 or CG_BF16");
  return launch_typed<float>(g, s);
}

void launch_layernorm_rows(const float *x, const int32_t *index, const float *w, const float *b,
                           float eps, void *y, int32_t y_dtype, int32_t n, int32_t d,
                           hipStream_t s) {
  if (n <= 0) return;
  const unsigned grid = unsigned((n + 3) / 4);
  if (d <= 256) layernorm_rows_kernel<4><<<grid, 256, 0, s>>>(x, index, w, b, eps, y, y_dtype, n, d);
  else if (d <= 512) layernorm_rows_kernel<8><<<grid, 256, 0, s>>>(x, index, w, b, eps, y, y_dtype, n, d);
  else if (d <= 1024) layernorm_rows_kernel<16><<<grid, 256, 0, s>>>(x, index, w, b, eps, y, y_dtype, n, d);
  else throw Error(CG_ERR_UNSUPPORTED, "LayerNorm width above 1024");
  CG_LAUNCHED();
}

void launch_convert(const float *x, void *y, int32_t dtype, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  convert_kernel<<<unsigned(blocks), 256, 0, s>>>(x, y, dtype, n);
  CG_LAUNCHED();
}

}  // namespace cg

using namespace cg;

extern "C" int cg_linear(const float *x, const float *w, const float *bias, float *y, int32_t m,
                         int32_t n, int32_t k, int32_t act, int32_t compute_dtype, void *stream) {
  return guarded([&] {
    CG_REQUIRE(act == CG_ACT_NONE || act == CG_ACT_GELU, CG_ERR_INVALID, "unknown activation");
    if (m == 0) return;
    CG_REQUIRE(x && w && y, CG_ERR_INVALID, "x, w and y are required");
    CG_REQUIRE(compute_dtype == CG_F32 || compute_dtype == CG_BF16, CG_ERR_INVALID,
               "compute dtype must be CG_F32 or CG_BF16");
    GemmArgs g{};
    g.M = m;
    g.N = n;
    g.K = k;
    g.compute = CG_F32;  // fp32 operands: the product is exact fp32 whatever compute_dtype asks
    g.A = x;
    g.lda = k;
    g.W = w;
    g.bias = bias;
    g.epi = act == CG_ACT_GELU ? EPI_GELU : EPI_STORE;
    g.out = y;
    g.out_dtype = CG_F32;
    g.ldo = n;
    launch_gemm(g, as_stream(stream));
  });
}

extern "C" int cg_linear_add_scale(const float *x, const float *w, const void *addend, int32_t addend_dtype,
                                   float *y, int32_t m, int32_t n, int32_t k, float scale,
                                   int32_t compute_dtype, void *stream) {
  return guarded([&] {
    if (m == 0) return;
    CG_REQUIRE(x && w && addend && y, CG_ERR_INVALID, "x, w, addend and y are required");
    CG_REQUIRE(compute_dtype == CG_F32 || compute_dtype == CG_BF16, CG_ERR_INVALID,
               "compute dtype must be CG_F32 or CG_BF16");
    CG_REQUIRE(addend_dtype == CG_F32 || addend_dtype == CG_BF16, CG_ERR_INVALID,
               "addend dtype must be CG_F32 or CG_BF16");
    GemmArgs g{};
    g.M = m;
    g.N = n;
    g.K = k;
    g.compute = CG_F32;
    g.A = x;
    g.lda = k;
    g.W = w;
    g.epi = EPI_SCALE_ADD;
    g.addend = addend;
    g.add_dtype = addend_dtype;
    g.round_c = compute_dtype == CG_BF16;
    g.ld_add = n;
    g.scale = scale;
    g.out = y;
    g.out_dtype = CG_F32;
    g.ldo = n;
    launch_gemm(g, as_stream(stream));
  });
}
