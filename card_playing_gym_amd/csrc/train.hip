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

#include "common.h"

namespace cg {
namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4;

// ---- strided GEMM ---------------------------------------------------------------------
// Tile 64 x 64, four waves (2 x 2), 16 k per LDS stage.  A(m, k) = A[m * sam + k * sak],
// B(k, n) = B[k * sbk + n * sbn].  MFMA 16x16x4 f32: lane (li, lg) gives A(row li, k lg) and
// B(k lg, col li); the result sits in lane (li, lg) as rows 4 lg + r, column li.
constexpr int GT_M = 64, GT_N = 64, GT_K = 16;

__global__ __launch_bounds__(256) void gemm_strided_kernel(int32_t M, int32_t N, int32_t K, float alpha,
                                                           const float *__restrict__ A, int64_t sam, int64_t sak,
                                                           const float *__restrict__ B, int64_t sbk, int64_t sbn,
                                                           float beta, float *__restrict__ C, int64_t ldc) {
  __shared__ float as[GT_K][GT_M + 4];
  __shared__ float bs[GT_K][GT_N + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.y * GT_M, n0 = blockIdx.x * GT_N;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Each thread stages 4 elements of A and 4 of B per k-stage; the faster-moving index
  // follows whichever stride is 1, so the global reads coalesce for either layout.
  const bool a_kfast = sak == 1, b_nfast = sbn == 1;
  for (int k0 = 0; k0 < K; k0 += GT_K) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * 256;  // 0 .. 1023 = 64 x 16
      int m, k;
      if (a_kfast) {
        m = idx / GT_K;
        k = idx % GT_K;
      } else {
        k = idx / GT_M;
        m = idx % GT_M;
      }
      const int gm = m0 + m, gk = k0 + k;
      as[k][m] = (gm < M && gk < K) ? A[int64_t(gm) * sam + int64_t(gk) * sak] : 0.f;
      int n, kb;
      if (b_nfast) {
        kb = idx / GT_N;
        n = idx % GT_N;
      } else {
        n = idx / GT_K;
        kb = idx % GT_K;
      }
      const int gn = n0 + n, gkb = k0 + kb;
      bs[kb][n] = (gn < N && gkb < K) ? B[int64_t(gkb) * sbk + int64_t(gn) * sbn] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < GT_K; ks += 4) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = as[ks + lg][wm * 32 + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = bs[ks + lg][wn * 32 + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 32 + i * 16 + 4 * lg + r, n = n0 + wn * 32 + j * 16 + li;
        if (m >= M || n >= N) continue;
        float *c = C + int64_t(m) * ldc + n;
        *c = alpha * acc[i][j][r] + (beta != 0.f ? beta * *c : 0.f);
      }
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

// dx = rstd (g - mean(g) - xhat mean(g xhat)), g = dy * w; per block of `rows_per_block`
// rows, partial dw = sum dy xhat and db = sum dy into part[blockIdx][0 / 1][d].  A NULL
// mean selects RMSNorm (no centring, no bias).
__global__ void norm_bwd_kernel(const float *__restrict__ x, const float *__restrict__ dy,
                                const float *__restrict__ w, const float *__restrict__ mean,
                                const float *__restrict__ rstd, float *__restrict__ dx, float *__restrict__ part,
                                int32_t n, int32_t d, int32_t rows_per_block) {
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
      dxr[k] = r * (gr[k] * w[k] - mg - xh * mgx);
      atomicAdd(&acc_lds[k], gr[k] * xh);  // LDS atomics: order within a block only
      atomicAdd(&acc_lds[d + k], gr[k]);
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < 2 * d; k += blockDim.x) part[int64_t(blockIdx.x) * 2 * d + k] = acc_lds[k];
}

// out[c] = sum_r in[r * ld + c] (+ out[c] when accumulate): column sums of per-block
// partials and bias gradients.
__global__ void column_sum_kernel(const float *__restrict__ in, int32_t rows, int32_t cols, int64_t ld,
                                  float *__restrict__ out, int32_t accumulate) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int r = 0; r < rows; ++r) s += in[int64_t(r) * ld + c];
  out[c] = accumulate ? out[c] + s : s;
}

// ---- GELU -------------------------------------------------------------------------------
__device__ __forceinline__ float gelu_exact(float u) { return 0.5f * u * (1.0f + erff(u * 0.70710678118654752f)); }

__global__ void gelu_fwd_kernel(const float *__restrict__ u, float *__restrict__ g, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    g[i] = gelu_exact(u[i]);
}

// du = dg * (Phi(u) + u phi(u)).
__global__ void gelu_bwd_kernel(const float *__restrict__ u, const float *__restrict__ dg, float *__restrict__ du,
                                int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float x = u[i];
    const float cdf = 0.5f * (1.0f + erff(x * 0.70710678118654752f));
    const float pdf = 0.3989422804014327f * expf(-0.5f * x * x);
    du[i] = dg[i] * (cdf + x * pdf);
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
};

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int D>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const AttnTrain a) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= a.n * a.H) return;
  const int t = item / a.H, h = item % a.H, hk = h / (a.H / a.KVH);
  const int64_t start = a.seq_start[a.seq_of[t]];
  float q[D];
#pragma unroll
  for (int d = 0; d < D; ++d) q[d] = a.q[int64_t(t) * a.ldq + h * D + d] * a.scale;
  float m = -INFINITY, l = 0.f, acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  for (int64_t j0 = start; j0 <= t; j0 += 64) {
    const int64_t j = j0 + lane;
    const bool ok = j <= t;
    float s = -INFINITY;
    if (ok) {
      const float *kr = a.k + j * a.ldk + hk * D;
      s = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) s = fmaf(q[d], kr[d], s);
    }
    const float mn = fmaxf(m, wave_max_f(s));
    const float p = ok ? expf(s - mn) : 0.f;
    const float corr = expf(m - mn);
    l = l * corr + wave_sum_f(p);
    const float *vr = a.v + (ok ? j : t) * a.ldv + hk * D;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * corr + p * vr[d];
    m = mn;
  }
  // acc holds each lane's share of sum_j p_j v_j: reduce over the wave.
  float *orow = a.out + (int64_t(t) * a.H + h) * D;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const float s = wave_sum_f(acc[d]);
    if (lane == 0) orow[d] = s / l;
  }
  if (lane == 0) a.lse_out[int64_t(t) * a.H + h] = m + logf(l);
}

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const AttnTrain a) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= a.n * a.H) return;
  const int t = item / a.H, h = item % a.H, hk = h / (a.H / a.KVH);
  const int64_t start = a.seq_start[a.seq_of[t]];
  const int64_t row = int64_t(t) * a.H + h;
  float q[D], go[D];
  float dpart = 0.f;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = a.q[int64_t(t) * a.ldq + h * D + d] * a.scale;
    go[d] = a.dout[row * D + d];
    dpart = fmaf(go[d], a.o[row * D + d], dpart);
  }
  const float dsum = dpart;  // every lane computed the full row sum
  const float lse = a.lse[row];
  float dq[D];
#pragma unroll
  for (int d = 0; d < D; ++d) dq[d] = 0.f;
  for (int64_t j0 = start; j0 <= t; j0 += 64) {
    const int64_t j = j0 + lane;
    if (j <= t) {
      const float *kr = a.k + j * a.ldk + hk * D, *vr = a.v + j * a.ldv + hk * D;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = fmaf(q[d], kr[d], s);
        dp = fmaf(go[d], vr[d], dp);
      }
      const float ds = expf(s - lse) * (dp - dsum);
#pragma unroll
      for (int d = 0; d < D; ++d) dq[d] = fmaf(ds, kr[d], dq[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const float s = wave_sum_f(dq[d]);
    if (lane == 0) a.dq[int64_t(t) * a.ldq + h * D + d] = s * a.scale;
  }
  if (lane == 0) a.dsum[row] = dsum;
}

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dkv_kernel(const AttnTrain a) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (item >= a.n * a.KVH) return;
  const int j = item / a.KVH, hk = item % a.KVH;
  const int G = a.H / a.KVH;
  const int64_t end = a.seq_start[a.seq_of[j] + 1];
  float kr[D], vr[D], dk[D], dv[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    kr[d] = a.k[int64_t(j) * a.ldk + hk * D + d];
    vr[d] = a.v[int64_t(j) * a.ldv + hk * D + d];
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  // Lanes take (query, head) pairs of the group: index i -> query j + i / G, head hk G + i % G.
  const int64_t pairs = (end - j) * G;
  for (int64_t i0 = 0; i0 < pairs; i0 += 64) {
    const int64_t i = i0 + lane;
    if (i < pairs) {
      const int64_t t = j + i / G;
      const int h = hk * G + int(i % G);
      const int64_t row = t * a.H + h;
      const float *qr = a.q + t * a.ldq + h * D, *gr = a.dout + row * D;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = fmaf(qr[d], kr[d], s);
        dp = fmaf(gr[d], vr[d], dp);
      }
      const float p = expf(s * a.scale - a.lse[row]);
      const float ds = p * (dp - a.dsum[row]);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dk[d] = fmaf(ds, qr[d], dk[d]);
        dv[d] = fmaf(p, gr[d], dv[d]);
      }
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const float sk = wave_sum_f(dk[d]), sv = wave_sum_f(dv[d]);
    if (lane == 0) {
      a.dk[int64_t(j) * a.ldk + hk * D + d] = sk * a.scale;
      a.dv[int64_t(j) * a.ldv + hk * D + d] = sv;
    }
  }
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

#define CG_HD_DISPATCH(KERNEL, D, GRID, ARGS, STREAM)                         \
  switch (D) {                                                                \
    case 8: KERNEL<8><<<GRID, 256, 0, STREAM>>>(ARGS); break;                 \
    case 16: KERNEL<16><<<GRID, 256, 0, STREAM>>>(ARGS); break;               \
    case 24: KERNEL<24><<<GRID, 256, 0, STREAM>>>(ARGS); break;               \
    case 32: KERNEL<32><<<GRID, 256, 0, STREAM>>>(ARGS); break;               \
    case 64: KERNEL<64><<<GRID, 256, 0, STREAM>>>(ARGS); break;               \
    default: throw Error(CG_ERR_UNSUPPORTED, "training attention: head_dim 8, 16, 24, 32 or 64"); \
  }

}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

int cg_gemm_strided(int32_t m, int32_t n, int32_t k, float alpha, const float *a, int64_t sam, int64_t sak,
                    const float *b, int64_t sbk, int64_t sbn, float beta, float *c, int64_t ldc, void *stream) {
  return guarded([&] {
    CG_REQUIRE(m >= 0 && n >= 0 && k >= 0, CG_ERR_INVALID, "negative GEMM size");
    if (m == 0 || n == 0) return;
    CG_REQUIRE(a && b && c, CG_ERR_INVALID, "a, b and c are required");
    const dim3 grid(unsigned((n + GT_N - 1) / GT_N), unsigned((m + GT_M - 1) / GT_M));
    CG_REQUIRE(grid.y <= 65535, CG_ERR_UNSUPPORTED, "GEMM: too many row tiles");
    gemm_strided_kernel<<<grid, 256, 0, as_stream(stream)>>>(m, n, k, alpha, a, sam, sak, b, sbk, sbn, beta, c, ldc);
    CG_LAUNCHED();
  });
}

int cg_layernorm_fwd(const float *x, const float *w, const float *b, float eps, float *y, float *mean, float *rstd,
                     int32_t n, int32_t d, void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(x && w && b && y && mean && rstd && d > 0, CG_ERR_INVALID, "LayerNorm operands are required");
    layernorm_fwd_kernel<<<blocks_of(n, 4), 256, 0, as_stream(stream)>>>(x, w, b, eps, y, mean, rstd, n, d);
    CG_LAUNCHED();
  });
}

size_t cg_norm_bwd_workspace_size(int32_t n, int32_t d) {
  const int64_t blocks = (int64_t(n) + 63) / 64;
  return size_t(std::max<int64_t>(blocks, 1)) * 2 * size_t(d) * 4;
}

int cg_norm_bwd(const float *x, const float *dy, const float *w, const float *mean, const float *rstd, float *dx,
                float *dw, float *db, int32_t n, int32_t d, void *workspace, size_t workspace_size,
                int32_t accumulate, void *stream) {
  return guarded([&] {
    if (n == 0) return;
    CG_REQUIRE(x && dy && w && rstd && dx && dw && d > 0, CG_ERR_INVALID, "norm backward operands are required");
    CG_REQUIRE(mean == nullptr || db != nullptr, CG_ERR_INVALID, "LayerNorm backward needs db");
    CG_REQUIRE(workspace && workspace_size >= cg_norm_bwd_workspace_size(n, d), CG_ERR_INVALID,
               "norm backward: workspace too small");
    hipStream_t s = as_stream(stream);
    const int rows = 64;
    const unsigned blocks = unsigned((int64_t(n) + rows - 1) / rows);
    float *part = static_cast<float *>(workspace);
    norm_bwd_kernel<<<blocks, 256, 2 * d * sizeof(float), s>>>(x, dy, w, mean, rstd, dx, part, n, d, rows);
    CG_LAUNCHED();
    column_sum_kernel<<<blocks_of(d, 256), 256, 0, s>>>(part, int32_t(blocks), d, 2 * d, dw, accumulate);
    CG_LAUNCHED();
    if (db) {
      column_sum_kernel<<<blocks_of(d, 256), 256, 0, s>>>(part + d, int32_t(blocks), d, 2 * d, db, accumulate);
      CG_LAUNCHED();
    }
  });
}

int cg_column_sum(const float *x, int32_t rows, int32_t cols, int64_t ld, float *out, int32_t accumulate,
                  void *stream) {
  return guarded([&] {
    if (cols == 0) return;
    CG_REQUIRE(x && out && rows >= 0, CG_ERR_INVALID, "column sum operands are required");
    column_sum_kernel<<<blocks_of(cols, 256), 256, 0, as_stream(stream)>>>(x, rows, cols, ld, out, accumulate);
    CG_LAUNCHED();
  });
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
    CG_REQUIRE(p && p->H > 0 && p->KVH > 0 && p->H % p->KVH == 0, CG_ERR_INVALID, "bad attention heads");
    if (p->n == 0) return;
    AttnTrain a{p->n, p->H, p->KVH, p->scale, p->seq_start, p->seq_of, p->q, p->k, p->v, p->ldq, p->ldk, p->ldv,
                nullptr, nullptr, nullptr, p->o, p->lse, nullptr, nullptr, nullptr, nullptr};
    CG_REQUIRE(a.q && a.k && a.v && a.out && a.lse_out && a.seq_start && a.seq_of, CG_ERR_INVALID,
               "attention forward operands are required");
    CG_HD_DISPATCH(attn_fwd_kernel, p->head_dim, blocks_of(int64_t(p->n) * p->H, 4), a, as_stream(stream));
    CG_LAUNCHED();
  });
}

int cg_attn_train_bwd(const cg_attn_train *p, const float *dout, float *dsum, float *dq, float *dk, float *dv,
                      void *stream) {
  return guarded([&] {
    CG_REQUIRE(p && p->H > 0 && p->KVH > 0 && p->H % p->KVH == 0, CG_ERR_INVALID, "bad attention heads");
    if (p->n == 0) return;
    AttnTrain a{p->n, p->H, p->KVH, p->scale, p->seq_start, p->seq_of, p->q, p->k, p->v, p->ldq, p->ldk, p->ldv,
                p->o, dout, p->lse, nullptr, nullptr, dsum, dq, dk, dv};
    CG_REQUIRE(a.q && a.k && a.v && a.o && a.dout && a.lse && dsum && dq && dk && dv, CG_ERR_INVALID,
               "attention backward operands are required");
    hipStream_t s = as_stream(stream);
    CG_HD_DISPATCH(attn_bwd_dq_kernel, p->head_dim, blocks_of(int64_t(p->n) * p->H, 4), a, s);
    CG_LAUNCHED();
    CG_HD_DISPATCH(attn_bwd_dkv_kernel, p->head_dim, blocks_of(int64_t(p->n) * p->KVH, 4), a, s);
    CG_LAUNCHED();
  });
}

}  // extern "C"
