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

// ---- strided GEMM ---------------------------------------------------------------------
// Tile 128 x 128, four waves (2 x 2, each 64 x 64 = 4 x 4 MFMA tiles), 16 k per LDS stage,
// double-buffered.  A(m, k) = A[m * sam + k * sak], B(k, n) = B[k * sbk + n * sbn]; tiles are
// staged through LDS with 16-byte loads along whichever index has stride 1.  MFMA 16x16x4
// f32: lane (li, lg) gives A(row li, k lg) and B(k lg, col li); the result sits in lane
// (li, lg) as rows 4 lg + r, column li.  Split K (grid.z > 1): slice z covers k in [z kc,
// (z + 1) kc) and writes its partial product to part[z] ([m, n]); a second pass sums them.
constexpr int GT_M = 128, GT_N = 128, GT_K = 16;
constexpr int GT_LD = GT_M + 4;  // LDS row (one k) of a staged operand tile, floats

// Loads a 128 x 16 (rows x k) operand tile with element (r, k) at p[r * sr + k * sk] into
// registers (`v`, two float4 per thread); rows >= rows_left or k >= k_left read 0.
struct TileRegs {
  float4 v[2];
};

__device__ __forceinline__ TileRegs load_tile(const float *__restrict__ p, int64_t sr, int64_t sk, int rows_left,
                                              int k_left, int tid, int mode) {
  TileRegs t;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int idx = tid + e * 256;  // 512 float4 = 2048 floats
    float4 v = {0.f, 0.f, 0.f, 0.f};
    if (mode == 1) {  // k contiguous: 128 rows x 4 groups of 4 k
      const int r = idx >> 2, k = (idx & 3) * 4;
      if (r < rows_left) {
        const float *q = p + int64_t(r) * sr + k;
        if (k + 3 < k_left) {
          v = *reinterpret_cast<const float4 *>(q);
        } else {
          if (k < k_left) v.x = q[0];
          if (k + 1 < k_left) v.y = q[1];
          if (k + 2 < k_left) v.z = q[2];
        }
      }
    } else if (mode == 2) {  // rows contiguous: 16 k x 32 groups of 4 rows
      const int k = idx >> 5, r = (idx & 31) * 4;
      if (k < k_left) {
        const float *q = p + int64_t(k) * sk + r;
        if (r + 3 < rows_left) {
          v = *reinterpret_cast<const float4 *>(q);
        } else {
          if (r < rows_left) v.x = q[0];
          if (r + 1 < rows_left) v.y = q[1];
          if (r + 2 < rows_left) v.z = q[2];
        }
      }
    } else {  // general strides: element by element, same slots as mode 1
      const int r = idx >> 2, k = (idx & 3) * 4;
      float x[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = (r < rows_left && k + c < k_left) ? p[int64_t(r) * sr + int64_t(k + c) * sk] : 0.f;
      v = float4{x[0], x[1], x[2], x[3]};
    }
    t.v[e] = v;
  }
  return t;
}

__device__ __forceinline__ void store_tile(float *lds, const TileRegs &t, int tid, int mode) {
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int idx = tid + e * 256;
    if (mode == 2) {
      const int k = idx >> 5, r = (idx & 31) * 4;
      *reinterpret_cast<float4 *>(lds + k * GT_LD + r) = t.v[e];
    } else {
      const int r = idx >> 2, k = (idx & 3) * 4;
      lds[(k + 0) * GT_LD + r] = t.v[e].x;
      lds[(k + 1) * GT_LD + r] = t.v[e].y;
      lds[(k + 2) * GT_LD + r] = t.v[e].z;
      lds[(k + 3) * GT_LD + r] = t.v[e].w;
    }
  }
}

__device__ __forceinline__ int tile_mode(const float *p, int64_t sr, int64_t sk) {
  const bool al = (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  if (sk == 1 && (sr & 3) == 0 && al) return 1;
  if (sr == 1 && (sk & 3) == 0 && al) return 2;
  return 0;
}

__global__ __launch_bounds__(256) void gemm_strided_kernel(int32_t M, int32_t N, int32_t K, int32_t kc, float alpha,
                                                           const float *__restrict__ A, int64_t sam, int64_t sak,
                                                           const float *__restrict__ B, int64_t sbk, int64_t sbn,
                                                           float beta, float *__restrict__ C, int64_t ldc,
                                                           float *__restrict__ part) {
  __shared__ __align__(16) float as[2][GT_K * GT_LD];
  __shared__ __align__(16) float bs[2][GT_K * GT_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.y * GT_M, n0 = blockIdx.x * GT_N;
  const int kbeg = blockIdx.z * kc, kend = min(K, kbeg + kc);
  const float *a0 = A + int64_t(m0) * sam, *b0 = B + int64_t(n0) * sbn;
  const int amode = tile_mode(a0, sam, sak), bmode = tile_mode(b0, sbn, sbk);
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  int buf = 0;
  if (kbeg < kend) {
    store_tile(as[0], load_tile(a0 + int64_t(kbeg) * sak, sam, sak, M - m0, kend - kbeg, tid, amode), tid, amode);
    store_tile(bs[0], load_tile(b0 + int64_t(kbeg) * sbk, sbn, sbk, N - n0, kend - kbeg, tid, bmode), tid, bmode);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += GT_K) {
    const bool more = k0 + GT_K < kend;
    TileRegs na, nb;
    if (more) {  // the next stage's loads fly during this stage's MFMAs
      na = load_tile(a0 + int64_t(k0 + GT_K) * sak, sam, sak, M - m0, kend - k0 - GT_K, tid, amode);
      nb = load_tile(b0 + int64_t(k0 + GT_K) * sbk, sbn, sbk, N - n0, kend - k0 - GT_K, tid, bmode);
    }
    const float *ta = as[buf], *tb = bs[buf];
#pragma unroll
    for (int ks = 0; ks < GT_K; ks += 4) {
      float af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = ta[(ks + lg) * GT_LD + wm * 64 + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = tb[(ks + lg) * GT_LD + wn * 64 + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      store_tile(as[buf ^ 1], na, tid, amode);
      store_tile(bs[buf ^ 1], nb, tid, bmode);
    }
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + 4 * lg + r, n = n0 + wn * 64 + j * 16 + li;
        if (m >= M || n >= N) continue;
        if (part) {
          part[(int64_t(blockIdx.z) * M + m) * N + n] = acc[i][j][r];
        } else {
          float *c = C + int64_t(m) * ldc + n;
          *c = alpha * acc[i][j][r] + (beta != 0.f ? beta * *c : 0.f);
        }
      }
}

// C[m, n] = alpha * sum_z part[z][m, n] + beta * C[m, n].
__global__ void gemm_reduce_kernel(int32_t M, int32_t N, int32_t slices, float alpha, const float *__restrict__ part,
                                   float beta, float *__restrict__ C, int64_t ldc) {
  const int64_t total = int64_t(M) * N;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    float s = 0.f;
    for (int z = 0; z < slices; ++z) s += part[int64_t(z) * total + i];
    float *c = C + (i / N) * ldc + i % N;
    *c = alpha * s + (beta != 0.f ? beta * *c : 0.f);
  }
}

// Split-K plan: enough (tile, slice) blocks to fill the chip when the output has few tiles
// and the reduction is long (weight gradients reduce over every token).
struct SplitK {
  int slices, kc;
};
SplitK split_k(int32_t m, int32_t n, int32_t k) {
  const int64_t tiles = int64_t((m + GT_M - 1) / GT_M) * ((n + GT_N - 1) / GT_N);
  int slices = 1;
  if (tiles < 512 && k >= 4 * GT_K * 16) {
    slices = int(std::min<int64_t>((512 + tiles - 1) / tiles, k / (GT_K * 16)));
    slices = std::max(1, std::min(slices, 64));
  }
  const int kc = ((k + slices - 1) / slices + GT_K - 1) / GT_K * GT_K;
  slices = (k + kc - 1) / kc;
  return {slices, kc};
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
// partials and bias gradients.  A block takes 64 columns x `chunk` rows: its four waves
// split the rows, each lane one column (coalesced rows), and meet in LDS; blockIdx.y's
// chunk lands in out[y][c] (a second pass sums the chunks).
__global__ __launch_bounds__(256) void column_sum_kernel(const float *__restrict__ in, int32_t rows, int32_t cols,
                                                         int64_t ld, float *__restrict__ out, int32_t accumulate,
                                                         int32_t chunk) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int r0 = blockIdx.y * chunk, r1 = min(rows, r0 + chunk);
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < cols) {
    int r = r0 + wave;
    for (; r + 12 < r1; r += 16) {
      s0 += in[int64_t(r) * ld + c];
      s1 += in[int64_t(r + 4) * ld + c];
      s2 += in[int64_t(r + 8) * ld + c];
      s3 += in[int64_t(r + 12) * ld + c];
    }
    for (; r < r1; r += 4) s0 += in[int64_t(r) * ld + c];
  }
  red[wave][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (wave == 0 && c < cols) {
    const float s = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    float *o = out + int64_t(blockIdx.y) * cols + c;
    *o = accumulate ? *o + s : s;
  }
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

// One lane per (token, head): a block is 64 consecutive tokens x up to four heads of one KV
// head's group (wave w = head hk G + 4 blockIdx.z + w), so every K / V tile staged in LDS
// serves up to 256 queries, and each lane runs its own softmax over the keys its token sees
// (no cross-lane reductions).
constexpr int AT = 32;  // keys per LDS tile

template <int D>
__device__ __forceinline__ float dot_lds(const float (&q)[D], const float *row) {
  float s = 0.f;
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    const float4 k = *reinterpret_cast<const float4 *>(row + d);
    s = fmaf(q[d], k.x, s);
    s = fmaf(q[d + 1], k.y, s);
    s = fmaf(q[d + 2], k.z, s);
    s = fmaf(q[d + 3], k.w, s);
  }
  return s;
}

// Stages keys [j0, j0 + AT) of KV head hk (rows past n read as 0) into kt / vt.
template <int D>
__device__ __forceinline__ void stage_kv(const AttnTrain &a, int hk, int64_t j0, float *kt, float *vt) {
  for (int i = threadIdx.x; i < AT * D / 4; i += blockDim.x) {
    const int r = i / (D / 4), c = (i % (D / 4)) * 4;
    const int64_t j = j0 + r;
    float4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
    if (j < a.n) {
      const float *kp = a.k + j * a.ldk + hk * D + c, *vp = a.v + j * a.ldv + hk * D + c;
      kv = float4{kp[0], kp[1], kp[2], kp[3]};
      vv = float4{vp[0], vp[1], vp[2], vp[3]};
    }
    *reinterpret_cast<float4 *>(kt + r * D + c) = kv;
    *reinterpret_cast<float4 *>(vt + r * D + c) = vv;
  }
}

template <int D>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const AttnTrain a) {
  __shared__ __align__(16) float kt[AT * D], vt[AT * D];
  const int G = a.H / a.KVH, hk = blockIdx.y;
  const int lane = threadIdx.x & 63, g = blockIdx.z * 4 + (threadIdx.x >> 6);
  const int64_t t0 = int64_t(blockIdx.x) * 64, t = t0 + lane;
  const int64_t t_last = min(int64_t(a.n) - 1, t0 + 63);
  const bool live = t < a.n && g < G;
  const int h = hk * G + min(g, G - 1);
  const int64_t start = live ? a.seq_start[a.seq_of[t]] : 0;
  const int64_t k_lo = a.seq_start[a.seq_of[t0]];
  float q[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = live ? a.q[t * a.ldq + h * D + d] * a.scale : 0.f;
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int64_t j0 = k_lo; j0 <= t_last; j0 += AT) {
    __syncthreads();
    stage_kv<D>(a, hk, j0, kt, vt);
    __syncthreads();
    float sc[AT];
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < AT; ++i) {
      const int64_t j = j0 + i;
      const bool ok = live && j >= start && j <= t;
      sc[i] = ok ? dot_lds<D>(q, kt + i * D) : -INFINITY;
      mt = fmaxf(mt, sc[i]);
    }
    if (mt == -INFINITY) continue;  // no key of this tile for this query
    const float mn = fmaxf(m, mt);
    const float corr = expf(m - mn);
    l *= corr;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] *= corr;
#pragma unroll
    for (int i = 0; i < AT; ++i) {
      const float p = expf(sc[i] - mn);
      l += p;
      const float *vr = vt + i * D;
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(vr + d);
        acc[d] = fmaf(p, v.x, acc[d]);
        acc[d + 1] = fmaf(p, v.y, acc[d + 1]);
        acc[d + 2] = fmaf(p, v.z, acc[d + 2]);
        acc[d + 3] = fmaf(p, v.w, acc[d + 3]);
      }
    }
    m = mn;
  }
  if (!live) return;
  const float inv = 1.0f / l;
  float *orow = a.out + (t * a.H + h) * D;
#pragma unroll
  for (int d = 0; d < D; ++d) orow[d] = acc[d] * inv;
  a.lse_out[t * a.H + h] = m + logf(l);
}

// dQ (and D = rowsum(dO * O)) per (token, head), with the forward's block layout.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const AttnTrain a) {
  __shared__ __align__(16) float kt[AT * D], vt[AT * D];
  const int G = a.H / a.KVH, hk = blockIdx.y;
  const int lane = threadIdx.x & 63, g = blockIdx.z * 4 + (threadIdx.x >> 6);
  const int64_t t0 = int64_t(blockIdx.x) * 64, t = t0 + lane;
  const int64_t t_last = min(int64_t(a.n) - 1, t0 + 63);
  const bool live = t < a.n && g < G;
  const int h = hk * G + min(g, G - 1);
  const int64_t row = t * a.H + h;
  const int64_t start = live ? a.seq_start[a.seq_of[t]] : 0;
  const int64_t k_lo = a.seq_start[a.seq_of[t0]];
  float q[D], go[D], dq[D];
  float dsum = 0.f;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = live ? a.q[t * a.ldq + h * D + d] * a.scale : 0.f;
    go[d] = live ? a.dout[row * D + d] : 0.f;
    dsum = fmaf(go[d], live ? a.o[row * D + d] : 0.f, dsum);
    dq[d] = 0.f;
  }
  const float lse = live ? a.lse[row] : 0.f;
  for (int64_t j0 = k_lo; j0 <= t_last; j0 += AT) {
    __syncthreads();
    stage_kv<D>(a, hk, j0, kt, vt);
    __syncthreads();
#pragma unroll 2
    for (int i = 0; i < AT; ++i) {
      const int64_t j = j0 + i;
      if (!(live && j >= start && j <= t)) continue;
      float kr[D];  // the key row once from LDS, for the score and the dQ update
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 k = *reinterpret_cast<const float4 *>(kt + i * D + d);
        kr[d] = k.x;
        kr[d + 1] = k.y;
        kr[d + 2] = k.z;
        kr[d + 3] = k.w;
      }
      float sc = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) sc = fmaf(q[d], kr[d], sc);
      const float p = expf(sc - lse);
      const float ds = p * (dot_lds<D>(go, vt + i * D) - dsum);
#pragma unroll
      for (int d = 0; d < D; ++d) dq[d] = fmaf(ds, kr[d], dq[d]);
    }
  }
  if (!live) return;
#pragma unroll
  for (int d = 0; d < D; ++d) a.dq[t * a.ldq + h * D + d] = dq[d] * a.scale;
  a.dsum[row] = dsum;
}

// dK / dV: one lane per key of a 64-key block of KV head blockIdx.y; the queries (token, head
// of the group) that can see those keys are staged in LDS QT tokens at a time.
constexpr int QT = 8;

template <int D>
__global__ __launch_bounds__(64) void attn_bwd_dkv_kernel(const AttnTrain a) {
  const int G = a.H / a.KVH, hk = blockIdx.y;
  extern __shared__ __align__(16) float qs[];  // [QT * G][2 D + 2]: q (scaled), dO, lse, D
  const int stride = 2 * D + 4;
  const int lane = threadIdx.x;
  const int64_t j0 = int64_t(blockIdx.x) * 64, j = j0 + lane;
  const bool live = j < a.n;
  const int64_t end = live ? a.seq_start[a.seq_of[j] + 1] : 0;
  const int64_t j_last = min(int64_t(a.n) - 1, j0 + 63);
  const int64_t q_hi = a.seq_start[a.seq_of[j_last] + 1];  // queries past it see none of these keys
  float kr[D], vr[D], dk[D], dv[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    kr[d] = live ? a.k[j * a.ldk + hk * D + d] : 0.f;
    vr[d] = live ? a.v[j * a.ldv + hk * D + d] : 0.f;
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  for (int64_t t0 = j0; t0 < q_hi; t0 += QT) {
    __syncthreads();
    for (int i = lane; i < QT * G * (D / 4); i += 64) {
      const int r = i / (D / 4), c = (i % (D / 4)) * 4;
      const int64_t t = t0 + r / G;
      const int h = hk * G + r % G;
      float *dst = qs + r * stride;
      if (t < a.n) {
        const float *qp = a.q + t * a.ldq + h * D + c, *gp = a.dout + (t * a.H + h) * D + c;
        *reinterpret_cast<float4 *>(dst + c) = float4{qp[0] * a.scale, qp[1] * a.scale, qp[2] * a.scale, qp[3] * a.scale};
        *reinterpret_cast<float4 *>(dst + D + c) = float4{gp[0], gp[1], gp[2], gp[3]};
        if (c == 0) {
          dst[2 * D] = a.lse[t * a.H + h];
          dst[2 * D + 1] = a.dsum[t * a.H + h];
        }
      } else {
        *reinterpret_cast<float4 *>(dst + c) = float4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<float4 *>(dst + D + c) = float4{0.f, 0.f, 0.f, 0.f};
        if (c == 0) {
          dst[2 * D] = 0.f;
          dst[2 * D + 1] = 0.f;
        }
      }
    }
    __syncthreads();
    for (int r = 0; r < QT * G; ++r) {
      const int64_t t = t0 + r / G;
      if (!(live && t >= j && t < end)) continue;
      const float *qrow = qs + r * stride;
      float qv[D], gv[D];  // the query and dO rows once from LDS, for the products and updates
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 a4 = *reinterpret_cast<const float4 *>(qrow + d);
        const float4 g4 = *reinterpret_cast<const float4 *>(qrow + D + d);
        qv[d] = a4.x;
        qv[d + 1] = a4.y;
        qv[d + 2] = a4.z;
        qv[d + 3] = a4.w;
        gv[d] = g4.x;
        gv[d + 1] = g4.y;
        gv[d + 2] = g4.z;
        gv[d + 3] = g4.w;
      }
      float sc = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        sc = fmaf(kr[d], qv[d], sc);
        dp = fmaf(vr[d], gv[d], dp);
      }
      const float p = expf(sc - qrow[2 * D]);
      const float ds = p * (dp - qrow[2 * D + 1]);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dk[d] = fmaf(ds, qv[d], dk[d]);
        dv[d] = fmaf(p, gv[d], dv[d]);
      }
    }
  }
  if (!live) return;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    a.dk[j * a.ldk + hk * D + d] = dk[d];  // q was staged scaled: dK = sum ds q scale
    a.dv[j * a.ldv + hk * D + d] = dv[d];
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


}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

size_t cg_gemm_workspace_size(int32_t m, int32_t n, int32_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  const SplitK sk = split_k(m, n, k);
  return sk.slices > 1 ? size_t(sk.slices) * size_t(m) * size_t(n) * 4 : 0;
}

int cg_gemm_strided(int32_t m, int32_t n, int32_t k, float alpha, const float *a, int64_t sam, int64_t sak,
                    const float *b, int64_t sbk, int64_t sbn, float beta, float *c, int64_t ldc, void *workspace,
                    size_t workspace_size, void *stream) {
  return guarded([&] {
    CG_REQUIRE(m >= 0 && n >= 0 && k >= 0, CG_ERR_INVALID, "negative GEMM size");
    if (m == 0 || n == 0) return;
    CG_REQUIRE(a && b && c, CG_ERR_INVALID, "a, b and c are required");
    const SplitK sk = split_k(m, n, k);
    const size_t need = cg_gemm_workspace_size(m, n, k);
    CG_REQUIRE(need == 0 || (workspace && workspace_size >= need), CG_ERR_INVALID,
               "GEMM: workspace too small, need " + std::to_string(need) + " bytes");
    const dim3 grid(unsigned((n + GT_N - 1) / GT_N), unsigned((m + GT_M - 1) / GT_M), unsigned(sk.slices));
    CG_REQUIRE(grid.y <= 65535, CG_ERR_UNSUPPORTED, "GEMM: too many row tiles");
    hipStream_t s = as_stream(stream);
    float *part = sk.slices > 1 ? static_cast<float *>(workspace) : nullptr;
    gemm_strided_kernel<<<grid, 256, 0, s>>>(m, n, k, sk.kc, alpha, a, sam, sak, b, sbk, sbn, beta, c, ldc, part);
    CG_LAUNCHED();
    if (part) {
      gemm_reduce_kernel<<<grid_1d(int64_t(m) * n), 256, 0, s>>>(m, n, sk.slices, alpha, part, beta, c, ldc);
      CG_LAUNCHED();
    }
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
    column_sum_kernel<<<dim3(blocks_of(d, 64), 1), 256, 0, s>>>(part, int32_t(blocks), d, 2 * d, dw, accumulate,
                                                                int32_t(blocks));
    CG_LAUNCHED();
    if (db) {
      column_sum_kernel<<<dim3(blocks_of(d, 64), 1), 256, 0, s>>>(part + d, int32_t(blocks), d, 2 * d, db,
                                                                  accumulate, int32_t(blocks));
      CG_LAUNCHED();
    }
  });
}

size_t cg_column_sum_workspace_size(int32_t rows, int32_t cols) {
  return rows > 2048 ? size_t((rows + 255) / 256) * size_t(std::max(cols, 0)) * 4 : 0;
}

int cg_column_sum(const float *x, int32_t rows, int32_t cols, int64_t ld, float *out, int32_t accumulate,
                  void *workspace, size_t workspace_size, void *stream) {
  return guarded([&] {
    if (cols == 0) return;
    CG_REQUIRE(x && out && rows >= 0, CG_ERR_INVALID, "column sum operands are required");
    hipStream_t s = as_stream(stream);
    if (rows <= 2048) {
      column_sum_kernel<<<dim3(blocks_of(cols, 64), 1), 256, 0, s>>>(x, rows, cols, ld, out, accumulate, rows);
      CG_LAUNCHED();
      return;
    }
    const size_t need = cg_column_sum_workspace_size(rows, cols);
    CG_REQUIRE(workspace && workspace_size >= need, CG_ERR_INVALID, "column sum: workspace too small");
    const int chunks = (rows + 255) / 256;
    float *part = static_cast<float *>(workspace);
    column_sum_kernel<<<dim3(blocks_of(cols, 64), unsigned(chunks)), 256, 0, s>>>(x, rows, cols, ld, part, 0, 256);
    CG_LAUNCHED();
    column_sum_kernel<<<dim3(blocks_of(cols, 64), 1), 256, 0, s>>>(part, chunks, cols, cols, out, accumulate, chunks);
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
    CG_REQUIRE(p && p->H > 0 && p->KVH > 0 && p->H % p->KVH == 0 && p->H / p->KVH <= 16, CG_ERR_INVALID,
               "training attention: H a multiple of KVH, at most 16 heads per KV head");
    if (p->n == 0) return;
    AttnTrain a{p->n, p->H, p->KVH, p->scale, p->seq_start, p->seq_of, p->q, p->k, p->v, p->ldq, p->ldk, p->ldv,
                nullptr, nullptr, nullptr, p->o, p->lse, nullptr, nullptr, nullptr, nullptr};
    CG_REQUIRE(a.q && a.k && a.v && a.out && a.lse_out && a.seq_start && a.seq_of, CG_ERR_INVALID,
               "attention forward operands are required");
    const int G = p->H / p->KVH;
    const dim3 grid(blocks_of(p->n, 64), unsigned(p->KVH), unsigned((G + 3) / 4));
    const unsigned threads = 64u * unsigned(std::min(G, 4));
    hipStream_t s = as_stream(stream);
    switch (p->head_dim) {
      case 8: attn_fwd_kernel<8><<<grid, threads, 0, s>>>(a); break;
      case 16: attn_fwd_kernel<16><<<grid, threads, 0, s>>>(a); break;
      case 24: attn_fwd_kernel<24><<<grid, threads, 0, s>>>(a); break;
      case 32: attn_fwd_kernel<32><<<grid, threads, 0, s>>>(a); break;
      case 64: attn_fwd_kernel<64><<<grid, threads, 0, s>>>(a); break;
      default: throw Error(CG_ERR_UNSUPPORTED, "training attention: head_dim 8, 16, 24, 32 or 64");
    }
    CG_LAUNCHED();
  });
}

int cg_attn_train_bwd(const cg_attn_train *p, const float *dout, float *dsum, float *dq, float *dk, float *dv,
                      void *stream) {
  return guarded([&] {
    CG_REQUIRE(p && p->H > 0 && p->KVH > 0 && p->H % p->KVH == 0 && p->H / p->KVH <= 16, CG_ERR_INVALID,
               "training attention: H a multiple of KVH, at most 16 heads per KV head");
    if (p->n == 0) return;
    AttnTrain a{p->n, p->H, p->KVH, p->scale, p->seq_start, p->seq_of, p->q, p->k, p->v, p->ldq, p->ldk, p->ldv,
                p->o, dout, p->lse, nullptr, nullptr, dsum, dq, dk, dv};
    CG_REQUIRE(a.q && a.k && a.v && a.o && a.dout && a.lse && dsum && dq && dk && dv, CG_ERR_INVALID,
               "attention backward operands are required");
    hipStream_t s = as_stream(stream);
    const int G = p->H / p->KVH;
    const dim3 grid(blocks_of(p->n, 64), unsigned(p->KVH), unsigned((G + 3) / 4));
    const dim3 grid_kv(blocks_of(p->n, 64), unsigned(p->KVH));
    const unsigned threads = 64u * unsigned(std::min(G, 4));
    const size_t dkv_lds = size_t(QT) * G * (2 * p->head_dim + 4) * sizeof(float);
    switch (p->head_dim) {
#define CG_BWD_CASE(DD)                                                  \
  case DD:                                                               \
    attn_bwd_dq_kernel<DD><<<grid, threads, 0, s>>>(a);                  \
    CG_LAUNCHED();                                                       \
    attn_bwd_dkv_kernel<DD><<<grid_kv, 64, dkv_lds, s>>>(a);             \
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
};

TrainDims dims_of(const cg_train_config &c, int32_t n) {
  TrainDims t{};
  t.n = n;
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
// m2, r2 (1), u (F); then x_last (d), mf, rf (1) and seq_of (n int32).
struct SavedLayer {
  float *xl, *h1, *m1, *r1, *qkv, *o, *lse, *x1, *h2, *m2, *r2, *u;
};

int64_t layer_floats(const TrainDims &t) { return t.n * (4 * t.d + 4 + t.QKV + t.Q + t.H + t.F); }

SavedLayer saved_layer(const TrainDims &t, void *saved, int64_t l) {
  float *p = static_cast<float *>(saved) + l * layer_floats(t);
  SavedLayer s{};
  auto take = [&](int64_t cols) {
    float *q = p;
    p += t.n * cols;
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
  return s;
}

struct SavedTail {
  float *x_last, *mf, *rf;
  int32_t *seq_of;
};
SavedTail saved_tail(const TrainDims &t, void *saved) {
  float *p = static_cast<float *>(saved) + t.L * layer_floats(t);
  return {p, p + t.n * t.d, p + t.n * t.d + t.n, reinterpret_cast<int32_t *>(p + t.n * t.d + 2 * t.n)};
}

size_t max_gemm_ws(const TrainDims &t) {
  size_t m = 0;
  const int64_t shapes[][3] = {{t.n, t.QKV, t.d}, {t.n, t.d, t.Q}, {t.n, t.F, t.d}, {t.n, t.d, t.F},
                               {t.QKV, t.d, t.n}, {t.d, t.Q, t.n}, {t.F, t.d, t.n}, {t.d, t.F, t.n},
                               {t.n, t.d, t.QKV}, {t.n, t.Q, t.d}, {t.n, t.d, t.F}};
  for (auto &sh : shapes) m = std::max(m, cg_gemm_workspace_size(int32_t(sh[0]), int32_t(sh[1]), int32_t(sh[2])));
  return m;
}

// Scratch of one call: GEMM split-K partials, then (backward) dx, dx1, dh (d each), g, dg, du (F),
// do (Q), dqkv (QKV), dsum (H), norm / column-sum partials.
struct Scratch {
  float *gemm_ws;
  size_t gemm_bytes;
  float *dx, *dx1, *dh, *g, *dg, *du, *dout, *dqkv, *dsum, *red;
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
  s.g = take(t.F);
  s.dg = take(t.F);
  s.du = take(t.F);
  s.dout = take(t.Q);
  s.dqkv = take(t.QKV);
  s.dsum = take(t.H);
  s.red = f;
  s.red_bytes = red_bytes_of(t);
  return s;
}

size_t scratch_bytes(const TrainDims &t) {
  const int64_t cols = 3 * t.d + 3 * t.F + t.Q + t.QKV + t.H;
  return (max_gemm_ws(t) + 255) / 256 * 256 + size_t(t.n * cols + 64 * 9) * 4 + red_bytes_of(t) + 256;
}

struct Gemm {
  const Scratch &s;
  hipStream_t st;
  // out[M, N] = alpha x[M, K] W[N, K]^T + beta out
  void nt(int64_t M, int64_t N, int64_t K, const float *x, const float *w, float *out, float beta = 0.f,
          float alpha = 1.f) const {
    ok(cg_gemm_strided(int32_t(M), int32_t(N), int32_t(K), alpha, x, K, 1, w, 1, K, beta, out, N, s.gemm_ws,
                       s.gemm_bytes, st));
  }
  // out[M, K] = dy[M, N] W[N, K]
  void nn(int64_t M, int64_t N, int64_t K, const float *dy, const float *w, float *out) const {
    ok(cg_gemm_strided(int32_t(M), int32_t(K), int32_t(N), 1.f, dy, N, 1, w, K, 1, 0.f, out, K, s.gemm_ws,
                       s.gemm_bytes, st));
  }
  // out[N, K] = dy[M, N]^T x[M, K]
  void tn(int64_t M, int64_t N, int64_t K, const float *dy, const float *x, float *out) const {
    ok(cg_gemm_strided(int32_t(N), int32_t(K), int32_t(M), 1.f, dy, 1, N, x, K, 1, 0.f, out, K, s.gemm_ws,
                       s.gemm_bytes, st));
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
  return a;
}

}  // namespace

extern "C" {

size_t cg_train_saved_size(const cg_train_config *c, int32_t n) {
  if (!c || n <= 0) return 0;
  const TrainDims t = dims_of(*c, n);
  return size_t(t.L * layer_floats(t) + t.n * t.d + 2 * t.n) * 4 + size_t(t.n) * 4 + 256;
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
    CG_REQUIRE((c->ple_width == 0 || ple) && (c->value_width == 0 || values), CG_ERR_INVALID,
               "training forward: ple / values lookups are required");
    const TrainDims t = dims_of(*c, n);
    hipStream_t st = as_stream(stream);
    const Scratch s = scratch_of(t, scratch);
    const Gemm gm{s, st};
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
      if (vi >= 0)
        ok(cg_add_strided(int32_t(t.n), int32_t(t.KVW), 1.f, values + vi * t.KVW, t.V, a.qkv + t.Q + t.KVW, t.QKV, st));
      const cg_attn_train at = attn_args(t, seq_start, tail.seq_of, a.qkv, a.o, a.lse);
      ok(cg_attn_train_fwd(&at, st));
      CG_HIP(hipMemcpyAsync(a.x1, a.xl, size_t(t.n * t.d) * 4, hipMemcpyDeviceToDevice, st));
      gm.nt(t.n, t.d, t.Q, a.o, w.out_w, a.x1, 1.f);
      ok(cg_layernorm_fwd(a.x1, w.ln_mlp_w, w.ln_mlp_b, c->eps, a.h2, a.m2, a.r2, int32_t(t.n), int32_t(t.d), st));
      gm.nt(t.n, t.F, t.d, a.h2, w.up_w, a.u);
      ok(cg_add_strided(int32_t(t.n), int32_t(t.F), 1.f, w.up_b, 0, a.u, t.F, st));
      ok(cg_gelu_fwd(a.u, s.g, t.n * t.F, st));
      CG_HIP(hipMemcpyAsync(x_next, a.x1, size_t(t.n * t.d) * 4, hipMemcpyDeviceToDevice, st));
      gm.nt(t.n, t.d, t.F, s.g, w.down_w, x_next, 1.f);
      ok(cg_add_strided(int32_t(t.n), int32_t(t.d), 1.f, w.down_b, 0, x_next, t.d, st));
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
    const TrainDims t = dims_of(*c, n);
    hipStream_t st = as_stream(stream);
    const Scratch s = scratch_of(t, scratch);
    const Gemm gm{s, st};
    const SavedTail tail = saved_tail(t, saved);
    const int32_t N = int32_t(t.n);
    ok(cg_norm_bwd(tail.x_last, dhidden, final_w, tail.mf, tail.rf, s.dx, grads->final_dw, grads->final_db, N,
                   int32_t(t.d), s.red, s.red_bytes, 0, st));
    if (dple) CG_HIP(hipMemsetAsync(dple, 0, size_t(t.n * t.P) * 4, st));
    if (dvalues) CG_HIP(hipMemsetAsync(dvalues, 0, size_t(t.n * t.V) * 4, st));
    for (int64_t l = t.L - 1; l >= 0; --l) {
      const cg_train_block &w = blocks[l];
      const cg_train_block_grads &gw = grads->blocks[l];
      const SavedLayer a = saved_layer(t, saved, l);
      if (dple)
        ple_slices(t.d, t.pd, [&](int64_t off, int64_t width, float scale) {
          ok(cg_add_strided(N, int32_t(width), scale, s.dx + off, t.d, dple + l * t.pd, t.P, st));
        });
      ok(cg_gelu_fwd(a.u, s.g, t.n * t.F, st));
      gm.tn(t.n, t.d, t.F, s.dx, s.g, gw.down_w);
      ok(cg_column_sum(s.dx, N, int32_t(t.d), t.d, gw.down_b, 0, s.red, s.red_bytes, st));
      gm.nn(t.n, t.d, t.F, s.dx, w.down_w, s.dg);
      ok(cg_gelu_bwd(a.u, s.dg, s.du, t.n * t.F, st));
      gm.tn(t.n, t.F, t.d, s.du, a.h2, gw.up_w);
      ok(cg_column_sum(s.du, N, int32_t(t.F), t.F, gw.up_b, 0, s.red, s.red_bytes, st));
      gm.nn(t.n, t.F, t.d, s.du, w.up_w, s.dh);
      ok(cg_norm_bwd(a.x1, s.dh, w.ln_mlp_w, a.m2, a.r2, s.dx1, gw.ln_mlp_w, gw.ln_mlp_b, N, int32_t(t.d), s.red,
                     s.red_bytes, 0, st));
      ok(cg_add_strided(N, int32_t(t.d), 1.f, s.dx, t.d, s.dx1, t.d, st));
      gm.tn(t.n, t.d, t.Q, s.dx1, a.o, gw.out_w);
      gm.nn(t.n, t.d, t.Q, s.dx1, w.out_w, s.dout);
      const cg_attn_train at = attn_args(t, seq_start, tail.seq_of, a.qkv, a.o, a.lse);
      ok(cg_attn_train_bwd(&at, s.dout, s.dsum, s.dqkv, s.dqkv + t.Q, s.dqkv + t.Q + t.KVW, st));
      const int32_t vi = c->value_index ? c->value_index[l] : -1;
      if (vi >= 0 && dvalues)
        ok(cg_add_strided(N, int32_t(t.KVW), 1.f, s.dqkv + t.Q + t.KVW, t.QKV, dvalues + vi * t.KVW, t.V, st));
      gm.tn(t.n, t.QKV, t.d, s.dqkv, a.h1, gw.qkv_w);
      gm.nn(t.n, t.QKV, t.d, s.dqkv, w.qkv_w, s.dh);
      ok(cg_norm_bwd(a.xl, s.dh, w.ln_attn_w, a.m1, a.r1, s.dx, gw.ln_attn_w, gw.ln_attn_b, N, int32_t(t.d), s.red,
                     s.red_bytes, 0, st));
      ok(cg_add_strided(N, int32_t(t.d), 1.f, s.dx1, t.d, s.dx, t.d, st));
    }
    CG_HIP(hipMemcpyAsync(dx, s.dx, size_t(t.n * t.d) * 4, hipMemcpyDeviceToDevice, st));
  });
}

}  // extern "C"
