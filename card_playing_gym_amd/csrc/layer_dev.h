// Device code of the fused per-layer tail (gfx950): the stage plan, LayerNorm statistics,
// GELU, the per-layer parameters staged in LDS and tail_body, the whole tail of one row
// block (launched by layer.hip's layer_tail_kernel).
#pragma once

#include "common.h"
#include "fragment.h"
#include "layer.h"

namespace cg {
namespace {

#ifndef TAIL_RING
#define TAIL_RING 2
#endif
// Stages of weights in flight per wave: two for 16- and 32-row blocks; one for 64-row
// blocks, whose four row tiles per fragment keep each stage's MFMAs busy four times as long
// (and whose accumulators leave no room for a second ring stage).
template <int BM>
constexpr int ring_of() { return BM >= 64 ? 1 : TAIL_RING; }

enum StageKind { ST_OUT, ST_UP, ST_DOWN, ST_QKV };

// MLP stage order.  Blocks of up to 32 rows run every up chunk first (each GELU output to
// its own LDS buffer), one barrier, then every down chunk: one block-wide wait for the MLP
// instead of one per chunk.  64-row blocks interleave up c, down c through two buffers
// (four would not fit in LDS beside the panel).
template <int BM>
constexpr bool ups_first() { return BM <= 32; }
template <int BM>
constexpr int hbufs_of() { return ups_first<BM>() ? 4 : 2; }

struct Plan {
  int nc, nq, n_post, S;
  bool ups_first;
};

__device__ __forceinline__ int stage_kind(const Plan &p, int s, int &chunk) {
  if (s < p.n_post) {
    if (s == 0) {
      chunk = 0;
      return ST_OUT;
    }
    if (p.ups_first) {
      chunk = s - 1 < p.nc ? s - 1 : s - 1 - p.nc;
      return s - 1 < p.nc ? ST_UP : ST_DOWN;
    }
    chunk = (s - 1) >> 1;
    return ((s - 1) & 1) ? ST_DOWN : ST_UP;
  }
  chunk = s - p.n_post;
  return ST_QKV;
}

__device__ __forceinline__ Slice stage_slice(const TailArgs &a, const Plan &p, int s, int cw) {
  int c;
  const int kind = stage_kind(p, s, c);
  const int d = a.d;
  const uint32_t kd = kblocks_of(d), kf = kblocks_of(a.d_ff);
  // Descriptors are rebuilt per stage from laundered pointers: four of them hoisted out of
  // the stage loop would hold 16 scalar registers for the whole kernel.
  if (kind == ST_OUT) return Slice{rsrc(opaque_ptr(a.w_out), uint32_t(d) * kd * 64), kd, cw / 16, 0};
  if (kind == ST_UP)
    return Slice{rsrc(opaque_ptr(a.w_up), uint32_t(a.d_ff) * kd * 64), kd, (PANEL * c + cw) / 16, 0};
  if (kind == ST_DOWN)
    return Slice{rsrc(opaque_ptr(a.w_down), uint32_t(d) * kf * 64), kf, cw / 16, (PANEL / 32) * c};
  return Slice{rsrc(opaque_ptr(a.w_qkv), uint32_t(a.n_qkv) * kd * 64), kd, (PANEL * c + cw) / 16, 0};
}

// LayerNorm statistics of rows held in the MFMA layout: v[i][j][r] is row 16 i + 4 lg + r,
// column cw + 16 j + li (columns >= d hold 0 and are excluded).  Each wave first takes the
// exact two-pass mean and centred sum of squares of its own columns (DPP sums over the
// fragment's 16 lanes, no barrier); then one thread per row merges the waves' (count, mean,
// M2) triples with Chan et al.'s pairwise formula, M2 = sum_w [M2_w + n_w (mean_w - mean)^2],
// and leaves (mean, rstd) in LDS: every lane then reads two values per row instead of
// repeating the merge (sixteen reads per row).  red holds 2 WAVES BM + 2 BM floats.
template <int BM>
__device__ __forceinline__ void row_stats(const f32x4 (&v)[BM / 16][FN], int cw, int d, float eps,
                                          float (&mean)[BM / 16][4], float (&rstd)[BM / 16][4],
                                          float *red, int wave, int li, int lg) {
  constexpr int FM = BM / 16;
  // Columns this wave holds (the same for every row): cw .. cw + 16 FN - 1, capped at d.
  const int nw = max(0, min(16 * FN, d - cw));
  const float inv_nw = nw > 0 ? 1.0f / float(nw) : 0.f;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        if (cw + 16 * j + li < d) sum += v[i][j][r];
      const float mw = sum16(sum) * inv_nw;
      float sq = 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        if (cw + 16 * j + li < d) sq += (v[i][j][r] - mw) * (v[i][j][r] - mw);
      const float m2 = sum16(sq);
      if (li == 0) {
        const int row = 16 * i + 4 * lg + r;
        red[(0 * WAVES + wave) * BM + row] = mw;
        red[(1 * WAVES + wave) * BM + row] = m2;
      }
    }
  lds_barrier();
  float *stat = red + 2 * WAVES * BM;  // [mean | rstd] x BM
  const int tid = threadIdx.x;
  if (tid < BM) {
    const float inv_d = 1.0f / float(d);
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w)
      total = fmaf(float(max(0, min(16 * FN, d - 16 * FN * w))), red[(0 * WAVES + w) * BM + tid], total);
    const float mu = total * inv_d;
    float m2 = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float n = float(max(0, min(16 * FN, d - 16 * FN * w)));
      const float dm = red[(0 * WAVES + w) * BM + tid] - mu;
      m2 += fmaf(n * dm, dm, red[(1 * WAVES + w) * BM + tid]);
    }
    stat[tid] = mu;
    stat[BM + tid] = rsqrtf(m2 * inv_d + eps);
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * i + 4 * lg + r;
      mean[i][r] = stat[row];
      rstd[i][r] = stat[BM + row];
    }
}

// LN(v) -> the panel (bf16, the next QKV stage's A operand), or, for the last block, the
// final norm -> hidden rows of readout tokens.
// Per-layer vectors and the block's token slots, staged in LDS by the kernel prologue.
struct Params {
  float *b_up, *b_down, *ln2_w, *ln2_b, *ln_w, *ln_b;  // [d_ff] and [PANEL] each
  int *tok_row, *tok_pos, *tok_out;                    // [BM] each
};

template <int BM>
__device__ __forceinline__ void next_prologue(const TailArgs &a, const Params &prm, const f32x4 (&v)[BM / 16][FN],
                                              unsigned char *panel, float *red, int m0, int cw,
                                              int wave, int li, int lg) {
  constexpr int FM = BM / 16;
  float mean[FM][4], rstd[FM][4];
  float lw[FN], lb[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = cw + 16 * j + li;
    lw[j] = prm.ln_w[n];
    lb[j] = prm.ln_b[n];
  }
  int out_row[FM][4];
  if (a.final_ln) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) out_row[i][r] = prm.tok_out[16 * i + 4 * lg + r];
  }
  row_stats<BM>(v, cw, a.d, a.eps, mean, rstd, red, wave, li, lg);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = cw + 16 * j + li;
    if (n >= a.d) continue;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * i + 4 * lg + r;
        const float y = fmaf((v[i][j][r] - mean[i][r]) * rstd[i][r], lw[j], lb[j]);
        if (a.final_ln) {
          if (out_row[i][r] >= 0) gst(a.hidden + int64_t(out_row[i][r]) * a.d + n, y);
        } else {
          *reinterpret_cast<bf16 *>(panel + row * ROWB + n * 2) = from_f32<bf16>(y);
        }
      }
  }
  if (!a.final_ln) lds_barrier();
}

__device__ __forceinline__ void store_kv(void *base, int dtype, int64_t index, float v) {
  if (dtype == CG_BF16) gst(static_cast<bf16 *>(base) + index, from_f32<bf16>(v));
  else if (dtype == CG_F16) gst(static_cast<f16 *>(base) + index, from_f32<f16>(v));
  else gst(static_cast<float *>(base) + index, v);
}

// MODE: 0 = first block's prologue (x = x_src, LN + QKV), 1 = post + next QKV, 2 = post +
// final norm.  NC / NQ: 256-wide chunks of d_ff / of the QKV width.  The stage sequence is
// a compile-time constant, so the fully unrolled stage loop folds every stage's kind and
// the weight registers flow from stage to stage without merges.
// Row block `blk` of one layer tail.  LDS: panel [BM rows of ROWB bytes], hbuf two or four more,
// red 2 * WAVES * BM + 2 * BM floats, dyn the Params (d_ff + 5 PANEL floats, then 3 BM ints).
template <int BM, int MODE, int NC, int NQ>
__device__ __forceinline__ void tail_body(const TailArgs &a, int blk, unsigned char *panel,
                                          unsigned char (*hbuf)[BM * ROWB], float *red, float *dyn) {
  constexpr int FM = BM / 16;
  constexpr int RING = ring_of<BM>();
  constexpr bool POST = MODE != 0, FINAL = MODE == 2;

  // The wave index is uniform: readfirstlane keeps its derived column ranges scalar.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cw = 16 * FN * wave;
  const int d = a.d;
  constexpr int N_POST = POST ? 1 + 2 * NC : 0;
  constexpr int S = N_POST + (FINAL ? 0 : NQ);
  Plan p;
  p.nc = NC;
  p.nq = FINAL ? 0 : NQ;
  p.n_post = N_POST;
  p.S = S;
  p.ups_first = ups_first<BM>();
  constexpr int HB = hbufs_of<BM>();
  static_assert(!ups_first<BM>() || NC <= HB, "one GELU buffer per d_ff chunk");
  const uint32_t xbytes = uint32_t(a.M) * uint32_t(d) * 4;

  // Prologue loads, issued before the weight stream (loads complete in order, so anything
  // issued after the ring's fragment loads would wait for them): this block's attention
  // rows (16-byte chunks, FM per thread at most) and the per-layer vectors.
  static_assert(BM * (PANEL / 8) <= FM * THREADS, "FM attention chunks per thread");
  const int m0_ = blk * BM;
  const int cpr = d / 8;
  uint4 arow[FM];
#pragma unroll
  for (int k = 0; k < FM; ++k) {
    const int c = tid + k * THREADS;
    arow[k] = uint4{0u, 0u, 0u, 0u};
    if (POST && c < BM * cpr) {
      const Rsrc ra = rsrc(a.attn, uint32_t(a.M) * uint32_t(d) * 2);
      arow[k] = bload16(ra, (uint32_t(m0_ + c / cpr) * d + 8 * (c % cpr)) * 2);
    }
  }
  constexpr int NB_UP = (4 * PANEL + THREADS - 1) / THREADS;
  float v_up[NB_UP], v_vec[5];
  int v_tok[3];
#pragma unroll
  for (int k = 0; k < NB_UP; ++k) {
    const int i = tid + k * THREADS;
    v_up[k] = POST && i < a.d_ff ? a.b_up[i] : 0.f;
  }
  {
    const bool in = tid < d;
    v_vec[0] = POST && in ? a.b_down[tid] : 0.f;
    v_vec[1] = POST && in ? a.ln2_w[tid] : 0.f;
    v_vec[2] = POST && in ? a.ln2_b[tid] : 0.f;
    v_vec[3] = in ? a.ln_w[tid] : 0.f;
    v_vec[4] = in ? a.ln_b[tid] : 0.f;
    const bool tin = tid < BM && m0_ + tid < a.M;
    v_tok[0] = tin && !a.final_ln ? a.tok_row[m0_ + tid] : -1;
    v_tok[1] = tin && !a.final_ln ? a.tok_pos[m0_ + tid] : 0;
    v_tok[2] = tin && a.final_ln ? a.tok_out[m0_ + tid] : -1;
  }

  // RING stages of weights in flight: stage s computes from wbuf[s % RING] and refills it
  // with stage s + RING's fragments (the stage sequence is unrolled, so the index is
  // static), so the weight stream keeps running through the epilogues' barriers.
  uint4 wbuf[RING][KS][FN];
#pragma unroll
  for (int r = 0; r < RING; ++r)
    if (S > r) load_slice(wbuf[r], stage_slice(a, p, r, cw), lane);

  Params prm;
  prm.b_up = dyn;
  prm.b_down = dyn + a.d_ff;
  prm.ln2_w = prm.b_down + PANEL;
  prm.ln2_b = prm.ln2_w + PANEL;
  prm.ln_w = prm.ln2_b + PANEL;
  prm.ln_b = prm.ln_w + PANEL;
  prm.tok_row = reinterpret_cast<int *>(prm.ln_b + PANEL);
  prm.tok_pos = prm.tok_row + BM;
  prm.tok_out = prm.tok_pos + BM;

  // Zero the LDS panels once: padding columns (k >= d, or past d_ff) stay zero.
  for (int o = tid * 16; o < BM * ROWB; o += THREADS * 16) {
    const uint4 z = {0u, 0u, 0u, 0u};
    *reinterpret_cast<uint4 *>(panel + o) = z;
#pragma unroll
    for (int h = 0; h < HB; ++h) *reinterpret_cast<uint4 *>(hbuf[h] + o) = z;
  }
#pragma unroll
  for (int k = 0; k < NB_UP; ++k) {
    const int i = tid + k * THREADS;
    if (i < a.d_ff) prm.b_up[i] = v_up[k];
  }
  if (tid < PANEL) {
    prm.b_down[tid] = v_vec[0];
    prm.ln2_w[tid] = v_vec[1];
    prm.ln2_b[tid] = v_vec[2];
    prm.ln_w[tid] = v_vec[3];
    prm.ln_b[tid] = v_vec[4];
  }
  if (tid < BM) {
    prm.tok_row[tid] = v_tok[0];
    prm.tok_pos[tid] = v_tok[1];
    prm.tok_out[tid] = v_tok[2];
  }
  lds_barrier();

  f32x4 acc[FM][FN], accd[FM][FN];
  zero<FM>(accd);
  {
    const int m0 = blk * BM;
    const int li = lane & 15, lg = lane >> 4;
    if (POST) {
      // Attention rows of this block -> panel (rows past M read as 0).
#pragma unroll
      for (int k = 0; k < FM; ++k) {
        const int c = tid + k * THREADS;
        if (c < BM * cpr) *reinterpret_cast<uint4 *>(panel + (c / cpr) * ROWB + 16 * (c % cpr)) = arow[k];
      }
      lds_barrier();
    } else {
      // First block's prologue: the conditioned input is the residual stream.
      const Rsrc rs = rsrc(a.x_src, xbytes);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * lg + r, n = cw + 16 * j + li;
            const float v = bloadf(rs, (uint32_t(m) * d + n) * 4);
            const bool ok = m < a.M && n < d;
            if (ok && a.x != a.x_src) gst(a.x + int64_t(m) * d + n, v);
            acc[i][j][r] = ok ? v : 0.f;
          }
      next_prologue<BM>(a, prm, acc, panel, red, m0, cw, wave, li, lg);
    }
  }

#pragma clang loop unroll(full)
  for (int s = 0; s < S; ++s) {
    const int m0 = opaque(blk * BM);
    const int lane_o = opaque_lane(lane);
    const int li = lane_o & 15, lg = lane_o >> 4;
    int c;
    const int kind = stage_kind(p, s, c);
    const bool refill = s + RING < S;
    const Slice nx = stage_slice(a, p, refill ? s + RING : s, cw);
    uint4(&cur)[KS][FN] = wbuf[s % RING];
    if (kind == ST_OUT) {
      // ---- out-proj + residual, then LN(ln_mlp) -> panel
      const Rsrc rs = rsrc(opaque_ptr(a.x_src), xbytes);
      float xr[FM][FN][4], lw[FN], lb[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = cw + 16 * j + li;
        lw[j] = prm.ln2_w[n];
        lb[j] = prm.ln2_b[n];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) xr[i][j][r] = bloadf(rs, (uint32_t(m0 + 16 * i + 4 * lg + r) * d + n) * 4);
      }
      // Issue the residual loads ahead of this stage's weight refills: loads complete in
      // order, so the epilogue then waits only for them, not for the next stage's weights.
      __builtin_amdgcn_sched_barrier(0);
      zero<FM>(acc);
      stage_mma<FM>(acc, panel, cur, nx, refill, lane_o);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * lg + r, n = cw + 16 * j + li;
            float v = 0.f;
            if (m < a.M && n < d) {
              v = acc[i][j][r] + xr[i][j][r];
              gst(a.x + int64_t(m) * d + n, v);
            }
            acc[i][j][r] = v;
          }
      float mean[FM][4], rstd[FM][4];
      row_stats<BM>(acc, cw, d, a.eps, mean, rstd, red, wave, li, lg);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = cw + 16 * j + li;
        if (n >= d) continue;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = 16 * i + 4 * lg + r;
            const float y = fmaf((acc[i][j][r] - mean[i][r]) * rstd[i][r], lw[j], lb[j]);
            *reinterpret_cast<bf16 *>(panel + row * ROWB + n * 2) = from_f32<bf16>(y);
          }
      }
      lds_barrier();
    } else if (kind == ST_UP) {
      // ---- up chunk c + GELU -> hbuf[c & 1]
      float bias[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = PANEL * c + cw + 16 * j + li;
        bias[j] = n < a.d_ff ? prm.b_up[n] : 0.f;
      }
      zero<FM>(acc);
      stage_mma<FM>(acc, panel, cur, nx, refill, lane_o);
      unsigned char *hb = hbuf[p.ups_first ? c : (c & 1)];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = cw + 16 * j + li;
        const bool ok = PANEL * c + col < a.d_ff;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = 16 * i + 4 * lg + r;
            const float g = ok ? gelu_fast(acc[i][j][r] + bias[j]) : 0.f;
            *reinterpret_cast<bf16 *>(hb + row * ROWB + col * 2) = from_f32<bf16>(g);
          }
      }
      // Down chunk c reads every wave's columns of GELU chunk c.
      if (!p.ups_first || c == p.nc - 1) lds_barrier();
    } else if (kind == ST_DOWN) {
      // ---- down chunk c (accumulates); after the last: residual (+PLE), next prologue
      const bool last = c == p.nc - 1;
      float xr[FM][FN][4], bias[FN];
      if (last) {
        const Rsrc rx = rsrc(opaque_ptr(a.x), xbytes);
        const Rsrc rp = rsrc(opaque_ptr(a.ple), a.ple ? uint32_t(a.M) * uint32_t(a.ld_ple) * 4 : 0u);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = cw + 16 * j + li;
          bias[j] = prm.b_down[n];
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t m = uint32_t(m0 + 16 * i + 4 * lg + r);
              float v = bloadf(rx, (m * d + n) * 4);
              if (a.ple)
                v = fmaf(bloadf(rp, (m * uint32_t(a.ld_ple) + a.ple_off + n % a.ple_dim) * 4), a.ple_scale, v);
              xr[i][j][r] = v;
            }
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // residual loads ahead of the weight refills
      stage_mma<FM>(accd, hbuf[p.ups_first ? c : (c & 1)], cur, nx, refill, lane_o);
      if (last) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = cw + 16 * j + li;
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int m = m0 + 16 * i + 4 * lg + r;
              float v = 0.f;
              if (m < a.M && n < d) {
                v = xr[i][j][r] + accd[i][j][r] + bias[j];
                gst(a.x + int64_t(m) * d + n, v);
              }
              accd[i][j][r] = v;
            }
        }
        next_prologue<BM>(a, prm, accd, panel, red, m0, cw, wave, li, lg);
      }
    } else {
      // ---- qkv chunk: q stored, k / v appended to the pool
      int trow[FM][4], tpos[FM][4];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          trow[i][r] = prm.tok_row[16 * i + 4 * lg + r];
          tpos[i][r] = prm.tok_pos[16 * i + 4 * lg + r];
        }
      zero<FM>(acc);
      stage_mma<FM>(acc, panel, cur, nx, refill, lane_o);
      // Per output column: its role (q / k / v / none) and, for k and v, the offset of its
      // (head, dim) inside a pool slot row; per token row: the slot's base offset.
      const int kvw = a.kv_heads * a.head_dim;
      int role[FN], col[FN];
      int64_t coff[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = PANEL * c + cw + 16 * j + li;
        role[j] = n >= a.n_qkv ? -1 : (n < a.q_cols ? 0 : (n < a.q_cols + kvw ? 1 : 2));
        const int kvc = n - a.q_cols - (role[j] == 2 ? kvw : 0);
        const int h = kvc / a.head_dim;
        col[j] = role[j] == 0 ? n : kvc;
        coff[j] = int64_t(h) * a.max_len * a.head_dim + (kvc - h * a.head_dim);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * i + 4 * lg + r;
          if (m >= a.M) continue;
          const int64_t slot = (int64_t(trow[i][r]) * a.kv_heads * a.max_len + tpos[i][r]) * a.head_dim;
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const float v = acc[i][j][r];
            if (role[j] == 0) {
              store_kv(a.q, a.q_dtype, int64_t(m) * a.q_cols + col[j], v);
            } else if (role[j] > 0 && trow[i][r] >= 0) {
              float val = v;
              if (role[j] == 2 && a.vemb_off >= 0) val += a.vemb[int64_t(m) * a.ld_vemb + a.vemb_off + col[j]];
              store_kv(role[j] == 2 ? a.vc : a.kc, a.kv_dtype, slot + coff[j], val);
            }
          }
        }
    }
  }
}



}  // namespace
}  // namespace cg
