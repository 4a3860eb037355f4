// Device code of the fused per-layer tail (gfx950): the stage plan, LayerNorm statistics,
// GELU, the per-layer parameters staged in LDS and tail_body, the whole tail of one row
// block (launched by layer.hip's layer_tail_kernel).
//
// Every stage product is formed transposed, out^T = W . A^T: the weight fragment is the
// MFMA's A operand and the LDS panel fragment its B operand (both keep the layouts the
// untransposed product uses, so the fragment-order weights are the same).  Lane (li, lg)
// of row tile i and column tile j then holds row 16 i + li at the four consecutive columns
// cw + 16 j + 4 lg .. +3, so every epilogue works on 16-byte runs of one row: residual rows
// load and store as float4, GELU / LayerNorm outputs go to LDS as one 8-byte write, q and
// the appended K / V leave as one 16- or 8-byte store per run, and a row's LayerNorm sums
// need two lane swaps (the four lane groups) instead of a 16-lane DPP reduction.
#pragma once

#include "common.h"
#include "fragment.h"
#include "layer.h"

namespace cg {
namespace {

#ifndef TAIL_RING
#define TAIL_RING 1
#endif
// Stages of weights in flight per wave beyond the one being multiplied.  One is enough:
// measured with two (128 more VGPRs per wave) against one, the kernel ran 21.5 / 21.3 us per
// decode layer (16 rows), 28.5 / 28.4 at 32 rows and 100.6 / 99.0 at 48 (the weight stream
// is bound by the L1 return path, not by the loads in flight); 64-row blocks have no room
// for two.
template <int BM>
constexpr int ring_of() { return BM > 48 ? 1 : TAIL_RING; }

enum StageKind { ST_OUT, ST_UP, ST_DOWN, ST_QKV };

// MLP stage order.  Blocks of up to 48 rows run every up chunk first (each GELU output to
// its own LDS buffer), one barrier, then every down chunk: one block-wide wait for the MLP
// instead of one per chunk; from 32 rows each chunk's GELU runs inside the next up chunk's
// k-steps, beside its MFMAs.  64-row blocks interleave up c, down c through two buffers (four would
// not fit in LDS beside the panel); a taller block would use one, with a barrier before each
// GELU chunk overwrites the one the last down chunk read.
template <int BM>
constexpr bool ups_first() { return BM <= 48; }
// The previous up chunk's GELU inside the next one's k-steps: measured faster at 32 rows
// (config 4: 1.787 -> 1.731 ms per step) and 48 (config 5: 2.805 -> 2.788), slower at 16
// (config 3: 1.140 -> 1.168), where a stage has two MFMAs per k-step to hide work behind.
template <int BM>
constexpr bool gelu_pipelined() { return ups_first<BM>() && BM >= 32; }
template <int BM>
constexpr int hbufs_of() { return ups_first<BM>() ? 4 : (BM <= 64 ? 2 : 1); }

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

// Weight fragment loads (cache-policy bits of the buffer instruction: 1 sc0, 2 nt).
#ifndef CG_W_CPOL
#define CG_W_CPOL 0
#endif
__device__ __forceinline__ uint4 wload16(Rsrc r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CG_W_CPOL);
  return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ void load_wslice(uint4 (&buf)[KS][FN], const Slice &s, int lane) {
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const uint32_t base = slice_base(s, j, lane);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) buf[ks][j] = wload16(s.w, base + 1024 * ks);
  }
}

// acc[i][j] += (W fragment j) x (panel rows 16 i + li)^T over all 256 k: the product of
// stage_mma (fragment.h) with the operands swapped, so the result tile is transposed
// (lane (li, lg) holds row 16 i + li, columns 4 lg .. +3 of the 16-column fragment j).
// The weight registers are refilled with the next stage's fragments as in stage_mma.
// `between(ks)` runs after k-step ks's MFMAs and refills are issued: independent VALU work
// (the previous up chunk's GELU) placed there executes while the matrix core multiplies.
struct NoWork {
  __device__ __forceinline__ void operator()(int) const {}
};
template <int FM, typename Between = NoWork>
__device__ __forceinline__ void stage_mma_t(f32x4 (&acc)[FM][FN], const unsigned char *lds,
                                            uint4 (&w)[KS][FN], const Slice &next, bool refill, int lane,
                                            Between between = NoWork{}) {
  const int li = lane & 15, lg = lane >> 4;
  uint32_t base[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) base[j] = slice_base(next, j, lane);
  auto a_frag = [&](int ks, int i) {
    return *reinterpret_cast<const uint4 *>(lds + (16 * i + li) * ROWB + (32 * ks + 8 * lg) * 2);
  };
  if constexpr (FM == 1) {
    uint4 af[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) af[ks] = a_frag(ks, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[0][j] = mma(w[ks][j], af[ks], acc[0][j]);
      if (refill) {
#pragma unroll
        for (int j = 0; j < FN; ++j) w[ks][j] = wload16(next.w, base[j] + 1024 * ks);
      }
      pin_refill();
      between(ks);
    }
  } else {
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
        for (int j = 0; j < FN; ++j) acc[i][j] = mma(w[ks][j], af[ks & 1][i], acc[i][j]);
      if (refill) {
#pragma unroll
        for (int j = 0; j < FN; ++j) w[ks][j] = wload16(next.w, base[j] + 1024 * ks);
      }
      pin_refill();
      between(ks);
    }
  }
}

// Sum over the four lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48): the columns of one row.
// v_permlane16/32_swap hand each lane its partner's value beside its own.
__device__ __forceinline__ float lane_groups_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Four values rounded to bf16 (nearest even; two v_cvt_pk_bf16_f32) as 8 bytes.  For the
// LDS panels only: a NaN keeps whatever quiet-NaN pattern the instruction gives.
__device__ __forceinline__ u32x2 pack_bf16x4(f32x4 v) {
  const bf16x4 h = __builtin_convertvector(v, bf16x4);
  return __builtin_bit_cast(u32x2, h);
}

__device__ __forceinline__ void st_nt(float *p, f32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(p)); }
__device__ __forceinline__ void st_nt(void *p, u32x2 v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x2 *>(p)); }

__device__ __forceinline__ f32x4 bload4f(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ f32x4 lds4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }

// Four consecutive values of `dtype` (fp32, bf16 or fp16) stored at p (aligned to their size):
// the 16-bit types through cvt4, the conversion cg_kv_write_step's stores use as well.
__device__ __forceinline__ void store4(void *p, int dtype, f32x4 v) {
  if (dtype == CG_BF16) st_nt(p, cvt4<bf16>(v));
  else if (dtype == CG_F16) st_nt(p, cvt4<f16>(v));
  else st_nt(static_cast<float *>(p), v);
}

// LayerNorm statistics of rows held transposed: v[i][j] is row 16 i + li at columns
// cw + 16 j + 4 lg .. +3 (16-column tiles at or past d hold 0 and are excluded).  Each wave
// first takes the exact two-pass mean and centred sum of squares of its own columns (in-lane
// sums, then the four lane groups); then one thread per row merges the waves' (count, mean,
// M2) triples with Chan et al.'s pairwise formula, M2 = sum_w [M2_w + n_w (mean_w - mean)^2],
// and leaves (mean, rstd) in LDS for every lane to read.  red holds 2 WAVES BM + 2 BM floats.
template <int BM>
__device__ __forceinline__ void row_stats_t(const f32x4 (&v)[BM / 16][FN], int cw, int d, float eps,
                                            float (&mean)[BM / 16], float (&rstd)[BM / 16], float *red,
                                            int wave, int li, int lg) {
  constexpr int FM = BM / 16;
  const int nw = max(0, min(16 * FN, d - cw));
  // Reciprocals of the column counts: exact for the powers of two of the usual widths.
  const float inv_nw = nw > 0 ? __builtin_amdgcn_rcpf(float(nw)) : 0.f;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      if (cw + 16 * j < d) sum += (v[i][j][0] + v[i][j][1]) + (v[i][j][2] + v[i][j][3]);
    const float mw = lane_groups_sum(sum) * inv_nw;
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      if (cw + 16 * j < d) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sq = fmaf(v[i][j][r] - mw, v[i][j][r] - mw, sq);
      }
    const float m2 = lane_groups_sum(sq);
    if (lg == 0) {
      red[(0 * WAVES + wave) * BM + 16 * i + li] = mw;
      red[(1 * WAVES + wave) * BM + 16 * i + li] = m2;
    }
  }
  lds_barrier();
  float *stat = red + 2 * WAVES * BM;  // [mean | rstd] x BM
  const int tid = threadIdx.x;
  if (tid < BM) {
    const float inv_d = __builtin_amdgcn_rcpf(float(d));
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
  for (int i = 0; i < FM; ++i) {
    mean[i] = stat[16 * i + li];
    rstd[i] = stat[BM + 16 * i + li];
  }
}

// Per-layer vectors, the QKV column map and the block's token slots, staged in LDS by the
// kernel prologue (layout: params_floats / params_bytes below).
struct Params {
  float *b_up, *b_down, *ln2_w, *ln2_b, *ln_w, *ln_b;  // [NC PANEL] (0 past d_ff) and [PANEL] each
  int2 *qkv_map;     // [3 PANEL / 4]: per run of four QKV columns {role (0 q, 1 k, 2 v, -1 none),
                     // offset (q: column; k / v: element offset inside a pool slot row)}
  int64_t *tok_slot;  // [BM]: element offset of the token's pool slot (head 0), -1: no write
  int *tok_out;       // [BM]
};

// LN(v; w, b) of the held rows -> the panel (bf16, the next stage's B operand).
template <int BM>
__device__ __forceinline__ void ln_to_panel(const f32x4 (&v)[BM / 16][FN], const float (&mean)[BM / 16],
                                            const float (&rstd)[BM / 16], const float *w, const float *b,
                                            unsigned char *panel, int cw, int d, int li, int lg) {
  constexpr int FM = BM / 16;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    if (cw + 16 * j >= d) continue;
    const int c0 = cw + 16 * j + 4 * lg;
    const f32x4 lw = lds4(w + c0), lb = lds4(b + c0);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      f32x4 y;
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = fmaf((v[i][j][r] - mean[i]) * rstd[i], lw[r], lb[r]);
      *reinterpret_cast<u32x2 *>(panel + (16 * i + li) * ROWB + c0 * 2) = pack_bf16x4(y);
    }
  }
}

// The next block's LayerNorm of the residual rows -> the panel, or, for the last block, the
// final norm -> hidden rows of readout tokens.
template <int BM>
__device__ __forceinline__ void next_prologue(const TailArgs &a, const Params &prm, const f32x4 (&v)[BM / 16][FN],
                                              unsigned char *panel, float *red, int cw, int wave, int li, int lg) {
  constexpr int FM = BM / 16;
  float mean[FM], rstd[FM];
  row_stats_t<BM>(v, cw, a.d, a.eps, mean, rstd, red, wave, li, lg);
  if (!a.final_ln) {
    ln_to_panel<BM>(v, mean, rstd, prm.ln_w, prm.ln_b, panel, cw, a.d, li, lg);
    lds_barrier();
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int out_row = prm.tok_out[16 * i + li];
    if (out_row < 0) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if (cw + 16 * j >= a.d) continue;
      const int c0 = cw + 16 * j + 4 * lg;
      const f32x4 lw = lds4(prm.ln_w + c0), lb = lds4(prm.ln_b + c0);
      f32x4 y;
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = fmaf((v[i][j][r] - mean[i]) * rstd[i], lw[r], lb[r]);
      float *dst = a.hidden + int64_t(out_row) * a.d + c0;
      if (a.hidden_vec) {
        st_nt(dst, y);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) gst(dst + r, y[r]);
      }
    }
  }
}

// A readout offset as torch indexing reads it (trunk.py:429): negative offsets count from
// the end of the sequence's len tokens; -1 when outside.
__device__ __forceinline__ int64_t readout_index(int64_t o, int64_t len) {
  if (o < 0) o += len;
  return o >= 0 && o < len ? o : -1;
}
// Token i of the step: (cache row or -1, clamped write position, output row or -1), as the
// reference writes it (trunk.py:417-420, kv_cache.py:84-105).  Rows outside the pool and
// negative positions are neither written nor attended and set their status word.
__device__ __forceinline__ void plan_token(const TailArgs &a, int i, int &row_out, int &pos_out, int &out_row) {
  int b, t;
  if (a.seq_start) {
    int lo = 0, hi = a.n_seqs - 1;  // last b with seq_start[b] <= i
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.seq_start[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    b = lo;
    t = int(i - a.seq_start[b]);
  } else {
    b = a.T == 1 ? i : i / a.T;
    t = i - b * a.T;
  }
  const int64_t row = a.rows ? a.rows[b] : int64_t(b);
  const int64_t p0 = a.positions[b];
  int64_t pos = p0 + t;
  if (pos > a.max_len - 1) pos = a.max_len - 1;
  const bool row_ok = row >= 0 && row < a.capacity, pos_ok = p0 >= 0;
  row_out = row_ok && pos_ok ? int(row) : -1;
  pos_out = row_ok && pos_ok ? int(pos) : 0;
  if (a.status && !row_ok) a.status[0] = 1;
  if (a.status && !pos_ok) a.status[1] = 1;
  if (a.readout) {
    const int64_t len = a.seq_start ? a.seq_start[b + 1] - a.seq_start[b] : int64_t(a.T);
    out_row = readout_index(a.readout[b], len) == t ? b : -1;
  } else {
    out_row = i;
  }
}

// MODE: 0 = first block's prologue (x = x_src, LN + QKV), 1 = post + next QKV, 2 = post +
// final norm.  NC / NQ: 256-wide chunks of d_ff / of the QKV width.  The stage sequence is
// a compile-time constant, so the fully unrolled stage loop folds every stage's kind and
// the weight registers flow from stage to stage without merges.
// Row block `blk` of one layer tail.  LDS: panel [BM rows of ROWB bytes], hbuf two or four more,
// red 2 * WAVES * BM + 2 * BM floats, dyn the Params ((NC + 5) PANEL floats, the QKV map, then 3 BM ints).
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
  // The residual rows the out-projection adds (the lane's own transposed tiles) are read
  // here too, so their latency overlaps the attention rows' instead of following it.
  // The first block's input rows (its embedding rows, or the conditioned rows) are read here
  // as well.
  f32x4 xr[FM][FN];
  bool id_ok[FM];
  {
    const int li = lane & 15, lg = lane >> 4;
    if (POST) {
      const Rsrc rs = rsrc(a.x_src, xbytes);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          xr[i][j] = bload4f(rs, (uint32_t(m0_ + 16 * i + li) * d + cw + 16 * j + 4 * lg) * 4);
    } else if (a.embed_table) {
      const Rsrc rt = rsrc(a.embed_table, uint32_t(a.vocab) * uint32_t(d) * 4);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0_ + 16 * i + li;
        const int64_t id = m < a.M ? a.ids[m] : 0;
        id_ok[i] = m < a.M && id >= 0 && id < a.vocab;
#pragma unroll
        for (int j = 0; j < FN; ++j)
          xr[i][j] = bload4f(rt, uint32_t((id_ok[i] ? id : 0) * d + cw + 16 * j + 4 * lg) * 4);
      }
    } else {
      const Rsrc rs = rsrc(a.x_src, xbytes);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const uint32_t off = (uint32_t(m0_ + 16 * i + li) * d + cw + 16 * j + 4 * lg) * 4;
          if (a.x_src_vec) {
            xr[i][j] = bload4f(rs, off);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) xr[i][j][r] = bloadf(rs, off + 4 * r);
          }
        }
    }
  }
  constexpr int NB_UP = (4 * PANEL + THREADS - 1) / THREADS;
  float v_up[NB_UP], v_vec[5];
  int v_tok[3];
  int2 v_map = int2{-1, 0};
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
    if (!POST && a.plan) {
      // The step's plan, formed here for this block's tokens and sequences.
      v_tok[0] = -1;
      v_tok[1] = 0;
      v_tok[2] = -1;
      if (tin) {
        const int i = m0_ + tid;
        plan_token(a, i, v_tok[0], v_tok[1], v_tok[2]);
        a.plan_row[i] = v_tok[0];
        a.plan_pos[i] = v_tok[1];
        a.plan_out[i] = v_tok[2];
        if (a.final_ln) v_tok[0] = -1;
      }
      const int sq = m0_ + tid;
      if (tid < BM && a.readout && sq < a.n_seqs) {
        const int64_t start = a.seq_start ? a.seq_start[sq] : int64_t(sq) * a.T;
        const int64_t stop = a.seq_start ? a.seq_start[sq + 1] : start + a.T;
        if (readout_index(a.readout[sq], stop - start) < 0) {
          if (a.status) a.status[2] = 1;
          if (a.hidden)
            for (int k = 0; k < d; ++k) a.hidden[int64_t(sq) * d + k] = 0.f;
        }
      }
    } else {
      v_tok[0] = tin && !a.final_ln ? a.tok_row[m0_ + tid] : -1;
      v_tok[1] = tin && !a.final_ln ? a.tok_pos[m0_ + tid] : 0;
      v_tok[2] = tin && a.final_ln ? a.tok_out[m0_ + tid] : -1;
    }
    // QKV column runs: role and offset of columns 4 tid .. +3 (head_dim is a multiple of 4).
    const int n = 4 * tid, kvw = a.kv_heads * a.head_dim;
    if (!a.final_ln && n < a.n_qkv) {
      if (n < a.q_cols) {
        v_map = int2{0, n};
      } else {
        const int role = n < a.q_cols + kvw ? 1 : 2;
        const int kvc = n - a.q_cols - (role == 2 ? kvw : 0);
        const int h = kvc / a.head_dim;
        v_map = int2{role, h * a.max_len * a.head_dim + (kvc - h * a.head_dim)};
      }
    }
  }

  // RING stages of weights in flight: stage s computes from wbuf[s % RING] and refills it
  // with stage s + RING's fragments (the stage sequence is unrolled, so the index is
  // static), so the weight stream keeps running through the epilogues' barriers.
  uint4 wbuf[RING][KS][FN];
#pragma unroll
  for (int r = 0; r < RING; ++r)
    if (S > r) load_wslice(wbuf[r], stage_slice(a, p, r, cw), lane);

  Params prm;
  prm.b_up = dyn;
  prm.b_down = dyn + NC * PANEL;  // b_up holds NC full chunks, zero past d_ff
  prm.ln2_w = prm.b_down + PANEL;
  prm.ln2_b = prm.ln2_w + PANEL;
  prm.ln_w = prm.ln2_b + PANEL;
  prm.ln_b = prm.ln_w + PANEL;
  prm.qkv_map = reinterpret_cast<int2 *>(prm.ln_b + PANEL);
  prm.tok_slot = reinterpret_cast<int64_t *>(prm.qkv_map + 3 * PANEL / 4);
  prm.tok_out = reinterpret_cast<int *>(prm.tok_slot + BM);

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
    if (i < NC * PANEL) prm.b_up[i] = v_up[k];  // v_up is 0 past d_ff
  }
  if (tid < PANEL) {
    prm.b_down[tid] = v_vec[0];
    prm.ln2_w[tid] = v_vec[1];
    prm.ln2_b[tid] = v_vec[2];
    prm.ln_w[tid] = v_vec[3];
    prm.ln_b[tid] = v_vec[4];
  }
  if (tid < 3 * PANEL / 4) prm.qkv_map[tid] = v_map;
  if (tid < BM) {
    prm.tok_slot[tid] = v_tok[0] < 0 ? int64_t(-1)
                                     : (int64_t(v_tok[0]) * a.kv_heads * a.max_len + v_tok[1]) * a.head_dim;
    prm.tok_out[tid] = v_tok[2];
  }
  lds_barrier();

  // x1 (the residual after the out-projection) stays in registers: the down projection's
  // chunks accumulate onto it (accd starts as x1), so it is never written to or read back
  // from memory and needs no registers of its own.
  f32x4 acc[FM][FN], accd[FM][FN];
  f32x4 prev[FM][FN];  // the previous up chunk's accumulators, before its GELU
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
      if (a.embed_table) {
        // ... formed here: the token's embedding row (read in the prologue) through the input
        // RMSNorm (trunk.py:104-115, rms_norm(x.float(), eps) * weight; fp32 rows, no rounding).
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int m = m0 + 16 * i + li;
          if (m < a.M && !id_ok[i] && a.status) a.status[3] = 1;
          float sq = 0.f;
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            f32x4 v = xr[i][j];
            if (!(id_ok[i] && cw + 16 * j < d)) v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < 4; ++r) sq = fmaf(v[r], v[r], sq);
            acc[i][j] = v;
          }
          sq = lane_groups_sum(sq);
          if (lg == 0) red[wave * BM + 16 * i + li] = sq;
        }
        lds_barrier();
        float *rms = red + 2 * WAVES * BM;
        if (tid < BM) {
          float total = 0.f;
#pragma unroll
          for (int w = 0; w < WAVES; ++w) total += red[w * BM + tid];
          rms[tid] = rsqrtf(total / float(d) + a.in_eps);
        }
        lds_barrier();
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int m = m0 + 16 * i + li;
          const float r = rms[16 * i + li];
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const int c0 = cw + 16 * j + 4 * lg;
            if (cw + 16 * j >= d) continue;
            const f32x4 g = *reinterpret_cast<const f32x4 *>(a.in_gain + c0);
            f32x4 x;
#pragma unroll
            for (int q = 0; q < 4; ++q) x[q] = acc[i][j][q] * r * g[q];
            acc[i][j] = x;
            if (m < a.M) st_nt(a.x + int64_t(m) * d + c0, x);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const int m = m0 + 16 * i + li, c0 = cw + 16 * j + 4 * lg;
            f32x4 v = xr[i][j];
            const bool ok = m < a.M && cw + 16 * j < d;
            if (!ok) v = f32x4{0.f, 0.f, 0.f, 0.f};
            if (ok && a.x != a.x_src) st_nt(a.x + int64_t(m) * d + c0, v);
            acc[i][j] = v;
          }
      }
      next_prologue<BM>(a, prm, acc, panel, red, cw, wave, li, lg);
    }
  }

#pragma clang loop unroll(full)
  for (int s = 0; s < S; ++s) {
    // Row and lane offsets are formed once and kept (172 VGPRs at 16 rows): re-forming them
    // in every stage through opaque() cost ~130 VALU instructions per wave and 1.8 %.
    const int m0 = blk * BM;
    const int lane_o = lane;
    const int li = lane_o & 15, lg = lane_o >> 4;
    int c;
    const int kind = stage_kind(p, s, c);
    const bool refill = s + RING < S;
    const Slice nx = stage_slice(a, p, refill ? s + RING : s, cw);
    uint4(&cur)[KS][FN] = wbuf[s % RING];
    if (kind == ST_OUT) {
      // ---- out-proj + residual (x1, kept; xr was read in the prologue and seeds the
      //      accumulators), then LN(ln_mlp) -> panel
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = xr[i][j];
      stage_mma_t<FM>(acc, panel, cur, nx, refill, lane_o);
      // Rows past M are exactly 0 already (their residual and attention rows read past the
      // buffers); columns past d read a neighbouring row's residual and are cleared (uniform).
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          accd[i][j] = acc[i][j];
          if (cw + 16 * j >= d) accd[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      float mean[FM], rstd[FM];
      row_stats_t<BM>(accd, cw, d, a.eps, mean, rstd, red, wave, li, lg);
      ln_to_panel<BM>(accd, mean, rstd, prm.ln2_w, prm.ln2_b, panel, cw, d, li, lg);
      lds_barrier();
    } else if (kind == ST_UP) {
      // ---- up chunk c (the bias seeds the accumulators) + GELU -> hbuf[c] (or hbuf[c & 1]
      //      when interleaved).  Columns past d_ff (a partial last chunk) must stay exactly 0:
      //      the down projection's fragments for those k are not zero.  Their weight loads
      //      read past the buffer (0) and the staged bias is 0 there, so GELU(0) = 0.
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const f32x4 bias = lds4(prm.b_up + PANEL * c + cw + 16 * j + 4 * lg);
#pragma unroll
        for (int i = 0; i < FM; ++i) acc[i][j] = bias;
      }
      // GELU of the bf16 Linear output (rounded to nearest even first, as autocast's Linear
      // returns it), rounded to bf16 again for the down projection's panel: one (row tile,
      // column tile) group of four values per lane.
      auto gelu_group = [&](const f32x4 (&v)[FM][FN], unsigned char *hb, int g) {
        const int i = g / FN, j = g % FN;
        *reinterpret_cast<u32x2 *>(hb + (16 * i + li) * ROWB + (cw + 16 * j + 4 * lg) * 2) =
            gelu_bf16x4(pack_bf16x4(v[i][j]));
      };
      constexpr int G = FM * FN;
      constexpr bool PIPE = gelu_pipelined<BM>();
      if (PIPE && c > 0) {
        // Up chunks run back to back: chunk c - 1's GELU is spread over chunk c's k-steps.
        unsigned char *hp = hbuf[c - 1];
        stage_mma_t<FM>(acc, panel, cur, nx, refill, lane_o, [&](int ks) {
#pragma unroll
          for (int g = 0; g < G; ++g)
            if (g * KS / G == ks) gelu_group(prev, hp, g);
        });
      } else {
        stage_mma_t<FM>(acc, panel, cur, nx, refill, lane_o);
      }
      unsigned char *hb = hbuf[p.ups_first ? c : (c % HB)];
      if (PIPE && c < p.nc - 1) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) prev[i][j] = acc[i][j];
      } else {
        // One GELU buffer: every wave has finished down chunk c - 1's reads of it.
        if (HB == 1 && c > 0) lds_barrier();
#pragma unroll
        for (int g = 0; g < G; ++g) gelu_group(acc, hb, g);
        // Down chunk c reads every wave's columns of GELU chunk c.
        if (!p.ups_first || c == p.nc - 1) lds_barrier();
      }
    } else if (kind == ST_DOWN) {
      // ---- down chunk c (accumulates); after the last: residual (+PLE), next prologue
      const bool last = c == p.nc - 1;
      f32x4 pl[FM][FN];
      if (last && a.ple) {
        const Rsrc rp = rsrc(opaque_ptr(a.ple), uint32_t(a.M) * uint32_t(a.ld_ple) * 4);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const uint32_t m = uint32_t(m0 + 16 * i + li);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int n = cw + 16 * j + 4 * lg + r;
              pl[i][j][r] = bloadf(rp, (m * uint32_t(a.ld_ple) + a.ple_off + n % a.ple_dim) * 4);
            }
          }
      }
      __builtin_amdgcn_sched_barrier(0);  // per-layer embedding loads ahead of the weight refills
      stage_mma_t<FM>(accd, hbuf[p.ups_first ? c : (c % HB)], cur, nx, refill, lane_o);
      if (last) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int c0 = cw + 16 * j + 4 * lg;
          const f32x4 bias = lds4(prm.b_down + c0);
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            const int m = m0 + 16 * i + li;
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
            if (m < a.M && cw + 16 * j < d) {
              v = accd[i][j] + bias;
              if (a.ple) v += pl[i][j] * a.ple_scale;
              st_nt(a.x + int64_t(m) * d + c0, v);
            }
            accd[i][j] = v;
          }
        }
        next_prologue<BM>(a, prm, accd, panel, red, cw, wave, li, lg);
      }
    } else {
      // ---- qkv chunk: q stored, k / v appended to the pool (four consecutive columns of one
      //      row per lane: one head's dims, head_dim being a multiple of 4)
      int64_t slot[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i) slot[i] = prm.tok_slot[16 * i + li];
      zero<FM>(acc);
      stage_mma_t<FM>(acc, panel, cur, nx, refill, lane_o);
      const int es = a.kv_dtype == CG_F32 ? 4 : 2;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int run = (PANEL * c + cw + 16 * j) / 4 + lg;
        const int2 e = prm.qkv_map[run];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int m = m0 + 16 * i + li;
          if (m >= a.M) continue;
          if (e.x == 0) {
            const uint32_t qo = uint32_t(m) * uint32_t(a.q_cols) + uint32_t(e.y);
            if (a.q_dtype == CG_F32) st_nt(static_cast<float *>(a.q) + qo, acc[i][j]);
            else store4(static_cast<char *>(a.q) + size_t(qo) * 2, a.q_dtype, acc[i][j]);
          } else if (e.x > 0 && slot[i] >= 0) {
            f32x4 val = acc[i][j];
            if (e.x == 2 && a.vemb_off >= 0) {
              const float *ve = a.vemb + int64_t(m) * a.ld_vemb + a.vemb_off +
                                (4 * run - a.q_cols - a.kv_heads * a.head_dim);
#pragma unroll
              for (int r = 0; r < 4; ++r) val[r] += ve[r];
            }
            store4(static_cast<char *>(e.x == 2 ? a.vc : a.kc) + (slot[i] + e.y) * es, a.kv_dtype, val);
          }
        }
      }
    }
  }
}

}  // namespace
}  // namespace cg
