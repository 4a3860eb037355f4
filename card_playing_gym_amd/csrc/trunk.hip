// The fused trunk: conditioning norms, the per-layer launch sequence of a ragged decode
// step, and the final LayerNorm at the readout tokens.
//
// One step = plan -> (per layer) [LN + QKV GEMM + KV append] -> [decode attention]
//   -> [out_proj GEMM + residual] -> [LN + up GEMM + GELU] -> [down GEMM + residual (+PLE)]
//   -> readout LayerNorm.
// This is DecoderBlock.forward_ragged / Trunk.forward_ragged (cardgym/nn/trunk.py:183-223,
// 391-429) with the gather copy and the masked full-span attention replaced by in-place
// attention over each row's own prefix.
#include <mutex>
#include <string>
#include <vector>

#include "attention.h"
#include "common.h"
#include "fragment.h"
#include "gemm.h"
#include "layer.h"

struct cg_trunk {
  cg_trunk_config cfg;
  int32_t head_dim;
  int32_t compute;
  std::vector<cg_layer_params> layers;
  const float *final_w;
  const float *final_b;
  // bf16 projections whose shape the fused layer kernel covers: weight copies are kept in
  // its fragment order instead of row-major.
  bool fused = false;
  // bf16 copies of the projection weights (compute == CG_BF16), one allocation.
  void *wbuf = nullptr;
  size_t wbuf_bytes = 0;
  std::vector<const void *> qkv_w, out_w, up_w, down_w;
};

namespace cg {
namespace {

constexpr size_t ALIGN = 256;
inline size_t align_up(size_t v) { return (v + ALIGN - 1) / ALIGN * ALIGN; }

struct Workspace {
  float *x;
  void *xn;  // LayerNorm of x, the A operand of the next projection (compute type)
  float *q;
  void *attn;
  void *h1;
  int32_t *tok_row;
  int32_t *tok_pos;
  int32_t *readout_tok;
  int32_t *tok_out;
  int32_t *order;  // (row, KV head) units by descending key tiles (the persistent attention)
  size_t bytes;
};

Workspace carve(const cg_trunk &t, int32_t n_tokens, int32_t n_seqs, char *base) {
  const int d = t.cfg.d_model, hd = t.cfg.n_heads * t.head_dim, ff = t.cfg.d_ff;
  const size_t act = t.compute == CG_BF16 ? 2 : 4;
  Workspace w{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char *p = base ? base + off : nullptr;
    off += align_up(bytes);
    return p;
  };
  w.x = reinterpret_cast<float *>(take(size_t(n_tokens) * d * 4));
  w.xn = take(size_t(n_tokens) * d * act);
  w.q = reinterpret_cast<float *>(take(size_t(n_tokens) * hd * 4));
  w.attn = take(size_t(n_tokens) * hd * act);
  w.h1 = take(size_t(n_tokens) * ff * act);
  w.tok_row = reinterpret_cast<int32_t *>(take(size_t(n_tokens) * 4));
  w.tok_pos = reinterpret_cast<int32_t *>(take(size_t(n_tokens) * 4));
  w.readout_tok = reinterpret_cast<int32_t *>(take(size_t(n_seqs > 0 ? n_seqs : 1) * 4));
  w.tok_out = reinterpret_cast<int32_t *>(take(size_t(n_tokens) * 4));
  w.order = reinterpret_cast<int32_t *>(take(size_t(n_seqs > 0 ? n_seqs : 1) * t.cfg.n_kv_heads * 4));
  w.bytes = off;
  return w;
}

// A readout offset as torch indexing reads it (trunk.py:429, x[batch, readout_offsets]):
// negative offsets count from the end of the sequence's len tokens; -1 when outside.
__device__ __forceinline__ int64_t readout_offset(int64_t o, int64_t len) {
  if (o < 0) o += len;
  return o >= 0 && o < len ? o : -1;
}

// Per-token cache slot (row, clamped write position), per-sequence readout token, and
// per-token output row (tok_out: the sequence whose readout the token is, or -1; every
// token is its own output row when readout is NULL).  Tokens whose row is outside the pool
// or whose position is negative are neither written nor attended, and sequences whose
// readout offset is outside their chunk get a zero hidden row; each case sets its status
// word (plain stores of 1: every writer stores the same value).
// Padded mode (seq_start NULL): token i belongs to sequence i / T.
__global__ void plan_kernel(const int64_t *__restrict__ seq_start, const int64_t *__restrict__ positions,
                            const int64_t *__restrict__ rows, const int64_t *__restrict__ readout,
                            int32_t n_seqs, int32_t n_tokens, int32_t T, int32_t max_len,
                            int32_t capacity, int32_t *__restrict__ tok_row,
                            int32_t *__restrict__ tok_pos, int32_t *__restrict__ readout_tok,
                            int32_t *__restrict__ tok_out, float *__restrict__ hidden, int32_t d,
                            int32_t *__restrict__ status) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_tokens) {
    int b, t;
    if (seq_start) {
      int lo = 0, hi = n_seqs - 1;  // last b with seq_start[b] <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (seq_start[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      b = lo;
      t = int(i - seq_start[b]);
    } else {
      b = i / T;
      t = i % T;
    }
    const int64_t row = rows ? rows[b] : int64_t(b);
    const int64_t p0 = positions[b];
    int64_t pos = p0 + t;
    if (pos > max_len - 1) pos = max_len - 1;
    const bool row_ok = row >= 0 && row < capacity, pos_ok = p0 >= 0;
    const bool ok = row_ok && pos_ok;
    tok_row[i] = ok ? int32_t(row) : -1;
    tok_pos[i] = ok ? int32_t(pos) : 0;
    if (status && !row_ok) status[0] = 1;
    if (status && !pos_ok) status[1] = 1;
    if (readout) {
      const int64_t len = seq_start ? seq_start[b + 1] - seq_start[b] : int64_t(T);
      tok_out[i] = readout_offset(readout[b], len) == t ? b : -1;
    } else {
      tok_out[i] = i;
    }
  }
  if (readout && i < n_seqs) {
    const int64_t start = seq_start ? seq_start[i] : int64_t(i) * T;
    const int64_t stop = seq_start ? seq_start[i + 1] : start + T;
    const int64_t o = readout_offset(readout[i], stop - start);
    int64_t r = start + o;
    if (o < 0) {
      r = -1;
      if (status) status[2] = 1;
      if (hidden)
        for (int k = 0; k < d; ++k) hidden[int64_t(i) * d + k] = 0.f;
    }
    readout_tok[i] = int32_t(r);
  }
}

// A step with sequences but no tokens: every readout offset is outside its (empty) chunk, so
// every hidden row is zero and the readout status word is set, as plan_kernel does per row.
__global__ void empty_readout_kernel(float *__restrict__ hidden, int32_t n_seqs, int32_t d,
                                     int32_t *__restrict__ status) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < int64_t(n_seqs) * d) hidden[i] = 0.f;
  if (i == 0 && status) status[2] = 1;
}

// One wave per row: y = rms_norm(src row) * gain; src row = table[ids[row]] or x[row].
// XT float: fp32 rows; XT bf16: bf16 rows whose normalised value rounds to bf16 before the
// gain (rms_norm(x.float()).to(x.dtype) * gain).
template <typename XT>
__global__ void rmsnorm_rows_kernel(const XT *__restrict__ x, const float *__restrict__ table,
                                    int32_t vocab, const int64_t *__restrict__ ids,
                                    const float *__restrict__ gain, float eps, float *__restrict__ y,
                                    int32_t n, int32_t d, int32_t *__restrict__ flag) {
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  float *out = y + int64_t(row) * d;
  float s = 0.f;
  if (ids) {
    const int64_t id = ids[row];
    if (id < 0 || id >= vocab) {
      for (int k = lane; k < d; k += 64) out[k] = 0.f;
      if (flag && lane == 0) flag[0] = 1;
      return;
    }
    const float *in = table + id * d;
    for (int k = lane; k < d; k += 64) s = fmaf(in[k], in[k], s);
    const float r = rsqrtf(wave_sum(s) / float(d) + eps);
    for (int k = lane; k < d; k += 64) out[k] = in[k] * r * gain[k];
    return;
  }
  const XT *in = x + int64_t(row) * d;
  for (int k = lane; k < d; k += 64) {
    const float v = to_f32(in[k]);
    s = fmaf(v, v, s);
  }
  const float r = rsqrtf(wave_sum(s) / float(d) + eps);
  for (int k = lane; k < d; k += 64) out[k] = to_f32(from_f32<XT>(to_f32(in[k]) * r)) * gain[k];
}

// The embedding form above for d = 64 Q with 16-byte aligned rows: four rows per wave, 16
// lanes per row, Q float4 per lane, so the id -> row -> sum chains of four rows overlap
// (one row per wave left the launch waiting on those latencies).
template <int Q>
__global__ void embed_rmsnorm_rows4_kernel(const float *__restrict__ table, int32_t vocab,
                                           const int64_t *__restrict__ ids, const float *__restrict__ gain,
                                           float eps, float *__restrict__ y, int32_t n, int32_t *__restrict__ flag) {
  constexpr int D = 64 * Q;
  const int lane = threadIdx.x & 63, l16 = lane & 15;
  const int row = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const bool live = row < n;
  const int64_t id = live ? ids[row] : 0;
  const bool ok = live && id >= 0 && id < vocab;
  if (live && !ok && l16 == 0 && flag) flag[0] = 1;
  const float4 *in = reinterpret_cast<const float4 *>(table + (ok ? id : 0) * D);
  float4 v[Q];
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    v[q] = ok ? in[l16 + 16 * q] : float4{0.f, 0.f, 0.f, 0.f};
    s = fmaf(v[q].x, v[q].x, s);
    s = fmaf(v[q].y, v[q].y, s);
    s = fmaf(v[q].z, v[q].z, s);
    s = fmaf(v[q].w, v[q].w, s);
  }
  const float r = rsqrtf(sum16(s) / float(D) + eps);
  if (!live) return;
  const float4 *g4 = reinterpret_cast<const float4 *>(gain);
  float4 *out = reinterpret_cast<float4 *>(y + int64_t(row) * D);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const float4 g = g4[l16 + 16 * q];  // a row with a bad id is written as zeros
    out[l16 + 16 * q] = ok ? float4{v[q].x * r * g.x, v[q].y * r * g.y, v[q].z * r * g.z, v[q].w * r * g.w}
                           : float4{0.f, 0.f, 0.f, 0.f};
  }
}

// fp32 -> bf16 (round to nearest even) weight copies.
__global__ void to_bf16_kernel(const float *__restrict__ src, bf16 *__restrict__ dst, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = from_f32<bf16>(src[i]);
}

unsigned rows_grid(int32_t n, int waves_per_block) {
  return unsigned((n + waves_per_block - 1) / waves_per_block);
}

// RMSNorm(table[ids]) * gain -> y [n, d] fp32: four rows per wave for the usual widths
// (16-byte aligned rows), one row per wave otherwise.  flag (may be NULL) = 1 on a bad id.
void launch_embed_rmsnorm(const float *table, int32_t vocab, const int64_t *ids, const float *gain, float eps,
                          float *y, int32_t n, int32_t d, int32_t *flag, hipStream_t s) {
  const bool aligned = ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(gain) |
                         reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  const unsigned grid4 = unsigned((int64_t(n) + 15) / 16);  // four waves of four rows
  if (aligned && d == 256) embed_rmsnorm_rows4_kernel<4><<<grid4, 256, 0, s>>>(table, vocab, ids, gain, eps, y, n, flag);
  else if (aligned && d == 128) embed_rmsnorm_rows4_kernel<2><<<grid4, 256, 0, s>>>(table, vocab, ids, gain, eps, y, n, flag);
  else if (aligned && d == 64) embed_rmsnorm_rows4_kernel<1><<<grid4, 256, 0, s>>>(table, vocab, ids, gain, eps, y, n, flag);
  else rmsnorm_rows_kernel<float><<<rows_grid(n, 4), 256, 0, s>>>(nullptr, table, vocab, ids, gain, eps, y, n, d, flag);
  CG_LAUNCHED();
}

void convert_weights(cg_trunk &t, hipStream_t s) {
  if (t.compute != CG_BF16) return;
  const int d = t.cfg.d_model, hd = t.cfg.n_heads * t.head_dim, ff = t.cfg.d_ff;
  const int qkv_rows = (t.cfg.n_heads + 2 * t.cfg.n_kv_heads) * t.head_dim;
  char *p = static_cast<char *>(t.wbuf);
  size_t off = 0;
  // W [rows, cols] fp32 -> bf16, row-major or in the fused kernel's fragment order.
  auto conv = [&](const float *src, int rows, int cols) {
    void *dst = p + off;
    if (t.fused) {
      off += align_up(packed_fragment_bytes(rows, cols));
      launch_pack_fragments(src, dst, rows, cols, s);
    } else {
      const int64_t n = int64_t(rows) * cols;
      off += align_up(size_t(n) * 2);
      int64_t blocks = (n + 255) / 256;
      if (blocks > 4096) blocks = 4096;
      to_bf16_kernel<<<unsigned(blocks), 256, 0, s>>>(src, static_cast<bf16 *>(dst), n);
      CG_LAUNCHED();
    }
    return static_cast<const void *>(dst);
  };
  for (int l = 0; l < t.cfg.n_layers; ++l) {
    const cg_layer_params &L = t.layers[l];
    t.qkv_w[l] = conv(L.qkv_w, qkv_rows, d);
    t.out_w[l] = conv(L.out_w, d, hd);
    t.up_w[l] = conv(L.mlp_up_w, ff, d);
    t.down_w[l] = conv(L.mlp_down_w, d, ff);
  }
}

size_t weight_bytes_per_layer(const cg_trunk &t) {
  const cg_trunk_config &c = t.cfg;
  const int hd = c.n_heads * t.head_dim;
  const int qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * t.head_dim;
  auto bytes = [&](int rows, int cols) {
    return align_up(t.fused ? packed_fragment_bytes(rows, cols) : size_t(rows) * cols * 2);
  };
  return bytes(qkv_rows, c.d_model) + bytes(c.d_model, hd) + bytes(c.d_ff, c.d_model) + bytes(c.d_model, c.d_ff);
}

}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

int cg_trunk_create(const cg_trunk_config *config, const cg_layer_params *layers,
                    const float *final_ln_w, const float *final_ln_b, int32_t compute_dtype,
                    cg_trunk **out) {
  cg_trunk *t = nullptr;
  int status = guarded([&] {
    CG_REQUIRE(config && layers && out && final_ln_w && final_ln_b, CG_ERR_INVALID,
               "config, layers, final norm and out are required");
    const cg_trunk_config &c = *config;
    CG_REQUIRE(c.d_model > 0 && c.n_layers > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.d_ff > 0,
               CG_ERR_INVALID, "trunk dimensions must be positive");
    CG_REQUIRE(c.d_model % c.n_heads == 0, CG_ERR_INVALID, "d_model must be divisible by n_heads");
    CG_REQUIRE(c.n_heads % c.n_kv_heads == 0, CG_ERR_INVALID, "n_kv_heads must divide n_heads");
    CG_REQUIRE(c.per_layer_dim >= 0 && c.value_width >= 0, CG_ERR_INVALID,
               "per_layer_dim and value_width must be non-negative");
    CG_REQUIRE(compute_dtype == CG_F32 || compute_dtype == CG_BF16, CG_ERR_INVALID,
               "compute dtype must be CG_F32 or CG_BF16");
    const int hd = c.d_model / c.n_heads;
    CG_REQUIRE(c.d_model % 8 == 0 && c.d_ff % 8 == 0, CG_ERR_UNSUPPORTED,
               "d_model and d_ff must be multiples of 8");
    CG_REQUIRE(hd == 8 || hd == 16 || hd == 24 || hd == 32 || hd == 64, CG_ERR_UNSUPPORTED,
               "head_dim must be 8, 16, 24, 32 or 64");
    t = new cg_trunk();
    t->cfg = c;
    t->head_dim = hd;
    t->compute = compute_dtype;
    t->layers.assign(layers, layers + c.n_layers);
    for (const cg_layer_params &L : t->layers) {
      CG_REQUIRE(L.ln_attn_w && L.ln_attn_b && L.qkv_w && L.out_w && L.ln_mlp_w && L.ln_mlp_b &&
                     L.mlp_up_w && L.mlp_up_b && L.mlp_down_w && L.mlp_down_b,
                 CG_ERR_INVALID, "a layer parameter is NULL");
      CG_REQUIRE(L.value_index < 0 || (L.value_index + 1) * c.n_kv_heads * hd <= c.value_width,
                 CG_ERR_INVALID, "value_index outside the value-embedding stream");
    }
    t->final_w = final_ln_w;
    t->final_b = final_ln_b;
    const int n = c.n_layers;
    t->qkv_w.resize(n);
    t->out_w.resize(n);
    t->up_w.resize(n);
    t->down_w.resize(n);
    for (int l = 0; l < n; ++l) {
      t->qkv_w[l] = t->layers[l].qkv_w;
      t->out_w[l] = t->layers[l].out_w;
      t->up_w[l] = t->layers[l].mlp_up_w;
      t->down_w[l] = t->layers[l].mlp_down_w;
    }
    if (compute_dtype == CG_BF16) {
#ifdef CG_TRUNK_NO_FUSED
      t->fused = false;  // measurement builds only
#else
      t->fused = tail_supported(c.d_model, c.d_ff, (c.n_heads + 2 * c.n_kv_heads) * hd, hd);
#endif
      t->wbuf_bytes = weight_bytes_per_layer(*t) * n;
      CG_HIP(hipMalloc(&t->wbuf, t->wbuf_bytes));
      convert_weights(*t, nullptr);
      CG_HIP(hipStreamSynchronize(nullptr));
    }
    *out = t;
  });
  if (status != CG_OK && t) {
    if (t->wbuf) (void)hipFree(t->wbuf);
    delete t;
  }
  return status;
}

int cg_trunk_refresh(cg_trunk *trunk, void *stream) {
  return guarded([&] {
    CG_REQUIRE(trunk != nullptr, CG_ERR_INVALID, "trunk is NULL");
    convert_weights(*trunk, as_stream(stream));
  });
}

int cg_trunk_destroy(cg_trunk *trunk) {
  return guarded([&] {
    if (!trunk) return;
    if (trunk->wbuf) CG_HIP(hipFree(trunk->wbuf));
    delete trunk;
  });
}

size_t cg_trunk_workspace_size(const cg_trunk *trunk, int32_t n_tokens, int32_t n_seqs) {
  if (!trunk || n_tokens < 0 || n_seqs < 0) return 0;
  return carve(*trunk, n_tokens, n_seqs, nullptr).bytes;
}

}  // extern "C"

namespace cg {
namespace {

// The step on a given workspace: cg_trunk_forward and cg_trunk_forward_static.
// Token ids instead of conditioned rows (cg_trunk_forward_tokens): x = rms_norm(table[ids]) * gain.
struct Embed {
  const float *table = nullptr;
  int32_t vocab = 0;
  const int64_t *ids = nullptr;
  const float *gain = nullptr;
  float eps = 0.f;
};

void trunk_forward(const cg_trunk *trunk, const cg_kv_layer *cache, const float *x, const float *ple,
                   const float *values, const cg_ragged *step, float *hidden, void *workspace,
                   size_t workspace_size, void *stream, const Embed &embed = Embed{}) {
  CG_REQUIRE(trunk && cache && step, CG_ERR_INVALID, "trunk, cache and step are required");
  // A step without tokens reads no rows (its empty inputs may come as NULL) and writes hidden
  // rows only for readouts.
  const bool no_tokens = step->n_tokens == 0;
  CG_REQUIRE(hidden || (no_tokens && !step->readout), CG_ERR_INVALID, "hidden is required");
  CG_REQUIRE(no_tokens || (x != nullptr) != (embed.table != nullptr), CG_ERR_INVALID,
             "exactly one of the input rows and the embedding table is required");
  CG_REQUIRE(!embed.table || no_tokens || (embed.ids && embed.gain && embed.vocab > 0), CG_ERR_INVALID,
             "token ids, the input norm gain and a positive vocabulary are required with the table");
  const cg_trunk &t = *trunk;
  const cg_trunk_config &c = t.cfg;
  const cg_ragged &r = *step;
  CG_REQUIRE(r.n_seqs >= 0 && r.n_tokens >= 0, CG_ERR_INVALID, "negative step size");
  CG_REQUIRE(r.positions != nullptr, CG_ERR_INVALID, "positions is NULL");
  CG_REQUIRE(r.seq_start || int64_t(r.n_seqs) * r.T == r.n_tokens, CG_ERR_INVALID,
             "padded step: n_tokens must equal n_seqs * T");
  CG_REQUIRE(r.n_tokens == 0 || c.per_layer_dim == 0 || ple, CG_ERR_INVALID,
             "This trunk expects a per-layer embedding lookup.");
  CG_REQUIRE(r.n_tokens == 0 || c.value_width == 0 || values, CG_ERR_INVALID,
             "This trunk expects a value-embedding lookup.");
  for (int l = 0; l < c.n_layers; ++l) {
    const cg_kv_layer &L = cache[l];
    check_layer(&L);
    CG_REQUIRE(L.kv_heads == c.n_kv_heads && L.head_dim == t.head_dim, CG_ERR_INVALID,
               "cache layout does not match the trunk");
    CG_REQUIRE(L.max_len == cache[0].max_len && L.capacity == cache[0].capacity &&
                   L.dtype == cache[0].dtype,
               CG_ERR_INVALID, "cache layers differ in shape");
  }
  CG_REQUIRE(r.rows || r.n_seqs <= cache[0].capacity, CG_ERR_RANGE,
             "dense rows: more sequences than cache rows");
  if (r.n_seqs == 0) return;
  if (r.n_tokens == 0) {
    if (r.readout) {
      const int64_t n = int64_t(r.n_seqs) * c.d_model;
      empty_readout_kernel<<<unsigned((n + 255) / 256), 256, 0, as_stream(stream)>>>(hidden, r.n_seqs, c.d_model,
                                                                                    r.status);
      CG_LAUNCHED();
    }
    return;
  }
  Workspace w = carve(t, r.n_tokens, r.n_seqs, static_cast<char *>(workspace));
  CG_REQUIRE(workspace && workspace_size >= w.bytes, CG_ERR_INVALID,
             "workspace too small: need " + std::to_string(w.bytes) + " bytes");
  hipStream_t s = as_stream(stream);
  const int d = c.d_model, H = c.n_heads, KVH = c.n_kv_heads, D = t.head_dim;
  const int N = r.n_tokens;
  const int max_len = cache[0].max_len;
  const int span = (r.span <= 0 || r.span > max_len) ? max_len : r.span;
  const int act_dtype = t.compute == CG_BF16 ? CG_BF16 : CG_F32;

  const float ple_scale = [&] {
    if (c.per_layer_dim == 0 || c.per_layer_dim == d) return 1.0f;
    const int repeats = (d + c.per_layer_dim - 1) / c.per_layer_dim;
    return 1.0f / sqrtf(float(repeats));
  }();
  // Queries of multi-token rows (packed chunks, prefill) are stored in the pool's 16-bit type
  // by the fused step (the reference rounds q to the cache dtype before the scores,
  // trunk.py:222), which the attention kernel loads as its MFMA operand as they are:
  // 139 -> 100 us per layer at config 5.  One-token decode keeps fp32 q, which that kernel
  // scales and rounds itself (the raw form measured 1-2.6 us slower per layer there, also
  // with the score scale folded into the exponent); the projections of the unfused path
  // write fp32.
  const bool multi_query = r.seq_start != nullptr || int64_t(H / KVH) * r.T > 16;
  const int q_dtype = (t.fused && multi_query && cache[0].dtype != CG_F32) ? cache[0].dtype : CG_F32;
  auto attn_args = [&](int l) {
    const cg_kv_layer &L = cache[l];
    AttnArgs a{};
    a.q = w.q;
    a.q_dtype = q_dtype;
    a.q_st = int64_t(H) * D;
    a.q_sh = D;
    a.q_sb = int64_t(r.T) * H * D;
    a.out = w.attn;
    a.out_dtype = act_dtype;
    a.o_st = int64_t(H) * D;
    a.o_sh = D;
    a.o_sb = int64_t(r.T) * H * D;
    a.k = L.k;
    a.v = L.v;
    a.kv_dtype = L.dtype;
    a.rows = r.rows;
    a.key_lengths = r.positions;
    a.kl_add = 1;
    a.seq_start = r.seq_start;
    a.n_tokens = N;
    a.n_seqs = r.n_seqs;
    a.n_heads = H;
    a.kv_heads = KVH;
    a.head_dim = D;
    a.T = r.T;
    a.max_len = max_len;
    a.capacity = L.capacity;
    a.span = span;
    a.scale_log2 = 1.4426950408889634f / sqrtf(float(D));
    return a;
  };
  // The fused path's first launch forms the plan of padded runs itself; packed runs keep a
  // launch for it (each token's sequence is a search over the chunk bounds, a chain of
  // dependent loads that measured 14 us longer per step inside the first launch at config 5).
  const bool plan_in_first = t.fused && !r.seq_start;
  if (!plan_in_first) {
    const int n = N > r.n_seqs ? N : r.n_seqs;
    plan_kernel<<<(n + 255) / 256, 256, 0, s>>>(r.seq_start, r.positions, r.rows, r.readout, r.n_seqs, N, r.T,
                                                max_len, cache[0].capacity, w.tok_row, w.tok_pos, w.readout_tok,
                                                w.tok_out, hidden, d, r.status);
    CG_LAUNCHED();
  }
  // The fused first launch reads the embedding rows through a buffer descriptor (a 32-bit
  // byte range) as float4 runs: tables of 4 GiB or more, or unaligned ones, take the
  // embedding norm as a launch of its own, whose rows the first launch then reads.
  const bool embed_in_first =
      embed.table && t.fused && int64_t(embed.vocab) * d * 4 < (int64_t(1) << 32) &&
      ((reinterpret_cast<uintptr_t>(embed.table) | reinterpret_cast<uintptr_t>(embed.gain)) & 15) == 0;
  if (embed.table && !embed_in_first) {
    launch_embed_rmsnorm(embed.table, embed.vocab, embed.ids, embed.gain, embed.eps, w.x, N, d,
                         r.status ? r.status + 3 : nullptr, s);
    x = w.x;
  }
  // Packed chunks on a 16-bit pool deal their units longest first: the unit order (by work)
  // is the same for every layer of the step, computed once here.  One-token decode runs take
  // the split kernel in unit order: with 32-key tiles and the last-wave merge it streams as
  // fast as the persistent kernel of the ordered entry points at spans of 2048-16384 keys
  // (324.9 / 342.1 / 353.3 / 370.4 against 330.1 / 335.1 / 351.6 / 387.0 us per launch for
  // 8192 x 2048 ... 1024 x 16384 rows of random lengths) without the order's 10-26 us launch
  // per step (config 4: 1.855-1.887 -> 1.837 ms per step).
#ifndef CG_PACKED_ORDER
#define CG_PACKED_ORDER 1
#endif
  const bool ordered = CG_PACKED_ORDER && r.seq_start && (cache[0].dtype == CG_BF16 || cache[0].dtype == CG_F16) &&
                       (D == 32 || D == 64);
  if (ordered) launch_attention_order(attn_args(0), w.order, s);
  auto attention = [&](int l) {
    AttnArgs a = attn_args(l);
    a.order = ordered ? w.order : nullptr;
    launch_decode_attention(a, s);
  };

  const int n_qkv = (H + 2 * KVH) * D;
  if (t.fused) {
    // bf16 projections: one fused launch per layer after its attention (layer.hip), plus
    // the first block's LN + QKV + append.
    auto base = [&] {
      TailArgs ta{};
      ta.M = N;
      ta.d = d;
      ta.d_ff = c.d_ff;
      ta.n_qkv = n_qkv;
      ta.q_cols = H * D;
      ta.kv_heads = KVH;
      ta.head_dim = D;
      ta.max_len = max_len;
      ta.kv_dtype = cache[0].dtype;
      ta.eps = c.eps;
      ta.q = w.q;
      ta.q_dtype = q_dtype;
      ta.tok_row = w.tok_row;
      ta.tok_pos = w.tok_pos;
      ta.vemb = values;
      ta.ld_vemb = c.value_width;
      ta.vemb_off = -1;
      ta.hidden = hidden;
      ta.hidden_vec = (reinterpret_cast<uintptr_t>(hidden) & 15) == 0;
      ta.tok_out = w.tok_out;
      return ta;
    };
    auto set_next = [&](TailArgs &ta, int nl) {
      if (nl == c.n_layers) {
        ta.final_ln = 1;
        ta.ln_w = t.final_w;
        ta.ln_b = t.final_b;
        return;
      }
      const cg_layer_params &Pn = t.layers[nl];
      ta.final_ln = 0;
      ta.ln_w = Pn.ln_attn_w;
      ta.ln_b = Pn.ln_attn_b;
      ta.w_qkv = t.qkv_w[nl];
      ta.kc = cache[nl].k;
      ta.vc = cache[nl].v;
      ta.vemb_off = (values && Pn.value_index >= 0) ? Pn.value_index * KVH * D : -1;
    };
    {
      TailArgs ta = base();
      ta.do_post = 0;
      ta.x_src = x;
      ta.x_src_vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
      ta.x = w.x;
      ta.plan = plan_in_first ? 1 : 0;
      ta.seq_start = r.seq_start;
      ta.positions = r.positions;
      ta.rows = r.rows;
      ta.readout = r.readout;
      ta.n_seqs = r.n_seqs;
      ta.T = r.T;
      ta.capacity = cache[0].capacity;
      ta.plan_row = w.tok_row;
      ta.plan_pos = w.tok_pos;
      ta.plan_out = w.tok_out;
      ta.status = r.status;
      if (embed_in_first) {
        ta.x_src = nullptr;
        ta.embed_table = embed.table;
        ta.vocab = embed.vocab;
        ta.ids = embed.ids;
        ta.in_gain = embed.gain;
        ta.in_eps = embed.eps;
      }
      set_next(ta, 0);
      launch_tail(ta, s);
    }
    // The tail of layer l: its post-attention half, then the next layer's QKV (or the
    // final norm).
    auto tail_of = [&](int l) {
      const cg_layer_params &P = t.layers[l];
      TailArgs ta = base();
      ta.do_post = 1;
      ta.attn = w.attn;
      ta.w_out = t.out_w[l];
      ta.w_up = t.up_w[l];
      ta.b_up = P.mlp_up_b;
      ta.w_down = t.down_w[l];
      ta.b_down = P.mlp_down_b;
      ta.ln2_w = P.ln_mlp_w;
      ta.ln2_b = P.ln_mlp_b;
      if (ple && c.per_layer_dim > 0) {
        ta.ple = ple;
        ta.ld_ple = int64_t(c.n_layers) * c.per_layer_dim;
        ta.ple_off = l * c.per_layer_dim;
        ta.ple_dim = c.per_layer_dim;
        ta.ple_scale = ple_scale;
      }
      ta.x_src = w.x;
      ta.x_src_vec = 1;
      ta.x = w.x;
      set_next(ta, l + 1);
      return ta;
    };
    for (int l = 0; l < c.n_layers; ++l) {
      attention(l);
      launch_tail(tail_of(l), s);
    }
    return;
  }

  if (x != w.x) CG_HIP(hipMemcpyAsync(w.x, x, size_t(N) * d * 4, hipMemcpyDeviceToDevice, s));
  launch_layernorm_rows(w.x, nullptr, t.layers[0].ln_attn_w, t.layers[0].ln_attn_b, c.eps, w.xn,
                        act_dtype, N, d, s);
  // Whole-row residual tiles fuse the next LayerNorm into the residual epilogue.
  const bool fused_ln = d <= 256;

  auto residual = [&](const void *A, int K, const void *W, const float *bias, const float *ln_w,
                      const float *ln_b, const float *ple_rows, int layer) {
    GemmArgs g{};
    g.M = N;
    g.N = d;
    g.K = K;
    g.compute = t.compute;
    g.A = A;
    g.lda = K;
    g.W = W;
    g.bias = bias;
    g.resid = w.x;
    g.ldr = d;
    if (ple_rows) {
      g.ple = ple_rows;
      g.ld_ple = int64_t(c.n_layers) * c.per_layer_dim;
      g.ple_off = layer * c.per_layer_dim;
      g.ple_dim = c.per_layer_dim;
      g.ple_scale = ple_scale;
    }
    if (ln_w && fused_ln) {
      g.epi = EPI_RESID_LN;
      g.ln_w = ln_w;
      g.ln_b = ln_b;
      g.eps = c.eps;
      g.out = w.xn;
      g.out_dtype = act_dtype;
      g.ldo = d;
      launch_gemm(g, s);
      return;
    }
    g.epi = EPI_RESID;
    launch_gemm(g, s);
    if (ln_w) launch_layernorm_rows(w.x, nullptr, ln_w, ln_b, c.eps, w.xn, act_dtype, N, d, s);
  };

  for (int l = 0; l < c.n_layers; ++l) {
    const cg_layer_params &P = t.layers[l];
    const cg_kv_layer &L = cache[l];
    {  // QKV projection of LN1(x) + append
      GemmArgs g{};
      g.M = N;
      g.N = (H + 2 * KVH) * D;
      g.K = d;
      g.compute = t.compute;
      g.A = w.xn;
      g.lda = d;
      g.W = t.qkv_w[l];
      g.epi = EPI_QKV;
      g.out = w.q;
      g.ldo = H * D;
      g.q_cols = H * D;
      g.kc = L.k;
      g.vc = L.v;
      g.kv_dtype = L.dtype;
      g.kv_heads = KVH;
      g.head_dim = D;
      g.max_len = max_len;
      g.tok_row = w.tok_row;
      g.tok_pos = w.tok_pos;
      g.vemb = values;
      g.ld_vemb = c.value_width;
      g.vemb_off = (values && P.value_index >= 0) ? P.value_index * KVH * D : -1;
      launch_gemm(g, s);
    }
    attention(l);
    // out_proj + residual, then LN2 -> xn
    residual(w.attn, H * D, t.out_w[l], nullptr, P.ln_mlp_w, P.ln_mlp_b, nullptr, l);
    {  // mlp[0] + GELU
      GemmArgs g{};
      g.M = N;
      g.N = c.d_ff;
      g.K = d;
      g.compute = t.compute;
      g.A = w.xn;
      g.lda = d;
      g.W = t.up_w[l];
      g.bias = P.mlp_up_b;
      g.epi = EPI_GELU;
      g.out = w.h1;
      g.out_dtype = act_dtype;
      g.ldo = c.d_ff;
      launch_gemm(g, s);
    }
    // mlp[2] + residual (+ PLE), then the next block's LN1 -> xn
    const bool last = l + 1 == c.n_layers;
    residual(w.h1, c.d_ff, t.down_w[l], P.mlp_down_b, last ? nullptr : t.layers[l + 1].ln_attn_w,
             last ? nullptr : t.layers[l + 1].ln_attn_b, (ple && c.per_layer_dim > 0) ? ple : nullptr, l);
  }
  const int rows_out = r.readout ? r.n_seqs : N;
  launch_layernorm_rows(w.x, r.readout ? w.readout_tok : nullptr, t.final_w, t.final_b, c.eps, hidden,
                        CG_F32, rows_out, d, s);
}

// The workspace of cg_trunk_forward_static: a file-scope device array, one copy per GPU (the
// code object's zero-initialised data, placed on each device when the library's code loads
// there and held until the process ends).  Host code never passes `scratch` itself to a
// kernel: its host-side name is only a stand-in; the device address of each GPU's copy comes
// from hipGetSymbolAddress, taken once per device with that device current.
__device__ __align__(256) unsigned char scratch[CG_TRUNK_STATIC_WORKSPACE];

std::mutex scratch_mutex;
std::vector<void *> scratch_address;  // per device ordinal, nullptr until first use

void *device_scratch() {
  int device = 0;
  CG_HIP(hipGetDevice(&device));
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (device >= int(scratch_address.size())) scratch_address.resize(size_t(device) + 1, nullptr);
  if (!scratch_address[device]) {
    void *ptr = nullptr;
    CG_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    CG_REQUIRE(ptr != nullptr, CG_ERR_HIP, "the static workspace has no device address");
    scratch_address[device] = ptr;
  }
  return scratch_address[device];
}

}  // namespace
}  // namespace cg

extern "C" {

int cg_trunk_forward_tokens(const cg_trunk *trunk, const cg_kv_layer *cache, const float *table, int32_t vocab,
                            const int64_t *ids, const float *gain, float eps, const float *ple, const float *values,
                            const cg_ragged *step, float *hidden, void *workspace, size_t workspace_size,
                            void *stream) {
  return guarded([&] {
    CG_REQUIRE(table != nullptr, CG_ERR_INVALID, "table is NULL");
    Embed e;
    e.table = table;
    e.vocab = vocab;
    e.ids = ids;
    e.gain = gain;
    e.eps = eps;
    trunk_forward(trunk, cache, nullptr, ple, values, step, hidden, workspace, workspace_size, stream, e);
  });
}

int cg_trunk_forward(const cg_trunk *trunk, const cg_kv_layer *cache, const float *x,
                     const float *ple, const float *values, const cg_ragged *step, float *hidden,
                     void *workspace, size_t workspace_size, void *stream) {
  return guarded([&] { trunk_forward(trunk, cache, x, ple, values, step, hidden, workspace, workspace_size, stream); });
}

int cg_trunk_forward_static(const cg_trunk *trunk, const cg_kv_layer *cache, const float *x,
                            const float *ple, const float *values, const cg_ragged *step, float *hidden,
                            void *stream) {
  return guarded([&] {
    CG_REQUIRE(trunk && step, CG_ERR_INVALID, "trunk and step are required");
    CG_REQUIRE(step->n_seqs >= 0 && step->n_tokens >= 0, CG_ERR_INVALID, "negative step size");
    const size_t need = carve(*trunk, step->n_tokens, step->n_seqs, nullptr).bytes;
    CG_REQUIRE(need <= CG_TRUNK_STATIC_WORKSPACE, CG_ERR_RANGE,
               "step needs " + std::to_string(need) + " workspace bytes; the static workspace holds " +
                   std::to_string(size_t(CG_TRUNK_STATIC_WORKSPACE)) + " (use cg_trunk_forward with a larger one)");
    trunk_forward(trunk, cache, x, ple, values, step, hidden, device_scratch(), CG_TRUNK_STATIC_WORKSPACE, stream);
  });
}

int cg_gelu_bf16(const void *x, void *y, int64_t n, void *stream) {
  return guarded([&] {
    CG_REQUIRE(n >= 0, CG_ERR_INVALID, "n must be non-negative");
    if (n == 0) return;
    CG_REQUIRE(x && y, CG_ERR_INVALID, "x and y are required");
    launch_gelu_apply(x, y, n, as_stream(stream));
  });
}

int cg_rmsnorm(const void *x, int32_t x_dtype, const float *gain, float eps, float *y, int32_t n, int32_t d,
               void *stream) {
  return guarded([&] {
    CG_REQUIRE(x && gain && y, CG_ERR_INVALID, "x, gain and y are required");
    CG_REQUIRE(n >= 0 && d > 0, CG_ERR_INVALID, "bad sizes");
    CG_REQUIRE(x_dtype == CG_F32 || x_dtype == CG_BF16, CG_ERR_INVALID, "x dtype must be CG_F32 or CG_BF16");
    if (n == 0) return;
    if (x_dtype == CG_BF16)
      rmsnorm_rows_kernel<bf16><<<rows_grid(n, 4), 256, 0, as_stream(stream)>>>(
          static_cast<const bf16 *>(x), nullptr, 0, nullptr, gain, eps, y, n, d, nullptr);
    else
      rmsnorm_rows_kernel<float><<<rows_grid(n, 4), 256, 0, as_stream(stream)>>>(
          static_cast<const float *>(x), nullptr, 0, nullptr, gain, eps, y, n, d, nullptr);
    CG_LAUNCHED();
  });
}

int cg_embed_rmsnorm(const float *table, int32_t vocab, const int64_t *ids, const float *gain,
                     float eps, float *y, int32_t n, int32_t d, int32_t *flag, void *stream) {
  return guarded([&] {
    CG_REQUIRE(table && ids && gain && y, CG_ERR_INVALID, "table, ids, gain and y are required");
    CG_REQUIRE(n >= 0 && d > 0 && vocab > 0, CG_ERR_INVALID, "bad sizes");
    if (n == 0) return;
    launch_embed_rmsnorm(table, vocab, ids, gain, eps, y, n, d, flag, as_stream(stream));
  });
}

}  // extern "C"
