// Internal interface of the fused per-layer kernel of the bf16 trunk step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cg {

// One launch does, for a block of token rows:
//   post  (do_post): x += attn . W_out^T; h = LN(x; ln2); x += GELU(h . W_up^T + b_up) . W_down^T
//                    + b_down (+ per-layer embedding);   (DecoderBlock._finish + Trunk._add_ple)
//   else           : x = x_src (the conditioned input; the first block's prologue)
//   then either  (final_ln == 0): h = LN(x; ln) ; [q | k | v] = h . W_qkv^T, q stored, k / v
//                    (+ value embedding) appended to the pool at each token's slot
//                    (the next block's _qkv + KVCache.write_step)
//   or           (final_ln == 1): hidden[tok_out[m]] = LN(x; ln) for readout tokens.
struct TailArgs {
  int32_t M;  // tokens
  int32_t d, d_ff, n_qkv, q_cols, kv_heads, head_dim, max_len, kv_dtype;
  float eps;

  int32_t do_post;
  const void *attn;  // [M, d] bf16 (attention output, heads x head_dim per token)
  // Weights in fragment order (launch_pack_fragments).
  const void *w_out;  // [d, d]
  const void *w_up;   // [d_ff, d]
  const float *b_up;  // [d_ff]
  const void *w_down;  // [d, d_ff]
  const float *b_down;  // [d]
  const float *ln2_w, *ln2_b;
  const float *ple;  // [M, ld_ple] or NULL
  int64_t ld_ple;
  int32_t ple_off, ple_dim;
  float ple_scale;

  const float *x_src;  // residual stream read
  float *x;            // residual stream written (may alias x_src)
  int32_t x_src_vec;   // x_src is 16-byte aligned (the first block reads it as float4 runs)

  int32_t final_ln;
  const float *ln_w, *ln_b;  // next block's ln_attn, or the final norm
  const void *w_qkv;         // [n_qkv, d]
  void *q;                   // [M, q_cols], type q_dtype (the pool's 16-bit type, or fp32)
  int32_t q_dtype;
  void *kc, *vc;
  const int32_t *tok_row, *tok_pos;
  const float *vemb;
  int64_t ld_vemb;
  int32_t vemb_off;  // < 0: none
  float *hidden;     // final_ln: [rows, d]
  int32_t hidden_vec;  // hidden is 16-byte aligned (rows written as float4 runs)
  const int32_t *tok_out;

  // MODE 0 only.  plan != 0: the launch forms the step's plan itself from its descriptors
  // (cg_ragged): per token its cache row, clamped write position and output row, written to
  // plan_row / plan_pos / plan_out (the tok_* arrays of the later launches); per sequence a
  // zero hidden row when its readout offset is outside its chunk; the status words.
  int32_t plan;
  const int64_t *seq_start, *positions, *rows, *readout;
  int32_t n_seqs, T, capacity;
  int32_t *plan_row, *plan_pos, *plan_out, *status;
  // embed_table != NULL: the input rows are formed here from token ids, x = rms_norm(
  // embed_table[ids]) * in_gain (eps in_eps; a row of an id outside [0, vocab) is zero).
  const float *embed_table;
  int32_t vocab;
  const int64_t *ids;
  const float *in_gain;
  float in_eps;
};

// The fused kernel reads its four weight matrices in MFMA fragment order: W [N, K] (fp32,
// row-major) -> bf16 blocks of 16 rows x 32 k, k zero-padded to a multiple of 32.
size_t packed_fragment_bytes(int N, int K);
void launch_pack_fragments(const float *src, void *dst, int N, int K, hipStream_t stream);

// Shapes the fused kernel is built for: d_model <= 256 and a multiple of 16, d_ff <= 1024
// and n_qkv <= 768, both multiples of 16, head_dim a multiple of 4 (each lane's run of four
// output columns stays inside one head); bf16 projections.
bool tail_supported(int d, int d_ff, int n_qkv, int head_dim);

// The fused layer kernel's GELU (bf16 in, bf16 out) over n values (a multiple of 4).
void launch_gelu_apply(const void *x, void *y, int64_t n, hipStream_t stream);

void launch_tail(const TailArgs &a, hipStream_t stream);

}  // namespace cg
