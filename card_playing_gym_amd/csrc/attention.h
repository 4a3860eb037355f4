// Internal launcher of the ragged decode-attention kernel, shared by the C-ABI op and the
// fused trunk.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cg {

struct AttnArgs {
  // Queries: element (b, head, t, d) of sequence b lives at
  //   (seq_start ? seq_start[b] * q_st : b * q_sb) + head * q_sh + t * q_st + d.
  const void *q;
  int32_t q_dtype;
  int64_t q_sb, q_sh, q_st;
  // Output, addressed like the queries with (o_sb, o_sh, o_st).
  void *out;
  int32_t out_dtype;
  int64_t o_sb, o_sh, o_st;
  // One layer of the pool, [capacity, kv_heads, max_len, head_dim].
  const void *k;
  const void *v;
  int32_t kv_dtype;
  const int64_t *rows;         // [n_seqs] or NULL (= b)
  const int64_t *key_lengths;  // [n_seqs]; the visible prefix is key_lengths[b] + kl_add + t
  int32_t kl_add;
  const int64_t *seq_start;    // [n_seqs + 1] packed token offsets, or NULL (T per sequence)
  int32_t n_seqs, n_heads, kv_heads, head_dim, T, max_len, capacity, span;
  int64_t n_tokens;            // packed mode: tokens in q / out (token ranges are clamped to it)
  float scale_log2;            // softmax scale * log2(e)
  // (row, KV head) units in descending order of work (launch_attention_order), or NULL.
  // With it, padded runs of up to 16 queries per unit on a 16-bit pool take the persistent
  // kernel (each wave walks several whole units back to back), and packed runs deal their
  // units longest first.
  const int32_t *order;
};

void launch_decode_attention(const AttnArgs &a, hipStream_t stream);

// Whether `a` (with an order) takes the persistent kernel, and the order it needs: one int
// per (row, KV head) unit, written by launch_attention_order from the same rows, key
// lengths and span (valid for every layer of one step).
bool attention_streams(const AttnArgs &a);
void launch_attention_order(const AttnArgs &a, int32_t *order, hipStream_t stream);

}  // namespace cg
