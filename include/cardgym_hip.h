/*
 * cardgym_hip.h -- C ABI of libcardgym_hip.so, the gfx950 (MI355X) kernels behind the
 * KV-cached ragged decode step of the cardgym GQA trunk.
 *
 * Conventions shared by every entry point:
 *   - Plain pointers and sizes only.  Every tensor pointer is a device pointer unless the
 *     comment says "host".  Tensors are dense row-major unless strides are passed.
 *   - Each call enqueues work on `stream` (a hipStream_t passed as void*; NULL = the
 *     null stream) and returns at once.  Nothing is read back to the host and nothing is
 *     allocated per call, so every call may be captured into a hipGraph.  The only calls
 *     that allocate are cg_trunk_create / cg_trunk_destroy.
 *   - The return value is a status (CG_OK = 0).  On failure, cg_last_error() returns the
 *     message for the calling thread.  No C++ exception crosses this boundary.
 *   - Integer index arrays that mirror PyTorch int64 tensors (rows, positions, offsets)
 *     are int64_t.
 *
 * Each declaration cites the reference interface it replaces (paths are into the
 * maxrlinder/card_playing_gym source tree).
 */
#ifndef CARDGYM_HIP_H
#define CARDGYM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------------- */
#define CG_OK 0
#define CG_ERR_INVALID 1     /* bad argument: shape, dtype, null pointer      -> ValueError   */
#define CG_ERR_UNSUPPORTED 2 /* valid but not built (e.g. head_dim 40)        -> ValueError   */
#define CG_ERR_RANGE 3       /* index or size out of range                    -> IndexError   */
#define CG_ERR_HIP 4         /* the HIP runtime reported an error             -> RuntimeError */

/* ---- element types ------------------------------------------------------------- */
#define CG_F32 0
#define CG_BF16 1
#define CG_F16 2

/* ---- activations for cg_linear ----------------------------------------------- */
#define CG_ACT_NONE 0
#define CG_ACT_GELU 1 /* exact erf GELU, torch.nn.GELU() */

/* Library version (major * 10000 + minor * 100 + patch). */
int cg_version(void);

/* Copies the calling thread's last error message into buf (always NUL-terminated);
 * returns the message length. */
size_t cg_last_error(char *buf, size_t size);

/* One layer of a KV pool: k and v are each [capacity, kv_heads, max_len, head_dim]
 * contiguous, element type `dtype`.  Mirrors KVCache.k[layer] / KVCache.v[layer]
 * (cardgym/nn/kv_cache.py:45-59). */
typedef struct cg_kv_layer {
  void *k;
  void *v;
  int32_t capacity;
  int32_t kv_heads;
  int32_t max_len;
  int32_t head_dim;
  int32_t dtype; /* CG_F32, CG_BF16 or CG_F16 */
} cg_kv_layer;

/* Strided source of new keys or values, logically [B, kv_heads, T, head_dim]; the
 * head_dim stride must be 1.  The reference passes transposed views of the QKV split
 * (cardgym/nn/trunk.py:147-152), hence the explicit strides. */
typedef struct cg_kv_source {
  const void *data;
  int32_t dtype;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_t;
} cg_kv_source;

/* KVCache.write_step (cardgym/nn/kv_cache.py:84-105): for every b < B, t < T and head,
 * cache[rows[b], head, positions[b*T + t], :] = new[b, head, t, :] cast to the cache
 * dtype (round to nearest even, NaN -> canonical quiet NaN, as Tensor.to).  rows may be
 * NULL for 0..B-1.  positions is int64 [B, T] (for T = 1 the reference's [B] form).
 * Positions must lie in [0, max_len); rows in [0, capacity): out-of-range entries are
 * skipped on the device and reported by cg_kv_check_indices. */
int cg_kv_write_step(const cg_kv_layer *layer, const int64_t *rows, const int64_t *positions,
                     const cg_kv_source *k_new, const cg_kv_source *v_new, int32_t B, int32_t T,
                     void *stream);

/* KVCache.write_range (cardgym/nn/kv_cache.py:65-82): positions start..start+T-1 of
 * rows (NULL = 0..B-1). */
int cg_kv_write_range(const cg_kv_layer *layer, const int64_t *rows, int32_t start,
                      const cg_kv_source *k_new, const cg_kv_source *v_new, int32_t B, int32_t T,
                      void *stream);

/* KVCache.read with explicit rows (cardgym/nn/kv_cache.py:107-120): gathers
 * [B, kv_heads, length, head_dim] copies of the first `length` positions of rows[b]
 * into k_out / v_out (cache dtype, contiguous).  rows NULL = 0..B-1. */
int cg_kv_read(const cg_kv_layer *layer, const int64_t *rows, int32_t B, int32_t length,
               void *k_out, void *v_out, void *stream);

/* KVCache.copy_rows (cardgym/nn/kv_cache.py:122-138) for one layer: the first `length`
 * positions of rows sources[i] are copied onto targets[i].  Sources and targets must not
 * overlap (the reference copies through a gathered temporary). */
int cg_kv_copy_rows(const cg_kv_layer *layer, const int64_t *sources, const int64_t *targets,
                    int32_t n, int32_t length, void *stream);

/* KVCache.copy_rows (cardgym/nn/kv_cache.py:122-138) for one chunk over n_layers layers of
 * one shape, with the reference's gather-then-write meaning: a target that is also a
 * source of the chunk receives the source's old contents.  Chunks where no pair writes a
 * row that a later pair reads (compaction: rows slide down) are copied at one read and one
 * write per byte; others are staged through the workspace.  workspace: 16-byte aligned, at
 * least cg_kv_copy_workspace_size bytes (the classification, then one layer's gathered
 * prefixes); a larger one stages that many more layers per launch.  At most 64 layers.
 * plan: CG_COPY_AUTO classifies the chunk on the device; CG_COPY_ORDERED is the caller's
 * promise that every row is inside the pool and no pair writes a row that a later pair
 * reads (it skips the classification and the staged launches; a broken promise gives
 * wrong contents, never an access outside the pool's rows). */
#define CG_COPY_AUTO 0
#define CG_COPY_ORDERED 1
size_t cg_kv_copy_workspace_size(const cg_kv_layer *layers, int32_t n_layers, int32_t n, int32_t length);
int cg_kv_copy_rows_layers(const cg_kv_layer *layers, int32_t n_layers, const int64_t *sources,
                           const int64_t *targets, int32_t n, int32_t length, int32_t plan, void *workspace,
                           size_t workspace_size, void *stream);

/* Validates row and position indices on the device (no host read-back): flag[0] is set
 * to 1 if any rows[b] is outside [0, capacity) or positions[i] outside [0, max_len).
 * flag must be zeroed by the caller.  n_pos is the length of positions. */
int cg_kv_check_indices(const cg_kv_layer *layer, const int64_t *rows, int32_t B,
                        const int64_t *positions, int32_t n_pos, int32_t *flag, void *stream);

/* Ragged GQA decode attention straight from the pool: the custom op
 * cardgym::decode_attention (cardgym/nn/cuda_decode.py:172-202) and the gather + masked
 * softmax fallback it replaces (cardgym/nn/trunk.py:216-256), without their
 * head_dim 32 / span 64 / fp16 limits.
 *   q       [B, n_heads, T, head_dim] with strides (q_sb, q_sh, q_st), type q_dtype
 *   rows    int64 [B] cache rows (NULL = 0..B-1)
 *   key_lengths int64 [B]: query t of row b sees keys < min(key_lengths[b] + t, span)
 *   out     [B, n_heads, T, head_dim] contiguous, type out_dtype
 * Scores, softmax and accumulation are fp32 whatever the storage types. */
int cg_decode_attention(const void *q, int32_t q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                        const cg_kv_layer *layer, const int64_t *rows, const int64_t *key_lengths,
                        int32_t B, int32_t n_heads, int32_t T, int32_t span, float scale, void *out,
                        int32_t out_dtype, void *stream);

/* cg_decode_attention with a work order, through the persistent kernel (same op and
 * meaning, cardgym/nn/cuda_decode.py:188-202; the trunk step itself runs decode waves
 * through the split kernel, which streams as fast without the order).  cg_decode_attention_order
 * writes order (int32 [B * kv_heads]: the (row, KV head) units sorted by their number of
 * 64-key tiles, longest first) for these rows, key lengths, T and span, and sets *streams
 * (if not NULL) to 1 when the persistent kernel applies (16-bit pool, head_dim 32 or 64,
 * G * T <= 16 queries per unit, span of at least 1024 keys: below it both kernels stream at
 * the same rate) -- otherwise it writes nothing and the ordered call runs the split kernel.  The order stays valid for every layer and call with the same rows,
 * key lengths, T and span; results do not depend on it beyond its being a permutation of
 * the units. */
int cg_decode_attention_order(const cg_kv_layer *layer, const int64_t *rows, const int64_t *key_lengths,
                              int32_t B, int32_t n_heads, int32_t T, int32_t span, int32_t *order,
                              int32_t *streams, void *stream);
int cg_decode_attention_ordered(const void *q, int32_t q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                const cg_kv_layer *layer, const int64_t *rows, const int64_t *key_lengths,
                                int32_t B, int32_t n_heads, int32_t T, int32_t span, float scale, void *out,
                                int32_t out_dtype, const int32_t *order, void *stream);

/* The packed-row form of cg_decode_attention, as the trunk step launches it: the
 * chunks of cardgym/nn/packing.py:36-40 ([start, end) bounds) instead of a padded run, with
 * the visibility rule of DecoderBlock.forward_ragged / _grouped_attention
 * (cardgym/nn/trunk.py:183-256, key_lengths = positions + 1, trunk.py:426):
 *   q       [n_tokens, n_heads, head_dim], token stride q_st, head stride q_sh, type q_dtype
 *   sequence b owns tokens seq_start[b] .. seq_start[b+1]-1 (int64 [n_seqs + 1]) and cache
 *   row rows[b] (NULL = b); its token t sees keys < min(positions[b] + 1 + t, span), i.e. its
 *   cached prefix and its own chunk up to itself (already written to the pool)
 *   out     [n_tokens, n_heads, head_dim] contiguous, type out_dtype */
int cg_decode_attention_packed(const void *q, int32_t q_dtype, int64_t q_st, int64_t q_sh,
                               const cg_kv_layer *layer, const int64_t *rows, const int64_t *positions,
                               const int64_t *seq_start, int32_t n_seqs, int32_t n_tokens, int32_t n_heads,
                               int32_t span, float scale, void *out, int32_t out_dtype, void *stream);
/* The unit order the trunk step uses for a packed run (no counterpart in the reference: a
 * scheduling aid).  cg_decode_attention_packed_order writes order (int32 [n_seqs * kv_heads]:
 * the (row, KV head) units sorted by 64-key tiles x 16-query tiles, most work first) for
 * these rows, positions, chunk bounds and span; cg_decode_attention_packed_ordered then deals
 * the units in that order (16-bit pools, head_dim 32 / 64; other pools ignore it).  Results
 * do not depend on the order beyond its being a permutation of the units, and it stays valid
 * for every layer of one step. */
int cg_decode_attention_packed_order(const cg_kv_layer *layer, const int64_t *rows, const int64_t *positions,
                                     const int64_t *seq_start, int32_t n_seqs, int32_t n_tokens, int32_t n_heads,
                                     int32_t span, int32_t *order, void *stream);
int cg_decode_attention_packed_ordered(const void *q, int32_t q_dtype, int64_t q_st, int64_t q_sh,
                                       const cg_kv_layer *layer, const int64_t *rows, const int64_t *positions,
                                       const int64_t *seq_start, int32_t n_seqs, int32_t n_tokens,
                                       int32_t n_heads, int32_t span, float scale, void *out,
                                       int32_t out_dtype, const int32_t *order, void *stream);

/* ---- fused trunk ------------------------------------------------------------------ */

/* TrunkConfig (cardgym/nn/trunk.py:39-91). */
typedef struct cg_trunk_config {
  int32_t d_model;
  int32_t n_layers;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t d_ff;
  int32_t per_layer_dim;  /* PLE width per layer, 0 = off */
  int32_t value_width;    /* columns of the value-embedding stream (n_value_layers * kv_width) */
  float eps;              /* LayerNorm epsilon (nn.LayerNorm default 1e-5) */
} cg_trunk_config;

/* One DecoderBlock's parameters (cardgym/nn/trunk.py:124-139), fp32 device tensors in
 * torch nn.Linear layout ([out, in] row-major).  value_index is the block's slot in the
 * value-embedding stream, or -1 (Trunk._value, trunk.py:314-316). */
typedef struct cg_layer_params {
  const float *ln_attn_w;
  const float *ln_attn_b;
  const float *qkv_w;      /* [(n_heads + 2 kv_heads) * head_dim, d_model] */
  const float *out_w;      /* [d_model, n_heads * head_dim] */
  const float *ln_mlp_w;
  const float *ln_mlp_b;
  const float *mlp_up_w;   /* [d_ff, d_model] */
  const float *mlp_up_b;   /* [d_ff] */
  const float *mlp_down_w; /* [d_model, d_ff] */
  const float *mlp_down_b; /* [d_model] */
  int32_t value_index;
} cg_layer_params;

typedef struct cg_trunk cg_trunk; /* opaque */

/* Builds a trunk over caller-owned fp32 parameters.  compute_dtype CG_F32 runs every
 * projection in fp32; CG_BF16 runs them as bf16 x bf16 with fp32 accumulation (the
 * projections of torch.autocast(bfloat16), trunk.py:143/156-157 under
 * cardgym/core/devices.py:32-43) from bf16 weight copies the handle owns.  layers is a
 * host array of n_layers entries; the pointers are kept, not copied.  Allocates. */
int cg_trunk_create(const cg_trunk_config *config, const cg_layer_params *layers,
                    const float *final_ln_w, const float *final_ln_b, int32_t compute_dtype,
                    cg_trunk **out);

/* Re-derives the handle's weight copies from the fp32 parameters (after the caller has
 * changed them, e.g. load_state_dict). */
int cg_trunk_refresh(cg_trunk *trunk, void *stream);

int cg_trunk_destroy(cg_trunk *trunk);

/* One ragged step (or prefill) over packed tokens.  Mirrors the metadata of
 * Trunk.forward_ragged (cardgym/nn/trunk.py:391-429) with packed-row descriptors
 * (cardgym/nn/packing.py:36-40):
 *   n_seqs sequences; sequence b owns tokens seq_start[b] .. seq_start[b+1]-1 of the
 *   packed [n_tokens, d_model] input (seq_start NULL = padded: T tokens each, n_tokens =
 *   n_seqs * T); positions[b] is its cache length before the step, rows[b] its cache row
 *   (NULL = b); token t of sequence b is written at min(positions[b] + t, max_len - 1)
 *   and its query sees keys < min(positions[b] + 1 + t, span).
 *   readout[b] (NULL = every token) is the offset within sequence b whose final-norm
 *   hidden state is returned. */
typedef struct cg_ragged {
  int32_t n_seqs;
  int32_t n_tokens;
  int32_t T;                 /* tokens per sequence when seq_start is NULL */
  int32_t span;              /* key cap; <= 0 means max_len */
  const int64_t *seq_start;  /* int64 [n_seqs + 1] or NULL */
  const int64_t *positions;  /* int64 [n_seqs] */
  const int64_t *rows;       /* int64 [n_seqs] or NULL */
  const int64_t *readout;    /* int64 [n_seqs] or NULL */
  int32_t *status;           /* int32 [4] device words or NULL: the step sets status[0] = 1
                                when some rows[b] is outside [0, capacity), status[1] = 1 when
                                some positions[b] is negative (those tokens are neither written
                                nor attended: where the reference's index_put would raise,
                                kv_cache.py:98-105), status[2] = 1 when some readout[b] is
                                outside [-len_b, len_b) of its sequence (a zero hidden row;
                                negative offsets count from the sequence's end, as torch
                                indexing does, trunk.py:429), status[3] = 1 when a token id of
                                cg_trunk_forward_tokens is outside the table (a zero input
                                row, where F.embedding would raise).  Never cleared by the
                                step. */
} cg_ragged;

/* Workspace bytes cg_trunk_forward needs for n_tokens tokens and n_seqs sequences. */
size_t cg_trunk_workspace_size(const cg_trunk *trunk, int32_t n_tokens, int32_t n_seqs);

/* Trunk.forward_ragged / Trunk.forward_prefill (cardgym/nn/trunk.py:376-429): every
 * block of the trunk over the packed tokens, appending their K/V to `cache` (an array of
 * n_layers cg_kv_layer, host), then the final LayerNorm at the readout tokens.
 *   x       fp32 [n_tokens, d_model], already conditioned (Trunk.condition); not modified
 *   ple     fp32 [n_tokens, n_layers * per_layer_dim] or NULL (Trunk._add_ple)
 *   values  fp32 [n_tokens, value_width] or NULL (value embeddings, added to V)
 *   hidden  fp32 [n_seqs, d_model] (readout given) or [n_tokens, d_model] (readout NULL) */
int cg_trunk_forward(const cg_trunk *trunk, const cg_kv_layer *cache, const float *x,
                     const float *ple, const float *values, const cg_ragged *step, float *hidden,
                     void *workspace, size_t workspace_size, void *stream);

/* SequenceModel.forward_ragged of a single-field token embedder (cardgym/nn/model.py:76-89:
 * embed, Trunk.condition's input RMSNorm, Trunk.forward_ragged; trunk.py:104-115, 285-312,
 * 391-429) from token ids: x = rms_norm(table[ids[i]], eps) * gain for the packed tokens
 * (ids int64 [n_tokens], table fp32 [vocab, d_model], gain fp32 [d_model]), then exactly
 * cg_trunk_forward.  With bf16 projections the rows are formed inside the first layer's
 * launch, together with the step's per-token plan, instead of in launches of their own
 * (when table and gain are 16-byte aligned and the table is under 4 GiB; otherwise the
 * embedding norm runs as a launch of its own first, with the same result). */
int cg_trunk_forward_tokens(const cg_trunk *trunk, const cg_kv_layer *cache, const float *table, int32_t vocab,
                            const int64_t *ids, const float *gain, float eps, const float *ple, const float *values,
                            const cg_ragged *step, float *hidden, void *workspace, size_t workspace_size,
                            void *stream);

/* No counterpart in the reference.  cg_trunk_forward for callers that cannot allocate its
 * workspace (code under HIP graph capture that must not call hipMalloc, tight serving loops,
 * harnesses that forbid allocation): the same kernels, run on a library-owned workspace, a
 * static device array of CG_TRUNK_STATIC_WORKSPACE bytes on each GPU the library runs on,
 * held until the process ends.  Allocates nothing.  A step whose
 * cg_trunk_workspace_size(trunk, n_tokens, n_seqs) exceeds the array is refused with
 * CG_ERR_RANGE (about 13,000 tokens of a d_model 256 / d_ff 1024 bf16 trunk, 6,500 fp32).
 * Every call on one GPU shares that GPU's array, which keeps the last call's contents (a step
 * writes every workspace byte before it reads it, so nothing needs clearing): calls that
 * overlap on one GPU (two streams, two host threads, concurrent graph replays) race on it,
 * and the caller must serialise them.  The first call on each device looks the array's
 * address up; make it outside stream capture. */
#define CG_TRUNK_STATIC_WORKSPACE (64u << 20)
int cg_trunk_forward_static(const cg_trunk *trunk, const cg_kv_layer *cache, const float *x,
                            const float *ple, const float *values, const cg_ragged *step, float *hidden,
                            void *stream);

/* GELU of the fused bf16 layer kernel (the MLP's nn.GELU, cardgym/nn/trunk.py:135, under
 * autocast: the bf16 output of mlp[0] in, bf16 out), exposed so that callers and tests can
 * check it: n bf16 values (n a multiple of 4, 8-byte aligned arrays) through the kernel's
 * GELU, x * Phi(x) with Phi from Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), rounded
 * to bf16 (nearest even). */
int cg_gelu_bf16(const void *x, void *y, int64_t n, void *stream);

/* ---- conditioning, embedding and heads ------------------------------------------ */

/* RMSNorm (cardgym/nn/trunk.py:104-115): y = rms_norm(x, eps).to(x.dtype) * gain, rows of
 * width d, fp32 out.  x_dtype CG_F32 (x float) or CG_BF16 (x bf16: the normalised value is
 * rounded to bf16 before the gain, as .to(x.dtype) does). */
int cg_rmsnorm(const void *x, int32_t x_dtype, const float *gain, float eps, float *y, int32_t n, int32_t d,
               void *stream);

/* Embedding lookup then RMSNorm: y[i] = rms_norm(table[ids[i]]) * gain, the synthetic
 * single-field embedder followed by Trunk.condition's input norm
 * (cardgym/nn/model.py:45-48, cardgym/nn/trunk.py:297-298).  Ids outside [0, vocab)
 * produce zero rows and set flag[0] = 1 when flag is not NULL. */
int cg_embed_rmsnorm(const float *table, int32_t vocab, const int64_t *ids, const float *gain,
                     float eps, float *y, int32_t n, int32_t d, int32_t *flag, void *stream);

/* y = act(x @ w^T + bias) for fp32 x [m, k], w [n, k], bias [n] or NULL: the nn.Linear
 * layers of the heads evaluated at readout rows (cardgym/rl/graphs.py:88-104,
 * cardgym/nn/model.py:12-17).  compute_dtype CG_BF16 rounds x and w to bf16 (autocast). */
int cg_linear(const float *x, const float *w, const float *bias, float *y, int32_t m, int32_t n,
              int32_t k, int32_t act, int32_t compute_dtype, void *stream);

/* y = (x @ w^T + addend) * scale for fp32 x [m, k], w [n, k], addend [m, n]: the per-layer
 * embedding stream of Trunk.condition, ple = (ple_lookup + ple_context(x)) / sqrt(2)
 * (cardgym/nn/trunk.py:301-306).  compute_dtype CG_BF16 (autocast) rounds the projection to
 * bf16 as the Linear's output; addend_dtype CG_BF16 (a bf16 lookup) also rounds the sum and
 * the scaled sum to bf16, as bf16 tensor arithmetic does.  The product itself is fp32. */
int cg_linear_add_scale(const float *x, const float *w, const void *addend, int32_t addend_dtype, float *y,
                        int32_t m, int32_t n, int32_t k, float scale, int32_t compute_dtype, void *stream);

/* ---- policy and value heads ------------------------------------------------------ */

/* The heads a rollout wave evaluates at every readout row (cardgym/rl/graphs.py:88-104):
 * policy logits nn.Linear(d_model, n_policy) and value_mlp(d_model, n_value) =
 * Linear(d_model, d_mid) -> GELU -> Linear(d_mid, n_value) (cardgym/nn/model.py:12-17),
 * in one launch with the rounding of bf16 autocast: operands rounded to bf16, fp32
 * accumulation, every Linear output and the GELU output rounded to bf16.  Replaces the
 * three autocast nn.Linear calls of SequenceModel's graphable heads.
 * Shapes: d_model and d_mid multiples of 16 up to 256, n_policy a multiple of 16 up to
 * 1024, 1 <= n_value <= 16.  Weights are fp32, row-major [out, in], read at create and
 * refresh time only (the handle keeps bf16 copies in the kernel's fragment order). */
typedef struct cg_heads cg_heads;

typedef struct {
  int32_t d_model, n_policy, d_mid, n_value;
} cg_heads_config;

int cg_heads_create(const cg_heads_config *config, const float *policy_w, const float *policy_b,
                    const float *value_w1, const float *value_b1, const float *value_w2,
                    const float *value_b2, cg_heads **out);

/* Re-derives the bf16 weight copies after the fp32 weights changed (an optimiser step). */
int cg_heads_refresh(cg_heads *heads, void *stream);

int cg_heads_destroy(cg_heads *heads);

/* logits fp32 [m, n_policy], values fp32 [m, n_value] from hidden fp32 [m, d_model]. */
int cg_heads_forward(const cg_heads *heads, const float *hidden, int32_t m, float *logits,
                     float *values, void *stream);

/* ---- policy sampling ------------------------------------------------------------- */

/* masked_probabilities (cardgym/rl/ppo.py:75-82): softmax of each row of fp32 logits over
 * its legal entries (mask bytes != 0), exactly 0 on illegal ones; numpy's float32 order
 * (max, exp(x - max), pairwise-summed normaliser, correctly rounded division).  Rows
 * without a legal entry give NaN rows, as numpy does.  Strides are in elements. */
int cg_masked_probabilities(const float *logits, int64_t ld_logits, const uint8_t *mask, int64_t ld_mask,
                            int32_t rows, int32_t width, float *probs, int64_t ld_probs, void *stream);

/* sample_rows (cardgym/rl/ppo.py:85-94): per row, the number of float32 running sums of
 * probs below the row's float64 uniform, clamped to the last legal index and replaced by
 * it when illegal; int64 indices.  Bit-exact with the reference for the same inputs. */
int cg_sample_rows(const float *probs, int64_t ld_probs, const uint8_t *mask, int64_t ld_mask,
                   const double *uniforms, int32_t rows, int32_t width, int64_t *sampled, void *stream);

/* Adds `delta` to every entry of the int64 array a (n entries): the synthetic driver's
 * "every game appended one token" position update, kept on the device. */
int cg_advance_positions(int64_t *positions, int32_t n, int64_t delta, void *stream);

/* ---- Piquet's token embedder (cardgym/games/piquet/model.py:128-341) ----------------------
 * PiquetEmbedding.forward for [n, 64] int64 tokens (32 fields, then 32 card codes):
 *   x      = sum of the 32 field rows of `fields` (row = token field + field_offsets[f])
 *            + CardGrid's summary of the cards                      -> bf16 [n, d_model]
 *   ple    = the same rows of `ple_fields`  (when ple_width > 0)     -> bf16 [n, ple_width]
 *   values = the same rows of `value_fields` (when value_width > 0)  -> bf16 [n, value_width]
 *   cards  = CardGrid.cards: code + rank embeddings, card_layers GridBlocks (rank
 *            convolution zero-padded, suit pooling, GELU MLP, residual), GridNorm
 *                                                                    -> fp32 [n, 32, 32]
 * with bf16 autocast's rounding (the CUDA one-hot GEMM path of model.py:255-270 for the
 * fields).  Parameters are the reference's fp32 tensors in their own layouts; the handle
 * keeps bf16 copies of the tables and the grid's matrices (cg_piquet_refresh after they
 * change) and reads the small vectors in place.  Field ids outside the table and card codes
 * outside [0, 12) contribute zero and set flag[0] = 1 (flag may be NULL). */
typedef struct {
  int32_t d_model, ple_width, value_width, table_rows;
  int32_t card_width, card_hidden, card_kernel, card_layers;
  float eps;
} cg_piquet_config;

typedef struct { /* one GridBlock (model.py:128-151) */
  const float *norm;     /* [width] */
  const float *along_w;  /* [hidden, width, kernel] (Conv1d) */
  const float *along_b;  /* [hidden] */
  const float *across_w; /* [hidden, width] */
  const float *out_w;    /* [width, hidden] */
  const float *out_b;    /* [width] */
} cg_piquet_block;

typedef struct cg_piquet cg_piquet;

int cg_piquet_create(const cg_piquet_config *config, const int32_t *field_offsets, const float *fields,
                     const float *ple_fields, const float *value_fields, const float *code, const float *rank,
                     const cg_piquet_block *blocks, const float *grid_norm, const float *summary,
                     cg_piquet **out);
int cg_piquet_refresh(cg_piquet *embedder, void *stream);
int cg_piquet_destroy(cg_piquet *embedder);
int cg_piquet_embed(const cg_piquet *embedder, const int64_t *tokens, int64_t ld_tokens, int32_t n, void *x,
                    void *ple, void *values, float *cards, int32_t *flag, void *stream);

/* ---- training side (fp32, or bf16 autocast): a packed-row trunk forward that keeps what its
 * backward needs,
 * and that backward (cardgym/nn/trunk.py:124-181, 285-374 under autograd; packed rows as in
 * cardgym/nn/packing.py:36-40).  The composition (which buffers each layer keeps, the order
 * of the backward) is card_playing_gym_amd/nn/train.py; these are its kernels. ---------- */

/* C = alpha op(A) op(B) + beta C with A(i, k) = a[i * sam + k * sak] and B(k, j) =
 * b[k * sbk + j * sbn]: every projection's forward, input gradient and weight gradient.
 * compute_dtype CG_F32, or CG_BF16 as under autocast: A and B rounded to bf16, fp32
 * accumulation, alpha op(A) op(B) rounded to bf16 before beta C is added. */
size_t cg_gemm_workspace_size(int32_t m, int32_t n, int32_t k); /* split-K partials, 0 if none */
int cg_gemm_strided(int32_t m, int32_t n, int32_t k, float alpha, const float *a, int64_t sam, int64_t sak,
                    const float *b, int64_t sbk, int64_t sbn, float beta, float *c, int64_t ldc,
                    int32_t compute_dtype, void *workspace, size_t workspace_size, void *stream);

/* nn.LayerNorm forward keeping (mean, rstd) per row. */
int cg_layernorm_fwd(const float *x, const float *w, const float *b, float eps, float *y, float *mean, float *rstd,
                     int32_t n, int32_t d, void *stream);

/* LayerNorm (mean != NULL) or gain-only RMSNorm (mean == NULL, db ignored) backward: dx per
 * row, plus residual (a gradient arriving around the norm, e.g. the residual stream's) when
 * not NULL; dw (and db) summed over the rows, added to dw / db when accumulate != 0. */
size_t cg_norm_bwd_workspace_size(int32_t n, int32_t d);
int cg_norm_bwd(const float *x, const float *dy, const float *w, const float *mean, const float *rstd, float *dx,
                const float *residual, float *dw, float *db, int32_t n, int32_t d, void *workspace,
                size_t workspace_size, int32_t accumulate, void *stream);

/* out[c] (+)= sum_r x[r * ld + c]: bias gradients (two passes over long columns). */
size_t cg_column_sum_workspace_size(int32_t rows, int32_t cols);
int cg_column_sum(const float *x, int32_t rows, int32_t cols, int64_t ld, float *out, int32_t accumulate,
                  void *workspace, size_t workspace_size, void *stream);

/* nn.GELU() (erf) and its backward du = dg * GELU'(u). */
int cg_gelu_fwd(const float *u, float *g, int64_t n, void *stream);
int cg_gelu_bwd(const float *u, const float *dg, float *du, int64_t n, void *stream);

/* dst[r, c] += alpha * src[r * ld_src + c] (ld_src 0: one row broadcast, a bias). */
int cg_add_strided(int32_t rows, int32_t cols, float alpha, const float *src, int64_t ld_src, float *dst,
                   int64_t ld_dst, void *stream);

/* Gain-only RMSNorm (trunk.py:104-115) keeping rstd per row. */
int cg_rmsnorm_fwd(const float *x, const float *w, float eps, float *y, float *rstd, int32_t n, int32_t d,
                   void *stream);

/* seq_of[t] = the packed sequence holding row t. */
int cg_seq_of(const int64_t *seq_start, int32_t n_seqs, int32_t *seq_of, void *stream);

/* Causal attention inside each packed sequence with GQA (F.scaled_dot_product_attention,
 * is_causal, enable_gqa: trunk.py:159-164).  q [n, H, D] at row stride ldq, k / v [n, KVH, D]
 * at ldk / ldv; o [n, H, D] dense; lse [n, H].  Forward writes o and lse; backward reads
 * them and writes dq / dk / dv at the strides of q / k / v (and dsum [n, H]).  q, k, v, o and
 * dout start 16-byte aligned and ldq / ldk / ldv are multiples of 4. */
typedef struct {
  int32_t n, H, KVH, head_dim;
  float scale;
  const int64_t *seq_start; /* [n_seqs + 1] */
  const int32_t *seq_of;    /* [n] */
  const float *q, *k, *v;
  int64_t ldq, ldk, ldv;
  float *o;
  float *lse;
  int32_t round_bf16; /* 1: o (forward) and dq / dk / dv (backward) rounded to bf16 */
} cg_attn_train;
int cg_attn_train_fwd(const cg_attn_train *p, void *stream);
int cg_attn_train_bwd(const cg_attn_train *p, const float *dout, float *dsum, float *dq, float *dk, float *dv,
                      void *stream);

/* The whole trunk under autograd (what card_playing_gym_amd/nn/train.py's TrunkFunction
 * runs): the forward keeps, per layer, the input, both norms' outputs and statistics, q / k /
 * v, the attention output and log-sum-exp, the residual after attention and the MLP's
 * pre-activation in `saved`; the backward reads them and writes every gradient.  x, ple,
 * values and the gradients are fp32 [n, width] rows of sequences packed back to back
 * (seq_start [n_seqs + 1]); saved and scratch start 16-byte aligned. */
typedef struct {
  int32_t d_model, n_layers, n_heads, n_kv_heads, d_ff, per_layer_dim, ple_width, value_width;
  float eps;
  const int32_t *value_index; /* host [n_layers]: the layer's slot in the value lookup, -1 none */
  int32_t bf16;               /* 1: bf16 autocast rounding points (GEMM operands and outputs, attention) */
} cg_train_config;

typedef struct { /* DecoderBlock parameters (trunk.py:124-139), fp32 */
  const float *ln_attn_w, *ln_attn_b, *qkv_w, *out_w, *ln_mlp_w, *ln_mlp_b, *up_w, *up_b, *down_w, *down_b;
} cg_train_block;

typedef struct {
  float *ln_attn_w, *ln_attn_b, *qkv_w, *out_w, *ln_mlp_w, *ln_mlp_b, *up_w, *up_b, *down_w, *down_b;
} cg_train_block_grads;

typedef struct {
  cg_train_block_grads *blocks; /* host array [n_layers] */
  float *final_dw, *final_db;
} cg_train_grads;

size_t cg_train_saved_size(const cg_train_config *c, int32_t n);
size_t cg_train_scratch_size(const cg_train_config *c, int32_t n);
int cg_trunk_train_forward(const cg_train_config *c, const cg_train_block *blocks, const float *final_w,
                           const float *final_b, const float *x, const float *ple, const float *values,
                           const int64_t *seq_start, int32_t n_seqs, int32_t n, float *hidden, void *saved,
                           size_t saved_size, void *scratch, size_t scratch_size, void *stream);
int cg_trunk_train_backward(const cg_train_config *c, const cg_train_block *blocks, const float *final_w,
                            const int64_t *seq_start, int32_t n, const float *dhidden, void *saved,
                            size_t saved_size, void *scratch, size_t scratch_size, const cg_train_grads *grads,
                            float *dx, float *dple, float *dvalues, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* CARDGYM_HIP_H */
