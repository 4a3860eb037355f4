// Internal interface of the MFMA projection kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cg {

// What happens to the fp32 accumulator C[M, N] = A . W^T.
enum EpiMode : int {
  EPI_STORE = 0,      // out = C + bias                                  (out_dtype)
  EPI_GELU = 1,       // out = gelu(C + bias)                            (out_dtype)
  EPI_RESID = 2,      // resid += C + bias + ple_scale * ple[m, ple_off + n % ple_dim]
  EPI_QKV = 3,        // q | k | v split; k, v (+ value embedding) appended to the KV pool
  EPI_SCALE_ADD = 4,  // out = (C + addend) * scale                      (out_dtype)
  EPI_RESID_LN = 5,   // EPI_RESID, then out = LayerNorm(resid row)      (out_dtype); N <= 256
};

struct GemmArgs {
  int32_t M, N, K;
  int32_t compute;  // CG_F32 or CG_BF16: storage type of A and W and operand type of the MFMA
  const void *A;    // [M, K] row-major, type `compute`
  int64_t lda;
  const void *W;    // [N, K] row-major, type `compute`
  const float *bias;
  // Epilogue.
  int32_t epi;
  void *out;
  int32_t out_dtype;
  int64_t ldo;
  float *resid;
  int64_t ldr;
  const float *ple;
  int64_t ld_ple;
  int32_t ple_off, ple_dim;
  float ple_scale;
  const void *addend;
  int32_t add_dtype;  // CG_F32, or CG_BF16: the sum and the scaled sum round to bf16
  int32_t round_c;    // round C + bias to bf16 first (an autocast Linear's output)
  int64_t ld_add;
  float scale;
  const float *ln_w, *ln_b;  // EPI_RESID_LN
  float eps;
  // EPI_QKV: columns [0, q_cols) -> q (fp32, ld ldo); then kv_heads * head_dim columns of
  // K and as many of V, appended at (tok_row[m], head, tok_pos[m]).
  int32_t q_cols;
  void *kc, *vc;
  int32_t kv_dtype, kv_heads, head_dim, max_len;
  const int32_t *tok_row, *tok_pos;
  const float *vemb;
  int64_t ld_vemb;
  int32_t vemb_off;  // < 0: no value embedding
};

void launch_gemm(const GemmArgs &g, hipStream_t stream);

// y[i] = LayerNorm(x[index ? index[i] : i]) (fp32 statistics), stored as y_dtype.
void launch_layernorm_rows(const float *x, const int32_t *index, const float *w, const float *b,
                           float eps, void *y, int32_t y_dtype, int32_t n, int32_t d,
                           hipStream_t stream);

// y = x (fp32) rounded to `dtype` (CG_BF16) or copied (CG_F32), n elements.
void launch_convert(const float *x, void *y, int32_t dtype, int64_t n, hipStream_t stream);

}  // namespace cg
