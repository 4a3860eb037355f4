// Masked softmax and inverse-CDF sampling of policy rows on the device (gfx950):
// cardgym/rl/ppo.py:75-94 (masked_probabilities, sample_rows), which the reference runs
// in numpy on the host after copying each wave's logits back (cardgym/rl/selfplay.py:
// 532-567).  One wave per row, reproducing numpy's float32 arithmetic order:
//   probabilities: max over the legal entries (NaN propagates), exp(x - max) on legal
//     entries and 0 elsewhere, the normaliser summed in numpy's pairwise order (blocks of
//     at most 128 with eight running sums, halves split at multiples of 8), and a
//     correctly rounded division.  Only the float32 exp can differ from numpy's (by an
//     ulp; numpy's exp is CPU-specific code).
//   sampling: the running float32 sum of each row in index order, compared as float64
//     with the row's uniform; the count of entries below it, clamped to the last legal
//     index and replaced by it when the entry is illegal.  Given the same probabilities
//     and uniforms the result is the reference's, bit for bit.
#include <cmath>

#include "common.h"

namespace cg {
namespace {

constexpr int ROWS_PER_BLOCK = 4;  // one wave per row
constexpr int MAX_WIDTH = 4096;    // six halvings leave blocks of at most 128 entries

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// numpy's float32 pairwise sum of w[off .. off + n) (n <= 128 << LEVEL), by the whole wave:
// a block of at most 128 keeps eight running sums r[j] = w[j] + w[j + 8] + ... (lane j),
// combined as ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)) and followed by the n % 8
// remaining entries one by one; larger ranges split at n / 2 rounded down to a multiple of
// 8.  Every lane returns the sum.
template <int LEVEL>
__device__ float pairwise_sum(const float *w, int off, int n, int lane) {
  if (n > 128) {
    if constexpr (LEVEL > 0) {
      int n2 = n / 2;
      n2 -= n2 % 8;
      const float left = pairwise_sum<LEVEL - 1>(w, off, n2, lane);
      return left + pairwise_sum<LEVEL - 1>(w, off + n2, n - n2, lane);
    }
  }
  const float *a = w + off;
  if (n < 8) {
    float res = 0.f;
    for (int i = 0; i < n; ++i) res += a[i];
    return res;
  }
  const int body = n - n % 8;
  float r = 0.f;
  if (lane < 8) {
    r = a[lane];
    for (int i = 8; i < body; i += 8) r += a[i + lane];
  }
  const float r0 = __shfl(r, 0, 64), r1 = __shfl(r, 1, 64), r2 = __shfl(r, 2, 64), r3 = __shfl(r, 3, 64);
  const float r4 = __shfl(r, 4, 64), r5 = __shfl(r, 5, 64), r6 = __shfl(r, 6, 64), r7 = __shfl(r, 7, 64);
  float res = ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7));
  for (int i = body; i < n; ++i) res += a[i];
  return res;
}

__global__ __launch_bounds__(64 * ROWS_PER_BLOCK) void masked_probabilities_kernel(
    const float *__restrict__ logits, int64_t ld_logits, const uint8_t *__restrict__ mask, int64_t ld_mask,
    int32_t rows, int32_t width, float *__restrict__ probs, int64_t ld_probs) {
  extern __shared__ float wrow[];  // [ROWS_PER_BLOCK][width]: the row's weights
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = blockIdx.x * ROWS_PER_BLOCK + wave;
  if (row >= rows) return;  // whole wave
  const float *x = logits + int64_t(row) * ld_logits;
  const uint8_t *legal = mask + int64_t(row) * ld_mask;
  float *w = wrow + wave * width;
  // max over the legal entries; a NaN among them makes it NaN, as numpy's max does
  float m = -INFINITY;
  int nan = 0;
  for (int i = lane; i < width; i += 64) {
    const float v = legal[i] ? x[i] : -INFINITY;
    if (v != v) nan = 1;
    else m = fmaxf(m, v);
  }
  m = wave_max(m);
  if (__any(nan)) m = NAN;
  for (int i = lane; i < width; i += 64) w[i] = legal[i] ? expf(x[i] - m) : 0.f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float total = pairwise_sum<6>(w, 0, width, lane);
  float *p = probs + int64_t(row) * ld_probs;
  for (int i = lane; i < width; i += 64) p[i] = w[i] / total;
}

__global__ __launch_bounds__(64 * ROWS_PER_BLOCK) void sample_rows_kernel(
    const float *__restrict__ probs, int64_t ld_probs, const uint8_t *__restrict__ mask, int64_t ld_mask,
    const double *__restrict__ uniforms, int32_t rows, int32_t width, int64_t *__restrict__ sampled) {
  extern __shared__ float prow[];  // [ROWS_PER_BLOCK][width rounded up to 4]
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = blockIdx.x * ROWS_PER_BLOCK + wave;
  if (row >= rows) return;  // whole wave
  const int w4 = (width + 3) & ~3;
  float *pr = prow + wave * w4;
  const float *p = probs + int64_t(row) * ld_probs;
  const uint8_t *legal = mask + int64_t(row) * ld_mask;
  int last = -1;
  for (int i = lane; i < w4; i += 64) {
    pr[i] = i < width ? p[i] : 0.f;
    if (i < width && legal[i]) last = i;
  }
  for (int o = 32; o > 0; o >>= 1) last = max(last, __shfl_xor(last, o, 64));
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // The running float32 sums in index order (np.cumsum), by one lane; the padding adds 0.
  if (lane == 0) {
    float c = 0.f;
    for (int i = 0; i < w4; i += 4) {
      float4 q = *reinterpret_cast<const float4 *>(pr + i);
      c = i == 0 ? q.x : c + q.x;
      q.x = c;
      c += q.y;
      q.y = c;
      c += q.z;
      q.z = c;
      c += q.w;
      q.w = c;
      *reinterpret_cast<float4 *>(pr + i) = q;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // float c < double u  <=>  c < t, t the least float >= u (NaN and +-inf included).
  const double u = uniforms[row];
  float t = float(u);
  if (double(t) < u) t = nextafterf(t, INFINITY);
  int below = 0;
  for (int i = lane; i < width; i += 64) below += pr[i] < t;
  for (int o = 32; o > 0; o >>= 1) below += __shfl_xor(below, o, 64);
  if (lane != 0) return;
  const int last_legal = last >= 0 ? last : width - 1;
  int s = below < last_legal ? below : last_legal;
  if (!legal[s]) s = last_legal;
  sampled[row] = s;
}

}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

int cg_masked_probabilities(const float *logits, int64_t ld_logits, const uint8_t *mask, int64_t ld_mask,
                            int32_t rows, int32_t width, float *probs, int64_t ld_probs, void *stream) {
  return guarded([&] {
    CG_REQUIRE(rows >= 0 && width >= 0, CG_ERR_INVALID, "rows and width must be non-negative");
    if (rows == 0 || width == 0) return;
    CG_REQUIRE(logits && mask && probs, CG_ERR_INVALID, "logits, mask and probs are required");
    CG_REQUIRE(ld_logits >= width && ld_mask >= width && ld_probs >= width, CG_ERR_INVALID,
               "row strides must be at least the width");
    CG_REQUIRE(width <= MAX_WIDTH, CG_ERR_UNSUPPORTED, "masked_probabilities: rows wider than 4096");
    const size_t lds = size_t(ROWS_PER_BLOCK) * width * 4;
    masked_probabilities_kernel<<<(rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK, 64 * ROWS_PER_BLOCK, lds,
                                  as_stream(stream)>>>(logits, ld_logits, mask, ld_mask, rows, width, probs, ld_probs);
    CG_LAUNCHED();
  });
}

int cg_sample_rows(const float *probs, int64_t ld_probs, const uint8_t *mask, int64_t ld_mask,
                   const double *uniforms, int32_t rows, int32_t width, int64_t *sampled, void *stream) {
  return guarded([&] {
    CG_REQUIRE(rows >= 0 && width >= 0, CG_ERR_INVALID, "rows and width must be non-negative");
    if (rows == 0) return;
    CG_REQUIRE(width > 0, CG_ERR_INVALID, "cannot sample from rows of width 0");
    CG_REQUIRE(probs && mask && uniforms && sampled, CG_ERR_INVALID, "probs, mask, uniforms and sampled are required");
    CG_REQUIRE(ld_probs >= width && ld_mask >= width, CG_ERR_INVALID, "row strides must be at least the width");
    CG_REQUIRE(width <= MAX_WIDTH, CG_ERR_UNSUPPORTED, "sample_rows: rows wider than 4096");
    const size_t lds = size_t(ROWS_PER_BLOCK) * ((width + 3) & ~3) * 4;
    sample_rows_kernel<<<(rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK, 64 * ROWS_PER_BLOCK, lds, as_stream(stream)>>>(
        probs, ld_probs, mask, ld_mask, uniforms, rows, width, sampled);
    CG_LAUNCHED();
  });
}

}  // extern "C"
