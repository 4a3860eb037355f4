// Policy and value heads at the readout rows in one launch (gfx950):
//
//   logits = h . Wp^T + bp                        (policy head, nn.Linear(d, n_policy))
//   values = GELU(h . W1^T + b1) . W2^T + b2      (value_mlp: Linear, GELU, Linear)
//
// cardgym/nn/model.py:12-17 evaluated at every readout row as the graphed wave does
// (cardgym/rl/graphs.py:88-104), with bf16 autocast's rounding: operands bf16, fp32
// accumulation, each Linear's output and the GELU's output rounded to bf16.
//
// A block owns 16 rows.  Its hidden rows go to an LDS panel (bf16) once; the policy chunks
// (256 columns each) and the value MLP's first layer are stages of fragment-order weights
// streamed from L2 into the eight waves' registers (the next stage's weights load during
// the current stage's MFMAs); the first layer's GELU output goes to a second LDS panel,
// and the n_value-wide second layer is a 16-lane dot product per (row, output).
#include "common.h"
#include "fragment.h"
#include "layer.h"

struct cg_heads {
  cg_heads_config cfg;
  const float *wp, *bp, *w1, *b1, *w2, *b2;
  void *packed = nullptr;  // Wp then W1, bf16 in fragment order
  size_t wp_bytes = 0, w1_bytes = 0;
};

// One block per (16 rows, stage) rather than per 16 rows (see heads_kernel).
#ifndef CG_HEADS_SPLIT
#define CG_HEADS_SPLIT 1
#endif

namespace cg {
namespace {

struct HeadArgs {
  int32_t M, d, n_policy, d_mid, n_value;
  const float *hidden;
  const void *wp, *w1;  // fragment order
  const float *bp, *b1, *w2, *b2;
  float *logits, *values;
};

__device__ __forceinline__ float round_bf16(float v) { return to_f32(from_f32<bf16>(v)); }

// SPLIT: the block's stage is blockIdx.y (policy chunk y < NP, else the value MLP), so the
// grid holds NP + 1 blocks per 16 rows; each reads its rows and one stage's weights.
// Otherwise one block runs every stage of its rows, the next stage's weights loading during
// the current one's MFMAs.
template <int NP, bool SPLIT>
__global__ __launch_bounds__(THREADS) void heads_kernel(const HeadArgs a) {
  constexpr int BM = 16;
  constexpr int S = NP + 1;  // NP policy chunks, then the value MLP's first layer
  __shared__ __align__(16) unsigned char panel[BM * ROWB];
  __shared__ __align__(16) unsigned char mid[BM * ROWB];
  __shared__ float w2s[16 * PANEL + 16];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int cw = 16 * FN * wave;
  const int m0 = blockIdx.x * BM;
  const int d = a.d;
  const uint32_t kd = kblocks_of(d);

  // This block's hidden rows, 8 floats per thread (rows past M read as 0).
  const int cpr = d / 8;
  const bool h_in = tid < BM * cpr;
  uint4 h0 = {0u, 0u, 0u, 0u}, h1 = {0u, 0u, 0u, 0u};
  if (h_in) {
    const Rsrc rh = rsrc(a.hidden, uint32_t(a.M) * uint32_t(d) * 4);
    const uint32_t off = (uint32_t(m0 + tid / cpr) * d + 8 * (tid % cpr)) * 4;
    h0 = bload16(rh, off);
    h1 = bload16(rh, off + 16);
  }
  auto slice = [&](int s) {
    if (s < NP) return Slice{rsrc(opaque_ptr(a.wp), uint32_t(a.n_policy) * kd * 64), kd, (PANEL * s + cw) / 16, 0};
    return Slice{rsrc(opaque_ptr(a.w1), uint32_t(a.d_mid) * kd * 64), kd, cw / 16, 0};
  };
  uint4 wbuf[2][KS][FN];
  load_slice(wbuf[0], slice(SPLIT ? int(blockIdx.y) : 0), lane);
  if (!SPLIT && S > 1) load_slice(wbuf[1], slice(1), lane);
  // The value MLP's second layer (W2 then b2, at most 16 x PANEL + 16 floats) is requested
  // now and parked in LDS after the first layer, so no global round trip follows the barrier.
  constexpr int W2R = (16 * PANEL + 16 + THREADS - 1) / THREADS;
  const bool value_block = !SPLIT || int(blockIdx.y) == NP;
  const int nw2 = a.n_value * a.d_mid;
  float w2r[W2R];
#pragma unroll
  for (int q = 0; q < W2R; ++q) {
    const int i = tid + q * THREADS;
    w2r[q] = !value_block ? 0.f : i < nw2 ? a.w2[i] : i < nw2 + a.n_value ? a.b2[i - nw2] : 0.f;
  }

  // Zero both panels (k >= d and mid columns >= d_mid stay zero), then the hidden rows.
  for (int o = tid * 16; o < BM * ROWB; o += THREADS * 16) {
    const uint4 z = {0u, 0u, 0u, 0u};
    *reinterpret_cast<uint4 *>(panel + o) = z;
    *reinterpret_cast<uint4 *>(mid + o) = z;
  }
  lds_barrier();
  if (h_in) {
    const float f[8] = {__uint_as_float(h0.x), __uint_as_float(h0.y), __uint_as_float(h0.z), __uint_as_float(h0.w),
                        __uint_as_float(h1.x), __uint_as_float(h1.y), __uint_as_float(h1.z), __uint_as_float(h1.w)};
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = uint32_t(from_f32<bf16>(f[2 * e]).bits) | uint32_t(from_f32<bf16>(f[2 * e + 1]).bits) << 16;
    *reinterpret_cast<uint4 *>(panel + (tid / cpr) * ROWB + 16 * (tid % cpr)) = uint4{w[0], w[1], w[2], w[3]};
  }
  lds_barrier();

  // ---- policy chunk s: logits (bias and output rounded like the bf16 Linear)
  auto policy_out = [&](const f32x4 (&acc)[1][FN], int s) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = PANEL * s + cw + 16 * j + li;
      if (n >= a.n_policy) continue;
      const float bias = round_bf16(a.bp[n]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 4 * lg + r;
        if (m < a.M) gst(a.logits + int64_t(m) * a.n_policy + n, round_bf16(acc[0][j][r] + bias));
      }
    }
  };
  // ---- value MLP, first layer: GELU of the rounded pre-activation -> mid panel
  auto value_mid = [&](const f32x4 (&acc)[1][FN]) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = cw + 16 * j + li;
      if (n >= a.d_mid) continue;
      const float bias = round_bf16(a.b1[n]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float g = gelu_fast(round_bf16(acc[0][j][r] + bias));
        *reinterpret_cast<bf16 *>(mid + (4 * lg + r) * ROWB + n * 2) = from_f32<bf16>(g);
      }
    }
  };

  f32x4 acc[1][FN];
  if constexpr (SPLIT) {
    const int s = int(blockIdx.y);
    zero<1>(acc);
    stage_mma<1>(acc, panel, wbuf[0], slice(s), false, opaque_lane(lane));
    if (s < NP) {
      policy_out(acc, s);
      return;
    }
    value_mid(acc);
  } else {
#pragma clang loop unroll(full)
    for (int s = 0; s < S; ++s) {
      const bool refill = s + 2 < S;
      const Slice nx = slice(refill ? s + 2 : s);
      uint4(&cur)[KS][FN] = wbuf[s & 1];
      zero<1>(acc);
      stage_mma<1>(acc, panel, cur, nx, refill, opaque_lane(lane));
      if (s < NP) policy_out(acc, s);
      else value_mid(acc);
    }
  }
#pragma unroll
  for (int q = 0; q < W2R; ++q) {
    const int i = tid + q * THREADS;
    if (i < nw2 + a.n_value) w2s[i] = round_bf16(w2r[q]);
  }
  lds_barrier();

  // ---- value MLP, second layer: one 16-lane group per (row, output)
  const int p = tid & 15;
  for (int idx = tid >> 4; idx < BM * a.n_value; idx += THREADS / 16) {
    const int row = idx / a.n_value, o = idx % a.n_value;
    float sum = 0.f;
    for (int k = p; k < a.d_mid; k += 16)
      sum = fmaf(to_f32(*reinterpret_cast<const bf16 *>(mid + row * ROWB + k * 2)), w2s[o * a.d_mid + k], sum);
    sum = sum16(sum);
    const int m = m0 + row;
    if (p == 0 && m < a.M) gst(a.values + int64_t(m) * a.n_value + o, round_bf16(sum + w2s[nw2 + o]));
  }
}

bool heads_supported(const cg_heads_config &c) {
  return c.d_model > 0 && c.d_model <= PANEL && c.d_model % 16 == 0 && c.n_policy > 0 && c.n_policy % 16 == 0 &&
         c.n_policy <= 4 * PANEL && c.d_mid > 0 && c.d_mid <= PANEL && c.d_mid % 16 == 0 && c.n_value >= 1 &&
         c.n_value <= 16;
}

void pack(cg_heads &h, hipStream_t s) {
  char *base = static_cast<char *>(h.packed);
  launch_pack_fragments(h.wp, base, h.cfg.n_policy, h.cfg.d_model, s);
  launch_pack_fragments(h.w1, base + h.wp_bytes, h.cfg.d_mid, h.cfg.d_model, s);
}

void release(cg_heads *h) {
  if (h->packed) (void)hipFree(h->packed);
  delete h;
}

}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

int cg_heads_create(const cg_heads_config *config, const float *policy_w, const float *policy_b,
                    const float *value_w1, const float *value_b1, const float *value_w2,
                    const float *value_b2, cg_heads **out) {
  cg_heads *h = nullptr;
  int status = guarded([&] {
    CG_REQUIRE(config && out, CG_ERR_INVALID, "config and out are required");
    CG_REQUIRE(policy_w && policy_b && value_w1 && value_b1 && value_w2 && value_b2, CG_ERR_INVALID,
               "every head weight and bias is required");
    CG_REQUIRE(heads_supported(*config), CG_ERR_UNSUPPORTED,
               "heads: d_model and d_mid must be multiples of 16 up to 256, n_policy a multiple of 16 "
               "up to 1024, n_value 1..16");
    h = new cg_heads();
    h->cfg = *config;
    h->wp = policy_w;
    h->bp = policy_b;
    h->w1 = value_w1;
    h->b1 = value_b1;
    h->w2 = value_w2;
    h->b2 = value_b2;
    h->wp_bytes = (packed_fragment_bytes(config->n_policy, config->d_model) + 255) & ~size_t(255);
    h->w1_bytes = packed_fragment_bytes(config->d_mid, config->d_model);
    CG_HIP(hipMalloc(&h->packed, h->wp_bytes + h->w1_bytes));
    pack(*h, nullptr);
    CG_HIP(hipStreamSynchronize(nullptr));
    *out = h;
  });
  if (status != CG_OK && h) release(h);
  return status;
}

int cg_heads_refresh(cg_heads *heads, void *stream) {
  return guarded([&] {
    CG_REQUIRE(heads != nullptr, CG_ERR_INVALID, "heads is NULL");
    pack(*heads, as_stream(stream));
  });
}

int cg_heads_destroy(cg_heads *heads) {
  return guarded([&] {
    if (heads) release(heads);
  });
}

int cg_heads_forward(const cg_heads *heads, const float *hidden, int32_t m, float *logits,
                     float *values, void *stream) {
  return guarded([&] {
    CG_REQUIRE(heads != nullptr, CG_ERR_INVALID, "heads is NULL");
    CG_REQUIRE(m >= 0, CG_ERR_INVALID, "negative row count");
    if (m == 0) return;
    CG_REQUIRE(hidden && logits && values, CG_ERR_INVALID, "hidden, logits and values are required");
    const cg_heads_config &c = heads->cfg;
    HeadArgs a{};
    a.M = m;
    a.d = c.d_model;
    a.n_policy = c.n_policy;
    a.d_mid = c.d_mid;
    a.n_value = c.n_value;
    a.hidden = hidden;
    a.wp = heads->packed;
    a.w1 = static_cast<const char *>(heads->packed) + heads->wp_bytes;
    a.bp = heads->bp;
    a.b1 = heads->b1;
    a.w2 = heads->w2;
    a.b2 = heads->b2;
    a.logits = logits;
    a.values = values;
    const unsigned blocks = unsigned((int64_t(m) + 15) / 16);
    const int np = (c.n_policy + PANEL - 1) / PANEL;
    const dim3 grid(blocks, CG_HEADS_SPLIT ? unsigned(np + 1) : 1u);
    hipStream_t s = as_stream(stream);
    switch (np) {
      case 1:
        heads_kernel<1, CG_HEADS_SPLIT><<<grid, THREADS, 0, s>>>(a);
        break;
      case 2:
        heads_kernel<2, CG_HEADS_SPLIT><<<grid, THREADS, 0, s>>>(a);
        break;
      case 3:
        heads_kernel<3, CG_HEADS_SPLIT><<<grid, THREADS, 0, s>>>(a);
        break;
      default:
        heads_kernel<4, CG_HEADS_SPLIT><<<grid, THREADS, 0, s>>>(a);
    }
    CG_LAUNCHED();
  });
}

}  // extern "C"
