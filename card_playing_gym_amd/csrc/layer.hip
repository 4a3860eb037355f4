// Fused per-layer kernel of the bf16 trunk step (gfx950).
//
// After a layer's attention, everything up to the next layer's attention runs in one
// launch per block of BM token rows (DecoderBlock._finish + Trunk._add_ple +
// DecoderBlock._qkv + KVCache.write_step of the next block, cardgym/nn/trunk.py:141-157,
// 318-333, cardgym/nn/kv_cache.py:84-105; for the last block the final LayerNorm at the
// readout tokens, trunk.py:429):
//
//   x1 = x + attn . W_out^T                     (stage "out")
//   h  = LN(x1; ln_mlp)                        -> LDS panel (bf16)
//   for each 256-wide chunk c of d_ff:         (stages "up c", "down c")
//     g_c = GELU(h . W_up[c]^T + b_up[c])      -> LDS (bf16, double-buffered)
//     acc += g_c . W_down[:, c]^T
//   x2 = x1 + acc + b_down (+ per-layer embedding)
//   h' = LN(x2; next ln_attn)                  -> LDS panel
//   [q | k | v] = h' . W_qkv^T                 (stages "qkv c"): q stored, k / v (+ value
//                                               embedding) written to the pool
//
// Work split: the block's eight waves split every stage's output columns (32 each); the
// panel (BM rows x 256 k, bf16) is read from LDS by all eight waves, the weights stream
// from L2 straight into each wave's registers: lane l loads 16 bytes of W row
// (col 16 j + l % 16) at k = 32 ks + 8 (l / 16), one v_mfma_f32_16x16x32_bf16 operand
// fragment, so weights never touch LDS.  Every product is formed transposed (W . A^T: the
// weight fragment is the MFMA's A operand), so a lane ends up holding four consecutive
// columns of one row (layer_dev.h).  Each fragment register is refilled with the next
// stage's fragment right after its MFMAs, so a stage of weights (128 KB per block) is in
// flight while the current one multiplies.  Row statistics of the LayerNorms reduce over
// the four lane groups with lane swaps, then over the eight waves in LDS.
#include "common.h"
#include "fragment.h"
#include "layer.h"
#include "layer_dev.h"

namespace cg {
namespace {

template <int BM, int MODE, int NC, int NQ>
__global__ __launch_bounds__(THREADS) void layer_tail_kernel(const TailArgs a) {
  __shared__ __align__(16) unsigned char panel[BM * ROWB];
  __shared__ __align__(16) unsigned char hbuf[hbufs_of<BM>()][BM * ROWB];
  __shared__ float red[2 * WAVES * BM + 2 * BM];
  extern __shared__ __align__(16) float dyn[];
  tail_body<BM, MODE, NC, NQ>(a, blockIdx.x, panel, hbuf, red, dyn);
}

// W [N, K] fp32 row-major -> bf16 fragment order (see Slice), k padded to 32 with zeros.
__global__ void pack_fragments_kernel(const float *__restrict__ src, bf16 *__restrict__ dst, int32_t N,
                                      int32_t K, int32_t kblocks) {
  const int64_t total = int64_t(N) * kblocks * 32;
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += int64_t(gridDim.x) * blockDim.x) {
    const int t = int(e & 7);
    const int lane = int((e >> 3) & 63);
    const int64_t blk = e >> 9;
    const int kb = int(blk % kblocks), nb = int(blk / kblocks);
    const int row = 16 * nb + (lane & 15), k = 32 * kb + 8 * (lane >> 4) + t;
    dst[e] = k < K ? from_f32<bf16>(src[int64_t(row) * K + k]) : bf16{0};
  }
}

}  // namespace

size_t packed_fragment_bytes(int N, int K) { return size_t(N) * ((K + 31) / 32) * 32 * 2; }

void launch_pack_fragments(const float *src, void *dst, int N, int K, hipStream_t s) {
  CG_REQUIRE(N % 16 == 0, CG_ERR_UNSUPPORTED, "fragment packing needs a multiple of 16 rows");
  const int kblocks = (K + 31) / 32;
  const int64_t total = int64_t(N) * kblocks * 32;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  pack_fragments_kernel<<<unsigned(blocks), 256, 0, s>>>(src, static_cast<bf16 *>(dst), N, K, kblocks);
  CG_LAUNCHED();
}

namespace {
// The fused kernel's GELU (gelu_bf16x4) over an array of bf16 values, four per thread.
__global__ __launch_bounds__(256) void gelu_apply_kernel(const uint2 *__restrict__ x, uint2 *__restrict__ y, int64_t n4) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += int64_t(gridDim.x) * blockDim.x) {
    const uint2 v = x[i];
    const u32x2_t g = gelu_bf16x4(u32x2_t{v.x, v.y});
    y[i] = uint2{g[0], g[1]};
  }
}
}  // namespace

void launch_gelu_apply(const void *x, void *y, int64_t n, hipStream_t s) {
  CG_REQUIRE(n % 4 == 0, CG_ERR_UNSUPPORTED, "GELU: a multiple of 4 values");
  CG_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 7) == 0, CG_ERR_UNSUPPORTED,
             "GELU: 8-byte aligned arrays");
  const int64_t n4 = n / 4;
  if (n4 == 0) return;
  int64_t blocks = (n4 + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  gelu_apply_kernel<<<unsigned(blocks), 256, 0, s>>>(static_cast<const uint2 *>(x), static_cast<uint2 *>(y), n4);
  CG_LAUNCHED();
}

bool tail_supported(int d, int d_ff, int n_qkv, int head_dim) {
  return d > 0 && d <= PANEL && d % 16 == 0 && d_ff > 0 && d_ff % 16 == 0 && d_ff <= 4 * PANEL &&
         n_qkv > 0 && n_qkv % 16 == 0 && n_qkv <= 3 * PANEL && head_dim > 0 && head_dim % 4 == 0;
}

namespace {
// Compute units of the current device (block rounds of the row-block choice below).
int device_cus() {
  static thread_local int dev = -1, cus = 256;
  int d = 0;
  if (hipGetDevice(&d) == hipSuccess && d != dev) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) == hipSuccess && n > 0) cus = n;
    dev = d;
  }
  return cus;
}

// Rows per block: one block per CU at a time (eight waves), so a launch takes
// ceil(blocks / CUs) rounds of one block's life, measured on MI355X at d 256 / d_ff 1024
// (kernel trace, configs 3 and 5 with the height forced) as about 17.5 us + 0.28 us per row:
// 22.6 / 25.7 / 30.5 / 35.4 us at 16 / 32 / 48 / 64 rows.  Most of a block's life is the
// weight stream (the layer's 1.38 MB from L2 into every CU), which does not grow with the
// rows.  16 rows keep the decode step (4096 rows) at one round of 256 blocks; config 4's
// 8192 rows take one round of 32-row blocks, config 5's ~35k packed rows three rounds of
// 48-row blocks (102 us against 122 at 32 rows and 120 at 64), prefill-sized launches 64.
// Taller blocks (80 and 96 rows, one weight stage in flight) measured 52 and 59 us per block
// and lost at both config 5 and prefill.
int tail_rows_per_block(int64_t M) {
#ifdef CG_TAIL_FORCE_BM
  if (M >= 0) return CG_TAIL_FORCE_BM;  // measurement builds only
#endif
  const int64_t cus = device_cus();
  int best = 16;
  double best_t = 1e30;
  for (int bm : {16, 32, 48, 64}) {
    const int64_t rounds = ((M + bm - 1) / bm + cus - 1) / cus;
    const double t = double(rounds) * (17.5 + 0.28 * bm);
    if (t < best_t - 1e-9) {
      best_t = t;
      best = bm;
    }
  }
  return best;
}
}  // namespace

void launch_tail(const TailArgs &a, hipStream_t s) {
  CG_REQUIRE(tail_supported(a.d, a.d_ff, a.n_qkv, a.head_dim), CG_ERR_UNSUPPORTED, "fused layer: unsupported shape");
  if (a.M <= 0) return;
  // 32-bit offsets: residual rows and queries through buffer descriptors and unsigned
  // products, slot-row offsets of the pool as int.
  CG_REQUIRE(int64_t(a.M) * a.d * 4 < (int64_t(1) << 32) && int64_t(a.M) * a.q_cols * 4 < (int64_t(1) << 32) &&
                 int64_t(a.kv_heads) * a.max_len * a.head_dim < (int64_t(1) << 31),
             CG_ERR_RANGE, "fused layer: step too large for 32-bit row offsets");
  const int bm = tail_rows_per_block(a.M);
  const int nc = (a.d_ff + PANEL - 1) / PANEL, nq = (a.n_qkv + PANEL - 1) / PANEL;
  const int mode = !a.do_post ? 0 : (a.final_ln ? 2 : 1);
  auto go = [&](auto k16, auto k32, auto k48, auto k64) {
    // Params (layer_dev.h): (nc + 5) PANEL floats, the QKV column map, token slots and rows.
    const size_t dyn = (size_t(nc) + 5) * PANEL * 4 + (3 * PANEL / 4) * 8 + size_t(bm) * (8 + 4);
    const unsigned grid = unsigned((a.M + bm - 1) / bm);
    if (bm == 64) k64<<<grid, THREADS, dyn, s>>>(a);
    else if (bm == 48) k48<<<grid, THREADS, dyn, s>>>(a);
    else if (bm == 32) k32<<<grid, THREADS, dyn, s>>>(a);
    else k16<<<grid, THREADS, dyn, s>>>(a);
    CG_LAUNCHED();
  };
#define CG_TAIL_CASE(MODE, NC, NQ)                                                       \
  if (mode == MODE && (MODE == 0 || nc == NC) && (MODE == 2 || nq == NQ))                \
    return go(layer_tail_kernel<16, MODE, NC, NQ>, layer_tail_kernel<32, MODE, NC, NQ>, \
              layer_tail_kernel<48, MODE, NC, NQ>, layer_tail_kernel<64, MODE, NC, NQ>)
  CG_TAIL_CASE(0, 1, 1); CG_TAIL_CASE(0, 1, 2); CG_TAIL_CASE(0, 1, 3);
  CG_TAIL_CASE(1, 1, 1); CG_TAIL_CASE(1, 1, 2); CG_TAIL_CASE(1, 1, 3);
  CG_TAIL_CASE(1, 2, 1); CG_TAIL_CASE(1, 2, 2); CG_TAIL_CASE(1, 2, 3);
  CG_TAIL_CASE(1, 3, 1); CG_TAIL_CASE(1, 3, 2); CG_TAIL_CASE(1, 3, 3);
  CG_TAIL_CASE(1, 4, 1); CG_TAIL_CASE(1, 4, 2); CG_TAIL_CASE(1, 4, 3);
  CG_TAIL_CASE(2, 1, 1); CG_TAIL_CASE(2, 2, 1); CG_TAIL_CASE(2, 3, 1); CG_TAIL_CASE(2, 4, 1);
#undef CG_TAIL_CASE
  throw Error(CG_ERR_UNSUPPORTED, "fused layer: unsupported chunk counts");
}

}  // namespace cg
