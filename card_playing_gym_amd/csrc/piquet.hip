// Piquet's token embedder on gfx950 (cardgym/games/piquet/model.py:128-341):
//
//   x      = sum_f fields[tok_f + off_f]  +  summary(cards)        (bf16, autocast)
//   ple    = sum_f ple_fields[tok_f + off_f]                       (bf16)
//   values = sum_f value_fields[tok_f + off_f]                     (bf16)
//   cards  = GridNorm(grid after the grid blocks)                  (fp32, [32 cards, width])
//
// with the card grid of each token: grid[s, r] = code[code of card (s, r)] + rank[r], then per
// block: n = GridNorm(grid); along = rank convolution of each suit row (zero padded) + bias;
// pooled = mean of n over suits; across = pooled . Wa^T; grid += out(GELU(along + across)).
// Rounding follows bf16 autocast: GEMM operands bf16 with fp32 accumulation and bf16 outputs
// (bias added before the rounding), GELU on its bf16 input, bf16 + bf16 rounded once; the
// residual grid and the norms stay fp32.
//
// Two launches.  piquet_fields_kernel: one thread per (token, 8 columns) of the three tables
// side by side (bf16 copies), summing the token's 32 field rows in fp32.  card_grid_kernel:
// 16 tokens per block, 8 waves; each wave carries two tokens (64 card rows = four 16-row
// MFMA tiles, the residual grid in its registers) through every grid block on its own --
// the convolution, the suit pooling and both projections stay inside the wave's tokens --
// then the block's 16 tokens form one 16-row tile for the summary projection.
#include <algorithm>

#include "common.h"
#include "fragment.h"
#include "layer.h"

namespace {
constexpr int MAX_LAYERS = 4;
constexpr int SUITS = 4, RANKS = 8, CARDS = 32, FIELDS = 32, WIDTH = 32;
}  // namespace

struct cg_piquet {
  cg_piquet_config cfg;
  int32_t offsets[FIELDS];
  const float *fields, *ple_fields, *value_fields, *code, *rank, *grid_norm, *summary;
  cg_piquet_block blocks[MAX_LAYERS];
  void *packed = nullptr;  // bf16: tables side by side, then per block conv / across / out
                           // fragments, then the summary's fragments
  size_t table_bytes = 0, conv_bytes = 0, across_bytes = 0, out_bytes = 0, summary_bytes = 0;
};

namespace cg {
namespace {

struct PiquetArgs {
  int32_t n, D, P, V, rows, layers, kw;
  int64_t ld_tokens;
  float eps;
  int32_t offsets[FIELDS];
  const int64_t *tokens;
  const bf16 *table;  // [rows, D + P + V]
  const float *code, *rank, *grid_norm;
  const float *norm[MAX_LAYERS], *along_b[MAX_LAYERS], *out_b[MAX_LAYERS];
  const void *conv[MAX_LAYERS], *across[MAX_LAYERS], *out[MAX_LAYERS];
  const void *summary;
  bf16 *x, *ple, *values;
  float *cards;
  int32_t *flag;
};

__device__ __forceinline__ float round_bf16(float v) { return to_f32(from_f32<bf16>(v)); }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return uint32_t(from_f32<bf16>(lo).bits) | (uint32_t(from_f32<bf16>(hi).bits) << 16);
}

// ---- field sums -------------------------------------------------------------------------
__global__ __launch_bounds__(256) void piquet_fields_kernel(const PiquetArgs a) {
  const int width = a.D + a.P + a.V;
  const int chunks = width / 8;
  const int64_t total = int64_t(a.n) * chunks;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t t = i / chunks;
    const int c = int(i % chunks);
    const int64_t *tok = a.tokens + t * a.ld_tokens;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    bool bad = false;
#pragma unroll 8
    for (int f = 0; f < FIELDS; ++f) {
      const int64_t id = tok[f] + a.offsets[f];
      if (id < 0 || id >= a.rows) {
        bad = true;
        continue;
      }
      const uint4 v = *reinterpret_cast<const uint4 *>(a.table + id * width + 8 * c);
      acc[0] += bf16_lo(v.x);
      acc[1] += bf16_hi(v.x);
      acc[2] += bf16_lo(v.y);
      acc[3] += bf16_hi(v.y);
      acc[4] += bf16_lo(v.z);
      acc[5] += bf16_hi(v.z);
      acc[6] += bf16_lo(v.w);
      acc[7] += bf16_hi(v.w);
    }
    if (bad && a.flag) a.flag[0] = 1;
    const uint4 out = {pack2(acc[0], acc[1]), pack2(acc[2], acc[3]), pack2(acc[4], acc[5]), pack2(acc[6], acc[7])};
    int col = 8 * c;
    bf16 *dst;
    int ld;
    if (col < a.D) {
      dst = a.x;
      ld = a.D;
    } else if (col < a.D + a.P) {
      dst = a.ple;
      ld = a.P;
      col -= a.D;
    } else {
      dst = a.values;
      ld = a.V;
      col -= a.D + a.P;
    }
    *reinterpret_cast<uint4 *>(dst + t * ld + col) = out;
  }
}

// ---- the card grid ----------------------------------------------------------------------
constexpr int GT = 16;          // tokens per block
constexpr int GWAVES = 8;       // two tokens per wave
constexpr int NROW = 80;        // LDS bytes per normalised card row: 32 bf16 + 16 pad
constexpr int MAX_PAD = 3;      // kernel taps up to 7
constexpr int PROW = CARDS * WIDTH * 2 + 16;  // LDS bytes per token of the summary panel

template <int H>
struct GridShape {
  static constexpr int HJ = H / 16;                 // hidden column tiles
  static constexpr int HK = H / 32;                 // out-projection k-steps
  static constexpr int HROW = H * 2 + 16;           // LDS bytes per GELU row
  static constexpr int NB = 2 * SUITS * (RANKS + 2 * MAX_PAD) * NROW;  // normalised rows
  static constexpr int HB = 2 * CARDS * HROW;                         // GELU rows
  static constexpr int SCRATCH = NB > HB ? NB : HB;
  static constexpr int ACROSS = 2 * RANKS * H * 2;
};

// Row statistics over the 32 columns a lane group holds as g[q][0..1][e]: the 16 lanes of a
// DPP row share the card rows (4 lg + e) and hold columns li and 16 + li.
__device__ __forceinline__ void rms_scale(const f32x4 (&g)[4][2], float eps, float (&inv)[4][4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ss = sum16(g[q][0][e] * g[q][0][e] + g[q][1][e] * g[q][1][e]);
      inv[q][e] = rsqrtf(ss * (1.0f / WIDTH) + eps);
    }
}

template <int H, int CT>
__global__ __launch_bounds__(64 * GWAVES) void card_grid_kernel(const PiquetArgs a) {
  using S = GridShape<H>;
  constexpr int HJ = S::HJ, HK = S::HK;
  __shared__ __align__(16) unsigned char scratch[GWAVES][S::SCRATCH];
  __shared__ __align__(16) unsigned char across_lds[GWAVES][S::ACROSS];
  __shared__ __align__(16) unsigned char panel[GT * PROW];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  unsigned char *nb = scratch[wave];
  unsigned char *hb = scratch[wave];  // the GELU rows reuse the normalised rows' space
  unsigned char *acr = across_lds[wave];
  const int t0 = blockIdx.x * GT + 2 * wave;  // this wave's first token
  const int pad = a.kw / 2, rs = RANKS + 2 * pad;

  // ---- the initial grid: code + rank embeddings, g[q][j][e] = grid[card row 16 q + 4 lg + e]
  //      [column 16 j + li]; card row = 32 (token) + card.
  f32x4 g[4][2];
  bool bad = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = min(t0 + q / 2, a.n - 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int card = (q & 1) * 16 + 4 * lg + e;
      int64_t code = a.tokens[int64_t(t) * a.ld_tokens + FIELDS + card];
      if (code < 0 || code >= 12) {
        bad = true;
        code = -1;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int w = 16 * j + li;
        const float ce = code >= 0 ? a.code[code * WIDTH + w] : 0.f;
        g[q][j][e] = ce + a.rank[(card & 7) * WIDTH + w];
      }
    }
  }
  if (bad && a.flag) a.flag[0] = 1;

  for (int layer = 0; layer < a.layers; ++layer) {
    // ---- n = GridNorm(grid) -> bf16 rows, each suit row framed by `pad` zero rows
    {
      float inv[4][4];
      rms_scale(g, a.eps, inv);
      float nw[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) nw[j] = a.norm[layer][16 * j + li];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int card = (q & 1) * 16 + 4 * lg + e;
          const int sr = (q >> 1) * SUITS + card / RANKS;
          unsigned char *row = nb + (sr * rs + pad + (card & 7)) * NROW;
#pragma unroll
          for (int j = 0; j < 2; ++j)
            *reinterpret_cast<bf16 *>(row + (16 * j + li) * 2) = from_f32<bf16>(g[q][j][e] * inv[q][e] * nw[j]);
        }
      // Zero frame rows (the GELU rows of the previous block overwrote them).
      for (int i = lane; i < 2 * SUITS * 2 * pad * 4; i += 64) {
        const int part = i & 3, k = (i >> 2) % (2 * pad), sr = (i >> 2) / (2 * pad);
        const int r = k < pad ? k : RANKS + k;
        *reinterpret_cast<uint4 *>(nb + (sr * rs + r) * NROW + 16 * part) = uint4{0u, 0u, 0u, 0u};
      }
    }
    __syncthreads();

    // ---- along: tap k of output rank o reads input rank o + k - pad
    f32x4 acc[4][HJ];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < HJ; ++j) acc[q][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4 *conv = static_cast<const uint4 *>(a.conv[layer]);
    for (int tap = 0; tap < a.kw; ++tap) {
      uint4 b[HJ];
#pragma unroll
      for (int j = 0; j < HJ; ++j) b[j] = conv[(tap * HJ + j) * 64 + lane];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int sr = (q >> 1) * SUITS + (q & 1) * 2 + li / RANKS;
        const uint4 av = *reinterpret_cast<const uint4 *>(nb + (sr * rs + (li & 7) + tap) * NROW + 16 * lg);
#pragma unroll
        for (int j = 0; j < HJ; ++j) acc[q][j] = mma(av, b[j], acc[q][j]);
      }
    }

    // ---- pooled (mean over suits, rounded to bf16) straight into an A fragment: row li =
    //      (token li / 8, rank li % 8), k = 8 lg .. 8 lg + 7
    {
      float p[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < SUITS; ++s) {
        const uint4 v = *reinterpret_cast<const uint4 *>(nb + (((li >> 3) * SUITS + s) * rs + pad + (li & 7)) * NROW + 16 * lg);
        p[0] += bf16_lo(v.x);
        p[1] += bf16_hi(v.x);
        p[2] += bf16_lo(v.y);
        p[3] += bf16_hi(v.y);
        p[4] += bf16_lo(v.z);
        p[5] += bf16_hi(v.z);
        p[6] += bf16_lo(v.w);
        p[7] += bf16_hi(v.w);
      }
      const uint4 pv = {pack2(0.25f * p[0], 0.25f * p[1]), pack2(0.25f * p[2], 0.25f * p[3]),
                        pack2(0.25f * p[4], 0.25f * p[5]), pack2(0.25f * p[6], 0.25f * p[7])};
      const uint4 *acw = static_cast<const uint4 *>(a.across[layer]);
#pragma unroll
      for (int j = 0; j < HJ; ++j) {
        const f32x4 c = mma(pv, acw[j * 64 + lane], f32x4{0.f, 0.f, 0.f, 0.f});
        // across rows 4 lg + e = (token (4 lg + e) / 8, rank (4 lg + e) % 8), column 16 j + li
#pragma unroll
        for (int e = 0; e < 4; ++e)
          *reinterpret_cast<bf16 *>(acr + ((4 * lg + e) * H + 16 * j + li) * 2) = from_f32<bf16>(c[e]);
      }
    }
    __syncthreads();

    // ---- GELU(along + bias + across) -> bf16 rows (hidden on k) for the out-projection
#pragma unroll
    for (int j = 0; j < HJ; ++j) {
      const int h = 16 * j + li;
      const float bias = round_bf16(a.along_b[layer][h]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int card = (q & 1) * 16 + 4 * lg + e;
          const float along = round_bf16(acc[q][j][e] + bias);
          const float across = to_f32(*reinterpret_cast<const bf16 *>(acr + (((q >> 1) * RANKS + (card & 7)) * H + h) * 2));
          const float m = round_bf16(along + across);
          *reinterpret_cast<bf16 *>(hb + ((q >> 1) * CARDS + card) * S::HROW + h * 2) = from_f32<bf16>(gelu_fast(m));
        }
    }
    __syncthreads();

    // ---- grid += out(GELU rows) + bias (bf16), fp32 residual
    {
      const uint4 *ow = static_cast<const uint4 *>(a.out[layer]);
      uint4 b[2][HK];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int ks = 0; ks < HK; ++ks) b[j][ks] = ow[(j * HK + ks) * 64 + lane];
      float ob[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) ob[j] = round_bf16(a.out_b[layer][16 * j + li]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 o[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int ks = 0; ks < HK; ++ks) {
          const uint4 av = *reinterpret_cast<const uint4 *>(hb + (q * 16 + li) * S::HROW + (32 * ks + 8 * lg) * 2);
#pragma unroll
          for (int j = 0; j < 2; ++j) o[j] = mma(av, b[j][ks], o[j]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) g[q][j][e] += round_bf16(o[j][e] + ob[j]);
      }
    }
    __syncthreads();
  }

  // ---- cards = GridNorm(grid): fp32 out, bf16 into the summary panel (token row, k = card
  //      * 32 + column)
  {
    float inv[4][4];
    rms_scale(g, a.eps, inv);
    float nw[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) nw[j] = a.grid_norm[16 * j + li];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = t0 + q / 2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int card = (q & 1) * 16 + 4 * lg + e;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int w = 16 * j + li;
          const float c = g[q][j][e] * inv[q][e] * nw[j];
          if (a.cards && t < a.n) gst(a.cards + (int64_t(t) * CARDS + card) * WIDTH + w, c);
          *reinterpret_cast<bf16 *>(panel + (2 * wave + q / 2) * PROW + (card * WIDTH + w) * 2) = from_f32<bf16>(c);
        }
      }
    }
  }
  __syncthreads();

  // ---- x += summary(cards): wave w owns output columns 16 CT w .. 16 CT (w + 1) - 1, K = 1024
  {
    constexpr int KB = CARDS * WIDTH / 32;  // 32 k-steps
    const uint4 *sw = static_cast<const uint4 *>(a.summary);
    f32x4 acc[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int G = 4;  // k-steps per group; the next group's weights load during this one
    uint4 cur[G][CT], nxt[G][CT];
#pragma unroll
    for (int k = 0; k < G; ++k)
#pragma unroll
      for (int c = 0; c < CT; ++c) cur[k][c] = sw[((wave * CT + c) * KB + k) * 64 + lane];
#pragma unroll
    for (int k0 = 0; k0 < KB; k0 += G) {
      if (k0 + G < KB) {
#pragma unroll
        for (int k = 0; k < G; ++k)
#pragma unroll
          for (int c = 0; c < CT; ++c) nxt[k][c] = sw[((wave * CT + c) * KB + k0 + G + k) * 64 + lane];
      }
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const uint4 av = *reinterpret_cast<const uint4 *>(panel + li * PROW + (32 * (k0 + k) + 8 * lg) * 2);
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[c] = mma(av, cur[k][c], acc[c]);
      }
      if (k0 + G < KB) {
#pragma unroll
        for (int k = 0; k < G; ++k)
#pragma unroll
          for (int c = 0; c < CT; ++c) cur[k][c] = nxt[k][c];
      }
    }
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int col = 16 * (wave * CT + c) + li;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = blockIdx.x * GT + 4 * lg + e;
        if (t >= a.n) continue;
        bf16 *xp = a.x + int64_t(t) * a.D + col;
        *xp = from_f32<bf16>(to_f32(*xp) + round_bf16(acc[c][e]));
      }
    }
  }
}

// ---- weight packing ------------------------------------------------------------------------
// Convolution weight [H, 32, KW] -> per tap, per 16-column tile, the B fragment of each lane:
// lane (li, lg) holds W[16 j + li][8 lg .. 8 lg + 7][tap].
__global__ void pack_conv_kernel(const float *__restrict__ w, bf16 *__restrict__ dst, int32_t H, int32_t kw) {
  const int64_t total = int64_t(kw) * H * WIDTH;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int e = int(i & 7), lane = int((i >> 3) & 63);
    const int64_t blk = i >> 9;
    const int j = int(blk % (H / 16)), tap = int(blk / (H / 16));
    const int h = 16 * j + (lane & 15), wcol = 8 * (lane >> 4) + e;
    dst[i] = from_f32<bf16>(w[(int64_t(h) * WIDTH + wcol) * kw + tap]);
  }
}

// Field tables side by side in bf16: dst[r, c] over [fields | ple | values].
__global__ void pack_table_kernel(const float *__restrict__ t0, const float *__restrict__ t1,
                                  const float *__restrict__ t2, bf16 *__restrict__ dst, int32_t rows, int32_t D,
                                  int32_t P, int32_t V) {
  const int width = D + P + V;
  const int64_t total = int64_t(rows) * width;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / width;
    const int c = int(i % width);
    float v;
    if (c < D) v = t0[r * D + c];
    else if (c < D + P) v = t1[r * P + (c - D)];
    else v = t2[r * V + (c - D - P)];
    dst[i] = from_f32<bf16>(v);
  }
}

unsigned grid_of(int64_t total) { return unsigned(std::min<int64_t>((total + 255) / 256, 4096)); }

void pack(cg_piquet &p, hipStream_t s) {
  const cg_piquet_config &c = p.cfg;
  char *base = static_cast<char *>(p.packed);
  pack_table_kernel<<<grid_of(int64_t(c.table_rows) * (c.d_model + c.ple_width + c.value_width)), 256, 0, s>>>(
      p.fields, p.ple_fields, p.value_fields, reinterpret_cast<bf16 *>(base), c.table_rows, c.d_model, c.ple_width,
      c.value_width);
  CG_LAUNCHED();
  char *at = base + p.table_bytes;
  for (int l = 0; l < c.card_layers; ++l) {
    pack_conv_kernel<<<grid_of(int64_t(c.card_kernel) * c.card_hidden * WIDTH), 256, 0, s>>>(
        p.blocks[l].along_w, reinterpret_cast<bf16 *>(at), c.card_hidden, c.card_kernel);
    CG_LAUNCHED();
    at += p.conv_bytes;
    launch_pack_fragments(p.blocks[l].across_w, at, c.card_hidden, WIDTH, s);
    at += p.across_bytes;
    launch_pack_fragments(p.blocks[l].out_w, at, WIDTH, c.card_hidden, s);
    at += p.out_bytes;
  }
  launch_pack_fragments(p.summary, at, c.d_model, CARDS * WIDTH, s);
}

size_t round256(size_t v) { return (v + 255) & ~size_t(255); }

bool piquet_supported(const cg_piquet_config &c) {
  return c.card_width == WIDTH && (c.card_hidden == 32 || c.card_hidden == 64) && c.card_kernel >= 1 &&
         c.card_kernel <= 2 * MAX_PAD + 1 && c.card_kernel % 2 == 1 && c.card_layers >= 0 &&
         c.card_layers <= MAX_LAYERS && c.d_model % 128 == 0 && c.d_model >= 128 && c.d_model <= 512 &&
         c.d_model % 8 == 0 && c.ple_width >= 0 && c.ple_width % 8 == 0 && c.value_width >= 0 &&
         c.value_width % 8 == 0 && c.table_rows > 0;
}

void release(cg_piquet *p) {
  if (p->packed) (void)hipFree(p->packed);
  delete p;
}

}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

int cg_piquet_create(const cg_piquet_config *config, const int32_t *field_offsets, const float *fields,
                     const float *ple_fields, const float *value_fields, const float *code, const float *rank,
                     const cg_piquet_block *blocks, const float *grid_norm, const float *summary,
                     cg_piquet **out) {
  cg_piquet *p = nullptr;
  int status = guarded([&] {
    CG_REQUIRE(config && out && field_offsets, CG_ERR_INVALID, "config, field_offsets and out are required");
    CG_REQUIRE(piquet_supported(*config), CG_ERR_UNSUPPORTED,
               "piquet embedder: card width 32, card hidden 32 or 64, odd card kernel up to 7, at most 4 grid "
               "blocks, d_model 128 / 256 / 384 / 512, table widths multiples of 8");
    const cg_piquet_config &c = *config;
    CG_REQUIRE(fields && code && rank && grid_norm && summary, CG_ERR_INVALID, "a required parameter is NULL");
    CG_REQUIRE((c.ple_width == 0) == (ple_fields == nullptr) && (c.value_width == 0) == (value_fields == nullptr),
               CG_ERR_INVALID, "ple / value tables must be given exactly when their width is non-zero");
    CG_REQUIRE(c.card_layers == 0 || blocks, CG_ERR_INVALID, "grid block parameters are required");
    for (int l = 0; l < c.card_layers; ++l) {
      const cg_piquet_block &b = blocks[l];
      CG_REQUIRE(b.norm && b.along_w && b.along_b && b.across_w && b.out_w && b.out_b, CG_ERR_INVALID,
                 "a grid block parameter is NULL");
    }
    p = new cg_piquet();
    p->cfg = c;
    for (int f = 0; f < FIELDS; ++f) p->offsets[f] = field_offsets[f];
    p->fields = fields;
    p->ple_fields = ple_fields;
    p->value_fields = value_fields;
    p->code = code;
    p->rank = rank;
    p->grid_norm = grid_norm;
    p->summary = summary;
    for (int l = 0; l < c.card_layers; ++l) p->blocks[l] = blocks[l];
    p->table_bytes = round256(size_t(c.table_rows) * (c.d_model + c.ple_width + c.value_width) * 2);
    p->conv_bytes = round256(size_t(c.card_kernel) * c.card_hidden * WIDTH * 2);
    p->across_bytes = round256(packed_fragment_bytes(c.card_hidden, WIDTH));
    p->out_bytes = round256(packed_fragment_bytes(WIDTH, c.card_hidden));
    p->summary_bytes = round256(packed_fragment_bytes(c.d_model, CARDS * WIDTH));
    const size_t total = p->table_bytes + size_t(c.card_layers) * (p->conv_bytes + p->across_bytes + p->out_bytes) +
                         p->summary_bytes;
    CG_HIP(hipMalloc(&p->packed, total));
    pack(*p, nullptr);
    CG_HIP(hipStreamSynchronize(nullptr));
    *out = p;
  });
  if (status != CG_OK && p) release(p);
  return status;
}

int cg_piquet_refresh(cg_piquet *p, void *stream) {
  return guarded([&] {
    CG_REQUIRE(p != nullptr, CG_ERR_INVALID, "piquet embedder is NULL");
    pack(*p, as_stream(stream));
  });
}

int cg_piquet_destroy(cg_piquet *p) {
  return guarded([&] {
    if (p) release(p);
  });
}

int cg_piquet_embed(const cg_piquet *p, const int64_t *tokens, int64_t ld_tokens, int32_t n, void *x, void *ple,
                    void *values, float *cards, int32_t *flag, void *stream) {
  return guarded([&] {
    CG_REQUIRE(p != nullptr, CG_ERR_INVALID, "piquet embedder is NULL");
    CG_REQUIRE(n >= 0, CG_ERR_INVALID, "negative token count");
    if (n == 0) return;
    const cg_piquet_config &c = p->cfg;
    CG_REQUIRE(tokens && x, CG_ERR_INVALID, "tokens and x are required");
    CG_REQUIRE(ld_tokens >= FIELDS + CARDS, CG_ERR_INVALID, "a token row holds 32 fields and 32 card codes");
    CG_REQUIRE((c.ple_width == 0 || ple) && (c.value_width == 0 || values), CG_ERR_INVALID,
               "ple / values outputs are required for non-zero table widths");
    PiquetArgs a{};
    a.n = n;
    a.D = c.d_model;
    a.P = c.ple_width;
    a.V = c.value_width;
    a.rows = c.table_rows;
    a.layers = c.card_layers;
    a.kw = c.card_kernel;
    a.ld_tokens = ld_tokens;
    a.eps = c.eps;
    for (int f = 0; f < FIELDS; ++f) a.offsets[f] = p->offsets[f];
    a.tokens = tokens;
    const char *base = static_cast<const char *>(p->packed);
    a.table = reinterpret_cast<const bf16 *>(base);
    a.code = p->code;
    a.rank = p->rank;
    a.grid_norm = p->grid_norm;
    const char *at = base + p->table_bytes;
    for (int l = 0; l < c.card_layers; ++l) {
      a.norm[l] = p->blocks[l].norm;
      a.along_b[l] = p->blocks[l].along_b;
      a.out_b[l] = p->blocks[l].out_b;
      a.conv[l] = at;
      at += p->conv_bytes;
      a.across[l] = at;
      at += p->across_bytes;
      a.out[l] = at;
      at += p->out_bytes;
    }
    a.summary = at;
    a.x = static_cast<bf16 *>(x);
    a.ple = static_cast<bf16 *>(ple);
    a.values = static_cast<bf16 *>(values);
    a.cards = cards;
    a.flag = flag;
    hipStream_t s = as_stream(stream);
    const int64_t chunks = int64_t(n) * ((c.d_model + c.ple_width + c.value_width) / 8);
    piquet_fields_kernel<<<grid_of(chunks), 256, 0, s>>>(a);
    CG_LAUNCHED();
    const unsigned blocks = unsigned((int64_t(n) + GT - 1) / GT);
    const int ct = c.d_model / 128;
    auto go = [&](auto kernel) {
      kernel<<<blocks, 64 * GWAVES, 0, s>>>(a);
      CG_LAUNCHED();
    };
    if (c.card_hidden == 64) {
      if (ct == 1) go(card_grid_kernel<64, 1>);
      else if (ct == 2) go(card_grid_kernel<64, 2>);
      else if (ct == 3) go(card_grid_kernel<64, 3>);
      else go(card_grid_kernel<64, 4>);
    } else {
      if (ct == 1) go(card_grid_kernel<32, 1>);
      else if (ct == 2) go(card_grid_kernel<32, 2>);
      else if (ct == 3) go(card_grid_kernel<32, 3>);
      else go(card_grid_kernel<32, 4>);
    }
  });
}

}  // extern "C"
