// Ragged GQA decode attention read straight from the KV pool.
//
// Replaces the gather + masked-softmax path of DecoderBlock.forward_ragged
// (cardgym/nn/trunk.py:216-256) and the fp16 / span<=64 CUDA op
// (cardgym/nn/cuda_decode.py:46-151).  Semantics: query t of sequence b, head hd, sees
// keys k < min(key_lengths[b] + t, span) of cache row rows[b], KV head hd / G; scores are
// q.k * scale, softmax in fp32, output sum_k p_k v_k.
//
// Layout of the work (gfx950, wave64):
//   * one workgroup per (sequence, KV head): the group's G query heads and all of the
//     sequence's new tokens share every K/V byte the workgroup reads, so the pool is read
//     once per (sequence, KV head) whatever G and T are;
//   * WAVES waves split the key range in 64-key blocks (wave w takes blocks w, w+WAVES..);
//   * inside a wave, lane = 4 * slot + e: slot (16 of them) owns keys 16 r + slot of each
//     block (r = 0..3), e owns head_dim / 4 consecutive dims.  A wave-wide load of one r
//     reads 16 consecutive keys = one contiguous 16 x head_dim segment of the row;
//   * each lane keeps its own running max / sum / accumulator per query (no cross-lane
//     traffic in the key loop except the 2-step quad reduction of the dot products); the
//     16 slots and the waves are merged once at the end (log-sum-exp merge);
//   * softmax in base 2 with log2(e) folded into the query scale.
#include <algorithm>
#include <type_traits>

#include "attention.h"
#include "attn_dev.h"

#include "common.h"

namespace cg {
namespace {

// DPP quad permutations: lane i of each group of 4 reads lane i^1 / i^2.
__device__ __forceinline__ float quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}

// Loads N consecutive elements of T as wide vectors and widens them to fp32.
template <typename T, int N>
__device__ __forceinline__ void load_widen(const T *__restrict__ p, float (&out)[N]) {
  constexpr int BYTES = N * int(sizeof(T));
  T tmp[N];
  if constexpr (BYTES % 16 == 0) {
    uint4 raw[BYTES / 16];
#pragma unroll
    for (int i = 0; i < BYTES / 16; ++i) raw[i] = reinterpret_cast<const uint4 *>(p)[i];
    __builtin_memcpy(tmp, raw, BYTES);
  } else if constexpr (BYTES % 8 == 0) {
    uint2 raw[BYTES / 8];
#pragma unroll
    for (int i = 0; i < BYTES / 8; ++i) raw[i] = reinterpret_cast<const uint2 *>(p)[i];
    __builtin_memcpy(tmp, raw, BYTES);
  } else if constexpr (BYTES % 4 == 0) {
    uint32_t raw[BYTES / 4];
#pragma unroll
    for (int i = 0; i < BYTES / 4; ++i) raw[i] = reinterpret_cast<const uint32_t *>(p)[i];
    __builtin_memcpy(tmp, raw, BYTES);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) tmp[i] = p[i];
  }
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = to_f32(tmp[i]);
}

constexpr int KEYS_PER_BLOCK = 64;
constexpr int QB = 4;  // queries per pass over the keys

template <typename TKV, int D, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void decode_attention_kernel(AttnArgs a) {
  constexpr int DPL = D / 4;
  __shared__ float merge_m[WAVES][QB], merge_l[WAVES][QB];
  __shared__ float merge_acc[WAVES][QB][D];

  const int unit = blockIdx.x;
  const int b = unit / a.kv_heads, h = unit % a.kv_heads;
  // The wave index is uniform: readfirstlane lets the compiler keep everything derived
  // from it (unit, row, descriptors) in scalar registers.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = lane >> 2, e = lane & 3;
  const int G = a.n_heads / a.kv_heads;

  const int64_t row = a.rows ? a.rows[b] : int64_t(b);
  int64_t tok0 = 0, count = a.T;
  if (a.seq_start) {
    // Packed descriptors come from the caller: clamp the range to the packed tokens.
    int64_t lo = a.seq_start[b], hi = a.seq_start[b + 1];
    lo = lo < 0 ? 0 : (lo > a.n_tokens ? a.n_tokens : lo);
    hi = hi < lo ? lo : (hi > a.n_tokens ? a.n_tokens : hi);
    tok0 = lo;
    count = hi - lo;
  }
  const int64_t q_base = a.seq_start ? tok0 * a.q_st : int64_t(b) * a.q_sb;
  const int64_t o_base = a.seq_start ? tok0 * a.o_st : int64_t(b) * a.o_sb;
  const int64_t kl = a.key_lengths[b] + a.kl_add;
  const bool row_ok = row >= 0 && row < a.capacity;

  const int64_t head_off = (row * a.kv_heads + h) * int64_t(a.max_len) * D + e * DPL;
  const TKV *__restrict__ kbase = static_cast<const TKV *>(a.k) + head_off;
  const TKV *__restrict__ vbase = static_cast<const TKV *>(a.v) + head_off;

  const int nq = int(count) * G;
  for (int qb = 0; qb < nq; qb += QB) {
    float q[QB][DPL];
    int lim[QB];
    int maxlim = 0;
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      const int m = qb + j;
      if (m < nq) {
        const int t = m / G, g = m % G;
        const int64_t qo = q_base + int64_t(h * G + g) * a.q_sh + int64_t(t) * a.q_st + e * DPL;
#pragma unroll
        for (int i = 0; i < DPL; ++i) q[j][i] = load_any(a.q, a.q_dtype, qo + i) * a.scale_log2;
        int64_t l = kl + t;
        if (l > a.span) l = a.span;
        if (!row_ok || l < 0) l = 0;
        lim[j] = int(l);
      } else {
#pragma unroll
        for (int i = 0; i < DPL; ++i) q[j][i] = 0.f;
        lim[j] = 0;
      }
      maxlim = lim[j] > maxlim ? lim[j] : maxlim;
    }

    float mx[QB], sum[QB], acc[QB][DPL];
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      mx[j] = NEG_BIG;
      sum[j] = 0.f;
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[j][i] = 0.f;
    }

    for (int kb = wave * KEYS_PER_BLOCK; kb < maxlim; kb += WAVES * KEYS_PER_BLOCK) {
      float kf[4][DPL], vf[4][DPL];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb + 16 * r + slot;
        if (key < maxlim) {
          load_widen<TKV, DPL>(kbase + int64_t(key) * D, kf[r]);
          load_widen<TKV, DPL>(vbase + int64_t(key) * D, vf[r]);
        } else {
#pragma unroll
          for (int i = 0; i < DPL; ++i) kf[r][i] = vf[r][i] = 0.f;
        }
      }
      float s[4][QB];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
          float p = 0.f;
#pragma unroll
          for (int i = 0; i < DPL; ++i) p = fmaf(q[j][i], kf[r][i], p);
          p += quad_xor1(p);
          p += quad_xor2(p);
          const int key = kb + 16 * r + slot;
          s[r][j] = key < lim[j] ? p : -INFINITY;
        }
      }
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        const float blk = fmaxf(fmaxf(s[0][j], s[1][j]), fmaxf(s[2][j], s[3][j]));
        const float mnew = fmaxf(mx[j], blk);
        const float corr = exp2f(mx[j] - mnew);
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = exp2f(s[r][j] - mnew);
        sum[j] = sum[j] * corr + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          float v = acc[j][i] * corr;
          v = fmaf(p[0], vf[0][i], v);
          v = fmaf(p[1], vf[1][i], v);
          v = fmaf(p[2], vf[2][i], v);
          v = fmaf(p[3], vf[3][i], v);
          acc[j][i] = v;
        }
        mx[j] = mnew;
      }
    }

    // Merge the 16 slots of the wave (lanes differing in bits 2..5).
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        const float mo = __shfl_xor(mx[j], off, 64);
        const float so = __shfl_xor(sum[j], off, 64);
        const float mnew = fmaxf(mx[j], mo);
        const float c1 = exp2f(mx[j] - mnew), c2 = exp2f(mo - mnew);
        sum[j] = sum[j] * c1 + so * c2;
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          const float ao = __shfl_xor(acc[j][i], off, 64);
          acc[j][i] = acc[j][i] * c1 + ao * c2;
        }
        mx[j] = mnew;
      }
    }

    if constexpr (WAVES > 1) {
      if (slot == 0) {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
          if (e == 0) {
            merge_m[wave][j] = mx[j];
            merge_l[wave][j] = sum[j];
          }
#pragma unroll
          for (int i = 0; i < DPL; ++i) merge_acc[wave][j][e * DPL + i] = acc[j][i];
        }
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int j = 0; j < QB; ++j) {
          float m = merge_m[0][j];
#pragma unroll
          for (int w = 1; w < WAVES; ++w) m = fmaxf(m, merge_m[w][j]);
          float l = 0.f, o[DPL];
#pragma unroll
          for (int i = 0; i < DPL; ++i) o[i] = 0.f;
#pragma unroll
          for (int w = 0; w < WAVES; ++w) {
            const float c = exp2f(merge_m[w][j] - m);
            l += merge_l[w][j] * c;
#pragma unroll
            for (int i = 0; i < DPL; ++i) o[i] += merge_acc[w][j][e * DPL + i] * c;
          }
          sum[j] = l;
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[j][i] = o[i];
        }
      }
      __syncthreads();
    }

    if (wave == 0 && slot == 0) {
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        const int m = qb + j;
        if (m < nq) {
          const int t = m / G, g = m % G;
          const int64_t oo = o_base + int64_t(h * G + g) * a.o_sh + int64_t(t) * a.o_st + e * DPL;
          const float inv = sum[j] > 0.f ? 1.0f / sum[j] : 0.f;
#pragma unroll
          for (int i = 0; i < DPL; ++i) store_any(a.out, a.out_dtype, oo + i, acc[j][i] * inv);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Matrix-core path (head_dim 32 / 64): one wave per (sequence, KV head), four independent
// waves per workgroup.  For each tile of KT keys:
//   S^T[key, query] = K . Q^T on MFMA: the A operand is 16 keys x 32 dims straight from the
//     pool (lane l reads 16 bytes of key l % 16 at dims 8 (l / 16): one coalesced load of
//     a contiguous 1 KB segment per 16 keys); the B operand is the group's queries
//     (G heads x the sequence's new tokens, 16 per column tile), pre-scaled by
//     scale * log2(e) and rounded to the cache type as the reference rounds q
//     (trunk.py:222).
//   Online softmax on the MFMA output layout: lane l holds keys 4 (l / 16) + i of query
//     column l % 16; the running max is shared by the four lanes of a column.
//   O^T[dim, query] += V^T . P^T on MFMA: P^T is the lane's own probabilities (the k
//     ordering of the product is chosen to match where the scores already are, so P never
//     moves between lanes); V^T is read from a padded per-wave LDS copy of the V tile.
// Query t of the sequence sees keys < min(key_lengths + t, span): per-column masks.
template <typename TKV, int D, int NQT>
__global__ __launch_bounds__(256) void decode_attention_mfma_kernel(AttnArgs a) {
  constexpr int ES = int(sizeof(TKV));
  constexpr bool F32 = ES == 4;
  constexpr int KT = F32 ? 32 : 64;   // keys per tile
  constexpr int NJ = KT / 16;         // 16-key score tiles per key tile
  constexpr int DK = D / 32;          // 32-dim slices of a key (S^T k-steps)
  constexpr int DH = D / 16;          // 16-dim slices of the output (O^T row tiles)
  constexpr int ROW = D * ES + 8;     // padded LDS row of V (bytes): conflict-free transposed reads
  __shared__ __align__(16) unsigned char vtile[4][KT * ROW];

  // The wave index is uniform: readfirstlane lets the compiler keep everything derived
  // from it (unit, row, pointers) in scalar registers.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int unit = blockIdx.x * 4 + wave;
  if (unit >= a.n_seqs * a.kv_heads) return;  // the whole wave leaves; no block barriers below
  const int b = unit / a.kv_heads, h = unit % a.kv_heads;
  const int li = lane & 15, lg = lane >> 4;
  const int G = a.n_heads / a.kv_heads;
  unsigned char *vt = vtile[wave];

  const int64_t row = a.rows ? a.rows[b] : int64_t(b);
  int64_t tok0 = 0, count = a.T;
  if (a.seq_start) {
    int64_t lo = a.seq_start[b], hi = a.seq_start[b + 1];
    lo = lo < 0 ? 0 : (lo > a.n_tokens ? a.n_tokens : lo);
    hi = hi < lo ? lo : (hi > a.n_tokens ? a.n_tokens : hi);
    tok0 = lo;
    count = hi - lo;
  }
  const int64_t q_base = a.seq_start ? tok0 * a.q_st : int64_t(b) * a.q_sb;
  const int64_t o_base = a.seq_start ? tok0 * a.o_st : int64_t(b) * a.o_sb;
  const int64_t kl = a.key_lengths[b] + a.kl_add;
  const bool row_ok = row >= 0 && row < a.capacity;
  const int64_t head_off = (row * a.kv_heads + h) * int64_t(a.max_len) * D;
  const TKV *__restrict__ kbase = static_cast<const TKV *>(a.k) + head_off;
  const TKV *__restrict__ vbase = static_cast<const TKV *>(a.v) + head_off;

  const int nq = int(count) * G;
  for (int qg = 0; qg < nq; qg += NQT * 16) {
    // ---- queries of this group: column li of tile qt is query qg + 16 qt + li ----------
    int lim[NQT];
    float qf[NQT][DK][8];
    int kend = 0;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const int m = qg + 16 * qt + li;
      int l = 0;
      if (m < nq) {
        const int t = m / G, g = m % G;
        const int64_t qo = q_base + int64_t(h * G + g) * a.q_sh + int64_t(t) * a.q_st;
#pragma unroll
        for (int dk = 0; dk < DK; ++dk)
#pragma unroll
          for (int e = 0; e < 8; ++e) qf[qt][dk][e] = load_any(a.q, a.q_dtype, qo + 32 * dk + 8 * lg + e) * a.scale_log2;
        int64_t lim64 = kl + t;
        if (lim64 > a.span) lim64 = a.span;
        l = (row_ok && lim64 > 0) ? int(lim64) : 0;
      } else {
#pragma unroll
        for (int dk = 0; dk < DK; ++dk)
#pragma unroll
          for (int e = 0; e < 8; ++e) qf[qt][dk][e] = 0.f;
      }
      lim[qt] = l;
      kend = l > kend ? l : kend;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int other = __shfl_xor(kend, o, 64);
      kend = other > kend ? other : kend;
    }

    f32x4 acc[NQT][DH];
    float mrun[NQT], lsum[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      mrun[qt] = NEG_BIG;
      lsum[qt] = 0.f;
#pragma unroll
      for (int dh = 0; dh < DH; ++dh) acc[qt][dh] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // B operands of S^T (16-bit paths): the queries in the cache's type.
    typename std::conditional<F32, float, typename Mfma16<typename std::conditional<F32, bf16, TKV>::type>::vec>::type
        qv[NQT][DK];
    if constexpr (!F32) {
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
        for (int dk = 0; dk < DK; ++dk) {
          f32x8 f;
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = qf[qt][dk][e];
          qv[qt][dk] = Mfma16<TKV>::from(f);
        }
    }

    // Global -> register staging of one tile: lane l holds 8 consecutive elements of key
    // 16 j + l % 16 at dims 32 dk + 8 (l / 16), for both K and V.
    constexpr int VEC = 8 * ES / 16;  // 16-byte vectors per 8 elements
    uint4 kr[NJ][DK][VEC], vr[NJ][DK][VEC];
    auto fetch = [&](int kb) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int key = kb + 16 * j + li;
        const bool ok = key < kend;
#pragma unroll
        for (int dk = 0; dk < DK; ++dk) {
          const int64_t off = int64_t(key) * D + 32 * dk + 8 * lg;
#pragma unroll
          for (int c = 0; c < VEC; ++c) {
            kr[j][dk][c] = ok ? reinterpret_cast<const uint4 *>(kbase + off)[c] : uint4{0u, 0u, 0u, 0u};
            vr[j][dk][c] = ok ? reinterpret_cast<const uint4 *>(vbase + off)[c] : uint4{0u, 0u, 0u, 0u};
          }
        }
      }
    };

    if (kend > 0) fetch(0);
    for (int kb = 0; kb < kend; kb += KT) {
      // V tile into LDS (row = key within the tile), K kept in registers.
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int dk = 0; dk < DK; ++dk)
#pragma unroll
          for (int c = 0; c < VEC; ++c) {
            unsigned char *dst = vt + (16 * j + li) * ROW + (32 * dk + 8 * lg) * ES + 16 * c;
            const uint4 v = vr[j][dk][c];
            reinterpret_cast<uint2 *>(dst)[0] = uint2{v.x, v.y};
            reinterpret_cast<uint2 *>(dst)[1] = uint2{v.z, v.w};
          }
      uint4 kcur[NJ][DK][VEC];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int dk = 0; dk < DK; ++dk)
#pragma unroll
          for (int c = 0; c < VEC; ++c) kcur[j][dk][c] = kr[j][dk][c];
      if (kb + KT < kend) fetch(kb + KT);  // next tile in flight during this one
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // ---- scores -------------------------------------------------------------------
      f32x4 sc[NQT][NJ];
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int dk = 0; dk < DK; ++dk) {
            if constexpr (F32) {
              float kf[8];
              __builtin_memcpy(kf, &kcur[j][dk][0], 32);
#pragma unroll
              for (int e = 0; e < 8; ++e)
                s4 = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[e], qf[qt][dk][e], s4, 0, 0, 0);
            } else {
              typename Mfma16<TKV>::vec kvec;
              __builtin_memcpy(&kvec, &kcur[j][dk][0], 16);
              s4 = Mfma16<TKV>::mma(kvec, qv[qt][dk], s4);
            }
          }
          sc[qt][j] = s4;
        }

      // ---- online softmax per query column --------------------------------------------
      float p[NQT][NJ][4];
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        float tmax = NEG_BIG;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + 16 * j + 4 * lg + i;
            const float v = key < lim[qt] ? sc[qt][j][i] : -INFINITY;
            sc[qt][j][i] = v;
            tmax = fmaxf(tmax, v);
          }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(mrun[qt], tmax);
        const float corr = fast_exp2(mrun[qt] - mnew);
        float psum = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[qt][j][i] = fast_exp2(sc[qt][j][i] - mnew);
            psum += p[qt][j][i];
          }
        lsum[qt] = lsum[qt] * corr + psum;
        mrun[qt] = mnew;
#pragma unroll
        for (int dh = 0; dh < DH; ++dh) acc[qt][dh] *= corr;
      }

      // ---- O^T += V^T . P^T --------------------------------------------------------------
      if constexpr (F32) {
#pragma unroll
        for (int dh = 0; dh < DH; ++dh)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float v = *reinterpret_cast<const float *>(vt + (16 * j + 4 * lg + i) * ROW + (16 * dh + li) * 4);
#pragma unroll
              for (int qt = 0; qt < NQT; ++qt)
                acc[qt][dh] = __builtin_amdgcn_mfma_f32_16x16x4f32(v, p[qt][j][i], acc[qt][dh], 0, 0, 0);
            }
      } else {
        // k slot 8 (l / 16) + e of a 32-key chunk c is key 32 c + 16 (e / 4) + 4 (l / 16) + e % 4.
#pragma unroll
        for (int c = 0; c < KT / 32; ++c) {
          typename Mfma16<TKV>::vec pv[NQT];
#pragma unroll
          for (int qt = 0; qt < NQT; ++qt) {
            f32x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = p[qt][2 * c + (e >> 2)][e & 3];
            pv[qt] = Mfma16<TKV>::from(f);
          }
#pragma unroll
          for (int dh = 0; dh < DH; ++dh) {
            unsigned short raw[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int key = 32 * c + 16 * (e >> 2) + 4 * lg + (e & 3);
              raw[e] = *reinterpret_cast<const unsigned short *>(vt + key * ROW + (16 * dh + li) * 2);
            }
            typename Mfma16<TKV>::vec vv;
            __builtin_memcpy(&vv, raw, 16);
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) acc[qt][dh] = Mfma16<TKV>::mma(vv, pv[qt], acc[qt][dh]);
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ---- normalise and store: lane l holds dims 16 dh + 4 (l / 16) + i of query column l % 16
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      float total = lsum[qt];
      total += __shfl_xor(total, 16, 64);
      total += __shfl_xor(total, 32, 64);
      const int m = qg + 16 * qt + li;
      if (m >= nq) continue;
      const int t = m / G, g = m % G;
      const float inv = total > 0.f ? 1.0f / total : 0.f;
      const int64_t oo = o_base + int64_t(h * G + g) * a.o_sh + int64_t(t) * a.o_st;
#pragma unroll
      for (int dh = 0; dh < DH; ++dh)
#pragma unroll
        for (int i = 0; i < 4; ++i) store_any(a.out, a.out_dtype, oo + 16 * dh + 4 * lg + i, acc[qt][dh][i] * inv);
    }
  }
}

// ---------------------------------------------------------------------------------------
// 16-bit pools (bf16 / fp16), head_dim 32 / 64: the same dataflow as above with the VALU
// and LDS work per key cut down.
//   * K / V tiles arrive through a buffer descriptor over the (row, KV head) segment,
//     unconditionally (keys past the visible range are clamped onto the last visible key,
//     whose value is finite, and get probability 0), so the loads land directly in the
//     registers the MFMAs read and the next tile's loads are in flight during this tile.
//   * Masks are applied only on tiles that reach past some query's limit.
//   * The per-query running max needs one cross-lane step per tile: the four lane groups
//     holding a query column's keys meet through v_permlane16/32_swap (VALU, no LDS).  The
//     running sum stays per lane and is merged once at the end.
//   * V^T fragments for O^T += V^T . P^T come from V rows stored as loaded in LDS through
//     ds_read_b64_tr_b16: within each 16-lane group, result lane i, element e is element
//     i % 4 of the 8 bytes lane 4 e + i / 4 addressed; lane j addressing key (j / 4) of a
//     4-key run at dims 4 (j % 4) .. +3 therefore receives 4 consecutive keys of dim j.
// SPLIT waves share one (sequence, KV head): wave p of the unit takes tiles p, p + SPLIT,
// ...; their partial (max, sum, O) merge in LDS at the end (SPLIT 1: four units per block).
#ifndef TR_WAVES_PER_EU
#define TR_WAVES_PER_EU 4
#endif
#ifndef TR_LAST_MERGES
#define TR_LAST_MERGES 1
#endif
// QRAW: the queries are stored in the cache type (16-byte aligned rows); they load as they
// are and the softmax scale multiplies the fp32 scores.  Otherwise any query type is read,
// scaled and rounded to the cache type.
// Waves per SIMD the split kernel is built for: multi-tile forms at head_dim 32 keep two.
template <int NQT, int D>
#ifndef TR_MQ_WAVES_PER_EU
#define TR_MQ_WAVES_PER_EU 2
#endif
constexpr int tr_waves_per_eu() { return D == 32 ? (NQT == 1 ? TR_WAVES_PER_EU : TR_MQ_WAVES_PER_EU) : 1; }

template <typename TKV, int D, int NQT, int SPLIT, int KT, int DEPTH, bool QRAW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(tr_waves_per_eu<NQT, D>())))
void decode_attention_tr_kernel(AttnArgs a) {
  static_assert(SPLIT == 1 || SPLIT == 2 || SPLIT == 4, "a block holds 4 / SPLIT whole units");
  static_assert(KT % 32 == 0, "key tiles are whole 32-key MFMA steps");
  constexpr int NJ = KT / 16;     // 16-key score tiles per key tile
  constexpr int DK = D / 32;      // 32-dim slices of a key (S^T k-steps)
  constexpr int DH = D / 16;      // 16-dim slices of the output (O^T row tiles)
  constexpr int ROW = D * 2 + 8;  // LDS bytes per V row (8-byte aligned, rows spread over banks)
  __shared__ __align__(16) unsigned char vtile[4][KT * ROW];
  // Partial results of the SPLIT waves of a unit: max and sum per query column, O^T tiles.
  __shared__ float part_m[SPLIT > 1 ? 4 : 1][NQT][16], part_l[SPLIT > 1 ? 4 : 1][NQT][16];
  __shared__ f32x4 part_o[SPLIT > 1 ? 4 : 1][NQT][DH][64];

  // The wave index is uniform: readfirstlane lets the compiler keep everything derived
  // from it (unit, row, descriptors) in scalar registers.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Packed chunks with an order (the units by descending work, written for this step) deal
  // the longest units first, so the launch does not end on a few long ones.  An entry
  // outside [0, U) computes nothing.
  int unit = blockIdx.x * (4 / SPLIT) + wave / SPLIT;
  if (a.order && a.seq_start) {
    const int U = a.n_seqs * a.kv_heads;
    unit = unit < U ? a.order[unit] : U;
    if (unit < 0) unit = U;
  }
  const int part = wave % SPLIT;
  // Block barriers below must be reached by every wave of the block the same number of
  // times.  SPLIT 4: the block is one unit, whose waves all leave together.  SPLIT 1: no
  // barriers.  SPLIT 2 (launched for padded runs only, where every unit has the same query
  // count and so the same loop trips): a unit past the end stays and runs the loops with
  // no visible key and no store.
  const bool unit_ok = unit < a.n_seqs * a.kv_heads;
  if (!unit_ok && SPLIT != 2) return;
  // One unit per block whose queries form a single group: its waves merge through an LDS
  // counter (the last one merges) instead of two block barriers.  The counter is cleared
  // behind one barrier that every wave of the block reaches (they all have the same unit).
  __shared__ int merge_count;
  bool last_merges = false;
  if constexpr (SPLIT == 4 && TR_LAST_MERGES) {
    const int nq0 = int(a.seq_start ? 0 : a.T) * (a.n_heads / a.kv_heads);
    last_merges = !a.seq_start && gridDim.y == 1 && nq0 <= NQT * 16;
    if (last_merges) {
      if (threadIdx.x == 0) merge_count = 0;
      __syncthreads();
    }
  }
  const int b = unit_ok ? unit / a.kv_heads : 0, h = unit_ok ? unit % a.kv_heads : 0;
  const int li = lane & 15, lg = lane >> 4;
  const int G = a.n_heads / a.kv_heads;
  unsigned char *vt = vtile[wave];

  const int64_t row = a.rows ? a.rows[b] : int64_t(b);
  int64_t tok0 = 0, count = a.T;
  if (a.seq_start) {
    int64_t lo = a.seq_start[b], hi = a.seq_start[b + 1];
    lo = lo < 0 ? 0 : (lo > a.n_tokens ? a.n_tokens : lo);
    hi = hi < lo ? lo : (hi > a.n_tokens ? a.n_tokens : hi);
    tok0 = lo;
    count = hi - lo;
  }
  const int64_t q_base = a.seq_start ? tok0 * a.q_st : int64_t(b) * a.q_sb;
  const int64_t o_base = a.seq_start ? tok0 * a.o_st : int64_t(b) * a.o_sb;
  const int64_t kl = a.key_lengths[b] + a.kl_add;
  const bool row_ok = unit_ok && row >= 0 && row < a.capacity;
  // This (row, head) segment: max_len keys of D elements.
  const int64_t seg = row_ok ? (row * a.kv_heads + h) * int64_t(a.max_len) * D : 0;
  const uint32_t seg_bytes = uint32_t(a.max_len) * D * 2;
  const Rsrc kres = kv_rsrc(static_cast<const TKV *>(a.k) + seg, seg_bytes);
  const Rsrc vres = kv_rsrc(static_cast<const TKV *>(a.v) + seg, seg_bytes);

  const int nq = int(count) * G;
  // Query groups of 16 NQT are dealt over the grid's y dimension (prefill: many per unit).
  // Multi-token rows: later query groups see more keys (causal), so the grid's y dimension
  // deals them first and the launch does not end on the longest items (64 x 512 prefill:
  // 15.42 -> 15.73 M tokens/s).
  const int y0 = int(gridDim.y - 1 - blockIdx.y);
  for (int qg = y0 * NQT * 16; qg < nq; qg += gridDim.y * NQT * 16) {
    // ---- key limits of this group's queries (column li of tile qt is query qg + 16 qt + li)
    int lim[NQT];
    int kmax = 0, kmin = 0x7fffffff;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const int m = qg + 16 * qt + li;
      int l = 0;
      if (m < nq) {
        int64_t lim64 = kl + m / G;
        if (lim64 > a.span) lim64 = a.span;
        l = (row_ok && lim64 > 0) ? int(lim64) : 0;
        kmin = min(kmin, l);
      }
      lim[qt] = l;
      kmax = max(kmax, l);
    }
    // Uniform bounds: keys below kmin are visible to every query, none at or past kend.
    const int kend = __builtin_amdgcn_readfirstlane(row16_max(kmax));
    const int kfull = __builtin_amdgcn_readfirstlane(row16_min(kmin));

    // Only the query tiles holding a query of the group run (a packed chunk of a few tokens
    // fills one or two of four): the group's body is instantiated for each live-tile count,
    // so every tile loop keeps a compile-time bound.
    const int live = (nq - qg + 15) / 16;
    auto group = [&](auto live_tiles) {
    constexpr int L = decltype(live_tiles)::value;
      // Lane l holds key 16 j + l % 16 of a tile at dims 32 dk + 8 (l / 16), for K and V.
      uint4 kr[DEPTH][NJ][DK], vr[DEPTH][NJ][DK];
      auto fetch = [&](int st, int kb) {
  #pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int key = min(kb + 16 * j + li, kend - 1);
  #pragma unroll
          for (int dk = 0; dk < DK; ++dk) {
            const uint32_t off = uint32_t(key * D + 32 * dk + 8 * lg) * 2;
            kr[st][j][dk] = kv_load16(kres, off);
            vr[st][j][dk] = kv_load16(vres, off);
          }
        }
      };
      // The first DEPTH key tiles are requested before the queries, so the latencies overlap.
      if (part * KT < kend) {
  #pragma unroll
        for (int st = 0; st < DEPTH; ++st) fetch(st, part * KT + st * SPLIT * KT);
      }

      // ---- queries.  QRAW: already rounded to the cache type unscaled, as the reference rounds
      //      q (q.to(cache.dtype), trunk.py:222), loaded 16 bytes per 8 dims; the scale (times
      //      log2 e) then multiplies the fp32 scores.  Otherwise scaled by the softmax scale *
      //      log2 e and rounded to the cache type; fp32 rows at 16-byte alignment load as two
      //      float4 per 8 dims. ----------------------------------------------------------------
      const bool q4 = !QRAW && a.q_dtype == CG_F32 &&
                      ((reinterpret_cast<uintptr_t>(a.q) & 15) | (a.q_sb & 3) | (a.q_sh & 3) | (a.q_st & 3) | (q_base & 3)) == 0;
      typename Mfma16<TKV>::vec qv[NQT][DK];
  #pragma unroll
      for (int qt = 0; qt < L; ++qt) {
        const int m = qg + 16 * qt + li;
        if constexpr (QRAW) {
  #pragma unroll
          for (int dk = 0; dk < DK; ++dk) {
            if (m < nq) {
              const int64_t qo = q_base + int64_t(h * G + m % G) * a.q_sh + int64_t(m / G) * a.q_st;
              qv[qt][dk] = *reinterpret_cast<const typename Mfma16<TKV>::vec *>(static_cast<const TKV *>(a.q) + qo +
                                                                                 32 * dk + 8 * lg);
            } else {
              f32x8 z;
  #pragma unroll
              for (int e = 0; e < 8; ++e) z[e] = 0.f;
              qv[qt][dk] = Mfma16<TKV>::from(z);
            }
          }
          continue;
        }
        f32x8 f[DK];
        if (m < nq) {
          const int t = m / G, g = m % G;
          const int64_t qo = q_base + int64_t(h * G + g) * a.q_sh + int64_t(t) * a.q_st;
          if (q4) {
  #pragma unroll
            for (int dk = 0; dk < DK; ++dk) {
              const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(a.q) + qo + 32 * dk + 8 * lg);
              const float4 x0 = src[0], x1 = src[1];
              f[dk][0] = x0.x * a.scale_log2;
              f[dk][1] = x0.y * a.scale_log2;
              f[dk][2] = x0.z * a.scale_log2;
              f[dk][3] = x0.w * a.scale_log2;
              f[dk][4] = x1.x * a.scale_log2;
              f[dk][5] = x1.y * a.scale_log2;
              f[dk][6] = x1.z * a.scale_log2;
              f[dk][7] = x1.w * a.scale_log2;
            }
          } else {
  #pragma unroll
            for (int dk = 0; dk < DK; ++dk)
  #pragma unroll
              for (int e = 0; e < 8; ++e) f[dk][e] = load_any(a.q, a.q_dtype, qo + 32 * dk + 8 * lg + e) * a.scale_log2;
          }
        } else {
  #pragma unroll
          for (int dk = 0; dk < DK; ++dk)
  #pragma unroll
            for (int e = 0; e < 8; ++e) f[dk][e] = 0.f;
        }
  #pragma unroll
        for (int dk = 0; dk < DK; ++dk) qv[qt][dk] = Mfma16<TKV>::from(f[dk]);
      }

      f32x4 acc[NQT][DH];
      float mrun[NQT], lsum[NQT];
      const float sm = QRAW ? a.scale_log2 : 1.0f;  // score scale applied in the exponent
  #pragma unroll
      for (int qt = 0; qt < L; ++qt) {
        mrun[qt] = NEG_BIG;
        lsum[qt] = 0.f;
  #pragma unroll
        for (int dh = 0; dh < DH; ++dh) acc[qt][dh] = f32x4{0.f, 0.f, 0.f, 0.f};
      }

      for (int kb0 = part * KT; kb0 < kend; kb0 += DEPTH * SPLIT * KT) {
  #pragma unroll
       for (int st = 0; st < DEPTH; ++st) {
        const int kb = kb0 + st * SPLIT * KT;
        if (st > 0 && kb >= kend) break;
        // ---- scores S^T[key, query] -----------------------------------------------------
        f32x4 sc[NQT][NJ];
  #pragma unroll
        for (int qt = 0; qt < L; ++qt)
  #pragma unroll
          for (int j = 0; j < NJ; ++j) {
            f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
            for (int dk = 0; dk < DK; ++dk) {
              typename Mfma16<TKV>::vec kvec;
              __builtin_memcpy(&kvec, &kr[st][j][dk], 16);
              s4 = Mfma16<TKV>::mma(kvec, qv[qt][dk], s4);
            }
            sc[qt][j] = s4;  // QRAW: raw q.k; the scale joins the exponent below
          }
        // ---- V rows -> LDS (as loaded), then the next tile's loads ----------------------
  #pragma unroll
        for (int j = 0; j < NJ; ++j)
  #pragma unroll
          for (int dk = 0; dk < DK; ++dk) {
            unsigned char *dst = vt + (16 * j + li) * ROW + (32 * dk + 8 * lg) * 2;
            reinterpret_cast<uint2 *>(dst)[0] = uint2{vr[st][j][dk].x, vr[st][j][dk].y};
            reinterpret_cast<uint2 *>(dst)[1] = uint2{vr[st][j][dk].z, vr[st][j][dk].w};
          }
        fetch(st, kb + DEPTH * SPLIT * KT);  // clamped: past kend it re-reads the last visible key

        // ---- mask (only tiles reaching past some query's limit) --------------------------
        if (kb + KT > kfull) {
  #pragma unroll
          for (int qt = 0; qt < L; ++qt)
  #pragma unroll
            for (int j = 0; j < NJ; ++j)
  #pragma unroll
              for (int i = 0; i < 4; ++i)
                if (kb + 16 * j + 4 * lg + i >= lim[qt]) sc[qt][j][i] = -INFINITY;
        }
        // ---- online softmax per query column ----------------------------------------------
        float p[NQT][NJ][4];
  #pragma unroll
        for (int qt = 0; qt < L; ++qt) {
          float tmax = NEG_BIG;
  #pragma unroll
          for (int j = 0; j < NJ; ++j)
  #pragma unroll
            for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, sc[qt][j][i]);
          // QRAW scores are unscaled: the maximum is taken on them (the scale is positive) and
          // the scale multiplies inside the exponent's FMA, p = 2^(s * scale - max).
          tmax = xor32_max(xor16_max(tmax)) * sm;
          const float mnew = fmaxf(mrun[qt], tmax);
          const float corr = fast_exp2(mrun[qt] - mnew);
          float psum = 0.f;
  #pragma unroll
          for (int j = 0; j < NJ; ++j)
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              p[qt][j][i] = fast_exp2(fmaf(sc[qt][j][i], sm, -mnew));
              psum += p[qt][j][i];
            }
          lsum[qt] = fmaf(lsum[qt], corr, psum);
          mrun[qt] = mnew;
  #pragma unroll
          for (int dh = 0; dh < DH; ++dh) acc[qt][dh] *= corr;
        }
        // ---- O^T += V^T . P^T (k slot 8 (l / 16) + e of chunk c is key
        //      32 c + 16 (e / 4) + 4 (l / 16) + e % 4) ------------------------------------------
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  #pragma unroll
        for (int c = 0; c < KT / 32; ++c) {
          typename Mfma16<TKV>::vec pv[NQT];
  #pragma unroll
          for (int qt = 0; qt < L; ++qt) {
            f32x8 f;
  #pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = p[qt][2 * c + (e >> 2)][e & 3];
            pv[qt] = Mfma16<TKV>::from(f);
          }
  #pragma unroll
          for (int dh = 0; dh < DH; ++dh) {
            const unsigned char *src = vt + (32 * c + 4 * lg + (li >> 2)) * ROW + (16 * dh + 4 * (li & 3)) * 2;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(src));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(src + 16 * ROW));
            typename Mfma16<TKV>::vec vv;
            __builtin_memcpy(&vv, &lo, 8);
            __builtin_memcpy(reinterpret_cast<char *>(&vv) + 8, &hi, 8);
  #pragma unroll
            for (int qt = 0; qt < L; ++qt) acc[qt][dh] = Mfma16<TKV>::mma(vv, pv[qt], acc[qt][dh]);
          }
        }
       }
      }

      if constexpr (SPLIT > 1) {
        // ---- merge the unit's SPLIT partial softmax states (log-sum-exp) ------------------
  #pragma unroll
        for (int qt = 0; qt < L; ++qt) {
          lsum[qt] = xor32_sum(xor16_sum(lsum[qt]));
          if (lg == 0) {
            part_m[wave][qt][li] = mrun[qt];
            part_l[wave][qt][li] = lsum[qt];
          }
  #pragma unroll
          for (int dh = 0; dh < DH; ++dh) part_o[wave][qt][dh][lane] = acc[qt][dh];
        }
        if (last_merges) {
          // The unit's last wave to get here merges and stores; the others leave at once
          // (no block barrier: a wave with one key tile does not wait for one with two).
          // One increment per wave (lane 0), its result broadcast to the wave.
          int done = 0;
          if (lane == 0) done = __hip_atomic_fetch_add(&merge_count, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
          done = __builtin_amdgcn_readfirstlane(done);
          if (done != SPLIT - 1) return;
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  #pragma unroll
          for (int qt = 0; qt < L; ++qt) {
            float mm = part_m[0][qt][li];
  #pragma unroll
            for (int w = 1; w < SPLIT; ++w) mm = fmaxf(mm, part_m[w][qt][li]);
            float l = 0.f;
  #pragma unroll
            for (int dh = 0; dh < DH; ++dh) acc[qt][dh] = f32x4{0.f, 0.f, 0.f, 0.f};
  #pragma unroll
            for (int w = 0; w < SPLIT; ++w) {
              const float c = fast_exp2(part_m[w][qt][li] - mm);
              l = fmaf(part_l[w][qt][li], c, l);
  #pragma unroll
              for (int dh = 0; dh < DH; ++dh) acc[qt][dh] += part_o[w][qt][dh][lane] * c;
            }
            lsum[qt] = l;
          }
        } else {
        __syncthreads();
        if (part == 0) {
  #pragma unroll
          for (int qt = 0; qt < L; ++qt) {
            float mm = part_m[wave][qt][li];
  #pragma unroll
            for (int w = 1; w < SPLIT; ++w) mm = fmaxf(mm, part_m[wave + w][qt][li]);
            float l = 0.f;
  #pragma unroll
            for (int dh = 0; dh < DH; ++dh) acc[qt][dh] = f32x4{0.f, 0.f, 0.f, 0.f};
  #pragma unroll
            for (int w = 0; w < SPLIT; ++w) {
              const float c = fast_exp2(part_m[wave + w][qt][li] - mm);
              l = fmaf(part_l[wave + w][qt][li], c, l);
  #pragma unroll
              for (int dh = 0; dh < DH; ++dh) acc[qt][dh] += part_o[wave + w][qt][dh][lane] * c;
            }
            lsum[qt] = l;
          }
        }
        __syncthreads();  // partials consumed before the next query group reuses them
        if (part != 0) return;
        }
      }
      // ---- normalise and store: lane l holds dims 16 dh + 4 (l / 16) + i of query column l % 16
      const bool o4 = a.out_dtype == (sizeof(TKV) == 2 && std::is_same<TKV, bf16>::value ? CG_BF16 : CG_F16) &&
                      ((reinterpret_cast<uintptr_t>(a.out) & 7) | (a.o_sb & 3) | (a.o_sh & 3) | (a.o_st & 3) | (o_base & 3)) == 0;
  #pragma unroll
      for (int qt = 0; qt < L; ++qt) {
        const float total = SPLIT > 1 ? lsum[qt] : xor32_sum(xor16_sum(lsum[qt]));
        const int m = qg + 16 * qt + li;
        if (m >= nq || !unit_ok) continue;
        const int t = m / G, g = m % G;
        const float inv = total > 0.f ? 1.0f / total : 0.f;
        const int64_t oo = o_base + int64_t(h * G + g) * a.o_sh + int64_t(t) * a.o_st;
        if (o4) {
          // 16-bit output: each lane's 4 consecutive dims as one 8-byte non-temporal store (a
          // dirty line left in L2 is written back while the next kernel streams).
  #pragma unroll
          for (int dh = 0; dh < DH; ++dh) {
            const TKV e0 = from_f32<TKV>(acc[qt][dh][0] * inv), e1 = from_f32<TKV>(acc[qt][dh][1] * inv);
            const TKV e2 = from_f32<TKV>(acc[qt][dh][2] * inv), e3 = from_f32<TKV>(acc[qt][dh][3] * inv);
            const uint64_t packed = uint64_t(e0.bits) | uint64_t(e1.bits) << 16 | uint64_t(e2.bits) << 32 |
                                    uint64_t(e3.bits) << 48;
            __builtin_nontemporal_store(packed, reinterpret_cast<uint64_t *>(static_cast<TKV *>(a.out) + oo + 16 * dh + 4 * lg));
          }
        } else {
  #pragma unroll
          for (int dh = 0; dh < DH; ++dh)
  #pragma unroll
            for (int i = 0; i < 4; ++i) store_any(a.out, a.out_dtype, oo + 16 * dh + 4 * lg + i, acc[qt][dh][i] * inv);
        }
      }
    };
    if constexpr (NQT == 1) {
      group(std::integral_constant<int, 1>{});
    } else if constexpr (NQT == 2) {
      if (live >= 2) group(std::integral_constant<int, 2>{});
      else group(std::integral_constant<int, 1>{});
    } else {
      if (live >= 4) group(std::integral_constant<int, NQT>{});
      else if (live == 3) group(std::integral_constant<int, 3>{});
      else if (live == 2) group(std::integral_constant<int, 2>{});
      else group(std::integral_constant<int, 1>{});
    }
  }
}

// ---- persistent decode attention ----------------------------------------------------------
// The split kernel above gives each (row, KV head) unit four waves that stream about one
// 64-key tile each at decode lengths, so a wave's life is mostly its start (queries, first
// tile round trip) and the merge.  Here a fixed grid of waves walks whole units back to
// back: wave w takes units order[w], order[2W - 1 - w], order[2W + w], ... of the units
// sorted by descending tile count (a snake deal, so every wave gets about the same number
// of tiles), and while the last tile of one unit is multiplied, the first tile and the
// queries of its next unit are already in flight.  One wave per unit: no merge.  Same
// arithmetic per tile as decode_attention_tr_kernel<.., NQT 1, SPLIT 1, KT 64, DEPTH 1>.
#ifndef STREAM_WAVES_PER_EU
#define STREAM_WAVES_PER_EU 4
#endif

// Waves per SIMD the kernel is built for (head_dim 64 needs twice the registers).
template <int D>
constexpr int stream_waves_per_eu() { return D == 32 ? STREAM_WAVES_PER_EU : 2; }

template <typename TKV, int D, bool QRAW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(stream_waves_per_eu<D>())))
void decode_attention_stream_kernel(AttnArgs a) {
  constexpr int KT = STREAM_KT;
  constexpr int NJ = KT / 16;     // 16-key score tiles per key tile
  constexpr int DK = D / 32;      // 32-dim slices of a key (S^T k-steps)
  constexpr int DH = D / 16;      // 16-dim slices of the output (O^T row tiles)
  constexpr int ROW = D * 2 + 8;  // LDS bytes per V row
  __shared__ __align__(16) unsigned char vtile[4][KT * ROW];
  typedef typename Mfma16<TKV>::vec QVec;

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int W = int(gridDim.x) * 4, w = int(blockIdx.x) * 4 + wave;
  const int U = a.n_seqs * a.kv_heads;
  const int G = a.n_heads / a.kv_heads;
  const int nq = a.T * G;  // <= 16: query column li is query li (token li / G, head li % G)
  unsigned char *vt = vtile[wave];
  const uint32_t seg_bytes = uint32_t(a.max_len) * D * 2;

  // One unit: its pool segment, key range and query / output bases.
  struct Unit {
    Rsrc kres, vres;
    int kend, kfull, lim;
    int64_t q_base, o_base;
  };
  // (An entry outside [0, U) -- an order not written for these arguments -- ends the walk.)
  auto unit_at = [&](int r) -> int {
    const int64_t idx = int64_t(r) * W + ((r & 1) ? W - 1 - w : w);
    const int u = idx < U ? a.order[idx] : -1;
    return u >= 0 && u < U ? u : -1;
  };
  auto describe = [&](int u, Unit &x) {
    const int b = u / a.kv_heads, h = u % a.kv_heads;
    const int64_t row = a.rows ? a.rows[b] : int64_t(b);
    const int64_t kl = a.key_lengths[b] + a.kl_add;
    const bool row_ok = row >= 0 && row < a.capacity;
    const int64_t seg = row_ok ? (row * a.kv_heads + h) * int64_t(a.max_len) * D : 0;
    x.kres = kv_rsrc(static_cast<const TKV *>(a.k) + seg, seg_bytes);
    x.vres = kv_rsrc(static_cast<const TKV *>(a.v) + seg, seg_bytes);
    int l = 0;
    if (li < nq) {
      int64_t lim64 = kl + li / G;
      if (lim64 > a.span) lim64 = a.span;
      l = (row_ok && lim64 > 0) ? int(lim64) : 0;
    }
    x.lim = l;
    x.kend = __builtin_amdgcn_readfirstlane(row16_max(l));
    x.kfull = __builtin_amdgcn_readfirstlane(row16_min(li < nq ? l : 0x7fffffff));
    x.q_base = int64_t(b) * a.q_sb + int64_t(h * G) * a.q_sh;
    x.o_base = int64_t(b) * a.o_sb + int64_t(h * G) * a.o_sh;
  };

  // Lane l holds key 16 j + l % 16 of a tile at dims 32 dk + 8 (l / 16), for K and V.
  uint4 kr[NJ][DK], vr[NJ][DK];
  auto fetch = [&](const Unit &x, int kb) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int key = min(kb + 16 * j + li, x.kend - 1);  // clamped onto the last visible key
#pragma unroll
      for (int dk = 0; dk < DK; ++dk) {
        const uint32_t off = uint32_t(key * D + 32 * dk + 8 * lg) * 2;
        kr[j][dk] = kv_load16(x.kres, off);
        vr[j][dk] = kv_load16(x.vres, off);
      }
    }
  };
  // Queries of column li (dims 32 dk + 8 lg .. +7), as loaded; converted at the unit's start.
  const bool q4 = !QRAW && a.q_dtype == CG_F32 &&
                  ((reinterpret_cast<uintptr_t>(a.q) & 15) | (a.q_sb & 3) | (a.q_sh & 3) | (a.q_st & 3)) == 0;
  uint4 qraw[QRAW ? DK : 2 * DK];
  auto load_q = [&](const Unit &x) {
#pragma unroll
    for (int dk = 0; dk < (QRAW ? DK : 2 * DK); ++dk) qraw[dk] = uint4{0u, 0u, 0u, 0u};
    if (li >= nq) return;
    const int64_t qo = x.q_base + int64_t(li % G) * a.q_sh + int64_t(li / G) * a.q_st;
    if constexpr (QRAW) {
#pragma unroll
      for (int dk = 0; dk < DK; ++dk)
        qraw[dk] = *reinterpret_cast<const uint4 *>(static_cast<const TKV *>(a.q) + qo + 32 * dk + 8 * lg);
    } else if (q4) {
#pragma unroll
      for (int dk = 0; dk < DK; ++dk) {
        const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const float *>(a.q) + qo + 32 * dk + 8 * lg);
        qraw[2 * dk] = src[0];
        qraw[2 * dk + 1] = src[1];
      }
    } else {
#pragma unroll
      for (int dk = 0; dk < DK; ++dk) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = load_any(a.q, a.q_dtype, qo + 32 * dk + 8 * lg + e);
        qraw[2 * dk] = uint4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
        qraw[2 * dk + 1] = uint4{__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]), __float_as_uint(f[7])};
      }
    }
  };
  auto queries = [&](QVec (&qv)[DK]) {
#pragma unroll
    for (int dk = 0; dk < DK; ++dk) {
      if constexpr (QRAW) {
        __builtin_memcpy(&qv[dk], &qraw[dk], 16);
      } else {
        const uint4 lo = qraw[2 * dk], hi = qraw[2 * dk + 1];
        f32x8 f;
        f[0] = __uint_as_float(lo.x) * a.scale_log2;
        f[1] = __uint_as_float(lo.y) * a.scale_log2;
        f[2] = __uint_as_float(lo.z) * a.scale_log2;
        f[3] = __uint_as_float(lo.w) * a.scale_log2;
        f[4] = __uint_as_float(hi.x) * a.scale_log2;
        f[5] = __uint_as_float(hi.y) * a.scale_log2;
        f[6] = __uint_as_float(hi.z) * a.scale_log2;
        f[7] = __uint_as_float(hi.w) * a.scale_log2;
        qv[dk] = Mfma16<TKV>::from(f);
      }
    }
  };

  int r = 0;
  int u = unit_at(0);
  if (u < 0) return;
  Unit cur;
  describe(u, cur);
  if (cur.kend > 0) fetch(cur, 0);
  load_q(cur);
  const bool o4 = a.out_dtype == (std::is_same<TKV, bf16>::value ? CG_BF16 : CG_F16) &&
                  ((reinterpret_cast<uintptr_t>(a.out) & 7) | (a.o_sb & 3) | (a.o_sh & 3) | (a.o_st & 3)) == 0;
  while (true) {
    QVec qv[DK];
    queries(qv);
    // The next unit's descriptors are read now, so its first tile can be requested while
    // this unit's last tile is multiplied.
    const int un = unit_at(r + 1);
    Unit nxt;
    if (un >= 0) describe(un, nxt);
    bool ahead = false;

    f32x4 acc[DH];
    float mrun = NEG_BIG, lsum = 0.f;
#pragma unroll
    for (int dh = 0; dh < DH; ++dh) acc[dh] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kb = 0; kb < cur.kend; kb += KT) {
      // ---- scores S^T[key, query] -------------------------------------------------------
      f32x4 sc[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dk = 0; dk < DK; ++dk) {
          QVec kvec;
          __builtin_memcpy(&kvec, &kr[j][dk], 16);
          s4 = Mfma16<TKV>::mma(kvec, qv[dk], s4);
        }
        sc[j] = QRAW ? s4 * a.scale_log2 : s4;
      }
      // ---- V rows -> LDS (as loaded), then the next tile: this unit's or the next unit's
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int dk = 0; dk < DK; ++dk) {
          unsigned char *dst = vt + (16 * j + li) * ROW + (32 * dk + 8 * lg) * 2;
          reinterpret_cast<uint2 *>(dst)[0] = uint2{vr[j][dk].x, vr[j][dk].y};
          reinterpret_cast<uint2 *>(dst)[1] = uint2{vr[j][dk].z, vr[j][dk].w};
        }
      if (kb + KT < cur.kend) {
        fetch(cur, kb + KT);
      } else if (un >= 0) {
        if (nxt.kend > 0) fetch(nxt, 0);
        load_q(nxt);
        ahead = true;
      }
      // ---- mask (only tiles reaching past some query's limit) ----------------------------
      if (kb + KT > cur.kfull) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kb + 16 * j + 4 * lg + i >= cur.lim) sc[j][i] = -INFINITY;
      }
      // ---- online softmax per query column -----------------------------------------------
      float p[NJ][4];
      float tmax = NEG_BIG;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, sc[j][i]);
      tmax = xor32_max(xor16_max(tmax));
      const float mnew = fmaxf(mrun, tmax);
      const float corr = fast_exp2(mrun - mnew);
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[j][i] = fast_exp2(sc[j][i] - mnew);
          psum += p[j][i];
        }
      lsum = fmaf(lsum, corr, psum);
      mrun = mnew;
#pragma unroll
      for (int dh = 0; dh < DH; ++dh) acc[dh] *= corr;
      // ---- O^T += V^T . P^T --------------------------------------------------------------
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int c = 0; c < KT / 32; ++c) {
        QVec pv;
        {
          f32x8 f;
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = p[2 * c + (e >> 2)][e & 3];
          pv = Mfma16<TKV>::from(f);
        }
#pragma unroll
        for (int dh = 0; dh < DH; ++dh) {
          const unsigned char *src = vt + (32 * c + 4 * lg + (li >> 2)) * ROW + (16 * dh + 4 * (li & 3)) * 2;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(src));
          const s16x4 hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(src + 16 * ROW));
          QVec vv;
          __builtin_memcpy(&vv, &lo, 8);
          __builtin_memcpy(reinterpret_cast<char *>(&vv) + 8, &hi, 8);
          acc[dh] = Mfma16<TKV>::mma(vv, pv, acc[dh]);
        }
      }
      // The next tile's V rows overwrite this one's only after every lane has read it.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ---- normalise and store: lane l holds dims 16 dh + 4 (l / 16) + i of query column l % 16
    {
      const float total = xor32_sum(xor16_sum(lsum));
      if (li < nq) {
        const float inv = total > 0.f ? 1.0f / total : 0.f;
        const int64_t oo = cur.o_base + int64_t(li % G) * a.o_sh + int64_t(li / G) * a.o_st;
        if (o4) {
#pragma unroll
          for (int dh = 0; dh < DH; ++dh) {
            const TKV e0 = from_f32<TKV>(acc[dh][0] * inv), e1 = from_f32<TKV>(acc[dh][1] * inv);
            const TKV e2 = from_f32<TKV>(acc[dh][2] * inv), e3 = from_f32<TKV>(acc[dh][3] * inv);
            const uint64_t packed = uint64_t(e0.bits) | uint64_t(e1.bits) << 16 | uint64_t(e2.bits) << 32 |
                                    uint64_t(e3.bits) << 48;
            __builtin_nontemporal_store(packed, reinterpret_cast<uint64_t *>(static_cast<TKV *>(a.out) + oo + 16 * dh + 4 * lg));
          }
        } else {
#pragma unroll
          for (int dh = 0; dh < DH; ++dh)
#pragma unroll
            for (int i = 0; i < 4; ++i) store_any(a.out, a.out_dtype, oo + 16 * dh + 4 * lg + i, acc[dh][i] * inv);
        }
      }
    }
    if (un < 0) break;
    if (!ahead) {  // this unit had no key: nothing was requested for the next one yet
      if (nxt.kend > 0) fetch(nxt, 0);
      load_q(nxt);
    }
    cur = nxt;
    ++r;
  }
}

// order = the units sorted by descending tile count (attn_dev.h: order_units).  One block.
__global__ __launch_bounds__(1024) void attention_order_kernel(const AttnArgs a, int32_t *__restrict__ order) {
  order_units(a, order);
}

#ifndef TR_SPLIT
#define TR_SPLIT 4
#endif
// Keys per tile of the one- and two-query-tile (decode) forms: 32-key tiles measured 51.9
// against 52.7 us per launch at config 3 (the driver's 20 steps), the same at longer rows.
#ifndef TR_KT
#define TR_KT 32
#endif
// Waves per unit for padded one-query-group runs (decode): 1, 2 or 4.
#ifndef TR_SPLIT_PADDED
#define TR_SPLIT_PADDED TR_SPLIT
#endif
#ifndef TR_DEPTH
#define TR_DEPTH 1
#endif
// Key tiles in flight per wave when one wave takes a whole multi-token item.
#ifndef TR_MQ_DEPTH
#define TR_MQ_DEPTH 1
#endif
#ifndef TR_ONE_WAVE_ITEMS
#define TR_ONE_WAVE_ITEMS 2048
#endif
// Keys per tile when one wave takes a whole multi-token item: 32-key tiles take the form
// from 202 to 143 VGPRs (three waves per SIMD instead of two) and measured 76.3 -> 74.6 us
// per launch at config 5, 33.5 -> 30.6 us at prefill.
#ifndef TR_MQ_KT
#define TR_MQ_KT 32
#endif

// The 16-bit-pool kernels for one query form (QRAW: queries stored in the cache type).
template <typename TKV, int D, bool QRAW>
void launch_tr(const AttnArgs &a, int queries, hipStream_t s) {
  const unsigned units = unsigned(int64_t(a.n_seqs) * a.kv_heads);
  const unsigned tr_grid = (units * TR_SPLIT + 3) / 4;
  if (queries <= 16 && !a.seq_start && TR_SPLIT_PADDED != TR_SPLIT)
    decode_attention_tr_kernel<TKV, D, 1, TR_SPLIT_PADDED, TR_KT, TR_DEPTH, QRAW>
        <<<(units * TR_SPLIT_PADDED + 3) / 4, 256, 0, s>>>(a);
  else if (queries <= 16)
    decode_attention_tr_kernel<TKV, D, 1, TR_SPLIT, TR_KT, TR_DEPTH, QRAW><<<tr_grid, 256, 0, s>>>(a);
  else if (queries <= 32)
    decode_attention_tr_kernel<TKV, D, 2, TR_SPLIT, TR_KT, TR_DEPTH, QRAW><<<tr_grid, 256, 0, s>>>(a);
  else {
    // Multi-token rows (prefill, chunks): one block row per 64 queries of a unit.  With
    // enough (unit, query group) items to fill the chip, or no query seeing more than one
    // 64-key tile, one wave takes a whole item (four per block); otherwise four waves
    // split its key tiles and merge.
    const dim3 grid_q(1, unsigned(std::min<int64_t>((int64_t(queries) + 63) / 64, 65535)));
    if (a.span <= 64 || int64_t(units) * grid_q.y >= TR_ONE_WAVE_ITEMS) {
      decode_attention_tr_kernel<TKV, D, 4, 1, TR_MQ_KT, TR_MQ_DEPTH, QRAW><<<dim3((units + 3) / 4, grid_q.y), 256, 0, s>>>(a);
    } else {
      decode_attention_tr_kernel<TKV, D, 4, TR_SPLIT, 64, 1, QRAW><<<dim3(tr_grid, grid_q.y), 256, 0, s>>>(a);
    }
  }
  CG_LAUNCHED();
}

int attention_cus() {
  static thread_local int dev = -1, cus = 256;
  int d = 0;
  if (hipGetDevice(&d) == hipSuccess && d != dev) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) == hipSuccess && n > 0) cus = n;
    dev = d;
  }
  return cus;
}

// The persistent kernel: as many blocks of four waves per CU (one wave per SIMD each) as
// its registers let reside, never more waves than units.
template <typename TKV, int D, bool QRAW>
void launch_stream(const AttnArgs &a, hipStream_t s) {
  const int64_t units = int64_t(a.n_seqs) * a.kv_heads;
  const int64_t blocks = std::min<int64_t>((units + 3) / 4, int64_t(attention_cus()) * stream_waves_per_eu<D>());
  decode_attention_stream_kernel<TKV, D, QRAW><<<unsigned(blocks), 256, 0, s>>>(a);
  CG_LAUNCHED();
}

template <typename TKV, int D>
void launch_mfma(const AttnArgs &a, int queries, hipStream_t s) {
  const unsigned grid = unsigned((int64_t(a.n_seqs) * a.kv_heads + 3) / 4);
  if constexpr (sizeof(TKV) == 2) {
    CG_REQUIRE(int64_t(a.max_len) * D * 2 < (int64_t(1) << 31), CG_ERR_UNSUPPORTED,
               "decode attention: one cache row of one head must stay below 2 GiB");
    constexpr int KV_CODE = std::is_same<TKV, bf16>::value ? CG_BF16 : CG_F16;
    const bool qraw = a.q_dtype == KV_CODE &&
                      ((reinterpret_cast<uintptr_t>(a.q) & 15) | (a.q_sb & 7) | (a.q_sh & 7) | (a.q_st & 7)) == 0;
    if (a.order && attention_streams(a))
      return qraw ? launch_stream<TKV, D, true>(a, s) : launch_stream<TKV, D, false>(a, s);
    if (qraw) return launch_tr<TKV, D, true>(a, queries, s);
    return launch_tr<TKV, D, false>(a, queries, s);
  } else {
    if (queries <= 16) decode_attention_mfma_kernel<TKV, D, 1><<<grid, 256, 0, s>>>(a);
    else if (queries <= 32) decode_attention_mfma_kernel<TKV, D, 2><<<grid, 256, 0, s>>>(a);
    else decode_attention_mfma_kernel<TKV, D, 4><<<grid, 256, 0, s>>>(a);
    CG_LAUNCHED();
  }
}

template <typename TKV, int D>
void launch_d(const AttnArgs &a, hipStream_t s) {
  constexpr int WAVES = 4;
  decode_attention_kernel<TKV, D, WAVES><<<a.n_seqs * a.kv_heads, 64 * WAVES, 0, s>>>(a);
  CG_LAUNCHED();
}

template <typename TKV>
void launch_kv(const AttnArgs &a, hipStream_t s) {
  // Queries per (sequence, KV head): G heads x tokens (packed chunks: up to 16 tokens).
  const int queries = (a.n_heads / a.kv_heads) * (a.seq_start ? 16 : a.T);
  if (a.head_dim == 32) return launch_mfma<TKV, 32>(a, queries, s);
  if (a.head_dim == 64) return launch_mfma<TKV, 64>(a, queries, s);
  switch (a.head_dim) {
    case 8:
      return launch_d<TKV, 8>(a, s);
    case 16:
      return launch_d<TKV, 16>(a, s);
    case 24:
      return launch_d<TKV, 24>(a, s);
    case 32:
      return launch_d<TKV, 32>(a, s);
    case 64:
      return launch_d<TKV, 64>(a, s);
  }
  throw Error(CG_ERR_UNSUPPORTED,
              "decode attention is built for head_dim 8, 16, 24, 32 and 64, not " +
                  std::to_string(a.head_dim));
}

}  // namespace

// Spans from which an ordered decode call takes the persistent kernel.  Measured on MI355X
// (bf16 pool, head_dim 32, 4 query heads per KV head): with up to 8-9 tiles per unit
// (config 3, span 538) both kernels stream at the same rate and the order costs a launch per
// step.  With the split kernel's earlier 64-key tiles and barrier merges, rows of up to 32
// tiles and a wide spread of lengths (config 4, span 2048) favoured the sorted deal (87.4 ->
// 80.8 us per launch); with 32-key tiles and the last-wave merge the split kernel matches
// it there (82.7 against 82.6-84.7 us), so the trunk step no longer orders decode waves.
#ifndef STREAM_MIN_SPAN
#define STREAM_MIN_SPAN 1024
#endif

bool attention_streams(const AttnArgs &a) {
  return a.span >= STREAM_MIN_SPAN && (a.kv_dtype == CG_BF16 || a.kv_dtype == CG_F16) &&
         (a.head_dim == 32 || a.head_dim == 64) && !a.seq_start && a.T >= 1 && a.kv_heads > 0 &&
         a.n_heads % a.kv_heads == 0 && int64_t(a.n_heads / a.kv_heads) * a.T <= 16 &&
         int64_t(a.max_len) * a.head_dim * 2 < (int64_t(1) << 31);
}

void launch_attention_order(const AttnArgs &a, int32_t *order, hipStream_t s) {
  if (int64_t(a.n_seqs) * a.kv_heads <= 0) return;
  attention_order_kernel<<<1, 1024, 0, s>>>(a, order);
  CG_LAUNCHED();
}

void launch_decode_attention(const AttnArgs &a, hipStream_t s) {
  CG_REQUIRE(a.n_heads > 0 && a.kv_heads > 0 && a.n_heads % a.kv_heads == 0, CG_ERR_INVALID,
             "n_heads must be a positive multiple of kv_heads");
  CG_REQUIRE(a.n_seqs >= 0, CG_ERR_INVALID, "negative batch");
  if (a.n_seqs == 0) return;
  switch (a.kv_dtype) {
    case CG_F32:
      return launch_kv<float>(a, s);
    case CG_BF16:
      return launch_kv<bf16>(a, s);
    case CG_F16:
      return launch_kv<f16>(a, s);
  }
  throw Error(CG_ERR_INVALID, "unknown cache dtype");
}

}  // namespace cg

using namespace cg;

namespace {
// The arguments of a padded run [B, n_heads, T, head_dim] (cg_decode_attention's layout).
AttnArgs padded_args(const void *q, int32_t q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                     const cg_kv_layer *layer, const int64_t *rows, const int64_t *key_lengths, int32_t B,
                     int32_t n_heads, int32_t T, int32_t span, float scale, void *out, int32_t out_dtype) {
  AttnArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_st = q_st;
  a.out = out;
  a.out_dtype = out_dtype;
  a.o_st = layer->head_dim;
  a.o_sh = int64_t(T) * layer->head_dim;
  a.o_sb = int64_t(n_heads) * T * layer->head_dim;
  a.k = layer->k;
  a.v = layer->v;
  a.kv_dtype = layer->dtype;
  a.rows = rows;
  a.key_lengths = key_lengths;
  a.kl_add = 0;
  a.seq_start = nullptr;
  a.n_seqs = B;
  a.n_heads = n_heads;
  a.kv_heads = layer->kv_heads;
  a.head_dim = layer->head_dim;
  a.T = T;
  a.max_len = layer->max_len;
  a.capacity = layer->capacity;
  a.span = (span <= 0 || span > layer->max_len) ? layer->max_len : span;
  a.scale_log2 = scale * 1.4426950408889634f;
  return a;
}
}  // namespace

extern "C" int cg_decode_attention(const void *q, int32_t q_dtype, int64_t q_sb, int64_t q_sh,
                                   int64_t q_st, const cg_kv_layer *layer, const int64_t *rows,
                                   const int64_t *key_lengths, int32_t B, int32_t n_heads,
                                   int32_t T, int32_t span, float scale, void *out,
                                   int32_t out_dtype, void *stream) {
  return cg_decode_attention_ordered(q, q_dtype, q_sb, q_sh, q_st, layer, rows, key_lengths, B, n_heads, T, span,
                                     scale, out, out_dtype, nullptr, stream);
}

extern "C" int cg_decode_attention_ordered(const void *q, int32_t q_dtype, int64_t q_sb, int64_t q_sh,
                                           int64_t q_st, const cg_kv_layer *layer, const int64_t *rows,
                                           const int64_t *key_lengths, int32_t B, int32_t n_heads, int32_t T,
                                           int32_t span, float scale, void *out, int32_t out_dtype,
                                           const int32_t *order, void *stream) {
  return guarded([&] {
    check_layer(layer);
    dtype_size(q_dtype);
    dtype_size(out_dtype);
    CG_REQUIRE(B >= 0 && T >= 0, CG_ERR_INVALID, "B and T must be non-negative");
    if (B == 0 || T == 0) return;  // empty tensors may carry NULL data pointers
    CG_REQUIRE(q && out && key_lengths, CG_ERR_INVALID, "q, out and key_lengths are required");
    AttnArgs a = padded_args(q, q_dtype, q_sb, q_sh, q_st, layer, rows, key_lengths, B, n_heads, T, span, scale,
                             out, out_dtype);
    a.order = order;
    launch_decode_attention(a, as_stream(stream));
  });
}

extern "C" int cg_decode_attention_order(const cg_kv_layer *layer, const int64_t *rows,
                                         const int64_t *key_lengths, int32_t B, int32_t n_heads, int32_t T,
                                         int32_t span, int32_t *order, int32_t *streams, void *stream) {
  return guarded([&] {
    check_layer(layer);
    CG_REQUIRE(B >= 0 && T >= 0, CG_ERR_INVALID, "B and T must be non-negative");
    CG_REQUIRE(n_heads > 0 && n_heads % layer->kv_heads == 0, CG_ERR_INVALID,
               "n_heads must be a positive multiple of kv_heads");
    AttnArgs a = padded_args(nullptr, CG_F32, 0, 0, 0, layer, rows, key_lengths, B, n_heads, T, span, 1.0f,
                             nullptr, CG_F32);
    const bool on = B > 0 && T > 0 && attention_streams(a);
    if (streams) *streams = on ? 1 : 0;
    if (!on) return;
    CG_REQUIRE(order && key_lengths, CG_ERR_INVALID, "order and key_lengths are required");
    launch_attention_order(a, order, as_stream(stream));
  });
}

namespace {
// The arguments of a packed run (cg_decode_attention_packed's layout).
AttnArgs packed_args(const void *q, int32_t q_dtype, int64_t q_st, int64_t q_sh, const cg_kv_layer *layer,
                     const int64_t *rows, const int64_t *positions, const int64_t *seq_start, int32_t n_seqs,
                     int32_t n_tokens, int32_t n_heads, int32_t span, float scale, void *out, int32_t out_dtype) {
  AttnArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_st = q_st;
  a.q_sh = q_sh;
  a.q_sb = 0;
  a.out = out;
  a.out_dtype = out_dtype;
  a.o_st = int64_t(n_heads) * layer->head_dim;
  a.o_sh = layer->head_dim;
  a.o_sb = 0;
  a.k = layer->k;
  a.v = layer->v;
  a.kv_dtype = layer->dtype;
  a.rows = rows;
  a.key_lengths = positions;
  a.kl_add = 1;
  a.seq_start = seq_start;
  a.n_tokens = n_tokens;
  a.n_seqs = n_seqs;
  a.n_heads = n_heads;
  a.kv_heads = layer->kv_heads;
  a.head_dim = layer->head_dim;
  a.T = 0;
  a.max_len = layer->max_len;
  a.capacity = layer->capacity;
  a.span = (span <= 0 || span > layer->max_len) ? layer->max_len : span;
  a.scale_log2 = scale * 1.4426950408889634f;
  return a;
}
}  // namespace

extern "C" int cg_decode_attention_packed(const void *q, int32_t q_dtype, int64_t q_st, int64_t q_sh,
                                          const cg_kv_layer *layer, const int64_t *rows,
                                          const int64_t *positions, const int64_t *seq_start,
                                          int32_t n_seqs, int32_t n_tokens, int32_t n_heads, int32_t span,
                                          float scale, void *out, int32_t out_dtype, void *stream) {
  return cg_decode_attention_packed_ordered(q, q_dtype, q_st, q_sh, layer, rows, positions, seq_start, n_seqs,
                                            n_tokens, n_heads, span, scale, out, out_dtype, nullptr, stream);
}

extern "C" int cg_decode_attention_packed_ordered(const void *q, int32_t q_dtype, int64_t q_st, int64_t q_sh,
                                                  const cg_kv_layer *layer, const int64_t *rows,
                                                  const int64_t *positions, const int64_t *seq_start,
                                                  int32_t n_seqs, int32_t n_tokens, int32_t n_heads,
                                                  int32_t span, float scale, void *out, int32_t out_dtype,
                                                  const int32_t *order, void *stream) {
  return guarded([&] {
    check_layer(layer);
    dtype_size(q_dtype);
    dtype_size(out_dtype);
    CG_REQUIRE(n_seqs >= 0 && n_tokens >= 0, CG_ERR_INVALID, "n_seqs and n_tokens must be non-negative");
    if (n_seqs == 0 || n_tokens == 0) return;
    CG_REQUIRE(q && out && positions && seq_start, CG_ERR_INVALID, "q, out, positions and seq_start are required");
    AttnArgs a = packed_args(q, q_dtype, q_st, q_sh, layer, rows, positions, seq_start, n_seqs, n_tokens, n_heads,
                             span, scale, out, out_dtype);
    a.order = order;
    launch_decode_attention(a, as_stream(stream));
  });
}

extern "C" int cg_decode_attention_packed_order(const cg_kv_layer *layer, const int64_t *rows,
                                                const int64_t *positions, const int64_t *seq_start,
                                                int32_t n_seqs, int32_t n_tokens, int32_t n_heads, int32_t span,
                                                int32_t *order, void *stream) {
  return guarded([&] {
    check_layer(layer);
    CG_REQUIRE(n_seqs >= 0 && n_tokens >= 0, CG_ERR_INVALID, "n_seqs and n_tokens must be non-negative");
    CG_REQUIRE(n_heads > 0 && n_heads % layer->kv_heads == 0, CG_ERR_INVALID,
               "n_heads must be a positive multiple of kv_heads");
    if (n_seqs == 0) return;
    CG_REQUIRE(order && positions && seq_start, CG_ERR_INVALID, "order, positions and seq_start are required");
    AttnArgs a = packed_args(nullptr, CG_F32, 0, 0, layer, rows, positions, seq_start, n_seqs, n_tokens, n_heads, span,
                             1.0f, nullptr, CG_F32);
    launch_attention_order(a, order, as_stream(stream));
  });
}
