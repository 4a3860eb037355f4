// KV pool operations: append (write_step), prefill write (write_range), gathered read,
// row compaction (copy_rows) and a device-side index check.
//
// Semantics follow cardgym/nn/kv_cache.py:65-138.  Every kernel bounds-checks its
// indices and skips out-of-range entries instead of faulting; cg_kv_check_indices
// reports them through a device flag.
#include <algorithm>
#include <climits>
#include <string>
#include <type_traits>

#include "common.h"

namespace cg {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string &message) { g_last_error = message; }

namespace {

// Four consecutive elements of a pool row from fp32 values: the 16-bit types through cvt4,
// the conversion the trunk step's fused append stores with.
template <typename TC>
__device__ __forceinline__ void put4(TC *dst, f32x4 v);
template <>
__device__ __forceinline__ void put4<float>(float *dst, f32x4 v) {
  *reinterpret_cast<f32x4 *>(dst) = v;
}
template <>
__device__ __forceinline__ void put4<bf16>(bf16 *dst, f32x4 v) {
  *reinterpret_cast<u32x2 *>(dst) = cvt4<bf16>(v);
}
template <>
__device__ __forceinline__ void put4<f16>(f16 *dst, f32x4 v) {
  *reinterpret_cast<u32x2 *>(dst) = cvt4<f16>(v);
}

// One thread per (b, t, head, run of VEC elements): VEC 4 when head_dim is a multiple of 4
// (every head_dim the trunk takes), 1 otherwise.  The write is a scatter of 64-128 byte rows,
// so the launch is bound by the number of rows, not bytes.  A source of the pool's own type
// is copied bit for bit (Tensor.to to the same dtype is the identity).
template <typename TC, typename TS, int VEC>
__global__ void kv_write_kernel(TC *__restrict__ kc, TC *__restrict__ vc, const TS *__restrict__ ks,
                                const TS *__restrict__ vs, int64_t ks_b, int64_t ks_h, int64_t ks_t,
                                int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                const int64_t *__restrict__ rows, const int64_t *__restrict__ positions,
                                int32_t start, int32_t B, int32_t T, int32_t KVH, int32_t L,
                                int32_t D, int32_t capacity) {
  const int runs = D / VEC;
  const int64_t total = int64_t(B) * T * KVH * runs;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int d = int(i % runs) * VEC;
    int64_t r = i / runs;
    const int h = int(r % KVH);
    r /= KVH;
    const int t = int(r % T);
    const int b = int(r / T);
    const int64_t row = rows ? rows[b] : int64_t(b);
    const int64_t pos = positions ? positions[int64_t(b) * T + t] : int64_t(start) + t;
    if (row < 0 || row >= capacity || pos < 0 || pos >= L) continue;
    const int64_t dst = ((row * KVH + h) * L + pos) * D + d;
    const TS *k = ks + b * ks_b + h * ks_h + t * ks_t + d;
    const TS *v = vs + b * vs_b + h * vs_h + t * vs_t + d;
    if constexpr (VEC == 1 || std::is_same<TC, TS>::value) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        kc[dst + e] = convert<TC>(k[e]);
        vc[dst + e] = convert<TC>(v[e]);
      }
    } else {
      put4(kc + dst, f32x4{to_f32(k[0]), to_f32(k[1]), to_f32(k[2]), to_f32(k[3])});
      put4(vc + dst, f32x4{to_f32(v[0]), to_f32(v[1]), to_f32(v[2]), to_f32(v[3])});
    }
  }
}

// Gathered read: out[b, h, p, :] = cache[rows[b], h, p, :] for p < length.  16-byte
// vectors when the row slice allows (it always does for head_dim * size % 16 == 0).
template <typename V>
__global__ void kv_gather_kernel(const V *__restrict__ kc, const V *__restrict__ vc, V *__restrict__ ko,
                                 V *__restrict__ vo, const int64_t *__restrict__ rows, int32_t B,
                                 int32_t KVH, int32_t L, int32_t length, int32_t vec_per_pos,
                                 int32_t capacity) {
  const int64_t per_head = int64_t(length) * vec_per_pos;
  const int64_t total = int64_t(B) * KVH * per_head;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t within = i % per_head;
    const int64_t bh = i / per_head;
    const int h = int(bh % KVH);
    const int b = int(bh / KVH);
    const int64_t row = rows ? rows[b] : int64_t(b);
    if (row < 0 || row >= capacity) continue;
    const int64_t src = (row * KVH + h) * int64_t(L) * vec_per_pos + within;
    ko[i] = kc[src];
    vo[i] = vc[src];
  }
}

// copy_rows: the first `length` positions of every head of sources[i] onto targets[i].
template <typename V>
__global__ void kv_copy_rows_kernel(V *__restrict__ kc, V *__restrict__ vc,
                                    const int64_t *__restrict__ sources,
                                    const int64_t *__restrict__ targets, int32_t n, int32_t KVH,
                                    int32_t L, int32_t length, int32_t vec_per_pos,
                                    int32_t capacity) {
  const int64_t per_head = int64_t(length) * vec_per_pos;
  const int64_t total = int64_t(n) * KVH * per_head;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t within = i % per_head;
    const int64_t bh = i / per_head;
    const int h = int(bh % KVH);
    const int j = int(bh / KVH);
    const int64_t s = sources[j], t = targets[j];
    if (s < 0 || s >= capacity || t < 0 || t >= capacity) continue;
    const int64_t head = int64_t(L) * vec_per_pos;
    const int64_t so = (s * KVH + h) * head + within, to = (t * KVH + h) * head + within;
    kc[to] = kc[so];
    vc[to] = vc[so];
  }
}

__global__ void kv_check_kernel(const int64_t *__restrict__ rows, int32_t B,
                                const int64_t *__restrict__ positions, int32_t n_pos,
                                int32_t capacity, int32_t L, int32_t *__restrict__ flag) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  bool bad = false;
  if (rows && i < B) bad |= rows[i] < 0 || rows[i] >= capacity;
  if (positions && i < n_pos) bad |= positions[i] < 0 || positions[i] >= L;
  if (bad) flag[0] = 1;
}

__global__ void advance_kernel(int64_t *__restrict__ a, int32_t n, int64_t delta) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] += delta;
}

inline unsigned grid_for(int64_t total, int block) {
  int64_t g = (total + block - 1) / block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return unsigned(g);
}

template <typename TC, typename TS>
void launch_write(const cg_kv_layer &L, const int64_t *rows, const int64_t *positions, int32_t start,
                  const cg_kv_source &k, const cg_kv_source &v, int32_t B, int32_t T,
                  hipStream_t s) {
  const bool vec = L.head_dim % 4 == 0;
  const int64_t total = int64_t(B) * T * L.kv_heads * (vec ? L.head_dim / 4 : L.head_dim);
  if (total == 0) return;
  auto go = [&](auto kernel) {
    kernel<<<grid_for(total, 256), 256, 0, s>>>(
        static_cast<TC *>(L.k), static_cast<TC *>(L.v), static_cast<const TS *>(k.data),
        static_cast<const TS *>(v.data), k.stride_b, k.stride_h, k.stride_t, v.stride_b, v.stride_h,
        v.stride_t, rows, positions, start, B, T, L.kv_heads, L.max_len, L.head_dim, L.capacity);
    CG_LAUNCHED();
  };
  if (vec) go(kv_write_kernel<TC, TS, 4>);
  else go(kv_write_kernel<TC, TS, 1>);
}

template <typename TC>
void dispatch_source(const cg_kv_layer &L, const int64_t *rows, const int64_t *positions,
                     int32_t start, const cg_kv_source &k, const cg_kv_source &v, int32_t B,
                     int32_t T, hipStream_t s) {
  switch (k.dtype) {
    case CG_F32:
      return launch_write<TC, float>(L, rows, positions, start, k, v, B, T, s);
    case CG_BF16:
      return launch_write<TC, bf16>(L, rows, positions, start, k, v, B, T, s);
    case CG_F16:
      return launch_write<TC, f16>(L, rows, positions, start, k, v, B, T, s);
  }
  throw Error(CG_ERR_INVALID, "unknown source dtype");
}

void write_common(const cg_kv_layer *layer, const int64_t *rows, const int64_t *positions,
                  int32_t start, const cg_kv_source *k, const cg_kv_source *v, int32_t B, int32_t T,
                  void *stream) {
  check_layer(layer);
  CG_REQUIRE(B >= 0 && T >= 0, CG_ERR_INVALID, "B and T must be non-negative");
  CG_REQUIRE(k && v, CG_ERR_INVALID, "k_new / v_new is NULL");
  if (int64_t(B) * T == 0) return;  // empty tensors may carry NULL data pointers
  CG_REQUIRE(k->data && v->data, CG_ERR_INVALID, "k_new / v_new data is NULL");
  CG_REQUIRE(k->dtype == v->dtype, CG_ERR_INVALID, "k_new and v_new must share a dtype");
  dtype_size(k->dtype);
  CG_REQUIRE(positions || start >= 0, CG_ERR_RANGE, "start must be non-negative");
  CG_REQUIRE(positions || int64_t(start) + T <= layer->max_len, CG_ERR_RANGE,
             "write_range past max_len");
  hipStream_t s = as_stream(stream);
  switch (layer->dtype) {
    case CG_F32:
      return dispatch_source<float>(*layer, rows, positions, start, *k, *v, B, T, s);
    case CG_BF16:
      return dispatch_source<bf16>(*layer, rows, positions, start, *k, *v, B, T, s);
    case CG_F16:
      return dispatch_source<f16>(*layer, rows, positions, start, *k, *v, B, T, s);
  }
}

// ---- copy_rows over many layers, overlap-safe -------------------------------------------
// The reference gathers each chunk before writing it (kv_cache.py:122-138): every pair's
// source is read before any target is written.  Two device-side facts about the chunk pick
// how that is met:
//   * a pair is "endangered" when its source row is some pair's target;
//   * the chunk is "ordered" when no pair writes a row that a LATER pair reads (pair i
//     writes t_i; every pair k with s_k == t_i has k <= i).
// An ordered chunk gives the same result when its pairs run one after the other, which is
// what the ordered kernel does: one thread per 16-byte slice of every (layer, head, K / V)
// prefix walks the pairs in order, and since a slice's reads and writes are all its own,
// reads may run ahead of writes.  That is one read and one write per byte, the case of
// compaction (survivors slide down to lower rows).  Any other chunk is staged: endangered
// prefixes are gathered into the workspace first, the rest is copied straight (a source
// that is no pair's target is never written).
constexpr int MAX_COPY_LAYERS = 64;
// Pairs in flight per wave and 16-byte accesses per lane of the ordered walk: 16 and 1
// measured 4.76 TB/s at config 3's compaction (8 and 2: 4.52; 12 / 24 / 32 and 1: 4.74 /
// 4.71 / 4.34; 16 and 2: 4.51; 8 and 4: 4.59).
#ifndef CG_WALK_UNROLL
#define CG_WALK_UNROLL 16
#endif
#ifndef CG_WALK_VPT
#define CG_WALK_VPT 1
#endif
struct LayerPtrs {
  void *k[MAX_COPY_LAYERS];
  void *v[MAX_COPY_LAYERS];
};

// Workspace header, in 32-bit words: [0] some pair is endangered, [1] the chunk is not
// ordered, [4, 4 + ceil(capacity / 32)) a bitmap of target rows, then per row 1 + the
// index of the last pair that reads it (0: none).
struct CopyHeader {
  uint32_t *flags, *bitmap;
  int32_t *last_reader;
  int64_t words;
};

inline int64_t copy_header_words(int32_t capacity) { return 4 + (int64_t(capacity) + 31) / 32 + capacity; }

inline CopyHeader copy_header(void *workspace, int32_t capacity) {
  uint32_t *w = static_cast<uint32_t *>(workspace);
  const int64_t bitmap_words = (int64_t(capacity) + 31) / 32;
  return {w, w + 4, reinterpret_cast<int32_t *>(w + 4 + bitmap_words), copy_header_words(capacity)};
}

size_t copy_header_bytes(int32_t capacity) { return (size_t(4) * size_t(copy_header_words(capacity)) + 255) / 256 * 256; }

size_t copy_bytes(const cg_kv_layer &L, int32_t n_layers, int32_t n, int32_t length) {
  return size_t(n) * n_layers * L.kv_heads * 2 * size_t(length) * L.head_dim * dtype_size(L.dtype);
}

__global__ void clear_words_kernel(uint32_t *__restrict__ words, int64_t count) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x)
    words[i] = 0;
}

__device__ __forceinline__ bool in_pool(int64_t row, int32_t capacity) { return row >= 0 && row < capacity; }

__device__ __forceinline__ bool is_marked(const uint32_t *bitmap, int64_t row) {
  return (bitmap[row >> 5] >> (row & 31)) & 1u;
}

// Pairs with a row outside the pool are skipped by every copy kernel, and ignored here.
__global__ void mark_pairs_kernel(const int64_t *__restrict__ sources, const int64_t *__restrict__ targets,
                                  int32_t n, int32_t capacity, uint32_t *__restrict__ bitmap,
                                  int32_t *__restrict__ last_reader) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = sources[i], t = targets[i];
  if (!in_pool(s, capacity) || !in_pool(t, capacity)) return;
  atomicOr(bitmap + (t >> 5), 1u << (t & 31));
  atomicMax(last_reader + s, i + 1);
}

__global__ void classify_pairs_kernel(const int64_t *__restrict__ sources, const int64_t *__restrict__ targets,
                                      int32_t n, int32_t capacity, const uint32_t *__restrict__ bitmap,
                                      const int32_t *__restrict__ last_reader, uint32_t *__restrict__ flags) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = sources[i], t = targets[i];
  if (!in_pool(s, capacity) || !in_pool(t, capacity)) {
    flags[1] = 1;  // only the staged kernels skip such pairs
    return;
  }
  if (is_marked(bitmap, s)) flags[0] = 1;        // every writer stores 1
  if (last_reader[t] > i + 1) flags[1] = 1;
}

// Ordered chunks: one wave per (layer, head, K / V, tile of 64 * VPT accesses of the
// prefix); each lane owns VPT accesses of the tile (lanes past the prefix's end repeat its
// last access, which the same lane instruction writes with the same value) and walks the
// pairs in order, U pairs' reads in flight ahead of their writes.  The loop has no
// branches, so a group's reads are all in flight together: a chunk with a pair outside the
// pool is never classed as ordered, and rows are clamped into the pool only so that a
// caller's broken promise (flags == nullptr) cannot reach outside it.
template <typename V, int U, int VPT>
__global__ void __launch_bounds__(64) ordered_copy_kernel(LayerPtrs lp, const int64_t *__restrict__ sources,
                                                          const int64_t *__restrict__ targets, int32_t n,
                                                          int32_t KVH, int32_t capacity, int64_t slot_vec,
                                                          int64_t seg_vec, int64_t tiles,
                                                          const uint32_t *__restrict__ flags) {
  if (flags && flags[1]) return;
  const int64_t tile = blockIdx.x % tiles;
  const int64_t r = blockIdx.x / tiles;
  const int c = int(r & 1), h = int((r >> 1) % KVH), l = int((r >> 1) / KVH);
  V *base = static_cast<V *>(c ? lp.v[l] : lp.k[l]) + h * slot_vec;
  int64_t e[VPT];
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    const int64_t x = tile * 64 * VPT + v * 64 + threadIdx.x;
    e[v] = x < seg_vec ? x : seg_vec - 1;
  }
  const int64_t row_stride = int64_t(KVH) * slot_vec;
  const int64_t last = capacity - 1;
  auto row = [&](int64_t x) { return base + (x < 0 ? 0 : x > last ? last : x) * row_stride; };
  int j = 0;
  for (; j + U <= n; j += U) {
    int64_t src[U], dst[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      src[u] = sources[j + u];
      dst[u] = targets[j + u];
    }
    V val[U][VPT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < VPT; ++v) val[u][v] = __builtin_nontemporal_load(row(src[u]) + e[v]);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < VPT; ++v) __builtin_nontemporal_store(val[u][v], row(dst[u]) + e[v]);
  }
  for (; j < n; ++j) {
    V val[VPT];
#pragma unroll
    for (int v = 0; v < VPT; ++v) val[v] = __builtin_nontemporal_load(row(sources[j]) + e[v]);
#pragma unroll
    for (int v = 0; v < VPT; ++v) __builtin_nontemporal_store(val[v], row(targets[j]) + e[v]);
  }
}

// Streams seg_vec accesses of V from src to dst, four in flight per thread; nothing
// copied here is read again soon, so both sides bypass the caches' retention.
template <typename V>
__device__ __forceinline__ void stream_copy(V *__restrict__ dst, const V *__restrict__ src, int64_t seg_vec) {
  constexpr int U = 4;
  for (int64_t e = threadIdx.x; e < seg_vec; e += int64_t(U) * blockDim.x) {
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (e + int64_t(u) * blockDim.x < seg_vec) r[u] = __builtin_nontemporal_load(src + e + int64_t(u) * blockDim.x);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (e + int64_t(u) * blockDim.x < seg_vec) __builtin_nontemporal_store(r[u], dst + e + int64_t(u) * blockDim.x);
  }
}

// Staged chunks (all chunks when `always`, else only those not classed as ordered).
// PHASE 0: without endangered pairs every prefix goes straight to its target; with them,
// only endangered prefixes move, into the workspace.  PHASE 1 (only with endangered
// pairs): endangered prefixes from the workspace, the rest straight from their sources.
// One workgroup per prefix at a time; V is the widest access that divides a position.
template <int PHASE, typename V>
__global__ void staged_copy_kernel(LayerPtrs lp, int32_t n_layers, const int64_t *__restrict__ sources,
                                   const int64_t *__restrict__ targets, int32_t KVH, int32_t capacity,
                                   int64_t slot_vec, int64_t seg_vec, int64_t segs, V *__restrict__ tmp,
                                   const uint32_t *__restrict__ flags, const uint32_t *__restrict__ bitmap,
                                   int32_t always) {
  if (!always && !flags[1]) return;
  const bool any = flags[0] != 0;
  if (PHASE == 1 && !any) return;
  for (int64_t seg = blockIdx.x; seg < segs; seg += gridDim.x) {
    const int c = int(seg & 1);
    const int h = int((seg >> 1) % KVH);
    const int l = int((seg >> 1) / KVH % n_layers);
    const int64_t j = (seg >> 1) / KVH / n_layers;
    const int64_t s = sources[j], t = targets[j];
    if (!in_pool(s, capacity) || !in_pool(t, capacity)) continue;
    const bool endangered = any && is_marked(bitmap, s);
    if (PHASE == 0 && any && !endangered) continue;
    V *base = static_cast<V *>(c ? lp.v[l] : lp.k[l]);
    V *staged = tmp + seg * seg_vec;
    const V *src = (PHASE == 1 && endangered) ? staged : base + (s * KVH + h) * slot_vec;
    V *dst = (PHASE == 0 && endangered) ? staged : base + (t * KVH + h) * slot_vec;
    stream_copy(dst, src, seg_vec);
  }
}

}  // namespace
}  // namespace cg

using namespace cg;

extern "C" {

int cg_version(void) { return 100; }

size_t cg_last_error(char *buf, size_t size) {
  const std::string &m = cg::g_last_error;
  if (buf && size) {
    size_t n = m.size() < size - 1 ? m.size() : size - 1;
    __builtin_memcpy(buf, m.data(), n);
    buf[n] = '\0';
  }
  return m.size();
}

int cg_kv_write_step(const cg_kv_layer *layer, const int64_t *rows, const int64_t *positions,
                     const cg_kv_source *k_new, const cg_kv_source *v_new, int32_t B, int32_t T,
                     void *stream) {
  return guarded([&] {
    CG_REQUIRE(positions != nullptr, CG_ERR_INVALID, "positions is NULL");
    write_common(layer, rows, positions, 0, k_new, v_new, B, T, stream);
  });
}

int cg_kv_write_range(const cg_kv_layer *layer, const int64_t *rows, int32_t start,
                      const cg_kv_source *k_new, const cg_kv_source *v_new, int32_t B, int32_t T,
                      void *stream) {
  return guarded([&] { write_common(layer, rows, nullptr, start, k_new, v_new, B, T, stream); });
}

int cg_kv_read(const cg_kv_layer *layer, const int64_t *rows, int32_t B, int32_t length,
               void *k_out, void *v_out, void *stream) {
  return guarded([&] {
    check_layer(layer);
    CG_REQUIRE(B >= 0 && length >= 0, CG_ERR_INVALID, "B and length must be non-negative");
    CG_REQUIRE(length <= layer->max_len, CG_ERR_RANGE, "read length past max_len");
    if (int64_t(B) * length == 0) return;
    CG_REQUIRE(k_out && v_out, CG_ERR_INVALID, "outputs are NULL");
    CG_REQUIRE(length <= layer->max_len, CG_ERR_RANGE, "read length past max_len");
    CG_REQUIRE(rows || B <= layer->capacity, CG_ERR_RANGE, "dense read past capacity");
    const int bytes = layer->head_dim * dtype_size(layer->dtype);
    hipStream_t s = as_stream(stream);
    const int64_t positions = int64_t(B) * layer->kv_heads * length;
    if (positions == 0) return;
    auto go = [&](auto tag) {
      using V = decltype(tag);
      const int vpp = bytes / int(sizeof(V));
      const int64_t total = positions * vpp;
      kv_gather_kernel<V><<<grid_for(total, 256), 256, 0, s>>>(
          static_cast<const V *>(layer->k), static_cast<const V *>(layer->v), static_cast<V *>(k_out),
          static_cast<V *>(v_out), rows, B, layer->kv_heads, layer->max_len, length, vpp,
          layer->capacity);
      CG_LAUNCHED();
    };
    if (bytes % 16 == 0) go(uint4{});
    else if (bytes % 8 == 0) go(uint2{});
    else if (bytes % 4 == 0) go(uint32_t{});
    else go(uint16_t{});
  });
}

int cg_kv_copy_rows(const cg_kv_layer *layer, const int64_t *sources, const int64_t *targets,
                    int32_t n, int32_t length, void *stream) {
  return guarded([&] {
    check_layer(layer);
    CG_REQUIRE(n >= 0 && length >= 0, CG_ERR_INVALID, "n and length must be non-negative");
    if (int64_t(n) * length == 0) return;
    CG_REQUIRE(sources && targets, CG_ERR_INVALID, "sources / targets are NULL");
    CG_REQUIRE(length <= layer->max_len, CG_ERR_RANGE, "copy length past max_len");
    const int bytes = layer->head_dim * dtype_size(layer->dtype);
    hipStream_t s = as_stream(stream);
    if (int64_t(n) * length == 0) return;
    auto go = [&](auto tag) {
      using V = decltype(tag);
      const int vpp = bytes / int(sizeof(V));
      const int64_t total = int64_t(n) * layer->kv_heads * length * vpp;
      kv_copy_rows_kernel<V><<<grid_for(total, 256), 256, 0, s>>>(
          static_cast<V *>(layer->k), static_cast<V *>(layer->v), sources, targets, n,
          layer->kv_heads, layer->max_len, length, vpp, layer->capacity);
      CG_LAUNCHED();
    };
    if (bytes % 16 == 0) go(uint4{});
    else if (bytes % 8 == 0) go(uint2{});
    else if (bytes % 4 == 0) go(uint32_t{});
    else go(uint16_t{});
  });
}

int cg_kv_check_indices(const cg_kv_layer *layer, const int64_t *rows, int32_t B,
                        const int64_t *positions, int32_t n_pos, int32_t *flag, void *stream) {
  return guarded([&] {
    check_layer(layer);
    CG_REQUIRE(flag != nullptr, CG_ERR_INVALID, "flag is NULL");
    const int n = B > n_pos ? B : n_pos;
    if (n <= 0) return;
    kv_check_kernel<<<(n + 255) / 256, 256, 0, as_stream(stream)>>>(
        rows, B, positions, n_pos, layer->capacity, layer->max_len, flag);
    CG_LAUNCHED();
  });
}

int cg_advance_positions(int64_t *positions, int32_t n, int64_t delta, void *stream) {
  return guarded([&] {
    CG_REQUIRE(positions || n == 0, CG_ERR_INVALID, "positions is NULL");
    if (n <= 0) return;
    advance_kernel<<<(n + 255) / 256, 256, 0, as_stream(stream)>>>(positions, n, delta);
    CG_LAUNCHED();
  });
}

size_t cg_kv_copy_workspace_size(const cg_kv_layer *layers, int32_t n_layers, int32_t n, int32_t length) {
  if (!layers || n_layers <= 0 || n < 0 || length < 0 || layers[0].capacity <= 0) return 0;
  return copy_header_bytes(layers[0].capacity) + copy_bytes(layers[0], 1, n, length);
}

int cg_kv_copy_rows_layers(const cg_kv_layer *layers, int32_t n_layers, const int64_t *sources,
                           const int64_t *targets, int32_t n, int32_t length, int32_t plan, void *workspace,
                           size_t workspace_size, void *stream) {
  return guarded([&] {
    CG_REQUIRE(layers && n_layers > 0, CG_ERR_INVALID, "layers are required");
    CG_REQUIRE(n_layers <= MAX_COPY_LAYERS, CG_ERR_UNSUPPORTED, "copy_rows: more than 64 layers in one call");
    CG_REQUIRE(n >= 0 && length >= 0, CG_ERR_INVALID, "n and length must be non-negative");
    CG_REQUIRE(plan == CG_COPY_AUTO || plan == CG_COPY_ORDERED, CG_ERR_INVALID, "copy_rows: unknown plan");
    const cg_kv_layer &L0 = layers[0];
    LayerPtrs lp{};
    for (int l = 0; l < n_layers; ++l) {
      const cg_kv_layer &L = layers[l];
      check_layer(&L);
      CG_REQUIRE(L.capacity == L0.capacity && L.kv_heads == L0.kv_heads && L.max_len == L0.max_len &&
                     L.head_dim == L0.head_dim && L.dtype == L0.dtype,
                 CG_ERR_INVALID, "copy_rows: layers differ in shape");
      lp.k[l] = L.k;
      lp.v[l] = L.v;
    }
    if (int64_t(n) * length == 0) return;
    CG_REQUIRE(sources && targets, CG_ERR_INVALID, "sources / targets are NULL");
    CG_REQUIRE(length <= L0.max_len, CG_ERR_RANGE, "copy length past max_len");
    const int64_t pos_bytes = int64_t(L0.head_dim) * dtype_size(L0.dtype);
    const size_t header = copy_header_bytes(L0.capacity);
    const size_t per_layer = copy_bytes(L0, 1, n, length);
    const size_t need = header + per_layer;
    CG_REQUIRE(workspace && workspace_size >= need, CG_ERR_INVALID,
               "copy_rows: workspace too small, need " + std::to_string(need) + " bytes");
    CG_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, CG_ERR_INVALID, "copy_rows: workspace must be 16-byte aligned");
    // Layers staged per launch: as many as the workspace holds.
    const int group = int(std::min<size_t>(size_t(n_layers), (workspace_size - header) / per_layer));
    const CopyHeader hd = copy_header(workspace, L0.capacity);
    void *tmp = static_cast<char *>(workspace) + header;
    hipStream_t s = as_stream(stream);
    auto go = [&](auto tag) {
      using V = decltype(tag);
      const int64_t slot_vec = int64_t(L0.max_len) * pos_bytes / int64_t(sizeof(V));
      const int64_t seg_vec = int64_t(length) * pos_bytes / int64_t(sizeof(V));
      // The ordered walk has one wave per tile of a prefix and n pairs per lane: used when
      // that fills the chip (>= 1024 waves of one access per lane) and the walk stays short.
      const int64_t slices = int64_t(n_layers) * L0.kv_heads * 2 * seg_vec;
      const bool walk = slices >= 64 * 1024 && n <= 4096;
      constexpr int VPT = CG_WALK_VPT;
      const int64_t tiles = (seg_vec + 64 * VPT - 1) / (64 * VPT);
      const unsigned walk_grid = unsigned(int64_t(n_layers) * L0.kv_heads * 2 * tiles);
      if (walk && plan == CG_COPY_ORDERED) {
        ordered_copy_kernel<V, CG_WALK_UNROLL, VPT><<<walk_grid, 64, 0, s>>>(
            lp, sources, targets, n, L0.kv_heads, L0.capacity, slot_vec, seg_vec, tiles, nullptr);
        CG_LAUNCHED();
        return;
      }
      clear_words_kernel<<<grid_for(hd.words, 256), 256, 0, s>>>(hd.flags, hd.words);
      CG_LAUNCHED();
      mark_pairs_kernel<<<(n + 255) / 256, 256, 0, s>>>(sources, targets, n, L0.capacity, hd.bitmap, hd.last_reader);
      CG_LAUNCHED();
      classify_pairs_kernel<<<(n + 255) / 256, 256, 0, s>>>(sources, targets, n, L0.capacity, hd.bitmap,
                                                            hd.last_reader, hd.flags);
      CG_LAUNCHED();
      if (walk) {
        ordered_copy_kernel<V, CG_WALK_UNROLL, VPT><<<walk_grid, 64, 0, s>>>(
            lp, sources, targets, n, L0.kv_heads, L0.capacity, slot_vec, seg_vec, tiles, hd.flags);
        CG_LAUNCHED();
      }
      for (int first = 0; first < n_layers; first += group) {
        const int count = std::min(group, n_layers - first);
        LayerPtrs sub{};
        for (int l = 0; l < count; ++l) {
          sub.k[l] = lp.k[first + l];
          sub.v[l] = lp.v[first + l];
        }
        const int64_t segs = int64_t(n) * count * L0.kv_heads * 2;
        const unsigned grid = unsigned(std::min<int64_t>(segs, 1024));
        staged_copy_kernel<0, V><<<grid, 256, 0, s>>>(sub, count, sources, targets, L0.kv_heads, L0.capacity,
                                                       slot_vec, seg_vec, segs, static_cast<V *>(tmp), hd.flags,
                                                       hd.bitmap, !walk);
        CG_LAUNCHED();
        staged_copy_kernel<1, V><<<grid, 256, 0, s>>>(sub, count, sources, targets, L0.kv_heads, L0.capacity,
                                                       slot_vec, seg_vec, segs, static_cast<V *>(tmp), hd.flags,
                                                       hd.bitmap, !walk);
        CG_LAUNCHED();
      }
    };
    using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
    using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
    if (pos_bytes % 16 == 0) go(u32x4{});
    else if (pos_bytes % 8 == 0) go(u32x2{});
    else if (pos_bytes % 4 == 0) go(uint32_t{});
    else go(uint16_t{});
  });
}

}  // extern "C"
