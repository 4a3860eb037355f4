// KV pool operations: append (write_step), prefill write (write_range), gathered read,
// row compaction (copy_rows) and a device-side index check.
//
// Semantics follow cardgym/nn/kv_cache.py:65-138.  Every kernel bounds-checks its
// indices and skips out-of-range entries instead of faulting; cg_kv_check_indices
// reports them through a device flag.
#include <string>

#include "common.h"

namespace cg {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string &message) { g_last_error = message; }

namespace {

// One thread per (b, t, head, element).  Each thread moves one element: the write is a
// scatter of 64-128 byte rows, so the launch is bound by the number of rows, not bytes.
template <typename TC, typename TS>
__global__ void kv_write_kernel(TC *__restrict__ kc, TC *__restrict__ vc, const TS *__restrict__ ks,
                                const TS *__restrict__ vs, int64_t ks_b, int64_t ks_h, int64_t ks_t,
                                int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                const int64_t *__restrict__ rows, const int64_t *__restrict__ positions,
                                int32_t start, int32_t B, int32_t T, int32_t KVH, int32_t L,
                                int32_t D, int32_t capacity) {
  const int64_t total = int64_t(B) * T * KVH * D;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int d = int(i % D);
    int64_t r = i / D;
    const int h = int(r % KVH);
    r /= KVH;
    const int t = int(r % T);
    const int b = int(r / T);
    const int64_t row = rows ? rows[b] : int64_t(b);
    const int64_t pos = positions ? positions[int64_t(b) * T + t] : int64_t(start) + t;
    if (row < 0 || row >= capacity || pos < 0 || pos >= L) continue;
    const int64_t dst = ((row * KVH + h) * L + pos) * D + d;
    kc[dst] = convert<TC>(ks[b * ks_b + h * ks_h + t * ks_t + d]);
    vc[dst] = convert<TC>(vs[b * vs_b + h * vs_h + t * vs_t + d]);
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
  const int64_t total = int64_t(B) * T * L.kv_heads * L.head_dim;
  if (total == 0) return;
  kv_write_kernel<TC, TS><<<grid_for(total, 256), 256, 0, s>>>(
      static_cast<TC *>(L.k), static_cast<TC *>(L.v), static_cast<const TS *>(k.data),
      static_cast<const TS *>(v.data), k.stride_b, k.stride_h, k.stride_t, v.stride_b, v.stride_h,
      v.stride_t, rows, positions, start, B, T, L.kv_heads, L.max_len, L.head_dim, L.capacity);
  CG_LAUNCHED();
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

}  // extern "C"
