// Pure data movement: KV append (slot-mapped row scatter), batched
// copy-on-write block copies over every layer, and the swap gather/scatter
// between pool blocks and a staging buffer. All HBM-bound byte copies:
// 16-byte vector accesses, consecutive lanes on consecutive 16-byte chunks
// of one row/block so each wave moves whole 128-byte lines.
#include <cstdarg>
#include <cstring>

#include <algorithm>

#include "pkv_common.h"

namespace pkv {

static thread_local std::string g_err;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// ------------------------------------------------------------ KV append ---
// One wave-sized group of lanes per (token, K|V) row; each lane moves VEC
// bytes. Rows of 1 KiB (8 KV heads x 64 dims x fp16) take one 64-lane pass.
template <typename V>
__global__ __launch_bounds__(256) void append_kernel(
    char* __restrict__ kpool, char* __restrict__ vpool, int64_t num_slots,
    const char* __restrict__ k, const char* __restrict__ v,
    const int32_t* __restrict__ slots, int64_t n_tokens, int32_t row_vecs,
    int32_t* status) {
  const int64_t total = n_tokens * 2 * (int64_t)row_vecs;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += stride) {
    const int64_t row = i / row_vecs;  // token * 2 + which
    const int32_t c = (int32_t)(i - row * row_vecs);
    const int64_t t = row >> 1;
    const int which = (int)(row & 1);
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) {
      if (c == 0 && which == 0) flag(status, PKV_STATUS_BAD_SLOT);
      continue;
    }
    const V* src = reinterpret_cast<const V*>(which ? v : k) + t * row_vecs + c;
    V* dst = reinterpret_cast<V*>(which ? vpool : kpool) + slot * row_vecs + c;
    *dst = __builtin_nontemporal_load(src);
  }
}

// --------------------------------------------------------- block copies ---
// Work unit = one (item, plane) block of `block_vecs` 16-byte vectors.
// mode 0: copy  pool[plane][src[i]] -> pool[plane][dst[i]]
// mode 1: gather pool[plane][ids[i]] -> staging[kv][layer][i]
// mode 2: scatter staging[kv][layer][i] -> pool[plane][ids[i]]
template <typename V, int MODE>
__global__ __launch_bounds__(256) void block_kernel(
    char* __restrict__ pool, int32_t n_planes, int64_t plane_vecs,
    int64_t block_vecs, int64_t num_blocks, const int32_t* __restrict__ a,
    const int32_t* __restrict__ b, int32_t n_items, char* __restrict__ staging,
    int32_t* status) {
  const int64_t unit = blockIdx.x;  // item * n_planes + plane
  const int32_t item = (int32_t)(unit / n_planes);
  const int32_t plane = (int32_t)(unit - (int64_t)item * n_planes);
  if (item >= n_items) return;
  V* base = reinterpret_cast<V*>(pool);
  const V* src;
  V* dst;
  if (MODE == 0) {
    const int64_t s = a[item], d = b[item];
    if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) {
      if (threadIdx.x == 0 && plane == 0) flag(status, PKV_STATUS_BAD_BLOCK);
      return;
    }
    if (s == d) return;
    src = base + plane * plane_vecs + s * block_vecs;
    dst = base + plane * plane_vecs + d * block_vecs;
  } else {
    const int64_t id = a[item];
    if (id < 0 || id >= num_blocks) {
      if (threadIdx.x == 0 && plane == 0) flag(status, PKV_STATUS_BAD_BLOCK);
      return;
    }
    // staging order is [kv][layer][item]; plane = layer * 2 + kv
    const int32_t layer = plane >> 1, kv = plane & 1;
    const int32_t n_layers = n_planes >> 1;
    V* st = reinterpret_cast<V*>(staging) +
            (((int64_t)kv * n_layers + layer) * n_items + item) * block_vecs;
    V* pb = base + plane * plane_vecs + id * block_vecs;
    if (MODE == 1) { src = pb; dst = st; } else { src = st; dst = pb; }
  }
  // Four loads in flight per thread before their stores. The loads are
  // ordinary (cached): copy-on-write sources repeat (shared prefixes), and a
  // repeated source is then read from L2. The stores stream (nontemporal).
  constexpr int U = 4;
  int64_t c = threadIdx.x;
  for (; c + (U - 1) * (int64_t)blockDim.x < block_vecs; c += U * (int64_t)blockDim.x) {
    V t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) t[u] = src[c + u * blockDim.x];
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(t[u], dst + c + u * blockDim.x);
  }
  for (; c < block_vecs; c += blockDim.x) __builtin_nontemporal_store(src[c], dst + c);
}

typedef int32_t v4i __attribute__((ext_vector_type(4)));

template <int MODE>
static int launch_blocks(char* pool, int32_t n_layers, int64_t plane_bytes,
                         int64_t block_bytes, int64_t num_blocks,
                         const int32_t* a, const int32_t* b, int32_t n_items,
                         char* staging, int32_t* status, hipStream_t stream) {
  if (n_layers <= 0 || plane_bytes <= 0 || block_bytes <= 0 || num_blocks <= 0)
    return fail(PKV_ERR_INVALID, "non-positive pool geometry");
  if (n_items < 0) return fail(PKV_ERR_INVALID, "negative item count");
  if (plane_bytes < block_bytes * num_blocks)
    return fail(PKV_ERR_INVALID, "plane_bytes smaller than num_blocks * block_bytes");
  if (n_items == 0) return PKV_OK;
  const int64_t units = (int64_t)n_items * n_layers * 2;
  if (units > 0x7fffffffLL) return fail(PKV_ERR_INVALID, "too many blocks in one call");
  const uintptr_t align = (uintptr_t)pool | (uintptr_t)staging;
  dim3 grid((unsigned)units), block(256);
  if (block_bytes % 16 == 0 && plane_bytes % 16 == 0 && align % 16 == 0) {
    hipLaunchKernelGGL((block_kernel<v4i, MODE>), grid, block, 0, stream, pool,
                       n_layers * 2, plane_bytes / 16, block_bytes / 16,
                       num_blocks, a, b, n_items, staging, status);
  } else if (block_bytes % 4 == 0 && plane_bytes % 4 == 0 && align % 4 == 0) {
    hipLaunchKernelGGL((block_kernel<int32_t, MODE>), grid, block, 0, stream,
                       pool, n_layers * 2, plane_bytes / 4, block_bytes / 4,
                       num_blocks, a, b, n_items, staging, status);
  } else if (block_bytes % 2 == 0 && plane_bytes % 2 == 0 && align % 2 == 0) {
    hipLaunchKernelGGL((block_kernel<int16_t, MODE>), grid, block, 0, stream,
                       pool, n_layers * 2, plane_bytes / 2, block_bytes / 2,
                       num_blocks, a, b, n_items, staging, status);
  } else {
    return fail(PKV_ERR_INVALID, "block size / alignment must be a multiple of 2 bytes");
  }
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}

// One step's metadata from a pinned host buffer to the device, read by the
// kernel through the buffer's device mapping: the copy is an ordinary
// kernel on the caller's stream, so the next kernel does not wait for a
// hand-off from a copy engine. 16-byte chunks when both ends and the size
// allow it, bytes otherwise.
template <typename V>
__global__ __launch_bounds__(256) void upload_kernel(V* __restrict__ dst,
                                                     const V* __restrict__ src, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_upload_pinned(void* dst, const void* host, int64_t bytes, void* stream) {
  if (bytes < 0) return fail(PKV_ERR_INVALID, "negative byte count");
  if (bytes == 0) return PKV_OK;
  if (!dst || !host) return fail(PKV_ERR_INVALID, "null buffer");
  void* src = nullptr;
  // only pinned memory the runtime maps for the device has a device pointer
  const hipError_t e = hipHostGetDevicePointer(&src, const_cast<void*>(host), 0);
  if (e != hipSuccess || !src)
    return fail(PKV_ERR_INVALID, "the source is not pinned host memory mapped for the device "
                "(%s)", hipGetErrorString(e));
  hipStream_t s = (hipStream_t)stream;
  const bool vec = ((uintptr_t)dst | (uintptr_t)src | (uintptr_t)bytes) % 16 == 0;
  const int64_t n = vec ? bytes / 16 : bytes;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 1024);
  if (vec)
    hipLaunchKernelGGL((upload_kernel<v4i>), dim3(grid), dim3(256), 0, s, (v4i*)dst,
                       (const v4i*)src, n);
  else
    hipLaunchKernelGGL((upload_kernel<unsigned char>), dim3(grid), dim3(256), 0, s,
                       (unsigned char*)dst, (const unsigned char*)src, n);
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}

int pkv_abi_version(void) { return 11; }

const char* pkv_last_error(void) { return g_err.c_str(); }

int pkv_append_kv(void* k_pool, void* v_pool, int64_t num_slots, const void* k,
                  const void* v, const int32_t* slot_mapping, int64_t n_tokens,
                  int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                  int32_t* status_word, void* stream) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(PKV_ERR_INVALID, "unsupported dtype code %d", dtype);
  if (n_kv_heads <= 0 || head_dim <= 0 || num_slots < 0 || n_tokens < 0)
    return fail(PKV_ERR_INVALID, "non-positive geometry");
  if (n_tokens == 0) return PKV_OK;
  if (!k_pool || !v_pool || !k || !v || !slot_mapping)
    return fail(PKV_ERR_INVALID, "null pointer argument");
  const int64_t row_bytes = (int64_t)n_kv_heads * head_dim * eb;
  const uintptr_t align = (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)k | (uintptr_t)v;
  hipStream_t s = (hipStream_t)stream;
  auto grid_for = [&](int64_t vecs) {
    int64_t total = n_tokens * 2 * vecs;
    int64_t blocks = (total + 255) / 256;
    return (unsigned)(blocks > 65536 ? 65536 : blocks);
  };
  if (row_bytes % 16 == 0 && align % 16 == 0) {
    const int64_t vecs = row_bytes / 16;
    hipLaunchKernelGGL((append_kernel<v4i>), dim3(grid_for(vecs)), dim3(256), 0, s,
                       (char*)k_pool, (char*)v_pool, num_slots, (const char*)k,
                       (const char*)v, slot_mapping, n_tokens, (int32_t)vecs, status_word);
  } else if (row_bytes % 4 == 0 && align % 4 == 0) {
    const int64_t vecs = row_bytes / 4;
    hipLaunchKernelGGL((append_kernel<int32_t>), dim3(grid_for(vecs)), dim3(256), 0, s,
                       (char*)k_pool, (char*)v_pool, num_slots, (const char*)k,
                       (const char*)v, slot_mapping, n_tokens, (int32_t)vecs, status_word);
  } else {
    const int64_t vecs = row_bytes / 2;
    hipLaunchKernelGGL((append_kernel<int16_t>), dim3(grid_for(vecs)), dim3(256), 0, s,
                       (char*)k_pool, (char*)v_pool, num_slots, (const char*)k,
                       (const char*)v, slot_mapping, n_tokens, (int32_t)vecs, status_word);
  }
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}

int pkv_copy_blocks(void* pool_base, int32_t n_layers, int64_t plane_bytes,
                    int64_t block_bytes, int64_t num_blocks, const int32_t* src,
                    const int32_t* dst, int32_t n_pairs, int32_t* status_word,
                    void* stream) {
  if (n_pairs > 0 && (!pool_base || !src || !dst))
    return fail(PKV_ERR_INVALID, "null pointer argument");
  return launch_blocks<0>((char*)pool_base, n_layers, plane_bytes, block_bytes,
                          num_blocks, src, dst, n_pairs, nullptr, status_word,
                          (hipStream_t)stream);
}

int pkv_gather_blocks(const void* pool_base, int32_t n_layers, int64_t plane_bytes,
                      int64_t block_bytes, int64_t num_blocks, const int32_t* ids,
                      int32_t n_ids, void* staging, int32_t* status_word,
                      void* stream) {
  if (n_ids > 0 && (!pool_base || !ids || !staging))
    return fail(PKV_ERR_INVALID, "null pointer argument");
  return launch_blocks<1>((char*)pool_base, n_layers, plane_bytes, block_bytes,
                          num_blocks, ids, nullptr, n_ids, (char*)staging,
                          status_word, (hipStream_t)stream);
}

int pkv_scatter_blocks(void* pool_base, int32_t n_layers, int64_t plane_bytes,
                       int64_t block_bytes, int64_t num_blocks, const int32_t* ids,
                       int32_t n_ids, const void* staging, int32_t* status_word,
                       void* stream) {
  if (n_ids > 0 && (!pool_base || !ids || !staging))
    return fail(PKV_ERR_INVALID, "null pointer argument");
  return launch_blocks<2>((char*)pool_base, n_layers, plane_bytes, block_bytes,
                          num_blocks, ids, nullptr, n_ids, (char*)staging,
                          status_word, (hipStream_t)stream);
}

}  // extern "C"
