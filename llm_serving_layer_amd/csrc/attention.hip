// Paged attention for arbitrary query lengths on gfx950 (chunked prefill,
// mixed prefill + decode), and the generic fallback used for any geometry
// the fast kernels do not cover.
//
//  * generic_kernel — any geometry, any query length, bottom-right causal;
//    used when prefill.hip's MFMA kernel does not cover the geometry or the
//    plan was tiled for another query tile.
//
// Numerics follow serving/backends/paged_torch.py:443-485: scores and
// softmax in fp32, probabilities rounded to the pool dtype, PV accumulated
// in fp32, output rounded to the pool dtype.
#include <algorithm>
#include <vector>

#include "pkv_common.h"

namespace pkv {

int run_fast_prefill(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                     const int32_t* cu_q, const int32_t* indptr, const int32_t* indices,
                     const int32_t* kv_lens, int32_t Hq, int32_t Hkv, int32_t D,
                     int32_t page_size, float scale, int32_t dtype, const int32_t* plan,
                     int32_t n_tiles, int32_t q_tile, int32_t* status, hipStream_t s,
                     bool* ran);

// ------------------------------------------------------------------ plans ---

int check_seq_pages(int32_t i, int32_t np, int32_t kv, int32_t last,
                           int32_t ps) {
  if (kv < 1) return fail(PKV_ERR_INVALID, "seq %d: kv_len=%d must be >= 1", i, kv);
  const int32_t need = (kv + ps - 1) / ps;
  if (np != need)
    return fail(PKV_ERR_INVALID,
                "seq %d: %d pages supplied but kv_len=%d with block_size=%d needs %d",
                i, np, kv, ps, need);
  const int32_t tail = kv - (np - 1) * ps;
  if (last != tail)
    return fail(PKV_ERR_INVALID,
                "seq %d: kv_last_page_len=%d but kv_len=%d over %d pages implies %d. "
                "An exact multiple of block_size must report %d, not 0.",
                i, last, kv, np, tail, ps);
  return PKV_OK;
}

}  // namespace pkv

using namespace pkv;

extern "C" int pkv_plan_prefill(const int32_t* cu_query_lens, const int32_t* kv_indptr,
                                const int32_t* kv_lens, const int32_t* kv_last_page_len,
                                int32_t n_seqs, int32_t page_size, int32_t q_tile,
                                int32_t* plan, int64_t plan_capacity,
                                int32_t* n_tiles_out) {
  if (n_seqs <= 0 || page_size <= 0 || q_tile <= 0)
    return fail(PKV_ERR_INVALID, "n_seqs, page_size and q_tile must be positive");
  if (cu_query_lens[0] != 0 || kv_indptr[0] != 0)
    return fail(PKV_ERR_INVALID, "cu_query_lens and kv_indptr must start at 0");
  struct Tile { int32_t seq, q0, ql; int64_t cost; };
  std::vector<Tile> tiles;
  for (int32_t i = 0; i < n_seqs; ++i) {
    const int32_t np = kv_indptr[i + 1] - kv_indptr[i];
    int rc = check_seq_pages(i, np, kv_lens[i], kv_last_page_len[i], page_size);
    if (rc) return rc;
    const int32_t ql = cu_query_lens[i + 1] - cu_query_lens[i];
    if (ql < 1 || ql > kv_lens[i])
      return fail(PKV_ERR_INVALID, "seq %d: query_len=%d outside [1, kv_len=%d]", i, ql,
                  kv_lens[i]);
    for (int32_t q0 = 0; q0 < ql; q0 += q_tile) {
      const int32_t n = std::min(q_tile, ql - q0);
      // keys visible to the tile's last row bound its work
      const int64_t keys = (int64_t)kv_lens[i] - ql + q0 + n;
      tiles.push_back({i, q0, n, keys * n});
    }
  }
  std::stable_sort(tiles.begin(), tiles.end(),
                   [](const Tile& a, const Tile& b) { return a.cost > b.cost; });
  if (4 * (int64_t)tiles.size() > plan_capacity)
    return fail(PKV_ERR_CAPACITY, "plan needs %lld entries, capacity %lld",
                (long long)(4 * tiles.size()), (long long)plan_capacity);
  int64_t o = 0;
  for (const Tile& t : tiles) {
    plan[o++] = t.seq; plan[o++] = t.q0; plan[o++] = t.ql; plan[o++] = 0;
  }
  *n_tiles_out = (int32_t)tiles.size();
  return PKV_OK;
}

namespace pkv {

// -------------------------------------------------------- generic kernel ---
// One wave per (query token, query head). Three passes over the visible keys
// (max, sum, weighted V) so the probabilities are normalised in fp32 and
// rounded to the pool dtype BEFORE the PV product, exactly the reference's
// order. Slow by design; used only where no fast kernel applies.
template <typename T>
__global__ __launch_bounds__(64) void generic_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kpool,
    const T* __restrict__ vpool, int64_t num_blocks,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ batch_idx, int32_t n_seqs, int32_t n_heads,
    int32_t n_kv_heads, int32_t D, int32_t ps, float scale, int32_t* status) {
  __shared__ float qs[256];
  __shared__ float pw[64];
  const int lane = threadIdx.x;
  const int tok = blockIdx.x / n_heads;
  const int hq = blockIdx.x - tok * n_heads;
  const int h = hq / (n_heads / n_kv_heads);
  int seq, j, q_len;
  if (cu_q) {
    seq = batch_idx[tok];
    if (seq < 0 || seq >= n_seqs) return;
    j = tok - cu_q[seq];
    q_len = cu_q[seq + 1] - cu_q[seq];
  } else {  // decode: token i is sequence i's only query
    seq = tok; j = 0; q_len = 1;
  }
  const int kv_len = kv_lens[seq];
  int n_keys = kv_len - q_len + j + 1;
  n_keys = n_keys < 0 ? 0 : (n_keys > kv_len ? kv_len : n_keys);
  const int32_t* pages = kv_indices + kv_indptr[seq];
  const int64_t row = (int64_t)n_kv_heads * D;

  for (int e = lane; e < D; e += 64)
    qs[e] = Elem<T>::to_f(q[((int64_t)tok * n_heads + hq) * D + e]);
  __syncthreads();

  auto key_row = [&](int key, const T* pool) -> const T* {
    int64_t page = pages[key / ps];
    if (page < 0 || page >= num_blocks) { flag(status, PKV_STATUS_BAD_PAGE); page = 0; }
    return pool + (page * ps + key % ps) * row + (int64_t)h * D;
  };
  auto score = [&](int key) -> float {
    const T* kr = key_row(key, kpool);
    float s = 0.f;
    for (int e = 0; e < D; ++e) s += qs[e] * Elem<T>::to_f(kr[e]);
    return s * scale;
  };

  float m = -INFINITY;
  for (int key = lane; key < n_keys; key += 64) m = fmaxf(m, score(key));
  m = wave_max(m);
  float l = 0.f;
  for (int key = lane; key < n_keys; key += 64) l += expf(score(key) - m);
  l = wave_sum(l);
  const float inv = n_keys > 0 ? 1.f / l : 0.f;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < n_keys; k0 += 64) {
    const int key = k0 + lane;
    float p = 0.f;
    if (key < n_keys) p = Elem<T>::to_f(Elem<T>::from_f(expf(score(key) - m) * inv));
    __syncthreads();
    pw[lane] = p;
    __syncthreads();
    const int nk = min(64, n_keys - k0);
    for (int u = 0; u < nk; ++u) {
      const T* vr = key_row(k0 + u, vpool);
      const float pu = pw[u];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int e = lane + 64 * c;
        if (e < D) acc[c] += pu * Elem<T>::to_f(vr[e]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int e = lane + 64 * c;
    if (e < D) out[((int64_t)tok * n_heads + hq) * D + e] = Elem<T>::from_f(acc[c]);
  }
}

template <typename T>
static int launch_generic(const void* q, void* out, const void* kp, const void* vp,
                          int64_t nb, const int32_t* cu_q, const int32_t* indptr,
                          const int32_t* indices, const int32_t* kv_lens,
                          const int32_t* bidx, int32_t n_seqs, int32_t n_tokens,
                          int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, float scale,
                          int32_t* status, hipStream_t s) {
  const int64_t blocks = (int64_t)n_tokens * Hq;
  if (blocks > 0x7fffffffLL) return fail(PKV_ERR_INVALID, "too many query rows");
  hipLaunchKernelGGL((generic_kernel<T>), dim3((unsigned)blocks), dim3(64), 0, s,
                     (const T*)q, (T*)out, (const T*)kp, (const T*)vp, nb, cu_q, indptr,
                     indices, kv_lens, bidx, n_seqs, Hq, Hkv, D, ps, scale, status);
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}

int check_geometry(int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, int32_t dtype) {
  if (!elem_bytes(dtype)) return fail(PKV_ERR_INVALID, "unsupported dtype code %d", dtype);
  if (Hq <= 0 || Hkv <= 0 || D <= 0 || ps <= 0)
    return fail(PKV_ERR_INVALID, "non-positive geometry");
  if (Hq % Hkv) return fail(PKV_ERR_INVALID, "n_heads %% n_kv_heads != 0");
  if (D > 256) return fail(PKV_ERR_INVALID, "head_dim %d > 256 is not supported", D);
  return PKV_OK;
}

}  // namespace pkv

namespace pkv {
int generic_decode(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                   const int32_t* indptr, const int32_t* indices, const int32_t* kv_lens,
                   int32_t n_seqs, int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, float scale,
                   int32_t dtype, int32_t* status, hipStream_t s) {
  if (dtype == PKV_DTYPE_F16)
    return launch_generic<_Float16>(q, out, kp, vp, nb, nullptr, indptr, indices, kv_lens,
                                    nullptr, n_seqs, n_seqs, Hq, Hkv, D, ps, scale, status, s);
  if (dtype == PKV_DTYPE_BF16)
    return launch_generic<__bf16>(q, out, kp, vp, nb, nullptr, indptr, indices, kv_lens,
                                  nullptr, n_seqs, n_seqs, Hq, Hkv, D, ps, scale, status, s);
  return launch_generic<float>(q, out, kp, vp, nb, nullptr, indptr, indices, kv_lens, nullptr,
                               n_seqs, n_seqs, Hq, Hkv, D, ps, scale, status, s);
}
}  // namespace pkv

extern "C" int pkv_attend_prefill(const void* q, void* out, const void* k_pool,
                                  const void* v_pool, int64_t num_blocks,
                                  const int32_t* cu_query_lens, const int32_t* kv_indptr,
                                  const int32_t* kv_indices, const int32_t* kv_lens,
                                  const int32_t* batch_indices, int32_t n_seqs,
                                  int32_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                                  int32_t head_dim, int32_t page_size, float scale,
                                  int32_t dtype, const int32_t* plan, int32_t n_tiles,
                                  int32_t q_tile, int32_t* status_word, void* stream) {
  int rc = check_geometry(n_heads, n_kv_heads, head_dim, page_size, dtype);
  if (rc) return rc;
  if (n_tokens <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  bool ran = false;
  rc = run_fast_prefill(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices,
                        kv_lens, n_heads, n_kv_heads, head_dim, page_size, scale, dtype, plan,
                        n_tiles, q_tile, status_word, s, &ran);
  if (rc || ran) return rc;
  if (dtype == PKV_DTYPE_F16)
    return launch_generic<_Float16>(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices, kv_lens, batch_indices, n_seqs, n_tokens, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
  if (dtype == PKV_DTYPE_BF16)
    return launch_generic<__bf16>(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices, kv_lens, batch_indices, n_seqs, n_tokens, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
  return launch_generic<float>(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices, kv_lens, batch_indices, n_seqs, n_tokens, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
}
