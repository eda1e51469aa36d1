// Paged attention for gfx950.
//
//  * decode_kernel   — every sequence has one query token. Split-K over the
//    sequence's pages: one wave per (partition, KV head). QK^T for the G
//    query heads that share the KV head is one 16x16x32 MFMA per 32 dims of
//    a 16-token page (the K rows of a page ARE the MFMA B operand: lane
//    (n, g) loads 16 contiguous bytes of token n's row). Softmax runs in
//    LDS; PV runs on the VALU with v_dot2 (two tokens per instruction, fp32
//    accumulation). Partitions spanning a whole sequence write the output;
//    the others write (m, l, o) partials that merge_kernel combines.
//  * generic_kernel  — any geometry, any query length, bottom-right causal.
//    The correctness fallback for shapes the fast kernels do not cover.
//
// Numerics follow serving/backends/paged_torch.py:443-485: scores and
// softmax in fp32, probabilities rounded to the pool dtype, PV accumulated
// in fp32, output rounded to the pool dtype.
#include <algorithm>
#include <vector>

#include "pkv_common.h"

namespace pkv {

// ------------------------------------------------------------------ plans ---

static int check_seq_pages(int32_t i, int32_t np, int32_t kv, int32_t last,
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

extern "C" int pkv_plan_decode(const int32_t* kv_indptr, const int32_t* kv_lens,
                               const int32_t* kv_last_page_len, int32_t n_seqs,
                               int32_t page_size, int32_t part_pages, int32_t* plan,
                               int64_t plan_capacity, int32_t* n_work_out,
                               int32_t* n_merge_out, int32_t* n_slots_out) {
  if (n_seqs <= 0 || page_size <= 0 || part_pages <= 0)
    return fail(PKV_ERR_INVALID, "n_seqs, page_size and part_pages must be positive");
  if (kv_indptr[0] != 0) return fail(PKV_ERR_INVALID, "kv_indptr must start at 0");
  struct Item { int32_t seq, first, np, slot; };
  std::vector<Item> items;
  std::vector<int32_t> merges;
  items.reserve(n_seqs);
  int32_t slots = 0;
  for (int32_t i = 0; i < n_seqs; ++i) {
    const int32_t np = kv_indptr[i + 1] - kv_indptr[i];
    int rc = check_seq_pages(i, np, kv_lens[i], kv_last_page_len[i], page_size);
    if (rc) return rc;
    const int32_t parts = (np + part_pages - 1) / part_pages;
    if (parts == 1) {
      items.push_back({i, 0, np, -1});
    } else {
      merges.insert(merges.end(), {i, slots, parts});
      for (int32_t p = 0; p < parts; ++p)
        items.push_back({i, p * part_pages, std::min(part_pages, np - p * part_pages),
                         slots + p});
      slots += parts;
    }
  }
  // Longest partitions first, so the short tail items fill in behind them.
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return a.np > b.np; });
  const int64_t need = 4 * (int64_t)items.size() + (int64_t)merges.size();
  if (need > plan_capacity)
    return fail(PKV_ERR_CAPACITY, "plan needs %lld entries, capacity %lld",
                (long long)need, (long long)plan_capacity);
  int64_t o = 0;
  for (const Item& it : items) {
    plan[o++] = it.seq; plan[o++] = it.first; plan[o++] = it.np; plan[o++] = it.slot;
  }
  for (int32_t v : merges) plan[o++] = v;
  *n_work_out = (int32_t)items.size();
  *n_merge_out = (int32_t)(merges.size() / 3);
  *n_slots_out = slots;
  return PKV_OK;
}

extern "C" int64_t pkv_decode_workspace_bytes(int32_t n_slots, int32_t n_heads,
                                              int32_t head_dim) {
  if (n_slots <= 0) return 0;
  return (int64_t)n_slots * n_heads * (head_dim + 2) * 4;
}

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

// ------------------------------------------------------ fast decode path ---

template <typename T> struct Mfma;
template <> struct Mfma<_Float16> {
  typedef f16x8 vec8;
  typedef f16x2 vec2;
  __device__ static f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static float dot2(vec2 a, vec2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <> struct Mfma<__bf16> {
  typedef bf16x8 vec8;
  typedef bf16x2_t vec2;
  __device__ static f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static float dot2(vec2 a, vec2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};

// D: head_dim (64 | 128). G: query heads per KV head (1 | 2 | 4).
// PP: pages per partition. Page size is fixed at 16 tokens (one MFMA N tile).
template <typename T, int D, int G, int PP>
__global__ __launch_bounds__(64) void decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kpool,
    const T* __restrict__ vpool, int64_t num_blocks,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ work,
    int32_t n_kv_heads, float scale_log2, float* __restrict__ part_o,
    float* __restrict__ part_ml, int32_t* status) {
  typedef typename Mfma<T>::vec8 vec8;
  typedef typename Mfma<T>::vec2 vec2;
  constexpr int PS = 16;
  constexpr int NCH = D / 32;        // MFMA k-chunks per 16-token tile
  constexpr int LPT = D / 8;         // lanes per token row in the PV layout
  constexpr int PAIRS = 64 / LPT;    // token pairs per PV pass
  constexpr int PASSES = PS / (2 * PAIRS);
  constexpr int NT = PP * PS;        // tokens per partition

  __shared__ float sc[NT * 4];
  __shared__ vec2 pl[(NT / 2) * G];

  const int lane = threadIdx.x;
  const int wi = blockIdx.x / n_kv_heads;
  const int h = blockIdx.x - wi * n_kv_heads;
  const int seq = work[4 * wi + 0];
  const int p0 = work[4 * wi + 1];
  const int np = work[4 * wi + 2];
  const int slot = work[4 * wi + 3];
  const int Hq = n_kv_heads * G;
  const int kv_len = kv_lens[seq];
  const int64_t row = (int64_t)n_kv_heads * D;

  // Page ids of this partition: lane j < np holds page j; broadcast later.
  int pid = 0;
  if (lane < np) pid = kv_indices[kv_indptr[seq] + p0 + lane];
  const bool bad = lane < np && (pid < 0 || (int64_t)pid >= num_blocks);
  if (bad) pid = 0;
  if (__builtin_amdgcn_ballot_w64(bad) && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);

  const int n = lane & 15;   // MFMA column (token in tile) / row (query head)
  const int g = lane >> 4;   // MFMA k-slot group

  // Q as the A operand: row n = query head h*G + n (zero rows beyond G).
  vec8 qa[NCH];
  {
    const T* qr = q + ((int64_t)seq * Hq + h * G + (n < G ? n : 0)) * D + g * (D / 4);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      vec8 t = *reinterpret_cast<const vec8*>(qr + c * 8);
      qa[c] = (n < G) ? t : vec8{};
    }
  }

  // Issue every K and V load of the partition before any arithmetic.
  vec8 kt[PP][NCH];
  vec8 vt[PP][PASSES][2];
  const int dc = lane % LPT;
  const int pr = lane / LPT;
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < np) {
      const int64_t page = __builtin_amdgcn_readlane(pid, j);
      const T* kr = kpool + (page * PS + n) * row + (int64_t)h * D + g * (D / 4);
#pragma unroll
      for (int c = 0; c < NCH; ++c) kt[j][c] = *reinterpret_cast<const vec8*>(kr + c * 8);
#pragma unroll
      for (int ps_ = 0; ps_ < PASSES; ++ps_) {
        const int t0 = 2 * (ps_ * PAIRS + pr);
        const T* vr = vpool + (page * PS + t0) * row + (int64_t)h * D + dc * 8;
        vt[j][ps_][0] = *reinterpret_cast<const vec8*>(vr);
        vt[j][ps_][1] = *reinterpret_cast<const vec8*>(vr + row);
      }
    }
  }

  // QK^T: one 16x16 tile of scores per page; lanes 0..15 hold rows 0..3.
  float mrun[G];
#pragma unroll
  for (int r = 0; r < G; ++r) mrun[r] = -INFINITY;
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < np) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NCH; ++c) s = Mfma<T>::mma(qa[c], kt[j][c], s);
      if (g == 0) {
        const bool live = (p0 + j) * PS + n < kv_len;
        f32x4 w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = live ? s[r] * scale_log2 : -INFINITY;
#pragma unroll
        for (int r = 0; r < G; ++r) mrun[r] = fmaxf(mrun[r], w[r]);
        *reinterpret_cast<f32x4*>(&sc[(j * PS + n) * 4]) = w;
      }
    } else if (g == 0) {
      const f32x4 w = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      *reinterpret_cast<f32x4*>(&sc[(j * PS + n) * 4]) = w;
    }
  }
  float m[G];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    float v = mrun[r];
#pragma unroll
    for (int s = 8; s >= 1; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    m[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));  // lanes 0..15 agree
  }
  __syncthreads();

  // Unnormalised probabilities p = 2^(s - m), rounded to the pool dtype and
  // stored as token pairs; row sums in fp32.
  float lsum[G];
#pragma unroll
  for (int r = 0; r < G; ++r) lsum[r] = 0.f;
#pragma unroll
  for (int u = 0; u < NT / 64; ++u) {
    const int t = lane + 64 * u;
    const f32x4 sv = *reinterpret_cast<const f32x4*>(&sc[t * 4]);
    T* plh = reinterpret_cast<T*>(pl);
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const float p = __builtin_amdgcn_exp2f(sv[r] - m[r]);
      lsum[r] += p;
      plh[((t >> 1) * G + r) * 2 + (t & 1)] = (T)p;
    }
  }
#pragma unroll
  for (int r = 0; r < G; ++r) lsum[r] = wave_sum(lsum[r]);
  __syncthreads();

  // PV on the VALU: acc[r][e] += p[r][t0] * V[t0][e] + p[r][t1] * V[t1][e].
  float acc[G][8];
#pragma unroll
  for (int r = 0; r < G; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < np) {
      const bool tail = (p0 + j + 1) * PS > kv_len;
#pragma unroll
      for (int ps_ = 0; ps_ < PASSES; ++ps_) {
        const int t0 = 2 * (ps_ * PAIRS + pr);
        vec8 v0 = vt[j][ps_][0], v1 = vt[j][ps_][1];
        if (tail) {  // never let an unwritten slot's bits reach the sum
          if ((p0 + j) * PS + t0 >= kv_len) v0 = vec8{};
          if ((p0 + j) * PS + t0 + 1 >= kv_len) v1 = vec8{};
        }
        vec2 pp[G];
#pragma unroll
        for (int r = 0; r < G; ++r) pp[r] = pl[((j * PS + t0) >> 1) * G + r];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          vec2 vp;
          vp[0] = v0[e];
          vp[1] = v1[e];
#pragma unroll
          for (int r = 0; r < G; ++r) acc[r][e] = Mfma<T>::dot2(pp[r], vp, acc[r][e]);
        }
      }
    }
  }
  // Sum over the token-pair lanes that share a dim chunk.
#pragma unroll
  for (int s = LPT; s < 64; s <<= 1)
#pragma unroll
    for (int r = 0; r < G; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] += __shfl_xor(acc[r][e], s, 64);

  if (pr == 0) {
    if (slot < 0) {
#pragma unroll
      for (int r = 0; r < G; ++r) {
        const float inv = 1.f / lsum[r];
        vec8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (T)(acc[r][e] * inv);
        *reinterpret_cast<vec8*>(out + ((int64_t)seq * Hq + h * G + r) * D + dc * 8) = o;
      }
    } else {
#pragma unroll
      for (int r = 0; r < G; ++r) {
        float* po = part_o + ((int64_t)slot * Hq + h * G + r) * D + dc * 8;
        *reinterpret_cast<f32x4*>(po) = f32x4{acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
        *reinterpret_cast<f32x4*>(po + 4) = f32x4{acc[r][4], acc[r][5], acc[r][6], acc[r][7]};
        if (lane == 0) {
          float* pm = part_ml + ((int64_t)slot * Hq + h * G + r) * 2;
          pm[0] = m[r];
          pm[1] = lsum[r];
        }
      }
    }
  }
}

// Combine a sequence's split-K partials: o = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s.
template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(
    T* __restrict__ out, const float* __restrict__ part_o,
    const float* __restrict__ part_ml, const int32_t* __restrict__ merges,
    int32_t n_heads, int32_t D) {
  const int seq = merges[3 * blockIdx.x + 0];
  const int s0 = merges[3 * blockIdx.x + 1];
  const int ns = merges[3 * blockIdx.x + 2];
  for (int idx = threadIdx.x; idx < n_heads * D; idx += blockDim.x) {
    const int hq = idx / D;
    float M = -INFINITY;
    for (int s = 0; s < ns; ++s) M = fmaxf(M, part_ml[((int64_t)(s0 + s) * n_heads + hq) * 2]);
    float L = 0.f, O = 0.f;
    for (int s = 0; s < ns; ++s) {
      const int64_t b = (int64_t)(s0 + s) * n_heads + hq;
      const float w = __builtin_amdgcn_exp2f(part_ml[b * 2] - M);
      L += w * part_ml[b * 2 + 1];
      O += w * part_o[b * D + (idx - hq * D)];
    }
    out[(int64_t)seq * n_heads * D + idx] = Elem<T>::from_f(O / L);
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

template <typename T, int D, int G, int PP>
static void launch_decode(const void* q, void* out, const void* kp, const void* vp,
                          int64_t nb, const int32_t* indptr, const int32_t* indices,
                          const int32_t* kv_lens, const int32_t* work, int32_t n_work,
                          int32_t Hkv, float scale_log2, float* po, float* pml,
                          int32_t* status, hipStream_t s) {
  hipLaunchKernelGGL((decode_kernel<T, D, G, PP>), dim3((unsigned)(n_work * Hkv)),
                     dim3(64), 0, s, (const T*)q, (T*)out, (const T*)kp, (const T*)vp,
                     nb, indptr, indices, kv_lens, work, Hkv, scale_log2, po, pml, status);
}

template <typename T, int D, int G>
static bool dispatch_pp(int32_t pp, const void* q, void* out, const void* kp,
                        const void* vp, int64_t nb, const int32_t* indptr,
                        const int32_t* indices, const int32_t* kv_lens,
                        const int32_t* work, int32_t n_work, int32_t Hkv, float sl2,
                        float* po, float* pml, int32_t* status, hipStream_t s) {
  switch (pp) {
    case 4: launch_decode<T, D, G, 4>(q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s); return true;
    case 8: launch_decode<T, D, G, 8>(q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s); return true;
    default: return false;
  }
}

template <typename T, int D>
static bool dispatch_g(int32_t G, int32_t pp, const void* q, void* out, const void* kp,
                       const void* vp, int64_t nb, const int32_t* indptr,
                       const int32_t* indices, const int32_t* kv_lens, const int32_t* work,
                       int32_t n_work, int32_t Hkv, float sl2, float* po, float* pml,
                       int32_t* status, hipStream_t s) {
  switch (G) {
    case 1: return dispatch_pp<T, D, 1>(pp, q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s);
    case 2: return dispatch_pp<T, D, 2>(pp, q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s);
    case 4: return dispatch_pp<T, D, 4>(pp, q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s);
    default: return false;
  }
}

template <typename T>
static bool dispatch_fast_decode(int32_t D, int32_t G, int32_t pp, const void* q,
                                 void* out, const void* kp, const void* vp, int64_t nb,
                                 const int32_t* indptr, const int32_t* indices,
                                 const int32_t* kv_lens, const int32_t* work,
                                 int32_t n_work, int32_t Hkv, float sl2, float* po,
                                 float* pml, int32_t* status, hipStream_t s) {
  switch (D) {
    case 64: return dispatch_g<T, 64>(G, pp, q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s);
    case 128: return dispatch_g<T, 128>(G, pp, q, out, kp, vp, nb, indptr, indices, kv_lens, work, n_work, Hkv, sl2, po, pml, status, s);
    default: return false;
  }
}

static int check_geometry(int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, int32_t dtype) {
  if (!elem_bytes(dtype)) return fail(PKV_ERR_INVALID, "unsupported dtype code %d", dtype);
  if (Hq <= 0 || Hkv <= 0 || D <= 0 || ps <= 0)
    return fail(PKV_ERR_INVALID, "non-positive geometry");
  if (Hq % Hkv) return fail(PKV_ERR_INVALID, "n_heads %% n_kv_heads != 0");
  if (D > 256) return fail(PKV_ERR_INVALID, "head_dim %d > 256 is not supported", D);
  return PKV_OK;
}

}  // namespace pkv

extern "C" int pkv_attend_decode(const void* q, void* out, const void* k_pool,
                                 const void* v_pool, int64_t num_blocks,
                                 const int32_t* kv_indptr, const int32_t* kv_indices,
                                 const int32_t* kv_lens, int32_t n_seqs, int32_t n_heads,
                                 int32_t n_kv_heads, int32_t head_dim, int32_t page_size,
                                 float scale, int32_t dtype, const int32_t* plan,
                                 int32_t n_work, int32_t n_merge, int32_t n_slots,
                                 int32_t part_pages, void* workspace, int64_t workspace_bytes,
                                 int32_t* status_word, void* stream) {
  int rc = check_geometry(n_heads, n_kv_heads, head_dim, page_size, dtype);
  if (rc) return rc;
  if (n_seqs <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int32_t G = n_heads / n_kv_heads;
  const bool fast_geom = page_size == 16 && (dtype == PKV_DTYPE_F16 || dtype == PKV_DTYPE_BF16) &&
                         (head_dim == 64 || head_dim == 128) && (G == 1 || G == 2 || G == 4);
  if (!fast_geom) {
    if (dtype == PKV_DTYPE_F16)
      return launch_generic<_Float16>(q, out, k_pool, v_pool, num_blocks, nullptr, kv_indptr, kv_indices, kv_lens, nullptr, n_seqs, n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
    if (dtype == PKV_DTYPE_BF16)
      return launch_generic<__bf16>(q, out, k_pool, v_pool, num_blocks, nullptr, kv_indptr, kv_indices, kv_lens, nullptr, n_seqs, n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
    return launch_generic<float>(q, out, k_pool, v_pool, num_blocks, nullptr, kv_indptr, kv_indices, kv_lens, nullptr, n_seqs, n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
  }
  if (!plan || n_work <= 0) return fail(PKV_ERR_INVALID, "decode needs a plan");
  if ((uintptr_t)q % 16 || (uintptr_t)out % 16 || (uintptr_t)k_pool % 16 ||
      (uintptr_t)v_pool % 16)
    return fail(PKV_ERR_INVALID, "q, out and the pools must be 16-byte aligned");
  float* po = nullptr;
  float* pml = nullptr;
  if (n_merge > 0) {
    const int64_t need = pkv_decode_workspace_bytes(n_slots, n_heads, head_dim);
    if (!workspace || n_slots <= 0 || workspace_bytes < need)
      return fail(PKV_ERR_CAPACITY, "split-K plan needs %lld workspace bytes, got %lld",
                  (long long)need, (long long)workspace_bytes);
    po = (float*)workspace;  // [n_slots][Hq][D] partial outputs, then [n_slots][Hq][2] (m, l)
    pml = po + (int64_t)n_slots * n_heads * head_dim;
  }
  const float sl2 = scale * kLog2e;
  bool ok;
  if (dtype == PKV_DTYPE_F16)
    ok = dispatch_fast_decode<_Float16>(head_dim, G, part_pages, q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens, plan, n_work, n_kv_heads, sl2, po, pml, status_word, s);
  else
    ok = dispatch_fast_decode<__bf16>(head_dim, G, part_pages, q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens, plan, n_work, n_kv_heads, sl2, po, pml, status_word, s);
  if (!ok) return fail(PKV_ERR_INVALID, "part_pages %d not supported (4 or 8)", part_pages);
  PKV_LAUNCH_CHECK();
  if (n_merge > 0) {
    const int32_t* merges = plan + 4 * (int64_t)n_work;
    if (dtype == PKV_DTYPE_F16)
      hipLaunchKernelGGL((merge_kernel<_Float16>), dim3(n_merge), dim3(256), 0, s,
                         (_Float16*)out, po, pml, merges, n_heads, head_dim);
    else
      hipLaunchKernelGGL((merge_kernel<__bf16>), dim3(n_merge), dim3(256), 0, s,
                         (__bf16*)out, po, pml, merges, n_heads, head_dim);
    PKV_LAUNCH_CHECK();
  }
  return PKV_OK;
}

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
  (void)plan; (void)n_tiles; (void)q_tile;
  if (n_tokens <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PKV_DTYPE_F16)
    return launch_generic<_Float16>(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices, kv_lens, batch_indices, n_seqs, n_tokens, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
  if (dtype == PKV_DTYPE_BF16)
    return launch_generic<__bf16>(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices, kv_lens, batch_indices, n_seqs, n_tokens, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
  return launch_generic<float>(q, out, k_pool, v_pool, num_blocks, cu_query_lens, kv_indptr, kv_indices, kv_lens, batch_indices, n_seqs, n_tokens, n_heads, n_kv_heads, head_dim, page_size, scale, status_word, s);
}
