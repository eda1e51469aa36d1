// Paged decode attention for gfx950 (every sequence has one query token).
//
// Work decomposition (planned on the host once per batch): each sequence's
// pages are cut into partitions of at most PP pages. A workgroup owns one
// partition; its waves own one KV head each, so the waves of a workgroup
// request the same pages together (the heads of a token row are adjacent in
// memory). The split depends only on the sequence's own length, so a
// sequence's result never depends on what it is batched with.
//
// Per wave (G query heads share the KV head, G <= 16):
//  1. one wave-wide load of the partition's page ids, broadcast by readlane;
//     every K and V load of the partition is issued before any arithmetic;
//  2. S^T = K Q^T with one 16x16x32 MFMA per 32 dims of a 16-token page: the
//     K rows of the page ARE the A operand (lane (token m, group g) holds
//     16 contiguous bytes of row m), Q^T the B operand (column n = query
//     head n, zero beyond G). The result leaves lane (head n, group g)
//     holding the scores of tokens 4g..4g+3 of the page for head n;
//  3. softmax in registers: mask past kv_len, the partition max and sum need
//     only an in-lane pass plus two cross-lane steps; p = 2^(s*scale*log2e -
//     m) is rounded to the pool dtype. Those four p values per lane are
//     exactly the A operand of a 16x16x16 MFMA (row = head, k = token);
//  4. PV on MFMA: the V page goes to LDS row-major, and ds_read_b64_tr_b16
//     hands each lane 4 consecutive tokens of one dim -- the B operand --
//     one read per 16 dims. Tokens past kv_len are zeroed in LDS so stale
//     bits can never reach the sum;
//  5. a partition that covers its whole sequence writes the output; otherwise
//     it writes (o, m, l) partials that merge_kernel combines in a second,
//     small launch. (Merging inside the same launch would need an agent-scope
//     release per partition; on a multi-XCD part that is an L2 write-back per
//     wave and measured ~10x slower than the extra launch.)
#include <algorithm>
#include <vector>

#include "pkv_common.h"

namespace pkv {

constexpr int kWorkInts = 8;  // {seq, page_base, n_pages, slot, kv_len, tok0, n_parts, slot0}

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <typename T> struct Mma;
template <> struct Mma<_Float16> {
  typedef f16x8 vec8;
  typedef f16x4 vec4;
  __device__ static f32x4 qk(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static f32x4 pv(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<__bf16> {
  typedef bf16x8 vec8;
  typedef bf16x4 vec4;
  __device__ static f32x4 qk(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static f32x4 pv(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                    __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  }
};

template <typename T, int D, int G, int PP>
__global__ __launch_bounds__(512) void decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kpool,
    const T* __restrict__ vpool, int64_t num_blocks, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ work, int32_t n_kv_heads, float scale_log2,
    float* __restrict__ part_o, float* __restrict__ part_ml, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  constexpr int PS = 16;
  constexpr int NCH = D / 32;   // QK MFMA k-chunks per page
  constexpr int NDB = D / 16;   // PV MFMA dim blocks
  constexpr int VL = D / 8;     // lanes per V row when loading (16 bytes each)
  constexpr int VROWS = 64 / VL;          // V rows per load instruction
  constexpr int VLOADS = PS / VROWS;      // load instructions per V page

  extern __shared__ __align__(16) unsigned char smem[];
  const int wave = threadIdx.x >> 6;
  T* vlds = reinterpret_cast<T*>(smem) + (size_t)wave * PP * PS * D;  // [PP][16][D]

  const int lane = threadIdx.x & 63;
  const int hw = blockDim.x >> 6;  // KV heads per workgroup
  const int groups_per_item = n_kv_heads / hw;
  const int wi = blockIdx.x / groups_per_item;
  const int h = (blockIdx.x - wi * groups_per_item) * hw + wave;
  const int32_t* w = work + kWorkInts * wi;
  const int seq = w[0], pbase = w[1], np = w[2], slot = w[3];
  const int kv_len = w[4], tok0 = w[5];
  const int Hq = n_kv_heads * G;
  const int64_t row = (int64_t)n_kv_heads * D;

  int pid = 0;
  if (lane < np) pid = kv_indices[pbase + lane];
  const bool bad = lane < np && (pid < 0 || (int64_t)pid >= num_blocks);
  if (bad) pid = 0;
  if (__builtin_amdgcn_ballot_w64(bad) && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);

  const int n = lane & 15;   // MFMA row/column index within a 16-lane block
  const int g = lane >> 4;   // MFMA k-group

  // Q^T as the QK B operand: column n = query head h*G + n (zero beyond G).
  vec8 qb[NCH];
  {
    const T* qr = q + ((int64_t)seq * Hq + h * G + (n < G ? n : 0)) * D + g * 8;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      vec8 t = *reinterpret_cast<const vec8*>(qr + c * 32);
      qb[c] = (n < G) ? t : vec8{};
    }
  }

  // Issue every K and V load of the partition.
  vec8 kt[PP][NCH];
  vec8 vt[PP][VLOADS];
  const int vr_ = lane / VL, vc_ = lane % VL;
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < np) {
      const int64_t page = __builtin_amdgcn_readlane(pid, j);
      const T* kr = kpool + (page * PS + n) * row + (int64_t)h * D + g * 8;
#pragma unroll
      for (int c = 0; c < NCH; ++c) kt[j][c] = *reinterpret_cast<const vec8*>(kr + c * 32);
#pragma unroll
      for (int u = 0; u < VLOADS; ++u)
        vt[j][u] = *reinterpret_cast<const vec8*>(vpool + (page * PS + u * VROWS + vr_) * row +
                                                  (int64_t)h * D + vc_ * 8);
    }
  }

  // V pages into LDS, row-major [token][dim]; rows past kv_len are zeroed.
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < np) {
#pragma unroll
      for (int u = 0; u < VLOADS; ++u) {
        const int t = u * VROWS + vr_;
        vec8 x = vt[j][u];
        if (tok0 + j * PS + t >= kv_len) x = vec8{};
        *reinterpret_cast<vec8*>(vlds + (j * PS + t) * D + vc_ * 8) = x;
      }
    }
  }

  // S^T per page; lane (n, g) holds tokens 4g..4g+3 of page j for head n.
  float s[PP][4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (j < np) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc = Mma<T>::qk(kt[j][c], qb[c], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool live = j < np && tok0 + j * PS + 4 * g + i < kv_len;
      s[j][i] = live ? acc[i] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, s[j][i]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));

  vec4 p[PP];
  float lsum = 0.f;
#pragma unroll
  for (int j = 0; j < PP; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = __builtin_amdgcn_exp2f(s[j][i] - mx);
      lsum += e;
      p[j][i] = (T)e;
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  __syncthreads();  // V tiles written by this wave are visible to its own LDS reads

  // O (rows = heads, cols = dims) += P V; B operand by transposing LDS reads.
  f32x4 o[NDB];
#pragma unroll
  for (int b = 0; b < NDB; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < np) {
      const T* base = vlds + (j * PS + 4 * g + (n >> 2)) * D + 4 * (n & 3);
#pragma unroll
      for (int b = 0; b < NDB; ++b) {
        const i16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(base + 16 * b));
        o[b] = Mma<T>::pv(p[j], __builtin_bit_cast(vec4, raw), o[b]);
      }
    }
  }

  // lane (dim column n, group g) holds heads 4g..4g+3 of dims 16b + n.
  if (slot < 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      const float li = __shfl(lsum, r, 64);  // lane r holds head r's sum
      if (r < G) {
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          out[((int64_t)seq * Hq + h * G + r) * D + 16 * b + n] = (T)(o[b][i] / li);
      }
    }
    return;
  }
  // Split sequence: unnormalised partial output and (m, l) per head.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * g + i;
    if (r < G) {
#pragma unroll
      for (int b = 0; b < NDB; ++b)
        part_o[((int64_t)slot * Hq + h * G + r) * D + 16 * b + n] = o[b][i];
    }
  }
  if (lane < G) {
    float* pm = part_ml + ((int64_t)slot * Hq + h * G + lane) * 2;
    pm[0] = mx;
    pm[1] = lsum;
  }
}

// Combine the split-K partials of one (sequence, KV head) per wave:
//   o = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s.
// Lanes first run over partitions to build the weights (held in LDS), then
// over output values; the partial loads of every partition are independent
// and issued back to back.
template <typename T, int D, int G>
__global__ __launch_bounds__(64) void merge_kernel(
    T* __restrict__ out, const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int32_t* __restrict__ merges, int32_t n_kv_heads) {
  constexpr int VALS = G * D / 64;
  __shared__ float wts[64][G];
  __shared__ float inv_l[G];
  const int lane = threadIdx.x;
  const int mi = blockIdx.x / n_kv_heads;
  const int h = blockIdx.x - mi * n_kv_heads;
  const int seq = merges[3 * mi], s0 = merges[3 * mi + 1], ns = merges[3 * mi + 2];
  const int Hq = n_kv_heads * G;

  float M[G];
#pragma unroll
  for (int r = 0; r < G; ++r) M[r] = -INFINITY;
  for (int c = 0; c < ns; c += 64)
    if (c + lane < ns) {
#pragma unroll
      for (int r = 0; r < G; ++r)
        M[r] = fmaxf(M[r], part_ml[((int64_t)(s0 + c + lane) * Hq + h * G + r) * 2]);
    }
#pragma unroll
  for (int r = 0; r < G; ++r) M[r] = wave_max(M[r]);

  float acc[VALS];
#pragma unroll
  for (int i = 0; i < VALS; ++i) acc[i] = 0.f;
  float L[G];
#pragma unroll
  for (int r = 0; r < G; ++r) L[r] = 0.f;
  for (int c = 0; c < ns; c += 64) {
    const int n = min(64, ns - c);
    if (lane < n) {
#pragma unroll
      for (int r = 0; r < G; ++r) {
        const int64_t b = ((int64_t)(s0 + c + lane) * Hq + h * G + r) * 2;
        const float w = __builtin_amdgcn_exp2f(part_ml[b] - M[r]);
        wts[lane][r] = w;
        L[r] += w * part_ml[b + 1];
      }
    }
    __syncthreads();
    int s = 0;
    for (; s + 4 <= n; s += 4) {  // four partitions' loads in flight at once
      float v[4][VALS];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float* po = part_o + ((int64_t)(s0 + c + s + u) * Hq + h * G) * D;
#pragma unroll
        for (int i = 0; i < VALS; ++i) v[u][i] = po[lane + 64 * i];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < VALS; ++i) acc[i] += wts[s + u][(lane + 64 * i) / D] * v[u][i];
    }
    for (; s < n; ++s) {
      const float* po = part_o + ((int64_t)(s0 + c + s) * Hq + h * G) * D;
#pragma unroll
      for (int i = 0; i < VALS; ++i) {
        const int idx = lane + 64 * i;
        acc[i] += wts[s][idx / D] * po[idx];
      }
    }
    __syncthreads();
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < G; ++r) inv_l[r] = 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < G; ++r) {
    const float tot = wave_sum(L[r]);
    if (lane == 0) inv_l[r] = 1.f / tot;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < VALS; ++i) {
    const int idx = lane + 64 * i;
    out[((int64_t)seq * Hq + h * G) * D + idx] = (T)(acc[i] * inv_l[idx / D]);
  }
}

template <typename T, int D, int G, int PP>
static void launch(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                   const int32_t* indices, const int32_t* work, int32_t n_work,
                   const int32_t* merges, int32_t n_merge, int32_t Hkv, float sl2, float* po,
                   float* pml, int32_t* status, hipStream_t s) {
  int hw = 1;  // waves (KV heads) per workgroup: the largest divisor of Hkv up to 8
  for (int c = 8; c >= 1; --c)
    if (Hkv % c == 0) { hw = c; break; }
  const size_t lds = (size_t)hw * PP * 16 * D * sizeof(T);
  hipLaunchKernelGGL((decode_kernel<T, D, G, PP>), dim3((unsigned)(n_work * (Hkv / hw))),
                     dim3(64 * hw), lds, s, (const T*)q, (T*)out, (const T*)kp,
                     (const T*)vp, nb, indices, work, Hkv, sl2, po, pml, status);
  if (n_merge > 0)
    hipLaunchKernelGGL((merge_kernel<T, D, G>), dim3((unsigned)(n_merge * Hkv)), dim3(64), 0,
                       s, (T*)out, po, pml, merges, Hkv);
}

typedef void (*LaunchFn)(const void*, void*, const void*, const void*, int64_t, const int32_t*,
                         const int32_t*, int32_t, const int32_t*, int32_t, int32_t, float,
                         float*, float*, int32_t*, hipStream_t);

template <typename T, int D, int G>
static LaunchFn pick_pp(int pp) {
  switch (pp) {
    case 2: return launch<T, D, G, 2>;
    case 4: return launch<T, D, G, 4>;
    case 8: return launch<T, D, G, 8>;
    default: return nullptr;
  }
}

template <typename T, int D>
static LaunchFn pick_g(int G, int pp) {
  switch (G) {
    case 1: return pick_pp<T, D, 1>(pp);
    case 2: return pick_pp<T, D, 2>(pp);
    case 4: return pick_pp<T, D, 4>(pp);
    case 8: return pick_pp<T, D, 8>(pp);
    case 16: return pick_pp<T, D, 16>(pp);
    default: return nullptr;
  }
}

template <typename T>
static LaunchFn pick(int D, int G, int pp) {
  switch (D) {
    case 64: return pick_g<T, 64>(G, pp);
    case 128: return pick_g<T, 128>(G, pp);
    default: return nullptr;
  }
}

static LaunchFn fast_decode(int32_t dtype, int32_t D, int32_t G, int32_t page_size, int32_t pp) {
  if (page_size != 16) return nullptr;
  if (dtype == PKV_DTYPE_F16) return pick<_Float16>(D, G, pp);
  if (dtype == PKV_DTYPE_BF16) return pick<__bf16>(D, G, pp);
  return nullptr;
}

// generic fallback lives in attention.hip
int generic_decode(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                   const int32_t* indptr, const int32_t* indices, const int32_t* kv_lens,
                   int32_t n_seqs, int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, float scale,
                   int32_t dtype, int32_t* status, hipStream_t s);
int check_seq_pages(int32_t i, int32_t np, int32_t kv, int32_t last, int32_t ps);
int check_geometry(int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, int32_t dtype);

}  // namespace pkv

using namespace pkv;

extern "C" int pkv_plan_decode(const int32_t* kv_indptr, const int32_t* kv_lens,
                               const int32_t* kv_last_page_len, int32_t n_seqs,
                               int32_t page_size, int32_t part_pages, int32_t* plan,
                               int64_t plan_capacity, int32_t* n_work_out,
                               int32_t* n_split_out, int32_t* n_slots_out) {
  if (n_seqs <= 0 || page_size <= 0 || part_pages <= 0)
    return fail(PKV_ERR_INVALID, "n_seqs, page_size and part_pages must be positive");
  if (kv_indptr[0] != 0) return fail(PKV_ERR_INVALID, "kv_indptr must start at 0");
  struct Item { int32_t v[kWorkInts]; };
  std::vector<Item> items;
  std::vector<int32_t> merges;
  items.reserve(n_seqs);
  int32_t slots = 0, split = 0;
  for (int32_t i = 0; i < n_seqs; ++i) {
    const int32_t np = kv_indptr[i + 1] - kv_indptr[i];
    int rc = check_seq_pages(i, np, kv_lens[i], kv_last_page_len[i], page_size);
    if (rc) return rc;
    const int32_t parts = (np + part_pages - 1) / part_pages;
    for (int32_t p = 0; p < parts; ++p) {
      const int32_t first = p * part_pages;
      items.push_back({{i, kv_indptr[i] + first, std::min(part_pages, np - first),
                        parts == 1 ? -1 : slots + p, kv_lens[i], first * page_size, parts,
                        parts == 1 ? -1 : slots}});
    }
    if (parts > 1) {
      merges.insert(merges.end(), {i, slots, parts});
      slots += parts;
      ++split;
    }
  }
  // Longest partitions first, so the short tail items fill in behind them.
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return a.v[2] > b.v[2]; });
  const int64_t need = (int64_t)kWorkInts * items.size() + (int64_t)merges.size();
  if (need > plan_capacity)
    return fail(PKV_ERR_CAPACITY, "plan needs %lld entries, capacity %lld", (long long)need,
                (long long)plan_capacity);
  int64_t o = 0;
  for (const Item& it : items)
    for (int k = 0; k < kWorkInts; ++k) plan[o++] = it.v[k];
  for (int32_t v : merges) plan[o++] = v;
  *n_work_out = (int32_t)items.size();
  *n_split_out = split;
  *n_slots_out = slots;
  return PKV_OK;
}

extern "C" int64_t pkv_decode_workspace_bytes(int32_t n_slots, int32_t n_heads,
                                              int32_t head_dim) {
  return n_slots > 0 ? (int64_t)n_slots * n_heads * (head_dim + 2) * 4 : 0;
}

extern "C" int pkv_attend_decode(const void* q, void* out, const void* k_pool,
                                 const void* v_pool, int64_t num_blocks,
                                 const int32_t* kv_indptr, const int32_t* kv_indices,
                                 const int32_t* kv_lens, int32_t n_seqs, int32_t n_heads,
                                 int32_t n_kv_heads, int32_t head_dim, int32_t page_size,
                                 float scale, int32_t dtype, const int32_t* plan,
                                 int32_t n_work, int32_t n_merge, int32_t n_slots,
                                 int32_t part_pages,
                                 void* workspace, int64_t workspace_bytes,
                                 int32_t* status_word, void* stream) {
  int rc = check_geometry(n_heads, n_kv_heads, head_dim, page_size, dtype);
  if (rc) return rc;
  if (n_seqs <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int32_t G = n_heads / n_kv_heads;
  LaunchFn fn = fast_decode(dtype, head_dim, G, page_size, part_pages);
  if (!fn)
    return generic_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                          n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype,
                          status_word, s);
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
  if ((int64_t)n_work * n_kv_heads > 0x7fffffffLL)
    return fail(PKV_ERR_INVALID, "too many work items");
  fn(q, out, k_pool, v_pool, num_blocks, kv_indices, plan, n_work,
     plan + (int64_t)kWorkInts * n_work, n_merge, n_kv_heads, scale * kLog2e, po, pml,
     status_word, s);
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}
