// Paged decode attention for gfx950 (every sequence has one query token).
//
// Work decomposition (planned on the host once per batch): a sequence's
// pages are cut into partitions of at most PP pages (split-K over the KV
// axis; the split depends only on that sequence's own length, so its result
// never depends on what it is batched with). A workgroup owns one partition
// and its waves own one KV head each, so they request the same pages
// together (the heads of a token row are adjacent in memory). One partition
// per wave, no loop and no barrier: the kernel keeps 5 waves per SIMD.
//
// Per wave and partition (G query heads share the KV head, G <= 16):
//  1. one wave-wide load of the partition's page ids, broadcast by readlane;
//     every K and V load of the partition is issued before any arithmetic;
//  2. S^T = K Q^T with one 16x16x32 MFMA per 32 dims of a 16-token page: the
//     K rows ARE the A operand (lane (token m, group g) holds 16 contiguous
//     bytes of row m), Q^T the B operand (column n = query head n, zero
//     beyond G). Lane (head n, group g) then holds the scores of tokens
//     4g..4g+3 of the page for head n;
//  3. softmax in registers: mask past kv_len, running max / sum over the
//     wave's partitions with one in-lane pass plus two cross-lane steps;
//     p = 2^(s*scale*log2e - m) rounded to the pool dtype -- four values per
//     lane that are exactly the A operand of a 16x16x16 MFMA;
//  4. PV on MFMA: the V page goes to LDS row-major and ds_read_b64_tr_b16
//     hands each lane 4 consecutive tokens of one dim, the B operand, one
//     read per 16 dims. Tokens past kv_len are zeroed so stale bits can
//     never reach the sum.
//
// Split sequences merge in the same launch. Each partition publishes its
// partial (o, m, l) with agent-scope stores, which write through the
// per-XCD L2 to the memory-side coherence point, waits until they have
// completed (s_waitcnt vmcnt(0)), then bumps an arrival counter for its
// (sequence, KV head). The wave that sees the last arrival reads the
// partials back with agent-scope loads (which do not hit a stale L2 line)
// and writes the output. This avoids a second launch and also avoids an
// agent-scope release fence, whose L2 write-back walks the whole cache and
// measured ~10x slower per wave than the merge itself.
//
// Fused append (optional): when the caller passes the step's new K/V rows,
// the wave that owns a sequence's last page writes the row of its head to
// slot_mapping's slot and patches the copy it already loaded, so a decode
// step costs one launch per layer instead of two. The patch is applied only
// when slot_mapping names the same slot as the page table, so the result is
// exactly "append, then attend".
#include <algorithm>
#include <vector>

#include "pkv_common.h"

namespace pkv {

// {seq, index of the partition's first page in kv_indices, n_pages, partial
//  slot (-1: the partition is the whole sequence), kv_len, first token,
//  n_partitions of the sequence, first slot of the sequence}
constexpr int kWorkInts = 8;
constexpr int kWaves = 8;

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

// Orders this wave's LDS writes before its own (cross-lane) LDS reads. A
// wave's LDS operations execute in order, so a compiler-level barrier with
// wavefront-scope fences is all that is needed (no s_barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T, int D, int G, int PP>
__global__ __launch_bounds__(kWaves * 64) void decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, T* __restrict__ kpool, T* __restrict__ vpool,
    int64_t num_blocks, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ work, int32_t n_kv_heads, float scale_log2,
    const T* __restrict__ k_new, const T* __restrict__ v_new,
    const int32_t* __restrict__ slot_mapping, float* part_o, float* part_ml,
    int32_t* counters, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  constexpr int PS = 16;
  constexpr int NCH = D / 32;   // QK MFMA k-chunks per page
  constexpr int NDB = D / 16;   // PV MFMA dim blocks
  constexpr int VL = D / 8;     // lanes per V row when loading (16 bytes each)
  constexpr int VROWS = 64 / VL;          // V rows per load instruction
  constexpr int VLOADS = PS / VROWS;      // load instructions per V page
  constexpr int TILE = PP * PS * D;       // V tile elements per wave

  extern __shared__ __align__(16) unsigned char smem[];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  T* vlds = reinterpret_cast<T*>(smem) + (size_t)wave * TILE;

  const int hw = blockDim.x >> 6;  // KV heads per workgroup
  const int groups_per_item = n_kv_heads / hw;
  const int wi = blockIdx.x / groups_per_item;
  const int h = (blockIdx.x - wi * groups_per_item) * hw + wave;
  const int32_t* w = work + kWorkInts * wi;
  const int seq = w[0], pbase = w[1], npp = w[2], slot = w[3];
  const int kv_len = w[4], tok0 = w[5], nparts = w[6], slot0 = w[7];
  const int Hq = n_kv_heads * G;
  const int64_t row = (int64_t)n_kv_heads * D;
  const int n = lane & 15;   // MFMA row/column within a 16-lane block
  const int g = lane >> 4;   // MFMA k-group
  const int vr_ = lane / VL, vc_ = lane % VL;

  int pid = 0;
  if (lane < npp) pid = kv_indices[pbase + lane];
  const bool bad = lane < npp && (pid < 0 || (int64_t)pid >= num_blocks);
  if (bad) pid = 0;
  if (__builtin_amdgcn_ballot_w64(bad) && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);

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
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < npp) {
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

  if (k_new && tok0 + npp * PS >= kv_len) {
    // This wave owns the sequence's newest token for head h.
    const int jl = npp - 1;
    const int tl = (kv_len - 1) % PS;
    const int64_t csr_slot = (int64_t)__builtin_amdgcn_readlane(pid, jl) * PS + tl;
    const int64_t new_slot = slot_mapping[seq];
    const bool in_range = new_slot >= 0 && new_slot < num_blocks * PS;
    if (!in_range && lane == 0) flag(status, PKV_STATUS_BAD_SLOT);
    const bool patch = new_slot == csr_slot;
    const T* kn = k_new + ((int64_t)seq * n_kv_heads + h) * D;
    const T* vn = v_new + ((int64_t)seq * n_kv_heads + h) * D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (n == tl) {
        const vec8 x = *reinterpret_cast<const vec8*>(kn + c * 32 + g * 8);
        if (in_range)
          *reinterpret_cast<vec8*>(kpool + new_slot * row + (int64_t)h * D + c * 32 + g * 8) = x;
#pragma unroll
        for (int j = 0; j < PP; ++j)  // static indices keep kt in registers
          if (patch && j == jl) kt[j][c] = x;
      }
    }
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      if (u * VROWS + vr_ == tl) {
        const vec8 x = *reinterpret_cast<const vec8*>(vn + vc_ * 8);
        if (in_range)
          *reinterpret_cast<vec8*>(vpool + new_slot * row + (int64_t)h * D + vc_ * 8) = x;
#pragma unroll
        for (int j = 0; j < PP; ++j)
          if (patch && j == jl) vt[j][u] = x;
      }
    }
  }

  // V pages into this wave's LDS tile, row-major [token][dim]; rows past
  // kv_len are zeroed.
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < npp) {
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
    if (j < npp) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc = Mma<T>::qk(kt[j][c], qb[c], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool live = j < npp && tok0 + j * PS + 4 * g + i < kv_len;
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
  wave_lds_sync();

  // O (rows = heads, cols = dims) += P V; B operand by transposing reads.
  f32x4 o[NDB];
#pragma unroll
  for (int b = 0; b < NDB; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < PP; ++j) {
    if (j < npp) {
      const T* base = vlds + (j * PS + 4 * g + (n >> 2)) * D + 4 * (n & 3);
#pragma unroll
      for (int b = 0; b < NDB; ++b) {
        const i16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + 16 * b));
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

  // ---- split sequence: publish, count, and the last arrival merges --------
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * g + i;
    if (r < G) {
#pragma unroll
      for (int b = 0; b < NDB; ++b)
        __hip_atomic_store(part_o + ((int64_t)slot * Hq + h * G + r) * D + 16 * b + n,
                           o[b][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (lane < G) {
    float* pm = part_ml + ((int64_t)slot * Hq + h * G + lane) * 2;
    __hip_atomic_store(pm, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(pm + 1, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Every partial store of this wave has completed at the coherence point
  // before the arrival is counted.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  int32_t* cnt = counters + (int64_t)seq * n_kv_heads + h;
  int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != nparts - 1) return;

  // Last arrival for (seq, h). Lanes run over partitions to get each head
  // row's max M and sum L, then, 64 partitions at a time, put the weights
  // 2^(m_s - M) in this wave's (now free) LDS tile and read the partial
  // outputs in batches of MB partitions with all of a lane's values at once:
  // a long sequence costs a few dependent round trips, not one per partition.
  float* wts = reinterpret_cast<float*>(vlds);  // [64][G]; the tile holds >= 64*G floats
  auto load_ml = [&](int c0, float* mr, float* lr) {
    const bool ok = c0 + lane < nparts;
    const int64_t b2 = ((int64_t)(slot0 + (ok ? c0 + lane : 0)) * Hq + h * G) * 2;
#pragma unroll
    for (int r = 0; r < G; ++r) {
      mr[r] = ok ? __hip_atomic_load(part_ml + b2 + 2 * r, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
      lr[r] = ok ? __hip_atomic_load(part_ml + b2 + 2 * r + 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    }
  };
  float mr[G], lr[G], M[G], L[G];
#pragma unroll
  for (int r = 0; r < G; ++r) { M[r] = -INFINITY; L[r] = 0.f; }
  for (int c0 = 0; c0 < nparts; c0 += 64) {
    load_ml(c0, mr, lr);
#pragma unroll
    for (int r = 0; r < G; ++r) M[r] = fmaxf(M[r], wave_max(mr[r]));
  }
  constexpr int VALS = (G * D + 63) / 64;
  constexpr int MB = VALS >= 16 ? 1 : 16 / VALS;  // partitions per load batch
  float acc[VALS];
#pragma unroll
  for (int i = 0; i < VALS; ++i) acc[i] = 0.f;
  for (int c0 = 0; c0 < nparts; c0 += 64) {
    if (nparts > 64) load_ml(c0, mr, lr);  // else still in registers
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const float wv = c0 + lane < nparts ? __builtin_amdgcn_exp2f(mr[r] - M[r]) : 0.f;
      L[r] += wave_sum(wv * lr[r]);
      wts[lane * G + r] = wv;
    }
    wave_lds_sync();
    const int cn = min(64, nparts - c0);
    for (int s0 = 0; s0 < cn; s0 += MB) {
      float v[MB][VALS];
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        const bool ok = s0 + u < cn;
        const float* po = part_o + ((int64_t)(slot0 + c0 + (ok ? s0 + u : 0)) * Hq + h * G) * D;
#pragma unroll
        for (int i = 0; i < VALS; ++i) {
          const int idx = lane + 64 * i;
          v[u][i] = (ok && idx < G * D)
                        ? __hip_atomic_load(po + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        if (s0 + u >= cn) break;
#pragma unroll
        for (int i = 0; i < VALS; ++i) {
          const int idx = lane + 64 * i;
          if (idx < G * D) acc[i] += wts[(s0 + u) * G + idx / D] * v[u][i];
        }
      }
    }
    wave_lds_sync();  // the next chunk rewrites the weights
  }
#pragma unroll
  for (int i = 0; i < VALS; ++i) {
    const int idx = lane + 64 * i;
    if (idx < G * D) {
      const int r = idx / D;
      float lr_ = L[0];
#pragma unroll
      for (int rr = 1; rr < G; ++rr)  // static indices keep L in registers
        if (r == rr) lr_ = L[rr];
      out[((int64_t)seq * Hq + h * G) * D + idx] = (T)(acc[i] / lr_);
    }
  }
  if (lane == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static int heads_per_workgroup(int Hkv) {
  for (int c = kWaves; c > 1; --c)
    if (Hkv % c == 0) return c;
  return 1;
}

template <typename T, int D, int G, int PP>
static void launch(const void* q, void* out, void* kp, void* vp, int64_t nb,
                   const int32_t* indices, const int32_t* work, int32_t n_work, int32_t Hkv,
                   float sl2, const void* kn, const void* vn, const int32_t* slots, float* po,
                   float* pml, int32_t* cnt, int32_t* status, hipStream_t s) {
  const int hw = heads_per_workgroup(Hkv);
  const size_t lds = (size_t)hw * PP * 16 * D * sizeof(T);
  hipLaunchKernelGGL((decode_kernel<T, D, G, PP>), dim3((unsigned)(n_work * (Hkv / hw))),
                     dim3(hw * 64), lds, s, (const T*)q, (T*)out, (T*)kp, (T*)vp, nb, indices,
                     work, Hkv, sl2, (const T*)kn, (const T*)vn, slots, po, pml, cnt, status);
}

typedef void (*LaunchFn)(const void*, void*, void*, void*, int64_t, const int32_t*,
                         const int32_t*, int32_t, int32_t, float, const void*, const void*,
                         const int32_t*, float*, float*, int32_t*, int32_t*, hipStream_t);

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
    case 128: return pp <= 4 ? pick_g<T, 128>(G, pp) : nullptr;
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

extern "C" int pkv_decode_fast_path(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                    int32_t page_size, int32_t dtype, int32_t part_pages) {
  if (n_kv_heads <= 0 || n_heads % n_kv_heads) return 0;
  return fast_decode(dtype, head_dim, n_heads / n_kv_heads, page_size, part_pages) ? 1 : 0;
}

extern "C" int pkv_plan_decode(const int32_t* kv_indptr, const int32_t* kv_lens,
                               const int32_t* kv_last_page_len, int32_t n_seqs,
                               int32_t page_size, int32_t part_pages, int32_t* plan,
                               int64_t plan_capacity, int32_t* n_work_out,
                               int32_t* n_slots_out) {
  if (n_seqs <= 0 || page_size <= 0 || part_pages <= 0)
    return fail(PKV_ERR_INVALID, "n_seqs, page_size and part_pages must be positive");
  if (kv_indptr[0] != 0) return fail(PKV_ERR_INVALID, "kv_indptr must start at 0");
  struct Item { int32_t v[kWorkInts]; };
  std::vector<Item> items;
  items.reserve(n_seqs);
  int32_t slots = 0;
  for (int32_t i = 0; i < n_seqs; ++i) {
    const int32_t np = kv_indptr[i + 1] - kv_indptr[i];
    int rc = check_seq_pages(i, np, kv_lens[i], kv_last_page_len[i], page_size);
    if (rc) return rc;
    const int32_t parts = (np + part_pages - 1) / part_pages;
    const int32_t slot0 = parts > 1 ? slots : -1;
    for (int32_t p = 0; p < parts; ++p) {
      const int32_t first = p * part_pages;
      items.push_back({{i, kv_indptr[i] + first, std::min(part_pages, np - first),
                        parts > 1 ? slots + p : -1, kv_lens[i], first * page_size, parts,
                        slot0}});
    }
    if (parts > 1) slots += parts;
  }
  // Longest partitions first, so the short tail items fill in behind them.
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return a.v[2] > b.v[2]; });
  const int64_t need = (int64_t)kWorkInts * items.size();
  if (need > plan_capacity)
    return fail(PKV_ERR_CAPACITY, "plan needs %lld entries, capacity %lld", (long long)need,
                (long long)plan_capacity);
  int64_t o = 0;
  for (const Item& it : items)
    for (int k = 0; k < kWorkInts; ++k) plan[o++] = it.v[k];
  *n_work_out = (int32_t)items.size();
  *n_slots_out = slots;
  return PKV_OK;
}

extern "C" int64_t pkv_decode_workspace_bytes(int32_t n_seqs, int32_t n_slots,
                                              int32_t n_heads, int32_t n_kv_heads,
                                              int32_t head_dim) {
  if (n_seqs <= 0 || n_kv_heads <= 0 || n_slots <= 0) return 0;
  const int64_t counters = ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256;
  return counters + (int64_t)n_slots * n_heads * (head_dim + 2) * 4;
}

extern "C" int pkv_attend_decode(const void* q, void* out, void* k_pool, void* v_pool,
                                 int64_t num_blocks, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* kv_lens,
                                 int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t page_size, float scale,
                                 int32_t dtype, const int32_t* plan, int32_t n_work,
                                 int32_t n_slots, int32_t part_pages, const void* k_new,
                                 const void* v_new, const int32_t* slot_mapping,
                                 void* workspace, int64_t workspace_bytes,
                                 int32_t* status_word, void* stream) {
  int rc = check_geometry(n_heads, n_kv_heads, head_dim, page_size, dtype);
  if (rc) return rc;
  if (n_seqs <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int32_t G = n_heads / n_kv_heads;
  LaunchFn fn = fast_decode(dtype, head_dim, G, page_size, part_pages);
  if (!fn) {
    if (k_new)
      return fail(PKV_ERR_INVALID, "a fused append needs the fast decode path "
                                   "(see pkv_decode_fast_path)");
    return generic_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                          n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype,
                          status_word, s);
  }
  if (!plan || n_work <= 0) return fail(PKV_ERR_INVALID, "decode needs a plan");
  if ((k_new == nullptr) != (v_new == nullptr) || (k_new && !slot_mapping))
    return fail(PKV_ERR_INVALID, "a fused append needs k_new, v_new and slot_mapping");
  const uintptr_t al = (uintptr_t)q | (uintptr_t)out | (uintptr_t)k_pool | (uintptr_t)v_pool |
                       (uintptr_t)k_new | (uintptr_t)v_new;
  if (al % 16) return fail(PKV_ERR_INVALID, "q, out, pools and new rows must be 16-byte aligned");
  float* po = nullptr;
  float* pml = nullptr;
  int32_t* cnt = nullptr;
  if (n_slots > 0) {
    const int64_t need =
        pkv_decode_workspace_bytes(n_seqs, n_slots, n_heads, n_kv_heads, head_dim);
    if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256)
      return fail(PKV_ERR_CAPACITY, "split-K plan needs %lld 256-byte-aligned workspace "
                  "bytes, got %lld", (long long)need, (long long)workspace_bytes);
    // [arrival counters, n_seqs * n_kv_heads, zero before the first launch and
    //  left zero by every launch][n_slots][Hq][D] partial outputs, then
    //  [n_slots][Hq][2] (m, l)
    cnt = (int32_t*)workspace;
    po = (float*)((char*)workspace + ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256);
    pml = po + (int64_t)n_slots * n_heads * head_dim;
  }
  if ((int64_t)n_work * n_kv_heads > 0x7fffffffLL)
    return fail(PKV_ERR_INVALID, "too many work items");
  fn(q, out, k_pool, v_pool, num_blocks, kv_indices, plan, n_work, n_kv_heads, scale * kLog2e,
     k_new, v_new, slot_mapping, po, pml, cnt, status_word, s);
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}
