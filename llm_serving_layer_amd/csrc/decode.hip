// Paged decode attention for gfx950 (every sequence has one query token).
//
// Work decomposition (planned on the host once per batch): a sequence's
// pages are cut into partitions of at most part_pages pages (split-K over
// the KV axis; the split depends only on that sequence's own length, so its
// result never depends on what it is batched with). A workgroup owns one
// partition and its waves own one KV head each, so they request the same
// pages together (the heads of a token row are adjacent in memory).
//
// A wave walks its partition GP pages at a time with an online softmax, and
// the next GP pages are always in flight while the current ones are used:
// the K registers are refilled as soon as S is computed, the V registers as
// soon as V has been copied to LDS. Per GP pages (G query heads share the KV
// head, G <= 16):
//  1. S^T = K Q^T with one 16x16x32 MFMA per 32 dims of a 16-token page: the
//     K rows ARE the A operand (lane (token m, group g) holds 16 contiguous
//     bytes of row m), Q^T the B operand (column n = query head n, zero
//     beyond G). Lane (head n, group g) then holds the scores of tokens
//     4g..4g+3 of the page for head n;
//  2. softmax in registers: mask past kv_len, running max / sum with one
//     in-lane pass plus two cross-lane steps; p = 2^(s*scale*log2e - m)
//     rounded to the pool dtype -- four values per lane that are exactly the
//     A operand of a 16x16x16 MFMA;
//  3. PV on MFMA: the V pages go to LDS row-major and ds_read_b64_tr_b16
//     hands each lane 4 consecutive tokens of one dim, the B operand, one
//     read per 16 dims. Tokens past kv_len are zeroed so stale bits can
//     never reach the sum.
//
// Split sequences merge in the same launch. Each partition publishes its
// partial (o, m, l) with 16-byte buffer stores carrying the sc1 (agent
// coherence) bit, which write through the per-XCD L2, waits until they have
// completed (s_waitcnt vmcnt(0)), then bumps an arrival counter for its
// (sequence, KV head). The wave that sees the last arrival reads the
// partials back with sc1 loads (never a stale L2 line) and writes the
// output. This avoids a second launch and an agent-scope release fence,
// whose L2 write-back walks the whole cache.
//
// Fused append (optional): when the caller passes the step's new K/V rows,
// the wave that owns a sequence's last page writes the row of its head to
// slot_mapping's slot and patches the copy it loaded, so a decode step costs
// one launch per layer instead of two. The patch is applied only when
// slot_mapping names the same slot as the page table, so the result is
// exactly "append, then attend" (the caller guarantees that no other
// sequence of the launch reads that slot).
#include <algorithm>
#include <vector>

#include "pkv_common.h"

namespace pkv {

// {seq, index of the partition's first page in kv_indices, n_pages, partial
//  slot (-1: the partition is the whole sequence), kv_len, first token,
//  n_partitions of the sequence, first slot of the sequence}
constexpr int kWorkInts = 8;
constexpr int kWaves = 4;         // KV heads (waves) per workgroup, at most
constexpr int kMaxPartPages = 64; // a partition's page ids fit one wave-wide load

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
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

// Buffer resource over the split-K workspace: raw (untyped) 32-bit records,
// hardware range check against `bytes` (out-of-range loads read 0, stores
// are dropped). kSc1 on a load/store = agent-scope coherent access.
constexpr int kSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}

// Layout of one partition's partial output: per (slot, KV head), NGR groups
// of 4 head rows, each NDB dim blocks of 16 lanes x 4 rows (float4 per
// lane) -- exactly the MFMA accumulator layout, so a wave stores and loads
// it with one 16-byte access per lane and dim block.
template <int D, int G> struct PartLayout {
  static constexpr int NGR = (G + 3) / 4;
  static constexpr int NDB = D / 16;
  static constexpr int FLOATS = NGR * NDB * 64;  // per (slot, KV head)
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kWaves * 64) void decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, T* __restrict__ kpool, T* __restrict__ vpool,
    int64_t num_blocks, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ work, int32_t n_kv_heads, float scale_log2,
    const T* __restrict__ k_new, const T* __restrict__ v_new,
    const int32_t* __restrict__ slot_mapping, float* part_o, float* part_ml,
    uint32_t o_bytes, uint32_t ml_bytes, int32_t* counters, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  typedef PartLayout<D, G> PL;
  constexpr int PS = 16;
  constexpr int GP = D <= 64 ? 4 : 2;   // pages per register tile
  constexpr int NCH = D / 32;           // QK MFMA k-chunks per page
  constexpr int NDB = D / 16;           // PV MFMA dim blocks
  constexpr int VL = D / 8;             // lanes per V row when loading (16 bytes each)
  constexpr int VROWS = 64 / VL;        // V rows per load instruction
  constexpr int VLOADS = PS / VROWS;    // load instructions per V page
  constexpr int TILE = GP * PS * D;     // V tile elements per wave
  constexpr int NGR = PL::NGR;

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

  // Lane j holds the partition's j-th page id (npp <= 64).
  int pid = 0;
  if (lane < npp) pid = kv_indices[pbase + lane];
  const bool bad = lane < npp && (pid < 0 || (int64_t)pid >= num_blocks);
  if (bad) pid = 0;
  if (__builtin_amdgcn_ballot_w64(bad) && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);

  // K/V loads go through a buffer resource per page: the page base is
  // wave-uniform (scalar registers) and every lane's offset within a page is
  // the same for all pages, so an address costs one VGPR, not two per load.
  // The resource's range is the page itself; nt: the pages are streamed once.
  const uint32_t page_bytes = (uint32_t)(PS * row * (int64_t)sizeof(T));
  const uint32_t koff = (uint32_t)((n * row + (int64_t)h * D + g * 8) * sizeof(T));
  const uint32_t voff = (uint32_t)((vr_ * row + (int64_t)h * D + vc_ * 8) * sizeof(T));
  const uint32_t vstep = (uint32_t)(VROWS * row * sizeof(T));
  constexpr int kNt = 2;
  vec8 kt[GP][NCH];
  vec8 vt[GP][VLOADS];
  auto load_k = [&](int p0) {
#pragma unroll
    for (int j = 0; j < GP; ++j) {
      if (p0 + j < npp) {
        const int64_t page = __builtin_amdgcn_readlane(pid, p0 + j);
        const __amdgpu_buffer_rsrc_t rk = ws_rsrc(kpool + page * PS * row, page_bytes);
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          kt[j][c] = __builtin_bit_cast(
              vec8, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + c * 32 * sizeof(T), 0, kNt));
      }
    }
  };
  auto load_v = [&](int p0) {
#pragma unroll
    for (int j = 0; j < GP; ++j) {
      if (p0 + j < npp) {
        const int64_t page = __builtin_amdgcn_readlane(pid, p0 + j);
        const __amdgpu_buffer_rsrc_t rv = ws_rsrc(vpool + page * PS * row, page_bytes);
#pragma unroll
        for (int u = 0; u < VLOADS; ++u)
          vt[j][u] = __builtin_bit_cast(
              vec8, __builtin_amdgcn_raw_buffer_load_b128(rv, voff, u * vstep, kNt));
      }
    }
  };
  load_k(0);
  load_v(0);

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

  // Fused append: the wave whose partition holds the newest token writes its
  // head's row now; the loaded copy is patched when its page is used.
  const bool owns_last = k_new != nullptr && tok0 + npp * PS >= kv_len;
  const int tl = (kv_len - 1) % PS;   // newest token's row within its page
  bool patch = false;
  if (owns_last) {
    const int64_t csr_slot = (int64_t)__builtin_amdgcn_readlane(pid, npp - 1) * PS + tl;
    const int64_t new_slot = slot_mapping[seq];
    const bool in_range = new_slot >= 0 && new_slot < num_blocks * PS;
    if (!in_range && lane == 0) flag(status, PKV_STATUS_BAD_SLOT);
    patch = new_slot == csr_slot;
    if (in_range) {
      const T* kn = k_new + ((int64_t)seq * n_kv_heads + h) * D;
      const T* vn = v_new + ((int64_t)seq * n_kv_heads + h) * D;
      if (lane < VL) {
        *reinterpret_cast<vec8*>(kpool + new_slot * row + (int64_t)h * D + lane * 8) =
            *reinterpret_cast<const vec8*>(kn + lane * 8);
        *reinterpret_cast<vec8*>(vpool + new_slot * row + (int64_t)h * D + lane * 8) =
            *reinterpret_cast<const vec8*>(vn + lane * 8);
      }
    }
  }

  const int ng = (npp + GP - 1) / GP;
  f32x4 o[NDB];
#pragma unroll
  for (int b = 0; b < NDB; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // per head n (replicated over g)

  for (int gi = 0; gi < ng; ++gi) {
    const int p0 = gi * GP;
    if (patch && gi == ng - 1) {
      const int jj = npp - 1 - p0;  // the newest page within this tile
      const T* kn = k_new + ((int64_t)seq * n_kv_heads + h) * D;
      const T* vn = v_new + ((int64_t)seq * n_kv_heads + h) * D;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (n == tl) {
          const vec8 x = *reinterpret_cast<const vec8*>(kn + c * 32 + g * 8);
#pragma unroll
          for (int j = 0; j < GP; ++j)  // static indices keep kt in registers
            if (j == jj) kt[j][c] = x;
        }
      }
#pragma unroll
      for (int u = 0; u < VLOADS; ++u) {
        if (u * VROWS + vr_ == tl) {
          const vec8 x = *reinterpret_cast<const vec8*>(vn + vc_ * 8);
#pragma unroll
          for (int j = 0; j < GP; ++j)
            if (j == jj) vt[j][u] = x;
        }
      }
    }

    // S^T per page; lane (n, g) holds tokens 4g..4g+3 of page j for head n.
    float s[GP][4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < GP; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (p0 + j < npp) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) acc = Mma<T>::qk(kt[j][c], qb[c], acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool live = p0 + j < npp && tok0 + (p0 + j) * PS + 4 * g + i < kv_len;
        s[j][i] = live ? acc[i] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[j][i]);
      }
    }
    if (gi + 1 < ng) load_k(p0 + GP);  // K registers are free again
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);  // finite: every tile has a live token
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);

    vec4 p[GP];
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < GP; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(s[j][i] - m_new);
        ls += e;
        p[j][i] = (T)e;
      }
    }
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    l_run = l_run * alpha + ls;
    m_run = m_new;

    // V pages into this wave's LDS tile, row-major [token][dim]; rows past
    // kv_len are zeroed. The previous tile's transposing reads are done.
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < GP; ++j) {
      if (p0 + j < npp) {
#pragma unroll
        for (int u = 0; u < VLOADS; ++u) {
          const int t = u * VROWS + vr_;
          vec8 x = vt[j][u];
          if (tok0 + (p0 + j) * PS + t >= kv_len) x = vec8{};
          *reinterpret_cast<vec8*>(vlds + (j * PS + t) * D + vc_ * 8) = x;
        }
      }
    }
    if (gi + 1 < ng) load_v(p0 + GP);  // V registers are free again

    // Rescale O: lane (n, g) holds head rows 4g+i, whose factor lives in lane 4g+i.
    if (gi > 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
        for (int b = 0; b < NDB; ++b) o[b][i] *= a;
      }
    }
    wave_lds_sync();

    // O (rows = heads, cols = dims) += P V; B operand by transposing reads.
#pragma unroll
    for (int j = 0; j < GP; ++j) {
      if (p0 + j < npp) {
        const T* base = vlds + (j * PS + 4 * g + (n >> 2)) * D + 4 * (n & 3);
#pragma unroll
        for (int b = 0; b < NDB; ++b) {
          const i16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + 16 * b));
          o[b] = Mma<T>::pv(p[j], __builtin_bit_cast(vec4, raw), o[b]);
        }
      }
    }
  }

  // lane (dim column n, group g) holds heads 4g..4g+3 of dims 16b + n.
  if (slot < 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      const float li = __shfl(l_run, r, 64);  // lane r holds head r's sum
      if (r < G) {
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          out[((int64_t)seq * Hq + h * G + r) * D + 16 * b + n] = (T)(o[b][i] / li);
      }
    }
    return;
  }

  // ---- split sequence: publish, count, and the last arrival merges --------
  const __amdgpu_buffer_rsrc_t ro = ws_rsrc(part_o, o_bytes);
  const uint32_t head_off = (uint32_t)(((int64_t)slot * n_kv_heads + h) * PL::FLOATS * 4);
  if (g < NGR) {
#pragma unroll
    for (int b = 0; b < NDB; ++b)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[b]), ro,
                                             head_off + ((g * NDB + b) * 16 + n) * 16, 0, kSc1);
  }
  if (lane < G) {
    const __amdgpu_buffer_rsrc_t rm = ws_rsrc(part_ml, ml_bytes);
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{m_run, l_run}), rm,
                                          (uint32_t)(((int64_t)slot * Hq + h * G + lane) * 8),
                                          0, kSc1);
  }
  // Every partial store of this wave has completed at the coherence point
  // before the arrival is counted.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  int32_t* cnt = counters + (int64_t)seq * n_kv_heads + h;
  int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != nparts - 1) return;

  // Last arrival for (seq, h). Lanes run over partitions for each head
  // row's max M and sum L; then, 64 partitions at a time, the weights
  // 2^(m_s - M) go to this wave's (now free) LDS tile as [partition][16
  // rows], and the partial outputs are read in the producers' own layout:
  // lane (n, g) takes row group rg = g % NGR of every SPLIT-th partition
  // starting at g / NGR, MB partitions per round trip, and the SPLIT lane
  // groups that share a row group are summed by shuffles at the end.
  constexpr int SPLIT = 4 / NGR;
  constexpr int MB = NDB >= 8 ? 2 : 4;
  const int rg = g % NGR, so = g / NGR;
  float* wts = reinterpret_cast<float*>(vlds);  // [64][16]; the tile holds >= 1024 floats
  const __amdgpu_buffer_rsrc_t rm = ws_rsrc(part_ml, ml_bytes);
  auto load_ml = [&](int c0, float* mr, float* lr) {
    const bool ok = c0 + lane < nparts;
    const uint32_t b2 = (uint32_t)(((int64_t)(slot0 + (ok ? c0 + lane : 0)) * Hq + h * G) * 8);
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const f32x2 ml =
          __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, b2 + 8 * r, 0, kSc1));
      mr[r] = ok ? ml[0] : -INFINITY;
      lr[r] = ok ? ml[1] : 0.f;
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
  f32x4 acc[NDB];
#pragma unroll
  for (int b = 0; b < NDB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nparts; c0 += 64) {
    if (nparts > 64) load_ml(c0, mr, lr);  // else still in registers
    f32x4 wv4[4];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float wv = 0.f;
      if (r < G) {
        wv = c0 + lane < nparts ? __builtin_amdgcn_exp2f(mr[r] - M[r]) : 0.f;
        L[r] += wave_sum(wv * lr[r]);
      }
      wv4[r / 4][r % 4] = wv;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) *reinterpret_cast<f32x4*>(wts + lane * 16 + 4 * k) = wv4[k];
    wave_lds_sync();
    const int cn = min(64, nparts - c0);
    for (int s0 = so; s0 < cn; s0 += SPLIT * MB) {
      f32x4 v[MB][NDB];
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        const int sl = s0 + u * SPLIT;
        const uint32_t off = (uint32_t)(((int64_t)(slot0 + c0 + (sl < cn ? sl : 0)) * n_kv_heads + h) *
                                        PL::FLOATS * 4);
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          v[u][b] = sl < cn ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                  ro, off + ((rg * NDB + b) * 16 + n) * 16, 0, kSc1))
                            : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        const int sl = s0 + u * SPLIT;
        if (sl < cn) {
          const f32x4 wr = *reinterpret_cast<const f32x4*>(wts + sl * 16 + 4 * rg);
#pragma unroll
          for (int b = 0; b < NDB; ++b) acc[b] += wr * v[u][b];
        }
      }
    }
    wave_lds_sync();  // the next chunk rewrites the weights
  }
#pragma unroll
  for (int b = 0; b < NDB; ++b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (SPLIT >= 4) acc[b][i] += __shfl_xor(acc[b][i], 16, 64);
      if (SPLIT >= 2) acc[b][i] += __shfl_xor(acc[b][i], 32, 64);
    }
  }
  if (so == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * rg + i;
      float lr_ = L[0];
#pragma unroll
      for (int rr = 1; rr < G; ++rr)  // static indices keep L in registers
        if (r == rr) lr_ = L[rr];
      if (r < G) {
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          out[((int64_t)seq * Hq + h * G + r) * D + 16 * b + n] = (T)(acc[b][i] / lr_);
      }
    }
  }
  if (lane == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static int heads_per_workgroup(int Hkv) {
  for (int c = kWaves; c > 1; --c)
    if (Hkv % c == 0) return c;
  return 1;
}

template <typename T, int D, int G>
static void launch(const void* q, void* out, void* kp, void* vp, int64_t nb,
                   const int32_t* indices, const int32_t* work, int32_t n_work, int32_t Hkv,
                   float sl2, const void* kn, const void* vn, const int32_t* slots, float* po,
                   float* pml, uint32_t o_bytes, uint32_t ml_bytes, int32_t* cnt,
                   int32_t* status, hipStream_t s) {
  constexpr int GP = D <= 64 ? 4 : 2;
  const int hw = heads_per_workgroup(Hkv);
  const size_t lds = (size_t)hw * GP * 16 * D * sizeof(T);
  hipLaunchKernelGGL((decode_kernel<T, D, G>), dim3((unsigned)(n_work * (Hkv / hw))),
                     dim3(hw * 64), lds, s, (const T*)q, (T*)out, (T*)kp, (T*)vp, nb, indices,
                     work, Hkv, sl2, (const T*)kn, (const T*)vn, slots, po, pml, o_bytes,
                     ml_bytes, cnt, status);
}

typedef void (*LaunchFn)(const void*, void*, void*, void*, int64_t, const int32_t*,
                         const int32_t*, int32_t, int32_t, float, const void*, const void*,
                         const int32_t*, float*, float*, uint32_t, uint32_t, int32_t*,
                         int32_t*, hipStream_t);

template <typename T, int D>
static LaunchFn pick_g(int G) {
  switch (G) {
    case 1: return launch<T, D, 1>;
    case 2: return launch<T, D, 2>;
    case 4: return launch<T, D, 4>;
    case 8: return launch<T, D, 8>;
    case 16: return launch<T, D, 16>;
    default: return nullptr;
  }
}

template <typename T>
static LaunchFn pick(int D, int G) {
  switch (D) {
    case 64: return pick_g<T, 64>(G);
    case 128: return pick_g<T, 128>(G);
    default: return nullptr;
  }
}

static LaunchFn fast_decode(int32_t dtype, int32_t D, int32_t G, int32_t page_size, int32_t pp) {
  if (page_size != 16 || pp < 1 || pp > kMaxPartPages) return nullptr;
  if (dtype == PKV_DTYPE_F16) return pick<_Float16>(D, G);
  if (dtype == PKV_DTYPE_BF16) return pick<__bf16>(D, G);
  return nullptr;
}

// Floats of partial output per (slot, KV head): the accumulator tile of
// ceil(G/4) groups of 4 head rows.
static int64_t part_floats(int32_t G, int32_t D) { return (int64_t)((G + 3) / 4) * 4 * D; }

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
  if (n_seqs <= 0 || page_size <= 0 || part_pages <= 0 || part_pages > kMaxPartPages)
    return fail(PKV_ERR_INVALID, "n_seqs and page_size must be positive and part_pages in "
                "[1, %d]", kMaxPartPages);
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
  // Longest partitions first, so the short tail items fill in behind them;
  // among equals, longer sequences first so their merges start early.
  std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) {
    return a.v[2] != b.v[2] ? a.v[2] > b.v[2] : a.v[4] > b.v[4];
  });
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
  if (n_heads % n_kv_heads) return 0;
  const int64_t counters = ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256;
  const int64_t po = (int64_t)n_slots * n_kv_heads * part_floats(n_heads / n_kv_heads, head_dim);
  return counters + (po + (int64_t)n_slots * n_heads * 2) * 4;
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
  uint32_t o_bytes = 0, ml_bytes = 0;
  if (n_slots > 0) {
    const int64_t need =
        pkv_decode_workspace_bytes(n_seqs, n_slots, n_heads, n_kv_heads, head_dim);
    if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256)
      return fail(PKV_ERR_CAPACITY, "split-K plan needs %lld 256-byte-aligned workspace "
                  "bytes, got %lld", (long long)need, (long long)workspace_bytes);
    // [arrival counters, n_seqs * n_kv_heads, zero before the first launch and
    //  left zero by every launch][n_slots][Hkv][part_floats] partial outputs,
    //  then [n_slots][Hq][2] (m, l)
    const int64_t pf = (int64_t)n_slots * n_kv_heads * part_floats(G, head_dim);
    const int64_t mlf = (int64_t)n_slots * n_heads * 2;
    if ((pf + mlf) * 4 > 0x7fffffffLL)
      return fail(PKV_ERR_INVALID, "split-K partials exceed 2 GiB; use larger partitions");
    cnt = (int32_t*)workspace;
    po = (float*)((char*)workspace + ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256);
    pml = po + pf;
    o_bytes = (uint32_t)(pf * 4);
    ml_bytes = (uint32_t)(mlf * 4);
  }
  if ((int64_t)n_work * n_kv_heads > 0x7fffffffLL)
    return fail(PKV_ERR_INVALID, "too many work items");
  fn(q, out, k_pool, v_pool, num_blocks, kv_indices, plan, n_work, n_kv_heads, scale * kLog2e,
     k_new, v_new, slot_mapping, po, pml, o_bytes, ml_bytes, cnt, status_word, s);
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}
