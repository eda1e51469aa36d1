// Chunked-prefill attention over a paged prefix on gfx950 matrix cores.
//
// One workgroup (4 waves) owns one KV head h and one tile of a sequence's
// query rows: 128 rows = BQ query tokens x G query heads (BQ = 128 / G), so
// every K/V tile it loads serves all G query heads of the KV head. Each wave
// owns 32 rows. Query row r of the tile is token r / G (of the tile) and
// query head h*G + r % G; it sits at absolute position kv_len - q_len +
// token (bottom-right causal alignment, as the reference's
// triu(diagonal = kv_len - q_len + 1) mask) and sees keys 0..position.
//
// The KV axis is walked 32 tokens (two pages) at a time. A tile of K and of
// V (those rows x head_dim of head h) goes straight from memory into one of
// four LDS buffers (a ring; direct-to-LDS buffer loads two tiles ahead,
// rows unpadded with their 16-byte chunks swizzled) and is read by every
// wave. All products are 32x32x16 MFMAs, so every LDS byte read feeds 32
// query rows:
//  * S^T = K Q^T: K rows from LDS as the A operand, Q^T held in registers
//    as the B operand. Lane (row n, group g) gets 16 scores of its query row
//    n: keys 8 i + 4 g + 0..3, i = 0..3;
//  * online softmax per query row, lane-local; the two half-waves holding a
//    row meet (v_permlane32_swap) only for a row max and for the final sum;
//  * O^T = V^T P^T: V^T from transposing LDS reads as the A operand, the
//    lane's own 8 probabilities of a 16-key block as the B operand (the
//    contraction index runs over keys 4 g + 0..3, 8 + 4 g + 0..3 of the
//    block). Every O^T accumulator of a lane belongs to its own query row,
//    so rescaling needs no cross-lane traffic.
// The running reference moves lazily: probabilities are taken against it,
// and only when some lane's sum of a tile's probabilities passes 2^12 is
// the row max taken and the accumulators rescaled, so probabilities stay at
// most 2^12 and o / l is unchanged. Tiles wholly below the causal diagonal
// skip the mask. Each wave's share of a tile lies within one page, so page
// ids are scalar reads and pages are buffer ranges: rows past kv_len read
// zeros without a memory access.
// Numerics as serving/backends/paged_torch.py:443-485: scores, softmax and
// accumulation in fp32; probabilities rounded to the pool dtype before PV.
// The scale must be positive (the row max is taken before scaling); other
// scales run the generic kernel.
#include "mfma.h"

namespace pkv {

constexpr int kPrefillRows = 128;   // query rows per workgroup (tokens x heads)
constexpr int kPrefillThreads = 256; // 4 waves x 32 rows

typedef float f32x16 __attribute__((ext_vector_type(16)));
template <typename T> struct Mma32;
template <> struct Mma32<_Float16> {
  __device__ static f32x16 mma(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma32<__bf16> {
  __device__ static f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// LDS of one workgroup: a ring of four K/V tile buffers, each its own
// variable (so the compiler's wait before a tile read covers only the loads
// into that buffer), rows unpadded with 16-byte chunks XOR-swizzled by row.
template <typename T, int D> struct PrefillLds {
  static constexpr int TT = 32;                        // KV tokens per tile
  static constexpr int RB = D * (int)sizeof(T);        // bytes of one head's row
  static constexpr int TILE = TT * RB;                 // one K (or V) tile
  static constexpr int LPT = TILE / (kPrefillThreads * 16);  // 16-byte loads per thread
};

// Row `row` of a tile stores its 16-byte chunk c at chunk position
// c ^ xr(row), xr a permutation of row & 7. Eight consecutive rows reading
// the same chunk (the K operand reads) then hit eight different chunk
// positions, and so do four consecutive rows reading chunks 2j and 2j + 1
// (the transposed V reads): both are free of bank conflicts.
__device__ __forceinline__ int xr(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }
// Byte offset of element `e` (of 2-byte elements) in row `row` of a tile.
template <int RB>
__device__ __forceinline__ int swz(int row, int e) {
  return row * RB + ((((e >> 3) ^ xr(row)) & 7) | ((e >> 3) & ~7)) * 16 + (e & 7) * 2;
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kpool,
    const T* __restrict__ vpool, int64_t num_blocks, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ plan,
    int32_t n_kv_heads, float scale_log2, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  typedef PrefillLds<T, D> L;
  constexpr int TT = L::TT;
  constexpr int PS = 16;
  constexpr int NH = TT / 32;            // 32-key halves per tile
  constexpr int NC = D / 16;             // QK k-chunks of 16 dims
  constexpr int NDH = D / 32;            // PV blocks of 32 dims
  constexpr int RB = L::RB;
  constexpr int CPR = RB / 16;           // 16-byte chunks per row
  constexpr int LPT = L::LPT;
  static_assert(LPT >= 1 && L::TILE == LPT * kPrefillThreads * 16, "whole 1 KiB wave loads");
  static_assert(64 % CPR == 0 && PS % (64 / CPR) == 0, "a wave load stays in one page");
  __shared__ __align__(16) unsigned char buf0[2 * L::TILE];
  __shared__ __align__(16) unsigned char buf1[2 * L::TILE];
  __shared__ __align__(16) unsigned char buf2[2 * L::TILE];
  __shared__ __align__(16) unsigned char buf3[2 * L::TILE];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31, g = lane >> 5;
  const int item = blockIdx.x / n_kv_heads;
  const int h = blockIdx.x - item * n_kv_heads;
  const int seq = plan[4 * item], qs = plan[4 * item + 1], qn = plan[4 * item + 2];
  const int q0 = cu_q[seq];
  const int q_len = cu_q[seq + 1] - q0;
  const int kv_len = kv_lens[seq];
  const int pbase = kv_indptr[seq];
  const int Hq = n_kv_heads * G;
  const int64_t row = (int64_t)n_kv_heads * D;
  const int base_pos = kv_len - q_len + qs;
  const int kv_end = base_pos + qn;
  const int ntiles = (kv_end + TT - 1) / TT;

  // This lane's query row (column n of every 32x32 tile) and Q^T as the B
  // operand of S^T = K Q^T: lane (n, g) holds Q[row][16c + 8g .. + 7].
  const int r = wave * 32 + n;
  const int tok = r / G;
  const bool valid = tok < qn;
  const int qpos = valid ? base_pos + tok : kv_len - 1;
  vec8 qb[NC];
  {
    const T* qr = q + ((int64_t)(q0 + qs + (valid ? tok : 0)) * Hq + h * G + r % G) * D + g * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const vec8 t = *reinterpret_cast<const vec8*>(qr + c * 16);
      qb[c] = valid ? t : vec8{};
    }
  }

  // Tiles past the end and rows at or past kv_len are outside their buffer
  // ranges: nothing is read for them. The ring starts zeroed, so what such
  // rows hold in LDS is finite and only ever meets zero probabilities.
  for (int i = tid; i < 2 * L::TILE / 16; i += kPrefillThreads) {
    reinterpret_cast<u32x4*>(buf0)[i] = u32x4{0u, 0u, 0u, 0u};
    reinterpret_cast<u32x4*>(buf1)[i] = u32x4{0u, 0u, 0u, 0u};
    reinterpret_cast<u32x4*>(buf2)[i] = u32x4{0u, 0u, 0u, 0u};
    reinterpret_cast<u32x4*>(buf3)[i] = u32x4{0u, 0u, 0u, 0u};
  }

  // Load k of a tile covers 64 x 16 bytes = 64 / CPR consecutive rows, all in
  // one page: its page id is wave-uniform, read with a scalar load a tile
  // ahead. (Scalar loads, so the vector-memory count holds tile loads only:
  // a plain vector load may complete before a direct-to-LDS load issued
  // earlier, so the count cannot prove a tile landed if the two mix.)
  const int npages = (kv_len + PS - 1) / PS;
  const uint32_t rowbytes = (uint32_t)(row * sizeof(T));
  // ids at or past this are out of range (kv_indices entries are int32)
  const uint32_t nb32 = num_blocks > 0x7fffffffLL ? 0x80000000u : (uint32_t)num_blocks;
  static_assert(TT % PS == 0, "a tile starts at a page boundary");
  auto page_of = [&](int t, int k) { return (t * TT + ((k * 4 + wave) * 64) / CPR) / PS; };
  auto load_ids = [&](int t, int* ids) {   // this wave's page ids for tile t
#pragma unroll
    for (int k = 0; k < LPT; ++k) {
      const int pg = min(page_of(t, k), npages - 1);
      ids[k] = __builtin_amdgcn_readfirstlane(kv_indices[pbase + pg]);
    }
  };
  auto load_tile = [&](int t, const int* ids, unsigned char* dst) {
#pragma unroll
    for (int k = 0; k < LPT; ++k) {
      const int c0 = (k * 4 + wave) * 64;            // first chunk of this wave load
      const int row0 = c0 / CPR;
      const int pg = page_of(t, k);
      const int raw = ids[k];
      const bool bad = (uint32_t)raw >= nb32;   // (negative ids too)
      if (bad && pg < npages && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);
      const int live_rows = bad ? 0 : min(PS, kv_len - pg * PS);   // <= 0 past the end
      const int64_t pid = bad ? 0 : raw;
      const uint32_t range = live_rows > 0 ? (uint32_t)live_rows * rowbytes : 0u;
      const __amdgpu_buffer_rsrc_t rk =
          ws_rsrc(const_cast<T*>(kpool) + pid * PS * row, range);
      const __amdgpu_buffer_rsrc_t rv =
          ws_rsrc(const_cast<T*>(vpool) + pid * PS * row, range);
      const int rr = row0 + lane / CPR;              // the lane's row of the tile
      const int lc = (((lane % CPR) ^ xr(rr)) & 7) | ((lane % CPR) & ~7);  // its chunk
      // (a tile starts at a page boundary: the row within its page is rr % PS)
      const uint32_t off = (uint32_t)(rr % PS) * rowbytes + (uint32_t)(h * RB + lc * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void*)(dst + c0 * 16), 16, off, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void*)(dst + L::TILE + c0 * 16), 16, off, 0,
          0, 0);
    }
  };

  // O^T accumulators: o[dh][rr] = O[row][32 dh + 8 (rr / 4) + 4 g + rr % 4].
  f32x16 o[NDH];
#pragma unroll
  for (int dh = 0; dh < NDH; ++dh) o[dh] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  // the transposing V reads: lane i of each 16-lane block points at key
  // (i / 4) of a 4-key group and dims 4 (i % 4) .. + 3 of its 16-dim block
  const int vrow = lane & 15;
  const int vcol = (lane & 16) + 4 * (vrow & 3);

  // P^T of the previous tile (the B operand of its PV), kept for the next step.
  vec8 pb[NH * 2];
#pragma unroll
  for (int i = 0; i < NH * 2; ++i) pb[i] = vec8{};
  // O^T += V^T P^T for a tile: V^T as the A operand, lane (dim, g) holding
  // V[key][dim] for keys 16 kb + 4 g + 0..3 and 16 kb + 8 + 4 g + 0..3.
  auto read_v = [&](const unsigned char* vl, vec8* va) {
#pragma unroll
    for (int kb = 0; kb < NH * 2; ++kb) {
      const int key = 16 * kb + 4 * g + (vrow >> 2);
#pragma unroll
      for (int dh = 0; dh < NDH; ++dh) {
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(vl + swz<RB>(key, vcol + 32 * dh)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(vl + swz<RB>(key + 8, vcol + 32 * dh)));
        va[kb * NDH + dh] = __builtin_bit_cast(
            vec8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
  };
  auto pv_mma = [&](const vec8* va) {
#pragma unroll
    for (int kb = 0; kb < NH * 2; ++kb) {
#pragma unroll
      for (int dh = 0; dh < NDH; ++dh) o[dh] = Mma32<T>::mma(va[kb * NDH + dh], pb[kb], o[dh]);
    }
  };
  auto pv = [&](const unsigned char* vl) {
    vec8 va[NH * 2 * NDH];
    read_v(vl, va);
    pv_mma(va);
  };

  // Tile t: S^T = K Q^T, then its softmax beside the previous tile's PV
  // (independent of it), which leaves tile t's probabilities in pb.
  auto compute = [&](int t, const unsigned char* kl, const unsigned char* vprev) {
    const int t0 = t * TT;
    const bool full = t0 + TT - 1 <= base_pos;
    // the previous tile's V operands, read while QK runs
    vec8 va[NH * 2 * NDH];
    read_v(vprev, va);
    // S^T = K Q^T: s[hf][rr] = score of key t0 + 32 hf + 8 (rr / 4) + 4 g + rr % 4.
    f32x16 s[NH];
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      s[hf] = f32x16{};
      const int kr = hf * 32 + n;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        s[hf] = Mma32<T>::mma(*reinterpret_cast<const vec8*>(kl + swz<RB>(kr, 16 * c + 8 * g)),
                              qb[c], s[hf]);
    }
    // Keys past the row's position are masked only on tiles that reach them.
    if (!full) {
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const int key = t0 + 32 * hf + 8 * (rr >> 2) + 4 * g + (rr & 3);
          if (key > qpos) s[hf][rr] = -INFINITY;
        }
      }
    }
    // The previous tile's PV (zero probabilities before the first tile), its
    // matrix instructions interleaved with the softmax's vector ones below.
    pv_mma(va);
    // Probabilities against the running reference m_run: 16-key block
    // (hf, qq) of P^T uses the lane's scores rr = 8 qq .. 8 qq + 7 in that
    // order.
    float ls = 0.f;
    auto probs = [&]() {
      ls = 0.f;
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hf][rr], scale_log2, -m_run));
          ls += e;
          pb[2 * hf + (rr >> 3)][rr & 7] = (T)e;
        }
      }
    };
    probs();
    // (pinned here: otherwise the compiler moves them behind the max test)
#pragma unroll
    for (int i = 0; i < NH * 2; ++i) {
      u32x4 w = __builtin_bit_cast(u32x4, pb[i]);
      asm volatile("" : "+v"(w));
      pb[i] = __builtin_bit_cast(vec8, w);
    }
    asm volatile("" : "+v"(ls));
#pragma unroll
    for (int i = 0; i < NH * 2 * NDH; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // then vector work
    }
    // Lazy rescale: the reference only moves when some lane's sum of its
    // probabilities passes 2^12, which bounds every one of them by 2^12
    // (within the pool dtype's range; NaN or inf counts as past it, as on the
    // first tile, whose reference is -inf); the result o / l does not depend
    // on which reference is used. Only then is the row max taken: it is at
    // least 8 above the reference (a sum past 2^12 over 16 keys has a term
    // past 2^8), so the reference grows, o (with the previous tile's PV
    // added) and l are rescaled and the probabilities taken again.
    if (__builtin_amdgcn_ballot_w64(!(ls <= 4096.f))) {
      // raw-score row max (scale_log2 > 0, so scaling commutes with max)
      float mx = -INFINITY;
#pragma unroll
      for (int hf = 0; hf < NH; ++hf) {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, s[hf][rr]);
      }
      mx = max_x32(mx) * scale_log2;
      const float m_new = fmaxf(m_run, mx);   // finite: key 0 is visible to every row
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int dh = 0; dh < NDH; ++dh) o[dh] *= alpha;
      probs();
    }
    // l_run: this lane's half of its row's keys; the halves meet at the end
    l_run += ls;
  };

  // The ring: tile t in buffer t % 4. Each step waits for its tile's loads
  // (this wave's, then every wave's at the barrier, which also ends every
  // wave's reads of the buffer the step then refills: the one of tile t - 2,
  // whose PV ran in the previous step), loads the pages of tile t + 2,
  // computes tile t beside the PV of tile t - 1, and loads the page ids of
  // tile t + 3.
  int ids0[LPT], ids1[LPT], ids2[LPT], ids3[LPT];   // page ids of tile j in ids(j % 4)
  load_ids(0, ids0);
  load_ids(1, ids1);
  __syncthreads();   // the zeroed ring before any load lands in it
  load_tile(0, ids0, buf0);
  load_ids(2, ids2);
  load_tile(1, ids1, buf1);
  auto step = [&](int t, unsigned char* cur, unsigned char* prev, unsigned char* nxt2,
                  int* ids_t2, int* ids_t3) {
    // Every tile load but the latest step's has landed; after the barrier,
    // every wave's have. (A fenced barrier would wait for all of them.)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LPT) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    load_tile(t + 2, ids_t2, nxt2);
    compute(t, cur, prev + L::TILE);
    // (after the tile's LDS reads: a scalar load in flight would make every
    // wait for them a wait for it too)
    load_ids(t + 3, ids_t3);
  };
  unsigned char* last = buf0;   // the buffer of the last tile computed
  for (int t = 0;; t += 4) {
    step(t, buf0, buf3, buf2, ids2, ids3);
    last = buf0;
    if (t + 1 >= ntiles) break;
    step(t + 1, buf1, buf0, buf3, ids3, ids0);
    last = buf1;
    if (t + 2 >= ntiles) break;
    step(t + 2, buf2, buf1, buf0, ids0, ids1);
    last = buf2;
    if (t + 3 >= ntiles) break;
    step(t + 3, buf3, buf2, buf1, ids1, ids2);
    last = buf3;
    if (t + 4 >= ntiles) break;
  }
  pv(last + L::TILE);   // the last tile's PV
  // the loads of the tiles past the end land in LDS before the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  l_run = sum_x32(l_run);
  if (valid) {
    const float inv = 1.f / l_run;
    T* orow = out + ((int64_t)(q0 + qs + tok) * Hq + h * G + r % G) * D + 4 * g;
#pragma unroll
    for (int dh = 0; dh < NDH; ++dh) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vec4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (T)(o[dh][4 * j + e] * inv);
        *reinterpret_cast<vec4*>(orow + 32 * dh + 8 * j) = v;
      }
    }
  }
}

template <typename T, int D, int G>
static void launch_prefill(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                           const int32_t* cu_q, const int32_t* indptr, const int32_t* indices,
                           const int32_t* kv_lens, const int32_t* plan, int32_t n_tiles,
                           int32_t Hkv, float sl2, int32_t* status, hipStream_t s) {
  hipLaunchKernelGGL((prefill_kernel<T, D, G>), dim3((unsigned)(n_tiles * Hkv)), dim3(kPrefillThreads), 0,
                     s, (const T*)q, (T*)out, (const T*)kp, (const T*)vp, nb, cu_q, indptr,
                     indices, kv_lens, plan, Hkv, sl2, status);
}

typedef void (*PrefillFn)(const void*, void*, const void*, const void*, int64_t, const int32_t*,
                          const int32_t*, const int32_t*, const int32_t*, const int32_t*,
                          int32_t, int32_t, float, int32_t*, hipStream_t);

template <typename T, int D>
static PrefillFn prefill_g(int G) {
  switch (G) {
    case 1: return launch_prefill<T, D, 1>;
    case 2: return launch_prefill<T, D, 2>;
    case 4: return launch_prefill<T, D, 4>;
    case 8: return launch_prefill<T, D, 8>;
    case 16: return launch_prefill<T, D, 16>;
    default: return nullptr;
  }
}

template <typename T>
static PrefillFn prefill_d(int D, int G) {
  switch (D) {
    case 64: return prefill_g<T, 64>(G);
    case 128: return prefill_g<T, 128>(G);
    default: return nullptr;
  }
}

// The MFMA prefill kernel for this geometry, or null (generic kernel).
PrefillFn fast_prefill(int32_t dtype, int32_t Hq, int32_t Hkv, int32_t D, int32_t page_size) {
  if (page_size != 16 || Hkv <= 0 || Hq % Hkv) return nullptr;
  const int G = Hq / Hkv;
  if (dtype == PKV_DTYPE_F16) return prefill_d<_Float16>(D, G);
  if (dtype == PKV_DTYPE_BF16) return prefill_d<__bf16>(D, G);
  return nullptr;
}

}  // namespace pkv

using namespace pkv;

extern "C" int pkv_prefill_q_tile(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                  int32_t page_size, int32_t dtype) {
  if (!fast_prefill(dtype, n_heads, n_kv_heads, head_dim, page_size)) return 0;
  return kPrefillRows / (n_heads / n_kv_heads);
}

namespace pkv {
int run_fast_prefill(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                     const int32_t* cu_q, const int32_t* indptr, const int32_t* indices,
                     const int32_t* kv_lens, int32_t Hq, int32_t Hkv, int32_t D,
                     int32_t page_size, float scale, int32_t dtype, const int32_t* plan,
                     int32_t n_tiles, int32_t q_tile, int32_t* status, hipStream_t s,
                     bool* ran) {
  *ran = false;
  PrefillFn fn = fast_prefill(dtype, Hq, Hkv, D, page_size);
  if (!fn || !plan || n_tiles <= 0 || q_tile != kPrefillRows / (Hq / Hkv) || !(scale > 0.f))
    return PKV_OK;
  if ((int64_t)n_tiles * Hkv > 0x7fffffffLL) return fail(PKV_ERR_INVALID, "too many tiles");
  if (((uintptr_t)q | (uintptr_t)kp | (uintptr_t)vp) % 16)
    return fail(PKV_ERR_INVALID, "q and pools must be 16-byte aligned");
  fn(q, out, kp, vp, nb, cu_q, indptr, indices, kv_lens, plan, n_tiles, Hkv, scale * kLog2e,
     status, s);
  PKV_LAUNCH_CHECK();
  *ran = true;
  return PKV_OK;
}
}  // namespace pkv
