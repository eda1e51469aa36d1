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
// V (those rows x head_dim of head h) is loaded two tiles ahead into
// registers, staged in one of two padded LDS buffers, and read by every
// wave. All products are 32x32x16 MFMAs, so every LDS byte read feeds 32
// query rows:
//  * S^T = K Q^T: K rows from LDS as the A operand, Q^T held in registers
//    as the B operand. Lane (row n, group g) gets 16 scores of its query row
//    n: keys 8 i + 4 g + 0..3, i = 0..3;
//  * online softmax per query row, lane-local but for one cross-lane step
//    per max / sum;
//  * O^T = V^T P^T: V^T from transposing LDS reads as the A operand, the
//    lane's own 8 probabilities of a 16-key block as the B operand (the
//    contraction index runs over keys 4 g + 0..3, 8 + 4 g + 0..3 of the
//    block). Every O^T accumulator of a lane belongs to its own query row,
//    so rescaling needs no cross-lane traffic.
// The running max moves lazily: only when a row's max grows by more than
// 2^8 (in exp2 units) are the accumulators rescaled, so probabilities stay
// at most 256 and o / l is unchanged. Tiles wholly below the causal
// diagonal skip the mask. Each wave's share of a tile lies within one page,
// so page ids are scalar reads and pages are buffer ranges: rows past
// kv_len read zeros without a memory access.
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

template <typename T, int D, int G>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kpool,
    const T* __restrict__ vpool, int64_t num_blocks, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ plan,
    int32_t n_kv_heads, float scale_log2, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  constexpr int TT = 32;                 // KV tokens per tile
  constexpr int PS = 16;
  constexpr int NH = TT / 32;            // 32-key halves per tile
  constexpr int NC = D / 16;             // QK k-chunks of 16 dims
  constexpr int NDH = D / 32;            // PV blocks of 32 dims
  constexpr int NT = kPrefillThreads;
  constexpr int RSB = D * (int)sizeof(T) + 16;
  constexpr int CPR = D * (int)sizeof(T) / 16;
  constexpr int CPT = TT * CPR / NT;
  static_assert(CPT >= 1 && TT * CPR % NT == 0, "tile must split evenly over the threads");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  auto lds_tile = [&](int buf, int kv) { return lds_raw + (buf * 2 + kv) * TT * RSB; };

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
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

  // Each wave's share of a tile lies in one page (its lanes cover 64 x 16
  // bytes of consecutive rows of a page), so the page id is a scalar read
  // and the page a buffer range: rows at or past kv_len and tiles past the
  // end read zeros without touching memory, and every tile issues the same
  // loads (exact wait counts in the pipelined loop).
  const int npages = (kv_len + PS - 1) / PS;
  const uint32_t rowbytes = (uint32_t)(row * sizeof(T));
  auto load_tile = [&](int t, vec8* kr, vec8* vr) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + NT * k;
      const int tk0 = t * TT + __builtin_amdgcn_readfirstlane((wave * 64 + NT * k) / CPR);
      const int pg = tk0 / PS;
      const int live_rows = min(PS, kv_len - pg * PS);   // <= 0 past the end
      const int raw = kv_indices[pbase + min(pg, npages - 1)];
      const bool bad = raw < 0 || (int64_t)raw >= num_blocks;
      if (bad && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);
      const int pid = __builtin_amdgcn_readfirstlane(bad ? 0 : raw);
      const __amdgpu_buffer_rsrc_t rk = ws_rsrc(const_cast<T*>(kpool) + (int64_t)pid * PS * row,
                                                live_rows > 0 ? live_rows * rowbytes : 0);
      const __amdgpu_buffer_rsrc_t rv = ws_rsrc(const_cast<T*>(vpool) + (int64_t)pid * PS * row,
                                                live_rows > 0 ? live_rows * rowbytes : 0);
      const uint32_t off = (uint32_t)(((c / CPR) % PS) * rowbytes + (h * D + (c % CPR) * 8) * sizeof(T));
      kr[k] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
      vr[k] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    }
  };
  auto stage = [&](int t, const vec8* kr, const vec8* vr) {
    unsigned char* kl = lds_tile(t & 1, 0);
    unsigned char* vl = lds_tile(t & 1, 1);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + NT * k;
      const int off = (c / CPR) * RSB + (c % CPR) * 16;
      *reinterpret_cast<vec8*>(kl + off) = kr[k];
      *reinterpret_cast<vec8*>(vl + off) = vr[k];
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

  auto compute = [&](int t) {
    const unsigned char* kl = lds_tile(t & 1, 0);
    const unsigned char* vl = lds_tile(t & 1, 1);
    const int t0 = t * TT;
    const bool full = t0 + TT - 1 <= base_pos;
    // S^T = K Q^T: s[hf][rr] = score of key t0 + 32 hf + 8 (rr / 4) + 4 g + rr % 4.
    f32x16 s[NH];
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      s[hf] = f32x16{};
      const unsigned char* kp = kl + (hf * 32 + n) * RSB + g * 16;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        s[hf] = Mma32<T>::mma(*reinterpret_cast<const vec8*>(kp + c * 32), qb[c], s[hf]);
    }
    // Raw-score row max (scale_log2 > 0, so scaling commutes with max);
    // keys past the row's position are masked only on tiles that reach them.
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
    float mx = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, s[hf][rr]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale_log2;
    // Lazy rescale: the reference max only moves when a row's max grows by
    // more than 2^8 (then p <= 256, exact in the pool dtype's range); the
    // result o / l does not depend on which reference is used.
    if (__builtin_amdgcn_ballot_w64(mx > m_run + 8.f)) {
      const float m_new = fmaxf(m_run, mx);   // finite: key 0 is visible to every row
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int dh = 0; dh < NDH; ++dh) o[dh] *= alpha;
    }
    // P^T as the B operand of O^T = V^T P^T: 16-key block (hf, qq) uses
    // the lane's scores rr = 8 qq .. 8 qq + 7 in that order.
    vec8 pb[NH * 2];
    float ls = 0.f;
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[hf][rr], scale_log2, -m_run));
        ls += e;
        pb[2 * hf + (rr >> 3)][rr & 7] = (T)e;
      }
    }
    ls += __shfl_xor(ls, 32, 64);
    l_run += ls;
#pragma unroll
    for (int kb = 0; kb < NH * 2; ++kb) {
      // V^T as the A operand: lane (dim, g) holds V[key][dim] for keys
      // 16 kb + 4 g + 0..3 and 16 kb + 8 + 4 g + 0..3.
      const unsigned char* vp = vl + (16 * kb + 4 * g + (vrow >> 2)) * RSB + vcol * (int)sizeof(T);
#pragma unroll
      for (int dh = 0; dh < NDH; ++dh) {
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(vp + 32 * dh * sizeof(T)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(vp + 8 * RSB + 32 * dh * sizeof(T)));
        const vec8 va = __builtin_bit_cast(
            vec8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dh] = Mma32<T>::mma(va, pb[kb], o[dh]);
      }
    }
  };

  vec8 kA[CPT], vA[CPT], kB[CPT], vB[CPT];
  load_tile(0, kA, vA);
  load_tile(1, kB, vB);
  stage(0, kA, vA);
  load_tile(2, kA, vA);
  __syncthreads();
  // two register sets, so unrolled by two; re-entered only after the
  // second half, so both halves' loads are in flight there
  for (int t = 0;; t += 2) {
    if (t + 1 < ntiles) stage(t + 1, kB, vB);
    load_tile(t + 3, kB, vB);
    compute(t);
    __syncthreads();
    if (t + 1 >= ntiles) break;
    if (t + 2 < ntiles) stage(t + 2, kA, vA);
    load_tile(t + 4, kA, vA);
    compute(t + 1);
    __syncthreads();
    if (t + 2 >= ntiles) break;
  }

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
  constexpr int TT = 32;
  const size_t lds = 2 * 2 * TT * (D * sizeof(T) + 16);  // two K+V tiles of TT padded rows
  hipLaunchKernelGGL((prefill_kernel<T, D, G>), dim3((unsigned)(n_tiles * Hkv)), dim3(kPrefillThreads), lds,
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
