// Chunked-prefill attention over a paged prefix on gfx950 matrix cores.
//
// One workgroup (4 waves) owns one KV head h and one tile of a sequence's
// query rows: 128 rows = BQ query tokens x G query heads (BQ = 128 / G), so
// every K/V tile it loads serves all G query heads of the KV head. Each wave
// owns two blocks of 16 rows. Query row r of the tile is token r / G (of the
// tile) and query head h*G + r % G; it sits at absolute position
// kv_len - q_len + token (bottom-right causal alignment, as the reference's
// triu(diagonal = kv_len - q_len + 1) mask) and sees keys 0..position.
//
// The KV axis is walked 64 tokens (4 pages; 32 for head_dim 128) at a time.
// A tile of K and of V (those rows x head_dim of head h) is loaded two tiles
// ahead into registers, staged in one of two padded LDS buffers, and read by
// every wave:
//  * S^T = K Q^T: 16x16x32 MFMA, K rows from LDS as the A operand, Q^T held
//    in registers as the B operand; lane (row n, group g) gets the scores of
//    tokens 4g..4g+3 of each page for its query row n;
//  * online softmax per query row (two cross-lane steps per max / sum);
//  * O += P V: 16x16x32 MFMA over two pages at a time. The probabilities a
//    lane holds for pages 2k and 2k+1 are its A operand as they are (the
//    contraction index runs over those 8 tokens in that order); the V B
//    operand is the matching pair of transposing LDS reads.
// Numerics as serving/backends/paged_torch.py:443-485: scores, softmax and
// accumulation in fp32; probabilities rounded to the pool dtype before PV.
#include "mfma.h"

namespace pkv {

constexpr int kPrefillRows = 128;  // query rows per workgroup (tokens x heads)
// One 16-row block per wave: 8 waves per workgroup at 108 VGPRs keep four
// waves per SIMD, which hides the score/softmax VALU work better than two
// row blocks per wave at half the waves.
constexpr int kPrefillRB = 1;
constexpr int kPrefillThreads = kPrefillRows / 16 / kPrefillRB * 64;

template <typename T, int D, int G>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kpool,
    const T* __restrict__ vpool, int64_t num_blocks, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ plan,
    int32_t n_kv_heads, float scale_log2, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  constexpr int BQ = kPrefillRows / G;   // query tokens per tile
  constexpr int TT = D <= 64 ? 64 : 32;  // KV tokens per tile (LDS stays under 64 KiB)
  constexpr int PS = 16;
  constexpr int NPG = TT / PS;           // pages per KV tile
  constexpr int NCH = D / 32;            // QK k-chunks
  constexpr int NDB = D / 16;            // PV dim blocks
  constexpr int RB = kPrefillRB;         // 16-row blocks per wave
  constexpr int NT = kPrefillThreads;
  constexpr int RSB = D * (int)sizeof(T) + 16;  // padded LDS row bytes
  constexpr int CPR = D * (int)sizeof(T) / 16;  // 16-byte chunks per head row
  constexpr int CPT = TT * CPR / NT;            // chunks per thread per tensor per tile
  static_assert(CPT >= 1 && TT * CPR % NT == 0, "tile must split evenly over the threads");
  // [buffer][K, V][TT rows of RSB bytes]
  extern __shared__ __align__(16) unsigned char lds_raw[];
  auto lds_tile = [&](int buf, int kv) { return lds_raw + (buf * 2 + kv) * TT * RSB; };

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int item = blockIdx.x / n_kv_heads;
  const int h = blockIdx.x - item * n_kv_heads;
  const int seq = plan[4 * item], qs = plan[4 * item + 1], qn = plan[4 * item + 2];
  const int q0 = cu_q[seq];
  const int q_len = cu_q[seq + 1] - q0;
  const int kv_len = kv_lens[seq];
  const int pbase = kv_indptr[seq];
  const int Hq = n_kv_heads * G;
  const int64_t row = (int64_t)n_kv_heads * D;
  const int base_pos = kv_len - q_len + qs;  // position of the tile's first query token
  const int kv_end = base_pos + qn;          // keys [0, kv_end) are visible to some row
  const int ntiles = (kv_end + TT - 1) / TT;

  // Per row block: Q^T (B operand), this lane's query row position.
  vec8 qb[RB][NCH];
  int qpos[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = (wave * RB + rb) * 16 + n;
    const int tok = r / G;
    const bool valid = tok < qn;
    // padding rows see every key so their running max stays finite
    qpos[rb] = valid ? base_pos + tok : kv_len - 1;
    const T* qr = q + ((int64_t)(q0 + qs + (valid ? tok : 0)) * Hq + h * G + r % G) * D + g * 8;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const vec8 t = *reinterpret_cast<const vec8*>(qr + c * 32);
      qb[rb][c] = valid ? t : vec8{};
    }
  }

  auto load_tile = [&](int t, vec8* kr, vec8* vr) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c = tid + NT * k;
      const int tok = t * TT + c / CPR;
      kr[k] = vec8{};
      vr[k] = vec8{};
      if (tok < kv_len) {
        int pid = kv_indices[pbase + tok / PS];
        if (pid < 0 || (int64_t)pid >= num_blocks) {
          flag(status, PKV_STATUS_BAD_PAGE);
          pid = 0;
        }
        const int64_t off = ((int64_t)pid * PS + tok % PS) * row + (int64_t)h * D + (c % CPR) * 8;
        kr[k] = *reinterpret_cast<const vec8*>(kpool + off);
        vr[k] = *reinterpret_cast<const vec8*>(vpool + off);
      }
    }
  };
  // Rows past kv_len were loaded as zeros, so V can never carry stale bits.
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

  f32x4 o[RB][NDB];
  float m_run[RB], l_run[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int b = 0; b < NDB; ++b) o[rb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](int t) {
    const unsigned char* kl = lds_tile(t & 1, 0);
    const unsigned char* vl = lds_tile(t & 1, 1);
    const int t0 = t * TT;
    const bool full = t0 + TT - 1 <= base_pos;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float sc[NPG][4];
      float mx = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < NPG; ++jj) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const unsigned char* kp = kl + (jj * PS + n) * RSB + g * 16;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          acc = Mma<T>::qk(*reinterpret_cast<const vec8*>(kp + c * 64), qb[rb][c], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // keys past the row's position (hence past kv_len) are masked;
          // a tile that ends at or before the first query's position needs none
          const bool live = full || t0 + jj * PS + 4 * g + i <= qpos[rb];
          sc[jj][i] = live ? acc[i] * scale_log2 : -INFINITY;
          mx = fmaxf(mx, sc[jj][i]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // finite: key 0 is visible to every row, and tiles run from key 0 up
      const float m_new = fmaxf(m_run[rb], mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run[rb] - m_new);
      vec8 pk[NPG / 2];
      float ls = 0.f;
#pragma unroll
      for (int jj = 0; jj < NPG; ++jj) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __builtin_amdgcn_exp2f(sc[jj][i] - m_new);
          ls += e;
          pk[jj / 2][(jj & 1) * 4 + i] = (T)e;
        }
      }
      ls += __shfl_xor(ls, 16, 64);
      ls += __shfl_xor(ls, 32, 64);
      l_run[rb] = l_run[rb] * alpha + ls;
      m_run[rb] = m_new;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
        for (int b = 0; b < NDB; ++b) o[rb][b][i] *= a;
      }
#pragma unroll
      for (int kk = 0; kk < NPG / 2; ++kk) {
        const unsigned char* v0 =
            vl + (2 * kk * PS + 4 * g + (n >> 2)) * RSB + 4 * (n & 3) * (int)sizeof(T);
        const unsigned char* v1 = v0 + PS * RSB;
#pragma unroll
        for (int b = 0; b < NDB; ++b) {
          const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4*)(v0 + 16 * b * sizeof(T)));
          const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4*)(v1 + 16 * b * sizeof(T)));
          const vec8 vb = __builtin_bit_cast(
              vec8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          o[rb][b] = Mma<T>::qk(pk[kk], vb, o[rb][b]);
        }
      }
    }
  };

  vec8 kA[CPT], vA[CPT], kB[CPT], vB[CPT];
  load_tile(0, kA, vA);
  if (ntiles > 1) load_tile(1, kB, vB);
  stage(0, kA, vA);
  if (ntiles > 2) load_tile(2, kA, vA);
  __syncthreads();
  for (int t = 0; t < ntiles; t += 2) {  // two register sets, so unrolled by two
    if (t + 1 < ntiles) stage(t + 1, kB, vB);
    if (t + 3 < ntiles) load_tile(t + 3, kB, vB);
    compute(t);
    __syncthreads();
    if (t + 1 < ntiles) {
      if (t + 2 < ntiles) stage(t + 2, kA, vA);
      if (t + 4 < ntiles) load_tile(t + 4, kA, vA);
      compute(t + 1);
      __syncthreads();
    }
  }

  // lane (dim column n, group g) holds rows 4g+i of each block, dims 16b + n.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (wave * RB + rb) * 16 + 4 * g + i;
      const int tok = r / G;
      const float li = __shfl(l_run[rb], 4 * g + i, 64);  // lane 4g+i holds row 4g+i's sum
      if (tok < qn) {
        T* orow = out + ((int64_t)(q0 + qs + tok) * Hq + h * G + r % G) * D + n;
#pragma unroll
        for (int b = 0; b < NDB; ++b) orow[16 * b] = (T)(o[rb][b][i] / li);
      }
    }
  }
}

template <typename T, int D, int G>
static void launch_prefill(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                           const int32_t* cu_q, const int32_t* indptr, const int32_t* indices,
                           const int32_t* kv_lens, const int32_t* plan, int32_t n_tiles,
                           int32_t Hkv, float sl2, int32_t* status, hipStream_t s) {
  constexpr int TT = D <= 64 ? 64 : 32;
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
  if (!fn || !plan || n_tiles <= 0 || q_tile != kPrefillRows / (Hq / Hkv)) return PKV_OK;
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
