// Greedy sampling on gfx950: the index of each row's largest logit, the
// scheduler's torch.argmax(logits, dim=-1) (serving/scheduler/scheduler.py:
// 752-757) done on the device, so a decode step hands the host one int64 per
// sequence instead of a row of logits.
//
// One workgroup (16 waves) per row. Threads stride over the row in 16-byte
// chunks, sixteen chunks in flight (256 KiB per workgroup: a whole 128 256
// fp16 row in one round trip; eight for bf16), each keeping its best (value,
// index); the 1024 candidates meet in a wave shuffle tree and then across the
// 16 waves. HBM-bound: a row of V logits is read once, so the loads carry the
// streaming hint (nt) and leave the caches to other data.
#include "mfma.h"

namespace pkv {

// The greedy order of torch's argmax: a NaN beats every number (its max
// reductions propagate NaN), a larger value beats a smaller one, and between
// equal values (two NaNs included) the smaller index wins.
__device__ __forceinline__ bool beats(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

constexpr int kArgmaxThreads = 1024;
// 16-byte chunks per thread per round (bf16 widens every element to fp32 for
// the max, and at 16 chunks its registers spill)
template <typename T> constexpr int kArgmaxInFlight = 16;
template <> constexpr int kArgmaxInFlight<__bf16> = 8;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// (Each bit cast of a chunk's word takes the word as a value, (unsigned)w[i]:
// this compiler bit-casts a vector element given as an lvalue from the
// vector's first element.)
//
// Per 16-byte chunk of logits: the largest number as a float (a NaN in the
// chunk is dropped here and found apart) and the chunk's largest magnitude
// bit pattern (M: per 16-bit half, or one 32-bit word), which exceeds kInf
// exactly when the chunk holds a NaN.
template <typename T> struct Chunk;
template <> struct Chunk<_Float16> {
  typedef u16x2 M;
  static constexpr unsigned kInf = 0x7c00u;
  __device__ static float max(const u32x4& w) {
    f16x2 m = __builtin_bit_cast(f16x2, (unsigned)w[0]);
#pragma unroll
    for (int i = 1; i < 4; ++i)
      m = __builtin_elementwise_max(m, __builtin_bit_cast(f16x2, (unsigned)w[i]));
    return fmaxf((float)m[0], (float)m[1]);
  }
  __device__ static u16x2 mag(const u32x4& w) {
    u16x2 m = __builtin_bit_cast(u16x2, w[0] & 0x7fff7fffu);
#pragma unroll
    for (int i = 1; i < 4; ++i)
      m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7fff7fffu));
    return m;
  }
};
template <> struct Chunk<__bf16> {
  typedef u16x2 M;
  static constexpr unsigned kInf = 0x7f80u;
  __device__ static float max(const u32x4& w) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      m = fmaxf(m, fmaxf(__builtin_bit_cast(float, w[i] << 16),
                         __builtin_bit_cast(float, w[i] & 0xffff0000u)));
    return m;
  }
  __device__ static u16x2 mag(const u32x4& w) { return Chunk<_Float16>::mag(w); }
};
template <> struct Chunk<float> {
  typedef unsigned M;
  static constexpr unsigned kInf = 0x7f800000u;
  __device__ static float max(const u32x4& w) {
    return fmaxf(fmaxf(__builtin_bit_cast(float, (unsigned)w[0]),
                       __builtin_bit_cast(float, (unsigned)w[1])),
                 fmaxf(__builtin_bit_cast(float, (unsigned)w[2]),
                       __builtin_bit_cast(float, (unsigned)w[3])));
  }
  __device__ static unsigned mag(const u32x4& w) {
    unsigned m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) m = ::max(m, w[i] & 0x7fffffffu);
    return m;
  }
};

__device__ __forceinline__ u16x2 mag_max(u16x2 a, u16x2 b) { return __builtin_elementwise_max(a, b); }
__device__ __forceinline__ unsigned mag_max(unsigned a, unsigned b) { return ::max(a, b); }

template <typename T>
__device__ __forceinline__ bool holds_nan(typename Chunk<T>::M m) {
  if constexpr (sizeof(T) == 4)
    return m > Chunk<T>::kInf;
  else
    return m[0] > Chunk<T>::kInf || m[1] > Chunk<T>::kInf;
}

// Element j of a 16-byte chunk as a float (a bit cast of the whole chunk,
// not a pointer cast, so the compiler cannot assume the two do not alias).
template <typename T>
__device__ __forceinline__ float elem(const u32x4& w, int j) {
  typedef T TV __attribute__((ext_vector_type(16 / sizeof(T))));
  return Elem<T>::to_f(__builtin_bit_cast(TV, w)[j]);
}

template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const T* __restrict__ logits,
                                                                int64_t vocab, int64_t stride,
                                                                int64_t* __restrict__ out) {
  constexpr int V = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  constexpr int NT = kArgmaxThreads;
  constexpr int U = kArgmaxInFlight<T>;
  const T* x = logits + (int64_t)blockIdx.x * stride;
  // Per thread, over its candidates in increasing index order: the first
  // index of the largest number (a strict > keeps the first of equals) and,
  // apart, the first NaN, which beats every number.
  const bool aligned = ((uintptr_t)x & 15) == 0;
  const int64_t nchunk = aligned ? vocab / V : 0;
  const int tid = threadIdx.x;
  // the thread's first candidate: it holds the best place while every value
  // seen is -inf (equal values keep the first)
  const int64_t first = tid < nchunk ? (int64_t)tid * V : nchunk * V + tid;
  float best = -INFINITY;
  int bi = first < vocab ? (int)first : 0x7fffffff, ni = 0x7fffffff;
  auto take = [&](float v, int i) {
    const bool gt = v > best;
    bi = gt ? i : bi;
    best = gt ? v : best;
    ni = min(ni, v != v ? i : 0x7fffffff);
  };
  // Rounds of U chunks a thread, all in flight at once (a 128 256-entry fp16
  // row is one round). Per chunk only its maximum and its largest magnitude
  // are computed (packed 16-bit max for fp16); the round's best chunk is then
  // searched element by element, and a chunk holding a NaN only when one
  // does.
  for (int64_t c0 = 0; c0 < nchunk; c0 += (int64_t)U * NT) {
    u32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + (int64_t)u * NT + tid;
      w[u] = c < nchunk ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + c * V))
                        : u32x4{0u, 0u, 0u, 0u};
    }
    float rb = -INFINITY;
    int rc = -1;                        // the round's first chunk with the largest number
    typename Chunk<T>::M mg{};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = c0 + (int64_t)u * NT + tid < nchunk;
      const float m = Chunk<T>::max(w[u]);
      const bool gt = in && m > rb;
      rb = gt ? m : rb;
      rc = gt ? u : rc;
      mg = in ? mag_max(mg, Chunk<T>::mag(w[u])) : mg;
    }
    if (rc >= 0 && rb > best) {         // the first element of chunk rc equal to rb
      u32x4 sel = w[0];
#pragma unroll
      for (int u = 1; u < U; ++u) sel = u == rc ? w[u] : sel;
      int j = V - 1;
#pragma unroll
      for (int k = V - 2; k >= 0; --k) j = elem<T>(sel, k) == rb ? k : j;
      best = rb;
      bi = (int)((c0 + (int64_t)rc * NT + tid) * V + j);
    }
    if (ni == 0x7fffffff && holds_nan<T>(mg)) {   // the thread's first NaN
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + (int64_t)u * NT + tid;
        if (ni == 0x7fffffff && c < nchunk) {
#pragma unroll
          for (int k = V - 1; k >= 0; --k) {
            const float v = elem<T>(w[u], k);
            ni = v != v ? (int)(c * V + k) : ni;
          }
        }
      }
    }
  }
  for (int64_t i = nchunk * V + tid; i < vocab; i += NT) take(Elem<T>::to_f(x[i]), (int)i);
  if (ni != 0x7fffffff) {   // a NaN: the first one is the thread's pick
    best = NAN;
    bi = ni;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (beats(ob, oi, best, bi)) { best = ob; bi = oi; }
  }
  __shared__ float wv[NT / 64];
  __shared__ int wi[NT / 64];
  if ((tid & 63) == 0) {
    wv[tid >> 6] = best;
    wi[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < NT / 64; ++w)
      if (beats(wv[w], wi[w], best, bi)) { best = wv[w]; bi = wi[w]; }
    out[blockIdx.x] = bi;
  }
}

}  // namespace pkv

using namespace pkv;

extern "C" int pkv_argmax_rows(const void* logits, int64_t n_rows, int64_t vocab,
                               int64_t row_stride, int32_t dtype, int64_t* out_ids,
                               void* stream) {
  if (n_rows < 0 || n_rows > 0x7fffffffLL)
    return fail(PKV_ERR_INVALID, "n_rows=%lld outside [0, 2^31)", (long long)n_rows);
  if (vocab <= 0 || vocab > 0x7fffffffLL)
    return fail(PKV_ERR_INVALID, "vocab=%lld outside [1, 2^31)", (long long)vocab);
  if (row_stride < vocab)
    return fail(PKV_ERR_INVALID, "row_stride=%lld is shorter than a row of %lld logits",
                (long long)row_stride, (long long)vocab);
  if (n_rows == 0) return PKV_OK;
  if (!logits || !out_ids) return fail(PKV_ERR_INVALID, "logits and out_ids must be non-null");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PKV_DTYPE_F16:
      hipLaunchKernelGGL(argmax_kernel<_Float16>, dim3((unsigned)n_rows), dim3(kArgmaxThreads), 0, s,
                         (const _Float16*)logits, vocab, row_stride, out_ids);
      break;
    case PKV_DTYPE_BF16:
      hipLaunchKernelGGL(argmax_kernel<__bf16>, dim3((unsigned)n_rows), dim3(kArgmaxThreads), 0, s,
                         (const __bf16*)logits, vocab, row_stride, out_ids);
      break;
    case PKV_DTYPE_F32:
      hipLaunchKernelGGL(argmax_kernel<float>, dim3((unsigned)n_rows), dim3(kArgmaxThreads), 0, s,
                         (const float*)logits, vocab, row_stride, out_ids);
      break;
    default:
      return fail(PKV_ERR_INVALID, "dtype=%d is not f16, bf16 or f32", dtype);
  }
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}
