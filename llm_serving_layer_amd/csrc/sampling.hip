// Greedy sampling on gfx950: the index of each row's largest logit, the
// scheduler's torch.argmax(logits, dim=-1) (serving/scheduler/scheduler.py:
// 752-757) done on the device, so a decode step hands the host one int64 per
// sequence instead of a row of logits.
//
// One workgroup (16 waves) per row. Threads stride over the row in 16-byte
// chunks, eight chunks in flight (128 KiB per workgroup, what one compute
// unit needs in flight to stream at its share of HBM bandwidth), each
// keeping its best (value, index); the 1024 candidates meet in a wave
// shuffle tree and then across the 16 waves. HBM-bound: a row of V logits
// is read once.
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
constexpr int kArgmaxInFlight = 8;   // 16-byte chunks per thread per round

template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const T* __restrict__ logits,
                                                                int64_t vocab, int64_t stride,
                                                                int64_t* __restrict__ out) {
  constexpr int V = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  constexpr int NT = kArgmaxThreads;
  constexpr int U = kArgmaxInFlight;
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
  int64_t c = tid;
  for (; c + (U - 1) * NT < nchunk; c += U * NT) {
    u32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = *reinterpret_cast<const u32x4*>(x + (c + u * NT) * V);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const T* e = reinterpret_cast<const T*>(&w[u]);
#pragma unroll
      for (int j = 0; j < V; ++j) take(Elem<T>::to_f(e[j]), (int)((c + u * NT) * V + j));
    }
  }
  for (; c < nchunk; c += NT) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(x + c * V);
    const T* e = reinterpret_cast<const T*>(&w);
#pragma unroll
    for (int j = 0; j < V; ++j) take(Elem<T>::to_f(e[j]), (int)(c * V + j));
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
