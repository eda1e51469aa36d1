// Shared helpers for the gfx950 paged-KV kernels: element types, error
// reporting for the C ABI, and wave-level reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/pagedkv.h"

namespace pkv {

// ---------------------------------------------------------------- errors ---

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define PKV_HIP_TRY(expr)                                                      \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return ::pkv::fail(PKV_ERR_HIP, "%s failed: %s", #expr,                  \
                         hipGetErrorString(e_));                               \
  } while (0)

// Report a launch error (bad configuration, missing code object) right away.
#define PKV_LAUNCH_CHECK()                                                     \
  do {                                                                         \
    hipError_t e_ = hipGetLastError();                                         \
    if (e_ != hipSuccess)                                                      \
      return ::pkv::fail(PKV_ERR_HIP, "kernel launch failed: %s",              \
                         hipGetErrorString(e_));                               \
  } while (0)

inline int elem_bytes(int32_t dtype) {
  switch (dtype) {
    case PKV_DTYPE_F16: return 2;
    case PKV_DTYPE_BF16: return 2;
    case PKV_DTYPE_F32: return 4;
    default: return 0;
  }
}

// ------------------------------------------------------------ type traits ---

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Elem;
template <> struct Elem<_Float16> {
  __device__ static float to_f(_Float16 x) { return (float)x; }
  __device__ static _Float16 from_f(float x) { return (_Float16)x; }
};
template <> struct Elem<__bf16> {
  __device__ static float to_f(__bf16 x) { return (float)x; }
  __device__ static __bf16 from_f(float x) { return (__bf16)x; }
};
template <> struct Elem<float> {
  __device__ static float to_f(float x) { return x; }
  __device__ static float from_f(float x) { return x; }
};

// ------------------------------------------------------- wave reductions ---
// 64-lane wavefront. __shfl_xor lowers to DPP / ds_swizzle / ds_bpermute as
// the pattern allows.

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ void flag(int32_t* status, int32_t bit) {
  if (status) atomicOr(status, bit);
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace pkv
