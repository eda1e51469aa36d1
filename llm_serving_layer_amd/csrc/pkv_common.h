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
// 64-lane wavefront, on the VALU only (no LDS round trips): DPP within rows
// of 16 lanes (quad permutes [1,0,3,2] and [2,3,0,1], then the half-row and
// row mirrors, which pair each lane with one holding the other 4- and
// 8-lane group's total), then the gfx950 row swaps: v_permlane16_swap
// exchanges the odd rows of one operand with the even rows of the other,
// v_permlane32_swap the upper half of one with the lower half of the other,
// so with both operands the same value the two results hold the two rows'
// (halves') values in every lane. Every step combines a lane's value with
// its partner's as a commutative op, so every lane ends with the same bits.

template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl, 0xf, 0xf, false));
}
// {the even row's value, the odd row's value} of each pair of 16-lane rows
__device__ __forceinline__ void rows16(float v, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  a = __builtin_bit_cast(float, (unsigned)r[0]);
  b = __builtin_bit_cast(float, (unsigned)r[1]);
}
// {the lower half's value, the upper half's value}
__device__ __forceinline__ void halves32(float v, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  a = __builtin_bit_cast(float, (unsigned)r[0]);
  b = __builtin_bit_cast(float, (unsigned)r[1]);
}
// sum / max over lanes l, l ^ 16 (the lane's pair of rows)
__device__ __forceinline__ float sum_x16(float v) { float a, b; rows16(v, a, b); return a + b; }
__device__ __forceinline__ float max_x16(float v) { float a, b; rows16(v, a, b); return fmaxf(a, b); }
// sum / max over lanes l, l ^ 32
__device__ __forceinline__ float sum_x32(float v) { float a, b; halves32(v, a, b); return a + b; }
__device__ __forceinline__ float max_x32(float v) { float a, b; halves32(v, a, b); return fmaxf(a, b); }

// lane l's value of v (l uniform), through a scalar register
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp<0x4E>(v));    // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0x141>(v));   // row_half_mirror
  v = fmaxf(v, dpp<0x140>(v));   // row_mirror
  return max_x32(max_x16(v));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return sum_x32(sum_x16(v));
}

__device__ __forceinline__ void flag(int32_t* status, int32_t bit) {
  if (status) atomicOr(status, bit);
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace pkv
