// gfx950 matrix-core and LDS helpers shared by the attention kernels.
#pragma once

#include "pkv_common.h"

namespace pkv {

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

// MFMA operand layouts used here (16x16 tiles, 64 lanes, lane l = 16 g + n):
//   16x16x32: A: lane holds A[n][8g .. 8g+7]; B: lane holds B[8g .. 8g+7][n];
//   16x16x16: A: lane holds A[n][4g .. 4g+3]; B: lane holds B[4g .. 4g+3][n];
//   C/D (both): lane holds D[4g + i][n], i = 0..3.
// ds_read_b64_tr_b16: within each 16-lane block, lane i receives element i
// of each of the 4 rows x 16 columns (16-bit) that the block's lanes point
// at (4 consecutive elements each) -- i.e. a transposed 4x16 tile.
// Orders this wave's LDS writes before its own (cross-lane) LDS reads. A
// wave's LDS operations execute in order, so a compiler-level barrier with
// wavefront-scope fences is all that is needed (no s_barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Buffer resource over [base, base + bytes): raw (untyped) records with a
// hardware range check (out-of-range loads read 0, stores are dropped). The
// base lives in scalar registers, so per-lane addresses are 32-bit offsets.
// Cache-policy bits of a buffer load/store: kSc1 = agent-scope coherent
// access (through to the memory-side coherence point), kNt = streaming.
constexpr int kNt = 2;
constexpr int kSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}

}  // namespace pkv
