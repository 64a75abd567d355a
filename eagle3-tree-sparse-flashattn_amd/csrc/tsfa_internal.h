// Internal declarations shared by the libtsfa HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tsfa.h"

namespace tsfa {

// ------------------------------------------------------------------ vectors
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

#define TSFA_LDS __attribute__((address_space(3)))

// Per-dtype MFMA 16x16x32 (fp32 accumulate).  Lane layouts (verified on
// gfx950): A[m][k] lane m + 16*(k/8), element k%8; B[k][n] lane n + 16*(k/8),
// element k%8; C[m][n] lane n + 16*(m/4), element m%4.
template <typename T> struct Mma;
template <> struct Mma<__bf16> {
  typedef bf16x8 vec8;
  __device__ static inline f32x4 run(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  typedef f16x8 vec8;
  __device__ static inline f32x4 run(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// ---------------------------------------------------------- host utilities
int device_cu_count(int* out);            // cached per device
int device_max_lds_per_block(int* out);   // cached per device

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace tsfa
