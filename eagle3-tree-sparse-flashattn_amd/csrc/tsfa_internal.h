// Internal declarations shared by the libtsfa HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tsfa.h"
#include "tsfa_plan.h"

namespace tsfa {

// ------------------------------------------------------------------ vectors
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

#define TSFA_LDS __attribute__((address_space(3)))

// Per-dtype MFMA 32x32x16 (fp32 accumulate).  Lane layouts (verified on
// gfx950): A[m][k] lane m + 32*(k/8), element k%8; B[k][n] lane n + 32*(k/8),
// element k%8; C[m][n] lane n + 32*((m/4)%2), element 4*(m/8) + m%4.
template <typename T> struct Mma;
template <> struct Mma<__bf16> {
  typedef bf16x8 vec8;
  __device__ static inline f32x16 run(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  typedef f16x8 vec8;
  __device__ static inline f32x16 run(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// ---------------------------------------------------------- host utilities
int device_cu_count(int* out);            // cached per device
int device_max_lds_per_block(int* out);   // cached per device


}  // namespace tsfa
