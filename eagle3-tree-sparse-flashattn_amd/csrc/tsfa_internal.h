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

// Division by a runtime-invariant divisor d >= 1 for dividends 0 <= n < 2^31:
// n / d == (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1 (Granlund and Montgomery, "Division by
// invariant integers using multiplication", 1994, Fig. 4.1; the sum cannot
// wrap because umulhi(n, m) <= n < 2^31).  A kernel's per-wave scalar
// divisions cost ~35 instructions each, on the scalar unit the CU's waves share.
struct FastDiv {
  uint32_t m, s, d;
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{(uint32_t)m, s, d};
}
__host__ __device__ inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (uint32_t)((((uint64_t)n * f.m) >> 32) + n) >> f.s;
}
__host__ __device__ inline uint32_t frem(uint32_t n, const FastDiv& f) { return n - fdiv(n, f) * f.d; }

// ---------------------------------------------------------- host utilities
int device_cu_count(int* out);            // cached per device
int device_max_lds_per_block(int* out);   // cached per device

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace tsfa
