// Shared device helpers and host-side error plumbing for the gfx950 kernels.
//
// Every exported entry point returns an int status (WANMI_OK or a negative code) and records a
// human-readable message retrievable with wanmi_last_error() on the calling thread.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/wanmi.h"

namespace wanmi {

// ------------------------------------------------------------------------------------------------
// Host: error recording
// ------------------------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

#define WANMI_REQUIRE(cond, code, ...)                                                             \
  do {                                                                                             \
    if (!(cond)) {                                                                                 \
      ::wanmi::set_error(__VA_ARGS__);                                                             \
      return (code);                                                                               \
    }                                                                                              \
  } while (0)

// Checks the launch that was just issued (configuration errors surface synchronously).
int check_launch(const char* what);

// ------------------------------------------------------------------------------------------------
// Device: vector types and bit helpers
// ------------------------------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// bf16 bits (held in the high half of an fp32) -> fp32, exact.
__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// fp32 -> bf16, round to nearest even, via the gfx950 packed converter (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_lo(pack_bf16x2(f, 0.0f)); }

// Biased fp32 exponent field of |f| (0 for zeros and subnormals), the MX block-max input.
__device__ __forceinline__ int exp_field(float f) { return (int)((__float_as_uint(f) >> 23) & 0xFFu); }

// 2^(127 - s) as an fp32 for an e8m0 shared exponent s in [0, 247] (always a normal float).
__device__ __forceinline__ float mx_inv_scale(int s) { return __uint_as_float((uint32_t)(254 - s) << 23); }

// Two fp32 -> two OCP e4m3fn codes (round to nearest even, hardware conversion on gfx950), packed
// into the low 16 bits.
__device__ __forceinline__ uint32_t cvt_e4m3x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}
__device__ __forceinline__ uint32_t cvt_e4m3x4(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

// Wavefront (64-lane) reductions via cross-lane shuffles.
__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Butterfly sum, offsets 32, 16, 8, 4, 2, 1: every lane ends with the same fp32 value (adds commute).
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace wanmi
