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

// Compute units of the current device (cached per device); 0 if the query fails.
int device_cu_count();

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
// Two values rounded to bf16 (round to nearest even, each on its own) by one packed conversion.
__device__ __forceinline__ void round_bf16_pair(float& a, float& b) {
  const uint32_t p = pack_bf16x2(a, b);
  a = bf16_lo(p);
  b = bf16_hi(p);
}

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
// Four bf16 values, packed two per word (low half first), times 2^(127 - s) -> four e4m3fn codes in
// one word, by the hardware's scaled conversion: `sc` carries the e8m0 exponent s in a float's
// exponent field (s << 23; s = 0 means 2^-127). For |value x 2^(127 - s)| < 256, the MX range, the
// codes equal cvt_e4m3x4 of the four values multiplied by mx_inv_scale(s) (checked exhaustively on
// MI355X over every bf16 input for s = 0 .. 247).
typedef short i16x2_t __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_e4m3x4_scaled(uint32_t p01, uint32_t p23, float sc) {
  i16x2_t r = {0, 0};
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2_t, p01), sc, false);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2_t, p23), sc, true);
  return __builtin_bit_cast(uint32_t, r);
}

// ------------------------------------------------------------------------------------------------
// Device: buffer descriptors and direct-to-LDS loads
// ------------------------------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// gfx9 buffer resource in four SGPRs: 48-bit base, stride 0, extent in bytes (loads at offsets at
// or past it return zero), raw 32-bit data format.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, bytes, 0x00020000u};
}

// Byte address of a __shared__ object inside the workgroup's LDS allocation.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Direct-to-LDS loads: lane l copies 16 (or 4) bytes from rsrc + voff to LDS address lds + 16 l
// (4 l); `lds` must be wave-uniform. They are issued as inline asm so that the compiler's wait-count
// pass does not see them: it cannot tell which LDS bytes an in-flight DMA writes, and would make
// every later LDS read wait for all outstanding loads (vmcnt(0)), which serializes a multi-stage
// pipeline. The caller therefore waits explicitly (s_waitcnt vmcnt(n) for its own loads, then a
// barrier) before any wave reads the destination.
// The compiler's hazard recognizer does not look inside inline asm, so each block starts with the
// wait states the load may need: an LDS DMA reads M0 and needs one wait state after an SALU write of
// M0 (the compiler writes the "{m0}" operand immediately before the block), and a vector memory
// instruction that reads an SGPR written by a VALU instruction (v_readlane / v_readfirstlane, which
// is how spilled SGPRs such as a resource or soffset are reloaded) needs five. s_nop 4 gives five.
// (With s_nop 0 a spill reload of the soffset right before the load made it read a stale offset.)
__device__ __forceinline__ void lds_dma_b128(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma_b32(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}
// The same with a wave-uniform byte offset `soff` (an SGPR) added to every lane's `voff`, so that
// per-stage and per-row-group offsets cost no VGPRs.
__device__ __forceinline__ void lds_dma_b128(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma_b32(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds) : "memory");
}
// The same 16-byte loads for the hot loops (the GEMM's k loop, the attention's K/V tiles), with only
// the one wait state M0 needs: there the resource and offset SGPRs are written by scalar
// instructions. The build checks that in the generated code (any vector instruction touching one of
// a load's SGPRs within five wait states before it) and, if it finds one, rebuilds the file with
// WANMI_DMA_ALL_WAITS, which gives these loads the full five as well.
#ifdef WANMI_DMA_ALL_WAITS
#define WANMI_DMA_HOT_NOP "s_nop 4\n\t"
#else
#define WANMI_DMA_HOT_NOP "s_nop 0\n\t"
#endif
__device__ __forceinline__ void lds_dma_b128_hot(u32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile(WANMI_DMA_HOT_NOP "buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma_b128_hot(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile(WANMI_DMA_HOT_NOP "buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds) : "memory");
}

// A 16-byte buffer store followed by two wait states. A VALU write of a VGPR that holds the data of
// a store wider than 64 bits must wait until the store has read it; the compiler's hazard check
// has been seen to miss that on gfx950 (a register of the data was overwritten by the very next
// instruction and some lanes stored the new value), so stores that the compiler may follow with a
// write of their data registers go through this: no instruction moves between the store and the
// nops. The build scans the generated code of every kernel for the pattern.
__device__ __forceinline__ void store_b128_guarded(u32x4 v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, 0);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 1" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Lane index recomputed on the spot (volatile, so not merged with earlier copies): code that runs
// after a register-heavy loop derives its lane-dependent addresses from this instead of keeping
// them live (and spilled) across the loop.
__device__ __forceinline__ int fresh_lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// max(x[l], x[l ^ 32]) in every lane l, with v_permlane32_swap (which exchanges one 32-lane half of
// its two operands): passing x as both operands, the two results hold x[l] and x[l ^ 32] in some
// order, so their max is the pair max whichever half the instruction swaps. No LDS, no lane id.
__device__ __forceinline__ int max_with_lane_xor32(int x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return max((int)r[0], (int)r[1]);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14)
constexpr int waitcnt_vm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }
constexpr int waitcnt_lgkm(int n) { return 0xF | (0x7 << 4) | ((n & 0xF) << 8) | (0x3 << 14); }

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
// v with a DPP lane permutation applied (bound_ctrl: lanes without a source read 0; every control
// used here has a source for every lane).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

// x[l] + x[l ^ 16] and x[l] + x[l ^ 32] in every lane, with v_permlane16_swap / v_permlane32_swap
// (each exchanges 16- or 32-lane groups of its two operands; with x as both, the pair of results is
// x[l] and x[l ^ 16] (x[l ^ 32]) in some order, and fp32 addition commutes).
__device__ __forceinline__ float add_lane_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_lane_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Butterfly sum over the 64 lanes in the order xor 1, 2, 4, 8, 16, 32, entirely in the VALU: quad
// permutes for 1 and 2; for 4 and 8 the half-row and row mirrors, which equal the xor partners once
// the quads (8-lane groups) hold one value each, as they do after the steps before; lane swaps for
// 16 and 32. Every lane ends with the same fp32 value.
__device__ __forceinline__ float wave_sum_f32_asc(float v) {
  v = v + dpp_f32<0xB1>(v);   // quad_perm(1,0,3,2): xor 1
  v = v + dpp_f32<0x4E>(v);   // quad_perm(2,3,0,1): xor 2
  v = v + dpp_f32<0x141>(v);  // row_half_mirror: xor 4 on uniform quads
  v = v + dpp_f32<0x140>(v);  // row_mirror: xor 8 on uniform 8-lane groups
  v = add_lane_xor16(v);
  return add_lane_xor32(v);
}
// The same maximum (order-free).
__device__ __forceinline__ float wave_max_f32_asc(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
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
