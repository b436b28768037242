// Fused adaptive LayerNorm + MXFP8 / ROW FP8 quantization for gfx950.
//
// One wavefront owns one row of H elements: lane l holds columns c*512 + 8l .. 8l+7 for chunk
// c < ceil(H/512), so every load and store is a 16-byte (or 8-byte) access and one chunk of a wave
// is a contiguous 1 KiB (512 B for codes) span of the row. The row makes exactly one HBM round trip.
//
// Statistics use a fixed summation order so the CPU oracle reproduces them bit for bit: every lane
// sums its own columns sequentially in fp32 (chunk by chunk, column order within a chunk), then the
// 64 lane sums combine in an xor butterfly (offsets 1, 2, 4, 8, 16, 32, done with DPP and lane swaps
// in the VALU rather than LDS permutes). Two passes:
//
//   LayerNorm: mu = S1 / H with S1 = sum x;  var = S2 / H with S2 = sum fl(fl(x - mu)^2)   (fp32)
//              rstd = fp32(1 / sqrt(fp64(var) + eps))
//   RMSNorm:   ms = S / H with S = sum fl(x^2);  rrms = fp32(1 / sqrt(fp64(ms) + eps))
//   y = bf16( ((x - mu) * rstd) * mul + add )         (fp32, each op rounded, no FMA)
//
// That is ~4 VALU ops per element for the statistics, which keeps the pass memory-bound: at 8 TB/s
// and 3 bytes moved per element there are only ~15 VALU ops per element to spend.
//
// Semantics follow _eager_adaln (vllm_omni_neuron/diffusion/quantization/adaln_kernels.py:51-84):
// gated residual add in fp32 then a bf16 round, normalization in fp32, modulation by fp32 mul/add,
// bf16 output; MX quantization follows _mx_dequant (kernels/nkilib/experimental/norm/
// adaln_quant_torch.py:151-175): shared exponent = block max biased exponent - 7, clamped at 0.
#include "wanmi_common.h"

namespace wanmi {

struct AdalnArgs {
  const uint16_t* hidden;
  const uint16_t* residual;
  const float* gate;
  const float* mul;
  const float* add;
  int64_t T;
  int H;
  int nch;
  float eps;
  int norm;
  int quant;
  void* out;
  uint8_t* scales;
  uint16_t* residual_out;
};

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer descriptor word 3

// A buffer descriptor over `bytes` bytes at `p`; accesses past the end read 0 / are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

__device__ __forceinline__ void load8f(__amdgpu_buffer_rsrc_t r, int lane, int c, float (&v)[8]) {
  const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 32, c * 2048, 0);
  const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 32 + 16, c * 2048, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = __uint_as_float(v0[j]);
    v[4 + j] = __uint_as_float(v1[j]);
  }
}

// Each tensor is addressed through a buffer descriptor based at the current row (scalar registers),
// one per-lane byte offset and the chunk offset in the scalar soffset field, so no per-chunk vector
// address is ever materialized; descriptor extents mask the columns past H in a partial chunk.
//
// kLdsMod (no residual, both modulation vectors given, H a multiple of 512 up to 5120; the block's
// three sites): the workgroup's eight waves (one row each) copy
// the fp32 mul and add vectors into LDS once (direct-to-LDS loads) and read them from there. Read
// per row from L2 instead, the two vectors are 8 bytes per column against the row's 2 (x) + 1
// (codes) -- four times the row's own traffic through the texture unit, the pass's busiest unit.
// The LDS copy holds, per vector, chunk c's first four floats of every lane (lane-major, 16 bytes
// each), then the second four, so that a lane's 16-byte reads of one chunk are consecutive across
// lanes (bank-conflict free). That instantiation also takes the norm type as a template parameter
// (kNorm), and its rows are whole chunks: with the runtime switches the compiler computed every
// variant of the per-value math and selected among them (five v_cndmask per value).
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

template <int NCH, bool kLdsMod = false, int kNorm = -1, int kQuant = -1, bool kRes = false>
__global__ __launch_bounds__(kLdsMod ? 512 : 256, kLdsMod ? 1 : (NCH <= 10 ? 4 : 2)) void adaln_quant_kernel(AdalnArgs a) {
#pragma clang fp contract(off)
  constexpr int kRows = kLdsMod ? 8 : 4;  // rows (waves) per workgroup
  constexpr int kVecs = kRes ? 3 : 2;     // vectors in LDS: mul, add (and the residual gate)
  __shared__ __attribute__((aligned(16))) float smod[kLdsMod ? kVecs * 2 * NCH * 64 * 4 : 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.H;
  const int nch = a.nch;
  const int64_t row = (int64_t)blockIdx.x * kRows + wave;
  const bool live = row < a.T;
  // every wave of the workgroup takes part in the vectors' copy (and its barrier); rows past T
  // load nothing (empty descriptor) and leave after it
  if (!kLdsMod && !live) return;
  const int64_t rbase = live ? row * (int64_t)H : 0;

  const __amdgpu_buffer_rsrc_t r_x = rsrc(a.hidden + rbase, live ? 2 * (int64_t)H : 0);
  uint32_t xp[NCH][4];  // the row's x as packed bf16 pairs (exact; also the residual sum)
  [[maybe_unused]] uint32_t rp[kRes ? NCH : 1][4];  // kRes: the residual row, combined after the barrier

  // ---- load (and optional gated residual add, x = bf16(h * gate + res)) ----
  if (!kLdsMod && a.residual) {
    const __amdgpu_buffer_rsrc_t r_r = rsrc(a.residual + rbase, 2 * (int64_t)H);
    const __amdgpu_buffer_rsrc_t r_ro = rsrc(a.residual_out + rbase, 2 * (int64_t)H);
    const __amdgpu_buffer_rsrc_t r_g = rsrc(a.gate, 4 * (int64_t)H);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c < nch) {
        const u32x4 hv = __builtin_amdgcn_raw_buffer_load_b128(r_x, lane * 16, c * 1024, 0);
        const u32x4 rv = __builtin_amdgcn_raw_buffer_load_b128(r_r, lane * 16, c * 1024, 0);
        float gv[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
        if (a.gate) load8f(r_g, lane, c, gv);
        u32x4 ov;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float h0 = bf16_lo(hv[j]), h1 = bf16_hi(hv[j]);
          if (a.gate) {
            h0 = h0 * gv[2 * j];
            h1 = h1 * gv[2 * j + 1];
          }
          ov[j] = pack_bf16x2(h0 + bf16_lo(rv[j]), h1 + bf16_hi(rv[j]));
          xp[c][j] = ov[j];
        }
        store_b128_guarded(ov, r_ro, lane * 16, c * 1024);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[c][j] = 0u;
      }
    }
  } else {
    [[maybe_unused]] const __amdgpu_buffer_rsrc_t r_r = rsrc(kRes && live ? a.residual + rbase : nullptr,
                                                            kRes && live ? 2 * (int64_t)H : 0);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c < nch) {
        const u32x4 hv = __builtin_amdgcn_raw_buffer_load_b128(r_x, lane * 16, c * 1024, 0);
        if constexpr (kRes) {
          const u32x4 rv = __builtin_amdgcn_raw_buffer_load_b128(r_r, lane * 16, c * 1024, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) rp[c][j] = rv[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[c][j] = hv[j];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[c][j] = 0u;
      }
    }
  }
  // Columns past H were read as zero through the descriptor extent.
  if constexpr (kLdsMod) {
    constexpr int kPerVec = 2 * NCH;  // 1 KiB loads per vector: halves x chunks
    const uint32_t base = lds_addr(smod);
    const u32x4 rm = buffer_rsrc(a.mul, 4u * (uint32_t)H), ra = buffer_rsrc(a.add, 4u * (uint32_t)H);
    // kRes: the gate is the third vector (all ones when absent: its loads read past an empty extent
    // as zero, so it is not used then)
    [[maybe_unused]] const u32x4 rgt = buffer_rsrc(a.gate, a.gate ? 4u * (uint32_t)H : 0u);
    for (int k = wave; k < kVecs * kPerVec; k += kRows) {
      const int kk = k % kPerVec, hh = kk / NCH, c = kk % NCH;
      const u32x4 rv = k < kPerVec ? rm : (k < 2 * kPerVec ? ra : rgt);
      lds_dma_b128(rv, (uint32_t)(c * 512 + 8 * lane + 4 * hh) * 4, base + (uint32_t)k * 1024);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    if (!live) return;
    if constexpr (kRes) {
      // x = bf16(h * gate + res) (the residual branch above, with the gate from LDS), written to
      // residual_out and normalized below
      const __amdgpu_buffer_rsrc_t r_ro = rsrc(a.residual_out + rbase, 2 * (int64_t)H);
      const float4* sm = reinterpret_cast<const float4*>(smod);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        float gv[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
        if (a.gate) {
          const float4 g0 = sm[(4 * NCH + c) * 64 + lane], g1 = sm[(5 * NCH + c) * 64 + lane];
          gv[0] = g0.x, gv[1] = g0.y, gv[2] = g0.z, gv[3] = g0.w, gv[4] = g1.x, gv[5] = g1.y, gv[6] = g1.z, gv[7] = g1.w;
        }
        u32x4 ov;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float h0 = bf16_lo(xp[c][j]), h1 = bf16_hi(xp[c][j]);
          if (a.gate) {
            h0 = h0 * gv[2 * j];
            h1 = h1 * gv[2 * j + 1];
          }
          ov[j] = pack_bf16x2(h0 + bf16_lo(rp[c][j]), h1 + bf16_hi(rp[c][j]));
          xp[c][j] = ov[j];
        }
        store_b128_guarded(ov, r_ro, lane * 16, c * 1024);
      }
    }
  }

  const int norm = kNorm >= 0 ? kNorm : a.norm;
  const bool has_mul = kLdsMod || a.mul != nullptr;
  const bool has_add = kLdsMod || a.add != nullptr;

  // ---- statistics (fixed-order fp32 sums, see the file header) ----
  float mu = 0.0f, rs = 1.0f;
  if (norm == WANMI_NORM_LAYER) {
    float s1 = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s1 = s1 + bf16_lo(xp[c][j]);
        s1 = s1 + bf16_hi(xp[c][j]);
      }
    s1 = wave_sum_f32_asc(s1);
    mu = s1 / (float)H;
    if constexpr (kNorm >= 0) {  // unpack x again below rather than hold all of it as fp32
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(xp[c][j]));
    }
    float s2 = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool ok = kLdsMod || ((c < nch) && (c * 512 + lane * 8 < H));  // (kLdsMod: whole chunks)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d0 = bf16_lo(xp[c][j]) - mu;
        const float d1 = bf16_hi(xp[c][j]) - mu;
        const float q0 = d0 * d0;
        const float q1 = d1 * d1;
        s2 = s2 + (ok ? q0 : 0.0f);
        s2 = s2 + (ok ? q1 : 0.0f);
      }
    }
    s2 = wave_sum_f32_asc(s2);
    const float var = s2 / (float)H;
    rs = (float)(1.0 / sqrt((double)var + (double)a.eps));
  } else if (norm == WANMI_NORM_RMS) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v0 = bf16_lo(xp[c][j]);
        const float v1 = bf16_hi(xp[c][j]);
        const float q0 = v0 * v0;
        const float q1 = v1 * v1;
        s = s + q0;
        s = s + q1;
      }
    s = wave_sum_f32_asc(s);
    const float ms = s / (float)H;
    rs = (float)(1.0 / sqrt((double)ms + (double)a.eps));
  }

  // Keep the per-chunk mul/add loads below the statistics: hoisted above them, all chunks' vectors
  // would be live at once (8 floats x 2 x NCH per lane) and halve occupancy.
  __builtin_amdgcn_sched_barrier(0);
  // mu through an empty asm, so that x - mu is computed again below instead of being kept from the
  // variance pass (the row's 8 NCH differences held in registers spilled)
  asm volatile("" : "+v"(mu));
  if constexpr (kNorm >= 0) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(xp[c][j]));
  }

  // ---- normalize + modulate (+ quantize + store), one chunk at a time ----
  // y = bf16(((x - mu) * rs) * mul + add). NONE and MX finish each chunk here; ROW keeps y in xp
  // for a second pass because its scale needs the whole row's max.
  const __amdgpu_buffer_rsrc_t r_m = rsrc(a.mul, 4 * (int64_t)H);
  const __amdgpu_buffer_rsrc_t r_a = rsrc(a.add, 4 * (int64_t)H);
  const int quant = kQuant >= 0 ? kQuant : a.quant;
  const int64_t out_row_bytes = quant == WANMI_QUANT_NONE ? 2 * (int64_t)H
                                : quant == WANMI_QUANT_MX  ? (int64_t)H
                                                             : (int64_t)H + 4;
  const __amdgpu_buffer_rsrc_t r_o =
      rsrc(reinterpret_cast<const uint8_t*>(a.out) + row * out_row_bytes, out_row_bytes);
  // the row's e8m0 scales (MX): one byte per 32 columns; bytes past H / 32 are dropped
  const __amdgpu_buffer_rsrc_t r_s = rsrc(quant == WANMI_QUANT_MX ? a.scales + row * (int64_t)(H / 32) : nullptr,
                                          quant == WANMI_QUANT_MX ? H / 32 : 0);
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (c < nch) {
      const bool ok = kLdsMod || c * 512 + lane * 8 < H;
      // y as packed bf16 pairs (two values per conversion) and as fp32
      uint32_t yp[4];
      float y[8];
      {
        float mv[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
        float av[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if constexpr (kLdsMod) {
          const float4* sm = reinterpret_cast<const float4*>(smod);
          const float4 m0 = sm[c * 64 + lane], m1 = sm[(NCH + c) * 64 + lane];
          const float4 a0 = sm[(2 * NCH + c) * 64 + lane], a1 = sm[(3 * NCH + c) * 64 + lane];
          mv[0] = m0.x, mv[1] = m0.y, mv[2] = m0.z, mv[3] = m0.w, mv[4] = m1.x, mv[5] = m1.y, mv[6] = m1.z, mv[7] = m1.w;
          av[0] = a0.x, av[1] = a0.y, av[2] = a0.z, av[3] = a0.w, av[4] = a1.x, av[5] = a1.y, av[6] = a1.z, av[7] = a1.w;
        } else {
          if (a.mul) load8f(r_m, lane, c, mv);
          if (a.add) load8f(r_a, lane, c, av);
        }
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float v = (j & 1) ? bf16_hi(xp[c][j >> 1]) : bf16_lo(xp[c][j >> 1]);
          if (norm == WANMI_NORM_LAYER) {
            v = (v - mu) * rs;
          } else if (norm == WANMI_NORM_RMS) {
            v = v * rs;
          }
          if (has_mul) v = v * mv[j];
          if (has_add) v = v + av[j];
          t[j] = v;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          yp[j] = ok ? pack_bf16x2(t[2 * j], t[2 * j + 1]) : 0u;  // columns past H stay zero
          y[2 * j] = bf16_lo(yp[j]);
          y[2 * j + 1] = bf16_hi(yp[j]);
        }
      }
      if (quant == WANMI_QUANT_NONE) {
        u32x4 ov;
#pragma unroll
        for (int j = 0; j < 4; ++j) ov[j] = yp[j];
        store_b128_guarded(ov, r_o, lane * 16, c * 1024);
      } else if (quant == WANMI_QUANT_MX) {
        // a 32-block is 4 consecutive lanes (col / 32 == c * 16 + lane / 4)
        // the largest exponent field is that of the largest |y|: the largest (bits & 0x7fff) of
        // the packed pairs
        u16x2 mag = {0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2, yp[j] & 0x7FFF7FFFu));
        int e = (int)(max(mag[0], mag[1]) >> 7);
        e = max(e, dpp_i32<0xB1>(e));  // quad_perm(1,0,3,2): lane ^ 1
        e = max(e, dpp_i32<0x4E>(e));  // quad_perm(2,3,0,1): lane ^ 2
        const int sexp = max(e - 7, 0);
        const float f = mx_inv_scale(sexp);
        u32x2 cv;
        cv[0] = cvt_e4m3x4(y[0] * f, y[1] * f, y[2] * f, y[3] * f);
        cv[1] = cvt_e4m3x4(y[4] * f, y[5] * f, y[6] * f, y[7] * f);
        __builtin_amdgcn_raw_buffer_store_b64(cv, r_o, lane * 8, c * 512, 0);
        // one byte per 4 lanes; the other lanes' offsets (and those of columns past H) lie past the
        // descriptor's extent and are dropped, so the store needs no branch
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)sexp, r_s, ok && (lane & 3) == 0 ? c * 16 + (lane >> 2) : H, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(y[j]));
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[c][j] = yp[j];
      }
    }
  }

  // ---- ROW: codes = e4m3(y / dq), dq = max(amax / 448, 1e-6), fp32 dq appended ----
  if (quant == WANMI_QUANT_ROW) {
    amax = wave_max_f32_asc(amax);
    const float dq = fmaxf(amax / 448.0f, 1e-6f);
    // The packed row is H + 4 bytes: codes through a descriptor over H bytes, then the scale.
    const __amdgpu_buffer_rsrc_t r_c =
        rsrc(reinterpret_cast<const uint8_t*>(a.out) + row * out_row_bytes, (int64_t)H);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c < nch) {
        float q[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          q[2 * j] = fminf(fmaxf(bf16_lo(xp[c][j]) / dq, -448.0f), 448.0f);
          q[2 * j + 1] = fminf(fmaxf(bf16_hi(xp[c][j]) / dq, -448.0f), 448.0f);
        }
        u32x2 cv;
        cv[0] = cvt_e4m3x4(q[0], q[1], q[2], q[3]);
        cv[1] = cvt_e4m3x4(q[4], q[5], q[6], q[7]);
        __builtin_amdgcn_raw_buffer_store_b64(cv, r_c, lane * 8, c * 512, 0);
      }
    }
    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dq), r_o, H, 0, 0);
  }
}

template <int NCH>
static void launch_adaln(const AdalnArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.T + 3) / 4;
  const int64_t blocks8 = (a.T + 7) / 8;  // the LDS instantiation: eight rows per workgroup
  if constexpr (NCH <= 10) {
    if constexpr (NCH == 10) {
      // the reference's residual sites (gated or not) with both modulation vectors, all three
      // vectors in LDS
      if (a.residual && a.mul && a.add && a.H == NCH * 512) {
        if (a.norm == WANMI_NORM_LAYER)
          hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_LAYER, -1, true>), dim3((unsigned)blocks8),
                             dim3(512), 0, stream, a);
        else if (a.norm == WANMI_NORM_RMS)
          hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_RMS, -1, true>), dim3((unsigned)blocks8),
                             dim3(512), 0, stream, a);
        else
          hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_NONE, -1, true>), dim3((unsigned)blocks8),
                             dim3(512), 0, stream, a);
        return;
      }
    }
    if (!a.residual && a.mul && a.add && a.H == NCH * 512) {
      if (a.norm == WANMI_NORM_LAYER && a.quant == WANMI_QUANT_MX)
        hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_LAYER, WANMI_QUANT_MX>), dim3((unsigned)blocks8),
                           dim3(512), 0, stream, a);
      else if (a.norm == WANMI_NORM_LAYER)
        hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_LAYER>), dim3((unsigned)blocks8), dim3(512), 0, stream, a);
      else if (a.norm == WANMI_NORM_RMS)
        hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_RMS>), dim3((unsigned)blocks8), dim3(512), 0, stream, a);
      else
        hipLaunchKernelGGL((adaln_quant_kernel<NCH, true, WANMI_NORM_NONE>), dim3((unsigned)blocks8), dim3(512), 0, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((adaln_quant_kernel<NCH, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

}  // namespace wanmi

extern "C" int wanmi_adaln_quant(const void* hidden, const void* residual, const float* gate,
                                 const float* mul, const float* add, int64_t T, int64_t H, float eps,
                                 int norm_type, int quant_type, void* out, uint8_t* scales,
                                 void* residual_out, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(T >= 0, WANMI_ERR_ARG, "wanmi_adaln_quant: T=%lld < 0", (long long)T);
  WANMI_REQUIRE(H > 0 && H % 32 == 0, WANMI_ERR_ARG,
                "wanmi_adaln_quant: H=%lld must be a positive multiple of 32", (long long)H);
  WANMI_REQUIRE(H <= 16384, WANMI_ERR_UNSUPPORTED, "wanmi_adaln_quant: H=%lld exceeds 16384",
                (long long)H);
  WANMI_REQUIRE(T < (1LL << 33), WANMI_ERR_ARG, "wanmi_adaln_quant: T=%lld too large", (long long)T);
  WANMI_REQUIRE(norm_type == WANMI_NORM_NONE || norm_type == WANMI_NORM_LAYER ||
                    norm_type == WANMI_NORM_RMS,
                WANMI_ERR_ARG, "wanmi_adaln_quant: unknown norm_type %d", norm_type);
  WANMI_REQUIRE(quant_type == WANMI_QUANT_NONE || quant_type == WANMI_QUANT_MX ||
                    quant_type == WANMI_QUANT_ROW,
                WANMI_ERR_ARG, "wanmi_adaln_quant: unknown quant_type %d", quant_type);
  WANMI_REQUIRE(!(eps < 0.0f), WANMI_ERR_ARG, "wanmi_adaln_quant: eps must be >= 0");
  if (T == 0) return WANMI_OK;
  WANMI_REQUIRE(hidden && out, WANMI_ERR_ARG, "wanmi_adaln_quant: hidden/out must not be null");
  WANMI_REQUIRE(quant_type != WANMI_QUANT_MX || scales, WANMI_ERR_ARG,
                "wanmi_adaln_quant: MX quantization needs a scales buffer");
  WANMI_REQUIRE(!residual || residual_out, WANMI_ERR_ARG,
                "wanmi_adaln_quant: residual given without residual_out");
  WANMI_REQUIRE(((uintptr_t)hidden % 16) == 0 && (!residual || ((uintptr_t)residual % 16) == 0) &&
                    (!residual_out || ((uintptr_t)residual_out % 16) == 0) &&
                    (!mul || ((uintptr_t)mul % 16) == 0) && (!add || ((uintptr_t)add % 16) == 0),
                WANMI_ERR_ARG, "wanmi_adaln_quant: tensors must be 16-byte aligned");
  WANMI_REQUIRE(!gate || ((uintptr_t)gate % 16) == 0, WANMI_ERR_ARG,
                "wanmi_adaln_quant: gate must be 16-byte aligned");
  WANMI_REQUIRE(((uintptr_t)out % 16) == 0, WANMI_ERR_ARG,
                "wanmi_adaln_quant: out must be 16-byte aligned");

  AdalnArgs a;
  a.hidden = static_cast<const uint16_t*>(hidden);
  a.residual = static_cast<const uint16_t*>(residual);
  a.gate = residual ? gate : nullptr;
  a.mul = mul;
  a.add = add;
  a.T = T;
  a.H = (int)H;
  a.nch = (int)((H + 511) / 512);
  a.eps = eps;
  a.norm = norm_type;
  a.quant = quant_type;
  a.out = out;
  a.scales = scales;
  a.residual_out = static_cast<uint16_t*>(residual_out);

  hipStream_t s = (hipStream_t)stream;
  if (a.nch <= 2) launch_adaln<2>(a, s);
  else if (a.nch <= 4) launch_adaln<4>(a, s);
  else if (a.nch <= 8) launch_adaln<8>(a, s);
  else if (a.nch <= 10) launch_adaln<10>(a, s);
  else if (a.nch <= 16) launch_adaln<16>(a, s);
  else if (a.nch <= 24) launch_adaln<24>(a, s);
  else if (a.nch <= 28) launch_adaln<28>(a, s);
  else launch_adaln<32>(a, s);
  return check_launch("wanmi_adaln_quant");
}
