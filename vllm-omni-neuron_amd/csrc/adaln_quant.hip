// Fused adaptive LayerNorm + MXFP8 / ROW FP8 quantization for gfx950.
//
// One wavefront owns one row of H elements: lane l holds columns c*512 + 8l .. 8l+7 for chunk
// c < ceil(H/512), so every load and store is a 16-byte (or 8-byte) access and one chunk of a wave
// is a contiguous 1 KiB (512 B for codes) span of the row. The row makes exactly one HBM round trip.
//
// Statistics are exact: each element is rounded once onto a fixed power-of-two grid chosen from
// the row's largest exponent E, so every partial sum is an integer below 2^53 and fp64 adds it
// without error in any order. The result therefore does not depend on how lanes or waves combine,
// and the CPU oracle reproduces it bit for bit with plain numpy.
//
//   LayerNorm: S1 = sum rint(x * 2^(165-E));          mu  = (S1 * 2^(E-165)) / H       (fp64)
//              S2 = sum rint((x-mu)^2 * 2^(289-2E));  var = (S2 * 2^(2E-289)) / H
//              rstd = 1 / sqrt(var + eps)  (fp64), then mu, rstd rounded to fp32
//   RMSNorm:   S  = sum rint(x^2 * 2^(291-2E));        rrms = 1 / sqrt(S*2^(2E-291)/H + eps)
//   y = bf16( ((x - mu) * rstd) * mul + add )         (fp32, each op rounded, no FMA)
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

// Exponent field of a bf16 held in the low / high half of a packed pair.
__device__ __forceinline__ int bexp_lo(uint32_t u) { return (int)((u >> 7) & 0xFFu); }
__device__ __forceinline__ int bexp_hi(uint32_t u) { return (int)((u >> 23) & 0xFFu); }

template <int NCH>
__global__ __launch_bounds__(256) void adaln_quant_kernel(AdalnArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int H = a.H;
  const int nch = a.nch;
  const int64_t row_stride_waves = (int64_t)gridDim.x * 4;

  for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < a.T; row += row_stride_waves) {
    uint32_t xp[NCH][4];  // the row's x as packed bf16 pairs (exact; also the residual sum)
    const int64_t rbase = row * (int64_t)H;

    // ---- load (and optional gated residual add) ----
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int col = c * 512 + lane * 8;
      const bool ok = (c < nch) && (col < H);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (ok) {
        v = *reinterpret_cast<const uint4*>(a.hidden + rbase + col);
        if (a.residual) {
          const uint4 r = *reinterpret_cast<const uint4*>(a.residual + rbase + col);
          const uint32_t hv[4] = {v.x, v.y, v.z, v.w};
          const uint32_t rv[4] = {r.x, r.y, r.z, r.w};
          float gv[8];
          if (a.gate) {
            const float4 g0 = *reinterpret_cast<const float4*>(a.gate + col);
            const float4 g1 = *reinterpret_cast<const float4*>(a.gate + col + 4);
            gv[0] = g0.x; gv[1] = g0.y; gv[2] = g0.z; gv[3] = g0.w;
            gv[4] = g1.x; gv[5] = g1.y; gv[6] = g1.z; gv[7] = g1.w;
          }
          uint32_t ov[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float h0 = bf16_lo(hv[j]), h1 = bf16_hi(hv[j]);
            if (a.gate) {
              h0 = h0 * gv[2 * j];
              h1 = h1 * gv[2 * j + 1];
            }
            const float s0 = h0 + bf16_lo(rv[j]);
            const float s1 = h1 + bf16_hi(rv[j]);
            ov[j] = pack_bf16x2(s0, s1);
          }
          v = make_uint4(ov[0], ov[1], ov[2], ov[3]);
          *reinterpret_cast<uint4*>(a.residual_out + rbase + col) = v;
        }
      }
      xp[c][0] = v.x;
      xp[c][1] = v.y;
      xp[c][2] = v.z;
      xp[c][3] = v.w;
    }

    // ---- statistics ----
    float mu = 0.0f, rs = 1.0f;
    if (a.norm != WANMI_NORM_NONE) {
      int e = 0;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) e = max(e, max(bexp_lo(xp[c][j]), bexp_hi(xp[c][j])));
      const int E = wave_max_i32(e);
      const double deps = (double)a.eps;
      if (a.norm == WANMI_NORM_LAYER) {
        double s1 = 0.0;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            s1 += rint(ldexp((double)bf16_lo(xp[c][j]), 165 - E));
            s1 += rint(ldexp((double)bf16_hi(xp[c][j]), 165 - E));
          }
        s1 = wave_sum_f64(s1);
        const double mu64 = ldexp(s1, E - 165) / (double)H;
        double s2 = 0.0;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const bool ok = (c < nch) && (c * 512 + lane * 8 < H);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const double d0 = (double)bf16_lo(xp[c][j]) - mu64;
            const double d1 = (double)bf16_hi(xp[c][j]) - mu64;
            const double q0 = rint(ldexp(d0 * d0, 289 - 2 * E));
            const double q1 = rint(ldexp(d1 * d1, 289 - 2 * E));
            s2 += ok ? q0 : 0.0;
            s2 += ok ? q1 : 0.0;
          }
        }
        s2 = wave_sum_f64(s2);
        const double var64 = ldexp(s2, 2 * E - 289) / (double)H;
        const double rstd64 = 1.0 / sqrt(var64 + deps);
        mu = (float)mu64;
        rs = (float)rstd64;
      } else {  // RMS
        double s = 0.0;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const double v0 = (double)bf16_lo(xp[c][j]);
            const double v1 = (double)bf16_hi(xp[c][j]);
            s += rint(ldexp(v0 * v0, 291 - 2 * E));
            s += rint(ldexp(v1 * v1, 291 - 2 * E));
          }
        s = wave_sum_f64(s);
        const double ms64 = ldexp(s, 2 * E - 291) / (double)H;
        rs = (float)(1.0 / sqrt(ms64 + deps));
      }
    }

    // ---- normalize + modulate: y = bf16(((x - mu) * rs) * mul + add), in place in xp ----
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int col = c * 512 + lane * 8;
      const bool ok = (c < nch) && (col < H);
      float mv[8], av[8];
      if (ok && a.mul) {
        const float4 m0 = *reinterpret_cast<const float4*>(a.mul + col);
        const float4 m1 = *reinterpret_cast<const float4*>(a.mul + col + 4);
        mv[0] = m0.x; mv[1] = m0.y; mv[2] = m0.z; mv[3] = m0.w;
        mv[4] = m1.x; mv[5] = m1.y; mv[6] = m1.z; mv[7] = m1.w;
      }
      if (ok && a.add) {
        const float4 b0 = *reinterpret_cast<const float4*>(a.add + col);
        const float4 b1 = *reinterpret_cast<const float4*>(a.add + col + 4);
        av[0] = b0.x; av[1] = b0.y; av[2] = b0.z; av[3] = b0.w;
        av[4] = b1.x; av[5] = b1.y; av[6] = b1.z; av[7] = b1.w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (!ok) {  // columns past H stay zero so row-wide reductions below ignore them
          xp[c][j] = 0u;
          continue;
        }
        float v0 = bf16_lo(xp[c][j]), v1 = bf16_hi(xp[c][j]);
        if (a.norm == WANMI_NORM_LAYER) {
          v0 = (v0 - mu) * rs;
          v1 = (v1 - mu) * rs;
        } else if (a.norm == WANMI_NORM_RMS) {
          v0 = v0 * rs;
          v1 = v1 * rs;
        }
        if (a.mul) {
          v0 = v0 * mv[2 * j];
          v1 = v1 * mv[2 * j + 1];
        }
        if (a.add) {
          v0 = v0 + av[2 * j];
          v1 = v1 + av[2 * j + 1];
        }
        xp[c][j] = pack_bf16x2(v0, v1);
      }
    }

    // ---- quantize + store ----
    if (a.quant == WANMI_QUANT_NONE) {
      uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int col = c * 512 + lane * 8;
        if ((c < nch) && (col < H))
          *reinterpret_cast<uint4*>(out + rbase + col) = make_uint4(xp[c][0], xp[c][1], xp[c][2], xp[c][3]);
      }
    } else if (a.quant == WANMI_QUANT_MX) {
      uint8_t* codes = reinterpret_cast<uint8_t*>(a.out);
      const int64_t sbase = row * (int64_t)(H / 32);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (c >= nch) break;  // uniform across the wave
        const int col = c * 512 + lane * 8;
        int e = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) e = max(e, max(bexp_lo(xp[c][j]), bexp_hi(xp[c][j])));
        e = max(e, __shfl_xor(e, 1, 64));
        e = max(e, __shfl_xor(e, 2, 64));
        const int s = max(e - 7, 0);
        const float f = mx_inv_scale(s);
        const uint32_t lo = cvt_e4m3x4(bf16_lo(xp[c][0]) * f, bf16_hi(xp[c][0]) * f,
                                       bf16_lo(xp[c][1]) * f, bf16_hi(xp[c][1]) * f);
        const uint32_t hi = cvt_e4m3x4(bf16_lo(xp[c][2]) * f, bf16_hi(xp[c][2]) * f,
                                       bf16_lo(xp[c][3]) * f, bf16_hi(xp[c][3]) * f);
        if (col < H) {
          *reinterpret_cast<uint2*>(codes + rbase + col) = make_uint2(lo, hi);
          if ((lane & 3) == 0) a.scales[sbase + col / 32] = (uint8_t)s;
        }
      }
    } else {  // ROW: codes = e4m3(y / dq), dq = max(amax / 448, 1e-6), fp32 dq appended
      float amax = 0.0f;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(xp[c][j])), fabsf(bf16_hi(xp[c][j]))));
      amax = wave_max_f32(amax);
      const float dq = fmaxf(amax / 448.0f, 1e-6f);
      uint8_t* prow = reinterpret_cast<uint8_t*>(a.out) + row * (int64_t)(H + 4);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int col = c * 512 + lane * 8;
        if ((c < nch) && (col < H)) {
          float q[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            q[2 * j] = fminf(fmaxf(bf16_lo(xp[c][j]) / dq, -448.0f), 448.0f);
            q[2 * j + 1] = fminf(fmaxf(bf16_hi(xp[c][j]) / dq, -448.0f), 448.0f);
          }
          uint32_t* dst = reinterpret_cast<uint32_t*>(prow + col);
          dst[0] = cvt_e4m3x4(q[0], q[1], q[2], q[3]);
          dst[1] = cvt_e4m3x4(q[4], q[5], q[6], q[7]);
        }
      }
      if (lane == 0) *reinterpret_cast<float*>(prow + H) = dq;
    }
  }
}

template <int NCH>
static void launch_adaln(const AdalnArgs& a, hipStream_t stream) {
  int64_t blocks = (a.T + 3) / 4;
  if (blocks > 1048576) blocks = 1048576;  // grid-stride loop covers the rest
  hipLaunchKernelGGL(adaln_quant_kernel<NCH>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
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
