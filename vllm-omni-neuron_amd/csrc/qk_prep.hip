// Q/K preparation for the Wan self/cross attention on gfx950.
//
// wanmi_qk_rmsnorm_rope: in place on a [S, heads*128] bf16 slab (row stride ld), per token:
//   x_hat = bf16(x * rrms * gamma),  rrms = 1 / sqrt(sum(x^2) / (heads*128) + eps)     (across heads)
//   then, if cos/sin are given, RoPE in fp32 on the pairs (a, b) of each head -- interleaved
//   channels (2i, 2i+1), Wan's own order, or the two halves (i, i+64), the rotate-half order of
//   channels de-interleaved per head (row_mx_loaders.py:26-39, row_mx_modules.py:51-76):
//   (a, b) -> bf16(a*cos - b*sin), bf16(a*sin + b*cos)
//   The two give the same bits on correspondingly permuted channels.
// and optionally the per-head maximum over tokens of ||x_out|| (the const-max bound's key norm).
// Reference: DistributedRMSNorm.forward (vllm_omni_neuron/diffusion/models/wan2_2/
// wan2_2_transformer.py:879-893) and apply_rotary_emb_wan (diffusion/layers/rope.py:8-34); the
// fused across-heads variant of the QKV kernel is qkv_cte.py:3781-3990. The key norm follows the
// bound assembly of ring_attention_const_max_fwd.py:296-360, 559-642.
//
// wanmi_transpose_heads: V (element (s, h, d) at v[s*ld + h*head_stride + d]) -> V^T
// [heads, 128, S_pad] with the key
// order inside every group of 16 stored as (0-3, 8-11, 4-7, 12-15), zero for keys >= S. That is
// the order in which the attention kernel's P^T registers hand keys to the PV MFMA, so each lane
// reads its 8 keys with a single 16-byte LDS load.
#include "wanmi_common.h"

namespace wanmi {

constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

struct QKNormArgs {
  uint16_t* x;
  int64_t S, ld;
  int heads, nch, tokens_per_wave;
  const float* gamma;
  const float* cos;  // [S, 64]
  const float* sin;  // [S, 64]
  float eps;
  float* maxnorm;  // [heads] or null (must be zeroed first)
  // optional: the queries' across-heads 1/rms from the QKV GEMM's per-128-column partial sums of
  // squares q_sumsq [S, qss_ld] (blocks 0 .. q_heads-1 in order), written to q_rr [S]
  const float* q_sumsq;
  int64_t qss_ld;
  int q_heads;
  float q_eps;
  float* q_rr;
  // optional (kOut instantiation): the result goes to out instead of back into x, element
  // (token t, head h, d) at out[t*out_ts + h*out_hs + d] (e.g. the head-major [N, S, 128] layout)
  uint16_t* out;
  int64_t out_ts, out_hs;
};


// Up to 40 heads (NCH <= 10) at most 128 VGPRs, four waves per SIMD: the 4095 waves of an S = 32760
// launch (8 tokens each) are then resident in one round over 256 CUs; at the 130 VGPRs the compiler
// would otherwise take, only three waves per SIMD fit and the last quarter of the grid runs as a
// second round (190 vs 159 us). Wider rows keep the registers they need.
// kHalves: rotate-half pairs (i, i+64) (the drop-in path for the reference's de-interleaved
// weights; it keeps the register budget but may spill a little), else interleaved pairs.
// Up to 40 heads the fp32 gamma (8 bytes per column, as much as the token's own bf16 read and write)
// is copied into LDS once per workgroup of 32 tokens instead of being read from L2 per token: per
// chunk, every lane's first four values (16 bytes, lane-major), then the second four.
template <int NCH, bool kHalves, bool kOut = false>
__global__ __launch_bounds__(256, (NCH <= 10 ? 4 : 2)) void qk_rmsnorm_rope_kernel(QKNormArgs a) {
#pragma clang fp contract(off)
  constexpr bool kLdsGamma = NCH <= 10;
  __shared__ __attribute__((aligned(16))) float sgam[kLdsGamma ? 2 * NCH * 64 * 4 : 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = a.heads * 128;
  const int64_t t0 = ((int64_t)blockIdx.x * 4 + wave) * a.tokens_per_wave;
  const __amdgpu_buffer_rsrc_t r_g = make_rsrc(a.gamma, 4 * (int64_t)W);
  if constexpr (kLdsGamma) {
    const u32x4 rg = buffer_rsrc(a.gamma, 4u * (uint32_t)W);  // columns past W read as zero
    const uint32_t base = lds_addr(sgam);
    for (int k = wave; k < 2 * NCH; k += 4) {
      const int hh = k / NCH, c = k % NCH;
      lds_dma_b128(rg, (uint32_t)(c * 512 + 8 * lane + 4 * hh) * 4, base + (uint32_t)k * 1024);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
  }
  float kmx[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) kmx[c] = 0.0f;

  if (a.q_rr != nullptr) {
    // lane i < tokens_per_wave: the Q 1/rms of token t0 + i, its partial sums added in block order
    // and the root taken in fp64 -- the operations, in the order, the attention's Q load performs on
    // the same partials (so the attention may read this instead, bit for bit)
    const int64_t tq = t0 + lane;
    const bool ok = lane < a.tokens_per_wave && tq < a.S;
    float qs = 0.0f;
    if (a.q_heads <= 40 && (a.qss_ld & 3) == 0) {
      // all ten 16-byte loads of the row in flight at once (a loop of dependent loads would wait a
      // memory round trip per partial before the wave's first token), through a descriptor over
      // the wave's rows whose last row ends at q_heads rounded up to 4 (within the row, as qss_ld
      // is a multiple of 4): lanes past the last token read zeros, and only the first q_heads
      // values are added
      const int64_t rows = min((int64_t)a.tokens_per_wave, a.S - t0);
      const int64_t qh4 = (a.q_heads + 3) & ~3;
      const __amdgpu_buffer_rsrc_t r_q =
          make_rsrc(a.q_sumsq + (rows > 0 ? t0 * a.qss_ld : 0), rows > 0 ? ((rows - 1) * a.qss_ld + qh4) * 4 : 0);
      u32x4 pv[10];
#pragma unroll
      for (int i = 0; i < 10; ++i)
        pv[i] = __builtin_amdgcn_raw_buffer_load_b128(r_q, (uint32_t)((lane * a.qss_ld + 4 * i) * 4), 0, 0);
#pragma unroll
      for (int i = 0; i < 10; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (4 * i + j < a.q_heads) qs = qs + __uint_as_float(pv[i][j]);
    } else if (ok) {
      const float* pq = a.q_sumsq + tq * a.qss_ld;
      for (int b = 0; b < a.q_heads; ++b) qs = qs + pq[b];
    }
    if (ok) a.q_rr[tq] = (float)(1.0 / sqrt((double)(qs / (float)(a.q_heads * 128)) + (double)a.q_eps));
  }

  for (int it = 0; it < a.tokens_per_wave; ++it) {
    const int64_t t = t0 + it;
    if (t >= a.S) break;  // wave-uniform
    const __amdgpu_buffer_rsrc_t r_x = make_rsrc(a.x + t * a.ld, 2 * (int64_t)W);
    uint32_t xp[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c < a.nch) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r_x, lane * 16, c * 1024, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[c][j] = v[j];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[c][j] = 0u;
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v0 = bf16_lo(xp[c][j]), v1 = bf16_hi(xp[c][j]);
        const float q0 = v0 * v0, q1 = v1 * v1;
        ss = ss + q0;
        ss = ss + q1;
      }
    ss = wave_sum_f32_asc(ss);
    const float rs = (float)(1.0 / sqrt((double)(ss / (float)W) + (double)a.eps));

    // interleaved: the lane's 4 pairs are the angles 4 (lane & 15) .. +3 of its head; halves: its 8
    // channels 8 (lane & 15) .. +7 are first-half (lane & 8 == 0) or second-half channels whose angles
    // are 8 (lane & 7) .. +7, paired with the same channels of lane ^ 8
    constexpr int kAngles = kHalves ? 8 : 4;
    float cs[kAngles], sn[kAngles];
    if (a.cos) {
      const __amdgpu_buffer_rsrc_t r_c = make_rsrc(a.cos + t * 64, 256);
      const __amdgpu_buffer_rsrc_t r_s = make_rsrc(a.sin + t * 64, 256);
      const uint32_t off = kHalves ? (uint32_t)(lane & 7) * 32 : (uint32_t)(lane & 15) * 16;
#pragma unroll
      for (int u = 0; u < kAngles / 4; ++u) {
        const u32x4 cv = __builtin_amdgcn_raw_buffer_load_b128(r_c, off + 16 * u, 0, 0);
        const u32x4 sv = __builtin_amdgcn_raw_buffer_load_b128(r_s, off + 16 * u, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          cs[4 * u + j] = __uint_as_float(cv[j]);
          sn[4 * u + j] = __uint_as_float(sv[j]);
        }
      }
    }
    const bool second_half = (lane & 8) != 0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c < a.nch) {
        u32x4 g0, g1;
        if constexpr (kLdsGamma) {
          g0 = reinterpret_cast<const u32x4*>(sgam)[c * 64 + lane];
          g1 = reinterpret_cast<const u32x4*>(sgam)[(NCH + c) * 64 + lane];
        } else {
          g0 = __builtin_amdgcn_raw_buffer_load_b128(r_g, lane * 32, c * 2048, 0);
          g1 = __builtin_amdgcn_raw_buffer_load_b128(r_g, lane * 32 + 16, c * 2048, 0);
        }
        const float gv[8] = {__uint_as_float(g0[0]), __uint_as_float(g0[1]), __uint_as_float(g0[2]),
                             __uint_as_float(g0[3]), __uint_as_float(g1[0]), __uint_as_float(g1[1]),
                             __uint_as_float(g1[2]), __uint_as_float(g1[3])};
        u32x4 ov;
        float n2 = 0.0f;
        // normalized + gamma, rounded to bf16 (the reference rounds after the norm)
        if constexpr (!kHalves) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float a0 = (bf16_lo(xp[c][j]) * rs) * gv[2 * j];
            float b0 = (bf16_hi(xp[c][j]) * rs) * gv[2 * j + 1];
            round_bf16_pair(a0, b0);
            if (a.cos) {
              const float ac = a0 * cs[j], bs = b0 * sn[j], as = a0 * sn[j], bc = b0 * cs[j];
              const float r0 = ac - bs, r1 = as + bc;
              a0 = r0;
              b0 = r1;
            }
            ov[j] = pack_bf16x2(a0, b0);
            const float fa = bf16_lo(ov[j]), fb = bf16_hi(ov[j]);
            n2 = n2 + fa * fa;
            n2 = n2 + fb * fb;
          }
        } else {
          float y[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            y[2 * j] = (bf16_lo(xp[c][j]) * rs) * gv[2 * j];
            y[2 * j + 1] = (bf16_hi(xp[c][j]) * rs) * gv[2 * j + 1];
            round_bf16_pair(y[2 * j], y[2 * j + 1]);
          }
          if (a.cos) {
            // pairs (i, i+64): first half x cos - x' sin, second half x cos + x' sin (x' = the
            // partner channel, held by lane ^ 8)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float o = __shfl_xor(y[k], 8, 64);
              const float xc = y[k] * cs[k], os = o * sn[k];
              y[k] = second_half ? xc + os : xc - os;
            }
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            ov[j] = pack_bf16x2(y[2 * j], y[2 * j + 1]);
            const float fa = bf16_lo(ov[j]), fb = bf16_hi(ov[j]);
            n2 = n2 + fa * fa;
            n2 = n2 + fb * fb;
          }
        }
        if constexpr (kOut) {
          // head c * 4 + (lane >> 4) of the chunk: 16 lanes write its 256 bytes, through a descriptor
          // based at the token (the host keeps every offset below 2^31)
          const __amdgpu_buffer_rsrc_t r_o = make_rsrc(a.out + t * a.out_ts, ((a.heads - 1) * a.out_hs + 128) * 2);
          store_b128_guarded(ov, r_o, (int)(((lane >> 4) * a.out_hs + (lane & 15) * 8) * 2), (int)(c * 8 * a.out_hs));
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(ov, r_x, lane * 16, c * 1024, 0);
        }
        if (a.maxnorm) {
          // one head = 16 consecutive lanes of a chunk (one DPP row): sum over the row with DPP
          // moves (quad xor 1, quad xor 2, half-row mirror, row mirror -- the pairs of an xor 1, 2,
          // 4, 8 butterfly, no LDS round trips); the max is kept on ||k||^2 and square-rooted once
          // at the end (sqrt is monotone and correctly rounded, so max(sqrt) = sqrt(max))
          n2 = n2 + dpp_f32<0xB1>(n2);   // quad_perm(1,0,3,2)
          n2 = n2 + dpp_f32<0x4E>(n2);   // quad_perm(2,3,0,1)
          n2 = n2 + dpp_f32<0x141>(n2);  // row_half_mirror
          n2 = n2 + dpp_f32<0x140>(n2);  // row_mirror
          kmx[c] = fmaxf(kmx[c], n2);
        }
      }
    }
  }
  if (a.maxnorm) {
    // Workgroup maximum first (through LDS), then one atomic per head per workgroup: every wave of
    // the grid finishes at about the same time, and per-wave atomics on the same few cache lines
    // serialize at the L2 (measured: 180 us of a 340 us launch).
    __shared__ float smax[4][NCH * 4];
    if ((lane & 15) == 0) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) smax[wave][c * 4 + (lane >> 4)] = kmx[c];
    }
    __syncthreads();
    const int hd = threadIdx.x;
    if (hd < a.heads) {
      const float m = fmaxf(fmaxf(smax[0][hd], smax[1][hd]), fmaxf(smax[2][hd], smax[3][hd]));
      // non-negative floats order like their bit patterns
      atomicMax(reinterpret_cast<unsigned int*>(a.maxnorm) + hd, __float_as_uint(sqrtf(m)));
    }
  }
}

__global__ void zero_f32_kernel(float* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

struct TransposeArgs {
  const uint16_t* v;  // element (s, h, d) at v[s*ld + h*hs + d]
  int64_t S, ld, hs;
  int heads;
  uint16_t* vt;
  int64_t S_pad;
};

// Block: one head, 64 keys. LDS tile [64 keys][128 d] padded to 130 bf16 per row so the column
// reads of the transpose hit distinct banks.
__global__ __launch_bounds__(256) void transpose_heads_kernel(TransposeArgs a) {
  __shared__ uint16_t tile[64][130];
  const int h = blockIdx.y;
  const int64_t s0 = (int64_t)blockIdx.x * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;  // 64 keys x 16 chunks of 8 d
    const int key = idx >> 4, ch = idx & 15;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (s0 + key < a.S) v = *reinterpret_cast<const uint4*>(a.v + (s0 + key) * a.ld + h * a.hs + ch * 8);
    uint32_t* dst = reinterpret_cast<uint32_t*>(&tile[key][ch * 8]);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
  }
  __syncthreads();
  // storage slot s of a 16-key group holds key kOrder[s]
  const int kOrder[16] = {0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;  // 128 d x 8 chunks of 8 slots
    const int d = idx >> 3, ch = idx & 7;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s_lo = ch * 8 + 2 * j, s_hi = s_lo + 1;
      const int k_lo = (s_lo & ~15) + kOrder[s_lo & 15];
      const int k_hi = (s_hi & ~15) + kOrder[s_hi & 15];
      w[j] = (uint32_t)tile[k_lo][d] | ((uint32_t)tile[k_hi][d] << 16);
    }
    if (s0 + ch * 8 < a.S_pad)
      *reinterpret_cast<uint4*>(a.vt + ((int64_t)h * 128 + d) * a.S_pad + s0 + ch * 8) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace wanmi

namespace wanmi {
static int qk_rmsnorm_rope_impl(void* x, int64_t S, int64_t ld, int heads, const float* gamma, const float* cos_tab,
                                const float* sin_tab, int rope_pairs, float eps, float* maxnorm, const float* q_sumsq,
                                int64_t q_sumsq_ld, int q_heads, float q_eps, float* q_rr, void* stream,
                                void* out = nullptr, int64_t out_ts = 0, int64_t out_hs = 0) {
  WANMI_REQUIRE(S >= 0 && heads > 0 && heads % 4 == 0 && heads <= 128, WANMI_ERR_ARG,
                "wanmi_qk_rmsnorm_rope: need S >= 0 and heads a positive multiple of 4 (<= 128), got S=%lld heads=%d",
                (long long)S, heads);
  WANMI_REQUIRE(ld >= heads * 128 && ld % 8 == 0, WANMI_ERR_ARG, "wanmi_qk_rmsnorm_rope: bad ld=%lld", (long long)ld);
  WANMI_REQUIRE((cos_tab == nullptr) == (sin_tab == nullptr), WANMI_ERR_ARG,
                "wanmi_qk_rmsnorm_rope: cos and sin must both be given or both be null");
  WANMI_REQUIRE(!(eps < 0.0f), WANMI_ERR_ARG, "wanmi_qk_rmsnorm_rope: eps must be >= 0");
  WANMI_REQUIRE(rope_pairs == WANMI_ROTATE_INTERLEAVED || rope_pairs == WANMI_ROTATE_HALVES, WANMI_ERR_ARG,
                "wanmi_qk_rmsnorm_rope: unknown rope_pairs %d", rope_pairs);
  hipStream_t s = (hipStream_t)stream;
  if (maxnorm) {
    hipLaunchKernelGGL(zero_f32_kernel, dim3((heads + 255) / 256), dim3(256), 0, s, maxnorm, heads);
    int st = check_launch("wanmi_qk_rmsnorm_rope(zero)");
    if (st) return st;
  }
  if (S == 0) return WANMI_OK;
  WANMI_REQUIRE(x && gamma, WANMI_ERR_ARG, "wanmi_qk_rmsnorm_rope: x and gamma must not be null");
  WANMI_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)gamma % 16) == 0 &&
                    (!cos_tab || (((uintptr_t)cos_tab % 16) == 0 && ((uintptr_t)sin_tab % 16) == 0)),
                WANMI_ERR_ARG, "wanmi_qk_rmsnorm_rope: tensors must be 16-byte aligned");
  QKNormArgs a;
  a.x = static_cast<uint16_t*>(x);
  a.S = S;
  a.ld = ld;
  a.heads = heads;
  a.nch = heads / 4;
  a.tokens_per_wave = 8;
  a.gamma = gamma;
  a.cos = cos_tab;
  a.sin = sin_tab;
  a.eps = eps;
  a.maxnorm = maxnorm;
  a.q_sumsq = q_sumsq;
  a.qss_ld = q_sumsq_ld;
  a.q_heads = q_heads;
  a.q_eps = q_eps;
  a.q_rr = q_rr;
  a.out = static_cast<uint16_t*>(out);
  a.out_ts = out_ts;
  a.out_hs = out_hs;
  const int64_t waves = (S + a.tokens_per_wave - 1) / a.tokens_per_wave;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (out) {
    WANMI_REQUIRE(a.nch <= 10, WANMI_ERR_UNSUPPORTED, "wanmi_qk_rmsnorm_rope_to: at most 40 heads");
    if (rope_pairs == WANMI_ROTATE_HALVES) {
      if (a.nch <= 4) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<4, true, true>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<10, true, true>), grid, dim3(256), 0, s, a);
    } else {
      if (a.nch <= 4) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<4, false, true>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<10, false, true>), grid, dim3(256), 0, s, a);
    }
    return check_launch("wanmi_qk_rmsnorm_rope_to");
  }
  if (rope_pairs == WANMI_ROTATE_HALVES) {
    if (a.nch <= 4) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<4, true>), grid, dim3(256), 0, s, a);
    else if (a.nch <= 10) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<10, true>), grid, dim3(256), 0, s, a);
    else if (a.nch <= 16) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<16, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<32, true>), grid, dim3(256), 0, s, a);
  } else {
    if (a.nch <= 4) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<4, false>), grid, dim3(256), 0, s, a);
    else if (a.nch <= 10) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<10, false>), grid, dim3(256), 0, s, a);
    else if (a.nch <= 16) hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<16, false>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(HIP_KERNEL_NAME(qk_rmsnorm_rope_kernel<32, false>), grid, dim3(256), 0, s, a);
  }
  return check_launch("wanmi_qk_rmsnorm_rope");
}
}  // namespace wanmi

extern "C" int wanmi_qk_rmsnorm_rope(void* x, int64_t S, int64_t ld, int heads, const float* gamma,
                                     const float* cos_tab, const float* sin_tab, int rope_pairs, float eps,
                                     float* maxnorm, void* stream) {
  wanmi::clear_error();
  return wanmi::qk_rmsnorm_rope_impl(x, S, ld, heads, gamma, cos_tab, sin_tab, rope_pairs, eps, maxnorm, nullptr, 0, 0,
                                     0.0f, nullptr, stream);
}

extern "C" int wanmi_qk_rmsnorm_rope_to(const void* x, int64_t S, int64_t ld, int heads, const float* gamma,
                                        const float* cos_tab, const float* sin_tab, int rope_pairs, float eps,
                                        void* out, int64_t out_token_stride, int64_t out_head_stride, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE((S == 0 || out) && ((uintptr_t)out % 16) == 0 && out_token_stride % 8 == 0 && out_head_stride % 8 == 0 &&
                    out_token_stride >= 0 && out_head_stride >= 0,
                WANMI_ERR_ARG,
                "wanmi_qk_rmsnorm_rope_to: out must be 16-byte aligned with strides that are multiples of 8 elements");
  WANMI_REQUIRE(heads > 0 && ((int64_t)(heads - 1) * out_head_stride + 128) * 2 < (1LL << 31), WANMI_ERR_UNSUPPORTED,
                "wanmi_qk_rmsnorm_rope_to: one token's heads span more than 2 GiB of out");
  return qk_rmsnorm_rope_impl(const_cast<void*>(x), S, ld, heads, gamma, cos_tab, sin_tab, rope_pairs, eps, nullptr,
                              nullptr, 0, 0, 0.0f, nullptr, stream, out, out_token_stride, out_head_stride);
}

extern "C" int wanmi_qk_rmsnorm_rope_qrr(void* x, int64_t S, int64_t ld, int heads, const float* gamma,
                                         const float* cos_tab, const float* sin_tab, int rope_pairs, float eps,
                                         float* maxnorm, const float* q_sumsq, int64_t q_sumsq_ld, int q_heads,
                                         float q_eps, float* q_rr, void* stream) {
  using namespace wanmi;
  clear_error();
  // no tokens: nothing is read or written, and empty q_sumsq / q_rr may have no storage
  WANMI_REQUIRE(S == 0 || (q_sumsq && q_rr && ((uintptr_t)q_sumsq % 4) == 0 && ((uintptr_t)q_rr % 4) == 0),
                WANMI_ERR_ARG, "wanmi_qk_rmsnorm_rope_qrr: q_sumsq and q_rr must be 4-byte aligned pointers");
  WANMI_REQUIRE(q_heads > 0 && q_sumsq_ld >= q_heads, WANMI_ERR_ARG,
                "wanmi_qk_rmsnorm_rope_qrr: need q_heads > 0 and q_sumsq_ld >= q_heads (q_heads=%d, ld=%lld)", q_heads,
                (long long)q_sumsq_ld);
  WANMI_REQUIRE(!(q_eps < 0.0f), WANMI_ERR_ARG, "wanmi_qk_rmsnorm_rope_qrr: q_eps must be >= 0");
  return qk_rmsnorm_rope_impl(x, S, ld, heads, gamma, cos_tab, sin_tab, rope_pairs, eps, maxnorm, q_sumsq, q_sumsq_ld,
                              q_heads, q_eps, q_rr, stream);
}

extern "C" int wanmi_transpose_heads(const void* v, int64_t S, int64_t ld, int64_t head_stride, int heads,
                                     void* vt, int64_t S_pad, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(S >= 0 && heads > 0 && heads <= 65535, WANMI_ERR_ARG, "wanmi_transpose_heads: bad S/heads");
  WANMI_REQUIRE(S_pad >= S && S_pad % 64 == 0, WANMI_ERR_ARG,
                "wanmi_transpose_heads: S_pad=%lld must be >= S and a multiple of 64", (long long)S_pad);
  WANMI_REQUIRE(ld >= 128 && ld % 8 == 0 && head_stride % 8 == 0, WANMI_ERR_ARG,
                "wanmi_transpose_heads: bad ld=%lld / head_stride=%lld", (long long)ld, (long long)head_stride);
  if (S_pad == 0) return WANMI_OK;
  WANMI_REQUIRE(v && vt, WANMI_ERR_ARG, "wanmi_transpose_heads: null pointer");
  WANMI_REQUIRE(((uintptr_t)v % 16) == 0 && ((uintptr_t)vt % 16) == 0, WANMI_ERR_ARG,
                "wanmi_transpose_heads: tensors must be 16-byte aligned");
  TransposeArgs a;
  a.v = static_cast<const uint16_t*>(v);
  a.S = S;
  a.ld = ld;
  a.hs = head_stride;
  a.heads = heads;
  a.vt = static_cast<uint16_t*>(vt);
  a.S_pad = S_pad;
  hipLaunchKernelGGL(transpose_heads_kernel, dim3((unsigned)(S_pad / 64), (unsigned)heads), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("wanmi_transpose_heads");
}
