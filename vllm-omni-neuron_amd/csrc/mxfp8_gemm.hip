// MXFP8 block-scaled GEMM for gfx950 with fused epilogues.
//
//   C[m, n] = epilogue( sum_k A[m, k] * 2^(sa[m, k/32]-127) * W[n, k] * 2^(sw[n, k/32]-127) )
//
// A (activations) is [M, K] e4m3fn with e8m0 scales [M, K/32]; W is the weight stored transposed,
// [N, K] e4m3fn with scales [N, K/32] -- both K-contiguous, the MX layout the adaLN kernel emits.
// The inner product runs on v_mfma_scale_f32_32x32x64_f8f6f4, which applies the e8m0 block scales
// in hardware, accumulating in fp32.
//
// Orientation: the MFMA's A operand is W (rows = output features n) and its B operand is A (columns
// = tokens m), so the accumulator of each lane holds four consecutive n of one token m per register
// group. Bias, GELU, bf16 rounding and the per-32 MX re-quantization along n are then lane-local
// (one exchange with lane ^ 32 completes a 32-wide block), and stores are 8-byte (bf16) or 4-byte
// (e4m3) vectors.
//
// Tiling: 256 (n) x 256 (m) x 128 (k) per workgroup of 4 waves, each wave a 128 x 128 block of
// 4 x 4 MFMA tiles (256 fp32 accumulators per lane). Operand tiles are staged through LDS in two
// stage buffers filled by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds, no VGPR round
// trip), with a 16-byte-chunk XOR swizzle (chunk ^ (row & 7)) so the MFMA operand reads of eight
// consecutive rows land on distinct banks. Each stage's loads are issued two stages ahead into the
// buffer just consumed; operands are read per 64-deep slice into ping-pong registers so LDS reads
// overlap the previous slice's MFMAs. Workgroup ids are remapped so each XCD (ids are
// dealt round-robin over 8 XCDs) works on a contiguous, L2-friendly group of tiles.
//
// Reference semantics: the ROW_MX projection epilogues of _qkv_cte_mx_impl / _dequant_row_mx
// (vllm_omni_neuron/kernels/nkilib/core/qkv/qkv_cte.py:3711-3750, 3996-4021) and of the MLP
// (kernels/nkilib/core/mlp/mlp_cte/mx/mlp_cte_mx_projection.py:630-668, GELU-tanh then
// quantize_mx in mlp_cte_mx_quantization.py:113-154); the torch statement is _mlp_ref_standard
// (kernels/nkilib/core/mlp/mlp_torch.py:401-599).
#include "wanmi_common.h"

namespace wanmi {

constexpr int TN = 256;  // weight rows (output features) per workgroup
constexpr int TM = 256;  // tokens per workgroup
constexpr int BK = 128;  // k bytes per stage (4 MX blocks)
constexpr int kStageBytes = TN * BK + TM * BK + TN * 4 + TM * 4;
constexpr int kGroupM = 8;
constexpr int kBufferRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3 (raw, 32-bit data)
// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14)
constexpr int kWaitVm18 = (18 & 0xF) | (0x7 << 4) | (0xF << 8) | ((18 >> 4) << 14);  // vmcnt <= 18
constexpr int kWaitLgkm0 = 0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14);               // lgkmcnt == 0

struct GemmArgs {
  const uint8_t* a;         // [M, lda]
  const uint8_t* a_scales;  // [M, K/32]
  const uint8_t* w;         // [N, K]
  const uint8_t* w_scales;  // [N, K/32]
  const float* row_scale;   // [M] or null
  const float* col_scale;   // [N] or null
  const float* bias;        // [N] or null
  const uint16_t* residual; // [M, ldo] bf16 (gated residual epilogue)
  const float* gate;        // [N]
  void* out;                // [M, ldo]
  uint8_t* out_scales;      // [M, N/32]
  int64_t M, N, K, lda, ldo;
  int epilogue;
};

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), tanh via exp of -2|u|
  const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  const float t = __expf(-2.0f * fabsf(u));
  float th = (1.0f - t) / (1.0f + t);
  th = copysignf(th, u);
  return 0.5f * x * (1.0f + th);
}

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 4); }


// MFMA operands of one 64-deep k slice of a wave's 128 x 128 block: 4 weight-row and 4 token-row
// fragments (32 bytes per lane each) and their e8m0 scale bytes.
struct SliceOperands {
  i32x8 w[4];
  i32x8 a[4];
  int ws[4];
  int as[4];
};

// Reads slice s (0 or 1) of an LDS stage. Lane data: bytes 0-15 = k[64s + 16h, +16),
// bytes 16-31 = k[64s + 32 + 16h, +16); the lane's scale byte is block 2s + h of its row.
__device__ __forceinline__ void read_slice(const uint8_t* base, int s, SliceOperands& op, int wn, int wm, int h,
                                           int r32) {
  const uint8_t* sw = base;
  const uint8_t* sa = base + TN * BK;
  const uint32_t* sws = reinterpret_cast<const uint32_t*>(base + TN * BK + TM * BK);
  const uint32_t* sas = sws + TN;
  const int c0 = s * 4 + h, c1 = s * 4 + 2 + h;
  const int sh = 8 * (2 * s + h);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rw = wn * 128 + i * 32 + r32;
    const uint4 x0 = *reinterpret_cast<const uint4*>(sw + swz(rw, c0));
    const uint4 x1 = *reinterpret_cast<const uint4*>(sw + swz(rw, c1));
    op.w[i] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    const int ra = wm * 128 + i * 32 + r32;
    const uint4 y0 = *reinterpret_cast<const uint4*>(sa + swz(ra, c0));
    const uint4 y1 = *reinterpret_cast<const uint4*>(sa + swz(ra, c1));
    op.a[i] = i32x8{(int)y0.x, (int)y0.y, (int)y0.z, (int)y0.w, (int)y1.x, (int)y1.y, (int)y1.z, (int)y1.w};
    op.ws[i] = (int)((sws[rw] >> sh) & 0xFFu);
    op.as[i] = (int)((sas[ra] >> sh) & 0xFFu);
  }
}

__device__ __forceinline__ void mfma_slice(const SliceOperands& op, f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(op.w[i], op.a[j], acc[i][j], 0, 0, 0, op.ws[i], 0,
                                                                   op.as[j]);
}

// One 32 x 32 accumulator tile: lane holds token m and n = ntile + 8*gi + 4*h + q (gi, q in 0..3).
template <int EPI>
__device__ __forceinline__ void epilogue_tile(const GemmArgs& g, const f32x16& a, int64_t m, int64_t ntile,
                                              int h) {
#pragma clang fp contract(off)
  const bool mok = m < g.M;
  const float rsc = (g.row_scale && mok) ? g.row_scale[m] : 1.0f;
  float v[16];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    const int64_t nb = ntile + gi * 8 + h * 4;
    float4 b = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g.bias) b = *reinterpret_cast<const float4*>(g.bias + nb);
    float4 cs = make_float4(1.f, 1.f, 1.f, 1.f);
    if (g.col_scale) cs = *reinterpret_cast<const float4*>(g.col_scale + nb);
    const float bb[4] = {b.x, b.y, b.z, b.w};
    const float cc[4] = {cs.x, cs.y, cs.z, cs.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float x = a[gi * 4 + q];
      if (g.row_scale) x = x * rsc;
      if (g.col_scale) x = x * cc[q];
      v[gi * 4 + q] = x + bb[q];
    }
  }
  if constexpr (EPI == WANMI_EPI_BF16 || EPI == WANMI_EPI_GELU_BF16) {
    uint16_t* out = reinterpret_cast<uint16_t*>(g.out);
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int64_t nb = ntile + gi * 8 + h * 4;
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = EPI == WANMI_EPI_GELU_BF16 ? gelu_tanh(v[gi * 4 + q]) : v[gi * 4 + q];
      if (mok)
        *reinterpret_cast<uint2*>(out + m * g.ldo + nb) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    }
  } else if constexpr (EPI == WANMI_EPI_GELU_MX) {
    float y[16];
    int e = 0;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      y[q] = round_bf16(gelu_tanh(v[q]));
      e = max(e, exp_field(y[q]));
    }
    e = max(e, __shfl_xor(e, 32, 64));  // lanes l and l^32 hold the two halves of the 32-block
    const int s = max(e - 7, 0);
    const float f = mx_inv_scale(s);
    uint8_t* codes = reinterpret_cast<uint8_t*>(g.out);
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int64_t nb = ntile + gi * 8 + h * 4;
      const uint32_t c4 = cvt_e4m3x4(y[gi * 4] * f, y[gi * 4 + 1] * f, y[gi * 4 + 2] * f, y[gi * 4 + 3] * f);
      if (mok) *reinterpret_cast<uint32_t*>(codes + m * g.ldo + nb) = c4;
    }
    if (mok && h == 0) g.out_scales[m * (g.N / 32) + ntile / 32] = (uint8_t)s;
  } else {  // gated residual: out = bf16(res + bf16(v) * gate)
    uint16_t* out = reinterpret_cast<uint16_t*>(g.out);
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int64_t nb = ntile + gi * 8 + h * 4;
      if (!mok) continue;
      const uint2 r = *reinterpret_cast<const uint2*>(g.residual + m * g.ldo + nb);
      const float4 gt = *reinterpret_cast<const float4*>(g.gate + nb);
      const float rr[4] = {bf16_lo(r.x), bf16_hi(r.x), bf16_lo(r.y), bf16_hi(r.y)};
      const float gg[4] = {gt.x, gt.y, gt.z, gt.w};
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float f = round_bf16(v[gi * 4 + q]);
        const float prod = f * gg[q];
        y[q] = rr[q] + prod;
      }
      *reinterpret_cast<uint2*>(out + m * g.ldo + nb) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    }
  }
}

template <int EPI, int I = 0>
__device__ __forceinline__ void epilogue_all(const GemmArgs& g, const f32x16 (&acc)[4][4], int64_t m0, int64_t n0,
                                             int wm, int wn, int lane) {
  if constexpr (I < 16) {
    constexpr int i = I / 4, j = I % 4;
    epilogue_tile<EPI>(g, acc[i][j], m0 + wm * 128 + j * 32 + (lane & 31), n0 + wn * 128 + i * 32, lane >> 5);
    epilogue_all<EPI, I + 1>(g, acc, m0, n0, wm, wn, lane);
  }
}

// kEvenStages: the pipelined, branch-free loop below (K a multiple of 256); otherwise a simple
// double-buffered loop that issues the next stage's loads after all reads of the current one.
template <bool kEvenStages>
__global__ __launch_bounds__(256, 1) void mxfp8_gemm_kernel(GemmArgs g) {
#pragma clang fp contract(off)
  // Two separate LDS objects: the compiler can then prove that the stage being read never aliases
  // the stage being filled by in-flight direct-to-LDS loads, and waits only on the latter's own.
  __shared__ __attribute__((aligned(16))) uint8_t smem0[kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t smem1[kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave >> 1, wm = wave & 1;
  const int64_t M = g.M, N = g.N, K = g.K;
  const int KB = (int)(K / 32);

  // ---- tile mapping: XCD-contiguous chunks, grouped along m ----
  const int tiles_n = (int)(N / TN);
  const int tiles_m = (int)((M + TM - 1) / TM);
  const int total = tiles_n * tiles_m;
  int pid = blockIdx.x;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  const int in_group = kGroupM * tiles_n;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int tm = first_m + (pid % in_group) % gsz;
  const int tn = (pid % in_group) / gsz;
  const int64_t n0 = (int64_t)tn * TN, m0 = (int64_t)tm * TM;

  // ---- global -> LDS staging: buffer loads straight into LDS (no VGPR round trip) ----
  // Wave w fills rows 64w .. 64w+63 of each operand tile, 8 rows (1 KiB) per instruction: lane l
  // lands in physical 16-byte slot l & 7 of row 8i + (l >> 3) and fetches the logical chunk the XOR
  // swizzle assigns to that slot. Token rows past M fall outside the activation buffer resource's
  // extent and read as zero (they are never stored).
  const int srow = lane >> 3;
  const int schunk = (lane & 7) ^ (srow & 7);
  const int64_t m_valid = min((int64_t)TM, M - m0);
  const __amdgpu_buffer_rsrc_t rs_w =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.w + n0 * K), (short)0, (int)(TN * K), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs_a =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.a + m0 * g.lda), (short)0, (int)(m_valid * g.lda), kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs_ws =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.w_scales + n0 * KB), (short)0, TN * KB, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs_as =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.a_scales + m0 * KB), (short)0, (int)(m_valid * KB), kBufferRsrcWord3);
  const uint32_t voff_w = (uint32_t)((wave * 64 + srow) * K + schunk * 16);
  const uint32_t voff_a = (uint32_t)((wave * 64 + srow) * g.lda + schunk * 16);
  const uint32_t voff_s = (uint32_t)((wave * 64 + lane) * KB);
  const uint32_t wstep = (uint32_t)(8 * K), astep = (uint32_t)(8 * g.lda);

#define WANMI_BLDS(rs, dst, bytes, voff) \
  __builtin_amdgcn_raw_ptr_buffer_load_lds((rs), (__attribute__((address_space(3))) void*)(dst), (bytes), (voff), 0, 0, 0)

#define WANMI_GEMM_ISSUE(kt, buf)                                                                \
  do {                                                                                           \
    const uint32_t k0_ = (uint32_t)(kt) * BK;                                                    \
    uint8_t* base_ = (buf) + wave * 64 * BK;                                                     \
    _Pragma("unroll") for (int i = 0; i < 8; ++i) {                                              \
      WANMI_BLDS(rs_w, base_ + i * 8 * BK, 16, voff_w + i * wstep + k0_);                         \
      WANMI_BLDS(rs_a, base_ + TN * BK + i * 8 * BK, 16, voff_a + i * astep + k0_);               \
    }                                                                                            \
    uint8_t* sbase_ = (buf) + TN * BK + TM * BK + wave * 64 * 4;                                 \
    WANMI_BLDS(rs_ws, sbase_, 4, voff_s + (kt) * 4);                                             \
    WANMI_BLDS(rs_as, sbase_ + TN * 4, 4, voff_s + (kt) * 4);                                    \
  } while (0)

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = (int)(K / BK);
  const int h = lane >> 5;
  const int r32 = lane & 31;

  if constexpr (!kEvenStages) {
    // stage kt in smem0 / smem1 alternately; the next stage's loads go into the other buffer
    // (read by nobody since the previous barrier) before this stage's MFMAs
    WANMI_GEMM_ISSUE(0, smem0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      uint8_t* cur = (kt & 1) ? smem1 : smem0;
      uint8_t* nxt = (kt & 1) ? smem0 : smem1;
      if (kt + 1 < KT) WANMI_GEMM_ISSUE(kt + 1, nxt);
      SliceOperands op;
      read_slice(cur, 0, op, wn, wm, h, r32);
      mfma_slice(op, acc);
      read_slice(cur, 1, op, wn, wm, h, r32);
      mfma_slice(op, acc);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  } else {
    // Pipeline (KT even, branch-free): stage kt lives in smem0 for even kt, smem1 for odd kt. The
    // loads of stage kt+2 go into the buffer stage kt was just read from (after a barrier confirms
    // every wave has read it), so each stage's loads have two stages of MFMA work to land; past the
    // end the stage index is clamped, re-loading the last stage into a buffer nobody reads again.
    // Within a stage the two 64-deep slices are read into ping-pong registers, each slice's LDS
    // reads overlapping the previous slice's MFMAs.
    WANMI_GEMM_ISSUE(0, smem0);
    WANMI_GEMM_ISSUE(1, smem1);
    __builtin_amdgcn_s_waitcnt(kWaitVm18);  // stage 0 landed (stage 1's 18 loads may be in flight)
    __syncthreads();
    SliceOperands opA, opB;
    read_slice(smem0, 0, opA, wn, wm, h, r32);
    for (int kt = 0; kt < KT; kt += 2) {
      // ---- stage kt (smem0) ----
      read_slice(smem0, 1, opB, wn, wm, h, r32);
      mfma_slice(opA, acc);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __syncthreads();  // every wave has read smem0
      WANMI_GEMM_ISSUE(min(kt + 2, KT - 1), smem0);
      __builtin_amdgcn_s_waitcnt(kWaitVm18);  // stage kt+1 (smem1) landed
      __syncthreads();
      read_slice(smem1, 0, opA, wn, wm, h, r32);
      mfma_slice(opB, acc);
      // ---- stage kt+1 (smem1) ----
      read_slice(smem1, 1, opB, wn, wm, h, r32);
      mfma_slice(opA, acc);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __syncthreads();  // every wave has read smem1
      WANMI_GEMM_ISSUE(min(kt + 3, KT - 1), smem1);
      __builtin_amdgcn_s_waitcnt(kWaitVm18);  // stage kt+2 (smem0) landed
      __syncthreads();
      read_slice(smem0, 0, opA, wn, wm, h, r32);  // past the last stage: a dead read
      mfma_slice(opB, acc);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load may still target LDS when the workgroup retires
#undef WANMI_GEMM_ISSUE
#undef WANMI_BLDS

  // ---- epilogue (expanded per tile and per epilogue kind, so accumulator indices are static) ----
  switch (g.epilogue) {
    case WANMI_EPI_BF16: epilogue_all<WANMI_EPI_BF16>(g, acc, m0, n0, wm, wn, lane); break;
    case WANMI_EPI_GELU_MX: epilogue_all<WANMI_EPI_GELU_MX>(g, acc, m0, n0, wm, wn, lane); break;
    case WANMI_EPI_GELU_BF16: epilogue_all<WANMI_EPI_GELU_BF16>(g, acc, m0, n0, wm, wn, lane); break;
    default: epilogue_all<WANMI_EPI_GATED_RESIDUAL>(g, acc, m0, n0, wm, wn, lane); break;
  }
}

}  // namespace wanmi

extern "C" int wanmi_mxfp8_gemm(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                                const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                                const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda,
                                int epilogue, void* out, int64_t ldo, uint8_t* out_scales,
                                const void* residual, const float* gate, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(M >= 0 && N > 0 && K > 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm: bad sizes M=%lld N=%lld K=%lld",
                (long long)M, (long long)N, (long long)K);
  WANMI_REQUIRE(N % TN == 0, WANMI_ERR_UNSUPPORTED, "wanmi_mxfp8_gemm: N=%lld must be a multiple of %d",
                (long long)N, TN);
  WANMI_REQUIRE(K % BK == 0, WANMI_ERR_UNSUPPORTED, "wanmi_mxfp8_gemm: K=%lld must be a multiple of %d",
                (long long)K, BK);
  WANMI_REQUIRE(epilogue >= WANMI_EPI_BF16 && epilogue <= WANMI_EPI_GATED_RESIDUAL, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: unknown epilogue %d", epilogue);
  WANMI_REQUIRE(lda >= K && lda % 16 == 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm: lda=%lld must be >= K and a multiple of 16",
                (long long)lda);
  WANMI_REQUIRE(ldo >= N && ldo % 4 == 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm: ldo=%lld must be >= N and a multiple of 4",
                (long long)ldo);
  if (M == 0) return WANMI_OK;
  WANMI_REQUIRE(a_codes && a_scales && w_codes && w_scales && out, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: null operand");
  WANMI_REQUIRE(epilogue != WANMI_EPI_GELU_MX || out_scales, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: GELU_MX epilogue needs out_scales");
  WANMI_REQUIRE(epilogue != WANMI_EPI_GATED_RESIDUAL || (residual && gate), WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: gated-residual epilogue needs residual and gate");
  WANMI_REQUIRE(((uintptr_t)a_codes % 16) == 0 && ((uintptr_t)w_codes % 16) == 0 &&
                    ((uintptr_t)a_scales % 4) == 0 && ((uintptr_t)w_scales % 4) == 0 &&
                    ((uintptr_t)out % 8) == 0 && (!bias || ((uintptr_t)bias % 16) == 0) &&
                    (!col_scale || ((uintptr_t)col_scale % 16) == 0) &&
                    (!gate || ((uintptr_t)gate % 16) == 0) && (!residual || ((uintptr_t)residual % 8) == 0),
                WANMI_ERR_ARG, "wanmi_mxfp8_gemm: misaligned operand");
  const int64_t tiles = (N / TN) * ((M + TM - 1) / TM);
  WANMI_REQUIRE(tiles < (1LL << 31), WANMI_ERR_ARG, "wanmi_mxfp8_gemm: problem too large");

  GemmArgs g;
  g.a = a_codes;
  g.a_scales = a_scales;
  g.w = w_codes;
  g.w_scales = w_scales;
  g.row_scale = row_scale;
  g.col_scale = col_scale;
  g.bias = bias;
  g.residual = static_cast<const uint16_t*>(residual);
  g.gate = gate;
  g.out = out;
  g.out_scales = out_scales;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldo = ldo;
  g.epilogue = epilogue;
  if ((K / BK) % 2 == 0)
    hipLaunchKernelGGL(mxfp8_gemm_kernel<true>, dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream, g);
  else
    hipLaunchKernelGGL(mxfp8_gemm_kernel<false>, dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream, g);
  return check_launch("wanmi_mxfp8_gemm");
}
