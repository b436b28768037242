// d-major bf16 attention output -> token-major MX activation, in one pass, for the o-projection drop-in.
//
// The reference's exact-attention call sites hand the o-projection a d-major tensor [B, N, 128, S]
// (wan2_2_transformer.py:815-819, 836) and its ROW_MX o-projection kernel quantizes it internally
// (row_mx_kernels.py:114-138). The GEMM here takes a token-major MX activation: codes [B*S, N*128]
// e4m3fn and one e8m0 scale per 32 consecutive channels, [B*S, N*4]. This kernel produces it from the
// d-major tensor directly, where a transpose copy and a separate quantization pass moved the tensor
// through HBM twice. The MX rule is the one of every other producer here (adaln_quant_torch.py:
// 151-175): shared exponent = the block's largest bf16 exponent field - 7, clamped at 0; codes =
// e4m3fn(x * 2^(127 - s)) by the hardware's scaled conversion. Bit-identical to the adaLN kernel's
// NO_NORM / MX mode on the transposed tensor.
//
// Workgroup: one (batch, head) and 64 tokens. Loads: each thread fetches 16-byte runs of 8 tokens of
// one channel (the tensor's contiguous axis) and scatters them into an LDS tile held token-major,
// [64 tokens][128 channels], rows padded to 130 bf16 (260 bytes) so that the 2-byte scatter and the
// 4-byte row reads both spread over the banks. Compute: thread (t, k) = (tid >> 2, tid & 3) owns the
// 32-channel block k of token t: 16 dword reads of its row segment, the block maximum, 32 codes as
// two 16-byte stores (four consecutive lanes write one token's 128 code bytes) and one scale byte.
#include "wanmi_common.h"

namespace wanmi {

struct DmajorMxArgs {
  const uint16_t* x;  // element (b, n, d, s) at x[b*bs + n*ns + d*ds + s]
  int64_t S, bs, ns, ds;
  int heads;
  uint8_t* codes;   // [B*S, heads*128]
  uint8_t* scales;  // [B*S, heads*4]
};

constexpr int kDmTokens = 64;
constexpr int kDmPitch = 130;  // bf16 per LDS row

__global__ __launch_bounds__(256) void dmajor_to_mx_kernel(DmajorMxArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[kDmTokens * kDmPitch];
  const int tid = threadIdx.x;
  const int n = blockIdx.y, b = blockIdx.z;
  const int64_t s0 = (int64_t)blockIdx.x * kDmTokens;
  // one descriptor over this (batch, head) plane; reads past its last element return zero
  const uint16_t* plane = a.x + b * a.bs + n * a.ns;
  const __amdgpu_buffer_rsrc_t r_x = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(plane), (short)0, (int)((127 * a.ds + a.S) * 2), 0x00020000);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;  // 128 channels x 8 runs of 8 tokens
    const int d = idx >> 3, tc = idx & 7;
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r_x, (int)((d * a.ds + s0 + tc * 8) * 2), 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      tile[(tc * 8 + 2 * j) * kDmPitch + d] = (uint16_t)(v[j] & 0xFFFFu);
      tile[(tc * 8 + 2 * j + 1) * kDmPitch + d] = (uint16_t)(v[j] >> 16);
    }
  }
  __syncthreads();
  const int t = tid >> 2, k = tid & 3;
  const int64_t s = s0 + t;
  // the block's 32 channels as 16 packed pairs (row offsets are multiples of 4 bytes)
  const uint32_t* row = reinterpret_cast<const uint32_t*>(tile + t * kDmPitch + 32 * k);
  uint32_t p[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = row[i];
  // the largest exponent field is that of the largest magnitude
  u16x2_t mag = {0, 0};
#pragma unroll
  for (int i = 0; i < 16; ++i) mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2_t, p[i] & 0x7FFF7FFFu));
  const int e = (int)(max(mag[0], mag[1]) >> 7);
  const int sx = max(e - 7, 0);
  const float sc = __uint_as_float((uint32_t)sx << 23);
  u32x4 c0, c1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c0[j] = cvt_e4m3x4_scaled(p[2 * j], p[2 * j + 1], sc);
    c1[j] = cvt_e4m3x4_scaled(p[8 + 2 * j], p[8 + 2 * j + 1], sc);
  }
  if (s < a.S) {
    const int64_t rowc = (int64_t)b * a.S + s;
    uint8_t* cdst = a.codes + rowc * (int64_t)a.heads * 128 + n * 128 + 32 * k;
    *reinterpret_cast<u32x4*>(cdst) = c0;
    *reinterpret_cast<u32x4*>(cdst + 16) = c1;
    a.scales[rowc * (int64_t)a.heads * 4 + n * 4 + k] = (uint8_t)sx;
  }
}

}  // namespace wanmi

extern "C" int wanmi_dmajor_to_mx(const void* x, int64_t B, int heads, int64_t S, int64_t b_stride, int64_t h_stride,
                                  int64_t d_stride, void* codes, uint8_t* scales, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(B >= 0 && S >= 0 && heads > 0 && heads <= 65535 && B <= 65535, WANMI_ERR_ARG,
                "wanmi_dmajor_to_mx: bad sizes B=%lld heads=%d S=%lld", (long long)B, heads, (long long)S);
  if (B == 0 || S == 0) return WANMI_OK;
  WANMI_REQUIRE(x && codes && scales, WANMI_ERR_ARG, "wanmi_dmajor_to_mx: null pointer");
  // 16-byte runs of 8 tokens: every run lies wholly inside or wholly past a channel row's S tokens and
  // the plane's extent, so no load straddles the end of the data
  WANMI_REQUIRE(S % 8 == 0 && d_stride >= S && d_stride % 8 == 0 && h_stride % 8 == 0 && b_stride % 8 == 0 &&
                    ((uintptr_t)x % 16) == 0 && ((uintptr_t)codes % 16) == 0,
                WANMI_ERR_UNSUPPORTED,
                "wanmi_dmajor_to_mx: needs S a multiple of 8, the token axis contiguous with strides that are "
                "multiples of 8 elements (d_stride >= S), and 16-byte aligned x and codes");
  WANMI_REQUIRE((127 * d_stride + S) * 2 < (1LL << 31), WANMI_ERR_UNSUPPORTED,
                "wanmi_dmajor_to_mx: one head's plane exceeds 2 GiB");
  DmajorMxArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.S = S;
  a.bs = b_stride;
  a.ns = h_stride;
  a.ds = d_stride;
  a.heads = heads;
  a.codes = static_cast<uint8_t*>(codes);
  a.scales = scales;
  const int64_t tiles = (S + kDmTokens - 1) / kDmTokens;
  WANMI_REQUIRE(tiles < (1LL << 31), WANMI_ERR_ARG, "wanmi_dmajor_to_mx: S too large");
  hipLaunchKernelGGL(dmajor_to_mx_kernel, dim3((unsigned)tiles, (unsigned)heads, (unsigned)B), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("wanmi_dmajor_to_mx");
}
