// Streaming device-to-device passes: the practical HBM rates that the memory-bound kernels here
// (the adaLN + quantization pass, the K normalization pass) are measured against, next to the
// nominal 8 TB/s. They have no counterpart in the reference; they are measurement infrastructure.
//
// One workgroup of 256 threads per 32 KiB chunk: each thread issues its eight 16-byte loads before
// any store (so every wave has 8 KiB in flight), then its 16-byte stores, non-temporal (cache
// policy 2, streamed past L2 as the kernels' own outputs are). The chunk's loads and stores go
// through buffer descriptors whose extent ends at the buffer's end: loads past the end read zero
// and stores past the end are dropped, so the tail needs no branch. A launch of one workgroup per
// chunk (not a persistent grid) lets the dispatcher refill CUs as chunks finish, which hides the
// memory latency best for a pass with no reuse (the adaLN kernel measured the same).
//
// hbm_stream_copy_kernel writes every byte it reads (a 1:1 read/write mix). hbm_stream_fold_kernel
// reads two bytes per byte it writes (the xor of each pair of 16-byte loads), the mix of the adaLN
// + MX pass (2 bytes of bf16 in, 1 byte of e4m3 out, plus 1/32 of a byte of scale): HBM reaches a
// different rate for each mix.
#include "wanmi_common.h"

namespace wanmi {

constexpr int kCopyThreads = 256;
constexpr int kCopyPerThread = 8;
constexpr int64_t kCopyChunk = (int64_t)kCopyThreads * kCopyPerThread * 16;  // 32 KiB

__global__ __launch_bounds__(kCopyThreads) void hbm_stream_copy_kernel(const uint8_t* src, uint8_t* dst, int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * kCopyChunk;
  const int64_t left = bytes - base;
  const uint32_t extent = (uint32_t)(left < kCopyChunk ? left : kCopyChunk);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src + base), (short)0, (int)extent, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(dst + base, (short)0, (int)extent, 0x00020000);
  u32x4 v[kCopyPerThread];
#pragma unroll
  for (int i = 0; i < kCopyPerThread; ++i)
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((i * kCopyThreads + threadIdx.x) * 16), 0, 0);
#pragma unroll
  for (int i = 0; i < kCopyPerThread; ++i) {
    __builtin_amdgcn_raw_buffer_store_b128(v[i], rd, (int)((i * kCopyThreads + threadIdx.x) * 16), 0, 2);
    // the store reads its data registers after it issues: keep them untouched for two wait states
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 1" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
}

__global__ __launch_bounds__(kCopyThreads) void hbm_stream_fold_kernel(const uint8_t* src, uint8_t* dst, int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * kCopyChunk;
  const int64_t left = bytes - base;
  const uint32_t extent = (uint32_t)(left < kCopyChunk ? left : kCopyChunk);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src + base), (short)0, (int)extent, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(dst + base / 2, (short)0, (int)(extent / 2), 0x00020000);
  u32x4 v[kCopyPerThread];
#pragma unroll
  for (int i = 0; i < kCopyPerThread; ++i)
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((i * kCopyThreads + threadIdx.x) * 16), 0, 0);
  // output 16-byte slot i*256 + t of the chunk's 16 KiB holds load 2i xor load 2i+1 of thread t
#pragma unroll
  for (int i = 0; i < kCopyPerThread / 2; ++i) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = v[2 * i][j] ^ v[2 * i + 1][j];
    __builtin_amdgcn_raw_buffer_store_b128(w, rd, (int)((i * kCopyThreads + threadIdx.x) * 16), 0, 2);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 1" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
}

}  // namespace wanmi

extern "C" int wanmi_hbm_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(bytes >= 0 && bytes % 16 == 0, WANMI_ERR_ARG,
                "wanmi_hbm_stream_copy: bytes=%lld must be a non-negative multiple of 16", (long long)bytes);
  if (bytes == 0) return WANMI_OK;
  WANMI_REQUIRE(src && dst && ((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0, WANMI_ERR_ARG,
                "wanmi_hbm_stream_copy: src and dst must be 16-byte aligned");
  const int64_t chunks = (bytes + kCopyChunk - 1) / kCopyChunk;
  WANMI_REQUIRE(chunks < (1LL << 31), WANMI_ERR_ARG, "wanmi_hbm_stream_copy: too large");
  hipLaunchKernelGGL(hbm_stream_copy_kernel, dim3((unsigned)chunks), dim3(kCopyThreads), 0, (hipStream_t)stream,
                     static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), bytes);
  return check_launch("wanmi_hbm_stream_copy");
}

extern "C" int wanmi_hbm_stream_fold(const void* src, void* dst, int64_t src_bytes, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(src_bytes >= 0 && src_bytes % kCopyChunk == 0, WANMI_ERR_ARG,
                "wanmi_hbm_stream_fold: src_bytes=%lld must be a non-negative multiple of %lld", (long long)src_bytes,
                (long long)kCopyChunk);
  if (src_bytes == 0) return WANMI_OK;
  WANMI_REQUIRE(src && dst && ((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0, WANMI_ERR_ARG,
                "wanmi_hbm_stream_fold: src and dst must be 16-byte aligned");
  const int64_t chunks = src_bytes / kCopyChunk;
  WANMI_REQUIRE(chunks < (1LL << 31), WANMI_ERR_ARG, "wanmi_hbm_stream_fold: too large");
  hipLaunchKernelGGL(hbm_stream_fold_kernel, dim3((unsigned)chunks), dim3(kCopyThreads), 0, (hipStream_t)stream,
                     static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), src_bytes);
  return check_launch("wanmi_hbm_stream_fold");
}
