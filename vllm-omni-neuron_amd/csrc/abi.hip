// Library-wide C ABI pieces: version, thread-local error message, launch checking, and the e4m3
// conversion test hook.
#include "wanmi_common.h"

#include <string.h>

namespace wanmi {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return WANMI_ERR_HIP;
  }
  return WANMI_OK;
}

__global__ void e4m3_encode_kernel(const float* __restrict__ in, uint8_t* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (uint8_t)(cvt_e4m3x2(in[i], 0.0f) & 0xFFu);
}

}  // namespace wanmi

extern "C" int wanmi_abi_version(void) { return WANMI_ABI_VERSION; }

extern "C" const char* wanmi_last_error(void) { return wanmi::g_last_error; }

extern "C" int wanmi_e4m3_encode(const float* in, uint8_t* out, int64_t n, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(n >= 0, WANMI_ERR_ARG, "wanmi_e4m3_encode: n=%lld < 0", (long long)n);
  if (n == 0) return WANMI_OK;
  WANMI_REQUIRE(in && out, WANMI_ERR_ARG, "wanmi_e4m3_encode: null pointer");
  const int threads = 256;
  const int64_t blocks = (n + threads - 1) / threads;
  WANMI_REQUIRE(blocks < (1LL << 31), WANMI_ERR_ARG, "wanmi_e4m3_encode: n too large");
  hipLaunchKernelGGL(e4m3_encode_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                     (hipStream_t)stream, in, out, n);
  return check_launch("wanmi_e4m3_encode");
}

namespace wanmi {

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

}  // namespace wanmi
