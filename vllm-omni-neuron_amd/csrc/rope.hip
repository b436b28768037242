// Wan 3D rotary-embedding tables on gfx950.
//
// WanRotaryPosEmbed (vllm_omni_neuron/diffusion/layers/rope.py:37-114) splits the head dimension
// into three axes -- time, height, width -- of t_dim = head_dim - 2 (2 (head_dim / 6)) and
// h_dim = w_dim = 2 (head_dim / 6) channels, and gives pair j of an axis of dim d at position p the
// angle p * theta^(-2j/d) (computed in fp64, cos/sin cast to fp32). A token of the latent grid
// (F, H, W) in raster order s = (f H + y) W + x takes its time pairs from f, height pairs from y and
// width pairs from x. The tables are built once per generation (T:1757), so this is a plain
// elementwise kernel: one thread per (token, pair), fp64 cos/sin of the angle, stores in the layout
// the caller asks for.
//
// The per-pair frequencies 1 / theta^(2j/d) are computed on the host in fp64 (64 values at most)
// and passed by value; the device computes the fp64 angle p * freq and its cos / sin.
#include "wanmi_common.h"

#include <math.h>

namespace wanmi {

constexpr int kMaxRopePairs = 128;  // head_dim <= 256

struct RopeArgs {
  double freq[kMaxRopePairs];  // per pair of the head: the axis frequency
  int axis[kMaxRopePairs];     // 0 = time (f), 1 = height (y), 2 = width (x)
  int64_t S;
  int grid_h, grid_w;
  int pairs;  // head_dim / 2
  int layout;
  float* cos;
  float* sin;
};

__global__ __launch_bounds__(256) void rope_tables_kernel(RopeArgs a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.S * a.pairs) return;
  const int64_t s = i / a.pairs;
  const int p = (int)(i - s * a.pairs);
  const int64_t hw = (int64_t)a.grid_h * a.grid_w;
  const int64_t f = s / hw;
  const int64_t y = (s / a.grid_w) % a.grid_h;
  const int64_t x = s % a.grid_w;
  const int ax = a.axis[p];
  const double pos = (double)(ax == 0 ? f : (ax == 1 ? y : x));
  const double ang = pos * a.freq[p];
  const float c = (float)cos(ang);
  const float sn = (float)sin(ang);
  if (a.layout == WANMI_ROPE_PAIRS) {
    a.cos[s * a.pairs + p] = c;
    a.sin[s * a.pairs + p] = sn;
  } else if (a.layout == WANMI_ROPE_INTERLEAVED) {
    const int64_t o = s * 2 * a.pairs + 2 * p;
    a.cos[o] = c;
    a.cos[o + 1] = c;
    a.sin[o] = sn;
    a.sin[o + 1] = sn;
  } else {  // WANMI_ROPE_ROTATE_HALF: cat([base, base])
    const int64_t o = s * 2 * a.pairs + p;
    a.cos[o] = c;
    a.cos[o + a.pairs] = c;
    a.sin[o] = sn;
    a.sin[o + a.pairs] = sn;
  }
}

}  // namespace wanmi

extern "C" int wanmi_rope_tables(int64_t frames, int64_t height, int64_t width, int head_dim, int64_t max_seq_len,
                                 double theta, int layout, float* cos_out, float* sin_out, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 2 * kMaxRopePairs, WANMI_ERR_ARG,
                "wanmi_rope_tables: head_dim=%d must be even and at most %d", head_dim, 2 * kMaxRopePairs);
  WANMI_REQUIRE(head_dim >= 6, WANMI_ERR_ARG, "wanmi_rope_tables: head_dim=%d leaves an axis without channels",
                head_dim);
  // rope.py builds the axis tables 2 * (head_dim / 6) wide but its forward slices them at head_dim / 3
  // (rope.py:54-55 against 91-95); where the two differ its slices cut pairs apart, which no per-pair
  // table reproduces
  WANMI_REQUIRE(head_dim / 3 == 2 * (head_dim / 6), WANMI_ERR_UNSUPPORTED,
                "wanmi_rope_tables: head_dim=%d: the reference's axis widths (%d) and forward split (%d) disagree",
                head_dim, 2 * (head_dim / 6), head_dim / 3);
  WANMI_REQUIRE(frames >= 0 && height >= 0 && width >= 0 && max_seq_len <= (1LL << 20), WANMI_ERR_ARG,
                "wanmi_rope_tables: grid sizes must be non-negative and max_seq_len at most 2^20");
  WANMI_REQUIRE(frames <= max_seq_len && height <= max_seq_len && width <= max_seq_len, WANMI_ERR_ARG,
                "wanmi_rope_tables: grid (%lld, %lld, %lld) exceeds max_seq_len=%lld", (long long)frames,
                (long long)height, (long long)width, (long long)max_seq_len);
  WANMI_REQUIRE(layout == WANMI_ROPE_PAIRS || layout == WANMI_ROPE_INTERLEAVED || layout == WANMI_ROPE_ROTATE_HALF,
                WANMI_ERR_ARG, "wanmi_rope_tables: unknown layout %d", layout);
  WANMI_REQUIRE(theta > 0.0, WANMI_ERR_ARG, "wanmi_rope_tables: theta must be positive");
  const int64_t S = frames * height * width;
  if (S == 0) return WANMI_OK;
  WANMI_REQUIRE(cos_out && sin_out, WANMI_ERR_ARG, "wanmi_rope_tables: null output");
  WANMI_REQUIRE(S <= (1LL << 40) / head_dim, WANMI_ERR_ARG, "wanmi_rope_tables: grid too large");
  RopeArgs a;
  const int hw_dim = 2 * (head_dim / 6);   // rope.py:54: h_dim = w_dim = 2 * (attention_head_dim // 6)
  const int t_dim = head_dim - 2 * hw_dim;  // rope.py:55
  const int dims[3] = {t_dim, hw_dim, hw_dim};
  int p = 0;
  for (int ax = 0; ax < 3; ++ax)
    for (int j = 0; j < dims[ax] / 2; ++j, ++p) {
      // rope.py:79: 1.0 / (theta ** (arange(0, dim, 2) / dim)), fp64
      a.freq[p] = 1.0 / pow(theta, (double)(2 * j) / (double)dims[ax]);
      a.axis[p] = ax;
    }
  a.S = S;
  a.grid_h = (int)height;
  a.grid_w = (int)width;
  a.pairs = head_dim / 2;
  a.layout = layout;
  a.cos = cos_out;
  a.sin = sin_out;
  const int64_t n = S * a.pairs;
  const int64_t blocks = (n + 255) / 256;
  WANMI_REQUIRE(blocks < (1LL << 31), WANMI_ERR_ARG, "wanmi_rope_tables: grid too large");
  hipLaunchKernelGGL(rope_tables_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("wanmi_rope_tables");
}
