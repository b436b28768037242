// Constant-max flash attention (non-causal) for gfx950, bf16 MFMA with fp32 accumulation.
//
//   o_i = sum_j exp(s q_i.k_j - c_i) v_j / max(sum_j exp(s q_i.k_j - c_i), 1e-37)
//   c_i = s * ||q_i|| * max_j ||k_j||           (per query row; Cauchy-Schwarz bound on s q_i.k_j)
//
// Softmax is invariant to the subtracted constant, so no running max and no rescaling of the
// accumulator are needed: the key loop is pure accumulation. Reference: the constant-max kernel
// and ring driver (vllm_omni_neuron/kernels/nkilib/experimental/attention/attention_const_max.py:
// 69-490, ring_attention_const_max_fwd.py:559-804); the exact-softmax statement is _torch_attend
// (diffusion/models/wan2_2/wan2_2_transformer.py:640-650). Here the whole key sequence of one GPU is
// a single "ring step", c_i is kept in fp32 (the reference rounds it to bf16; the result does not
// depend on c), and exp runs as exp2 with log2(e) folded into the scale.
//
// Mapping: a workgroup owns 256 queries of one head (8 waves x 32) and walks the keys in tiles of
// 64. Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (K from LDS as the A operand,
// its 32 queries' Q fragments resident in registers as the B operand), so every lane ends up owning
// one query column: the row sum of P is lane-local and P^T is already laid out as the B operand of
// O^T = V^T P^T -- no transpose of P. V^T comes pre-transposed with keys permuted inside groups of
// 16 (wanmi_transpose_heads) to match P^T's register order. ||q_i|| is taken from the same bf16
// Q fragments the MFMA consumes.
#include "wanmi_common.h"

#include <mutex>

namespace wanmi {

constexpr int kAttnRsrcWord3 = 0x00020000;
constexpr int kWaves = 8;          // waves per workgroup, 32 queries each
constexpr int BQ = 32 * kWaves;    // queries per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int BKV = 64;            // keys per LDS tile (two 32-key halves)
constexpr int kStages = 4;         // LDS ring depth in tiles
constexpr float kSumFloor = 1e-37f;
constexpr int kCrossHeadsPerGroupMax = 20;  // heads per workgroup, short key sequences (upper bound)

// Heads per workgroup of attention_head_group_kernel: the divisor c >= 2 of `heads` (at most
// kCrossHeadsPerGroupMax) whose grid of blocks * heads / c workgroups finishes first when every CU
// takes one at a time, each costing c heads plus a fixed part (the first three key tiles, the
// queries' norm sum, the last head's drain) of about 0.3 head, measured at 32760 queries over 512
// keys: 389.4 / 379.9 / 371.8 us with 5 / 10 / 20 heads per workgroup, 4 / 2 / 1 rounds of 256.
// The larger group wins a tie. 20 heads at 32760 queries (128 blocks), 8 at 75600 (296 blocks).
inline int cross_heads_per_group(int64_t blocks, int heads, int cus) {
  int best_c = 1;
  int64_t best = INT64_MAX;
  for (int c = 2; c <= kCrossHeadsPerGroupMax && c <= heads; ++c) {
    if (heads % c) continue;
    const int64_t wgs = blocks * (heads / c);
    const int64_t cost = ((wgs + cus - 1) / cus) * (10 * c + 3);
    if (cost <= best) {
      best = cost;
      best_c = c;
    }
  }
  return best_c;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kAttnRsrcWord3);
}

struct AttnArgs {
  const uint16_t* q;  // element (h, s, d) at q[h*q_hs + s*q_ss + d]
  int64_t q_hs, q_ss;
  const uint16_t* k;
  int64_t k_hs, k_ss;
  const uint16_t* vt;  // [heads, 128, vt_ld] (keys permuted within 16-groups)
  int64_t vt_ld;
  const float* kmax;  // [heads]
  int64_t Sq, Sk;
  int heads;
  float scale;       // softmax scale s
  float scale_log2;  // s * log2(e)
  int out_mode;
  void* out;
  int64_t o_hs, o_ss, o_ds;  // token-major: (h, s, d) at o_hs*h + o_ss*s + d; d-major: + o_ds*d + s
  uint8_t* out_scales;       // MX: [Sq, heads*4] at (s, h*4 + dtile)
  int64_t os_ss;
  // Fused Q preparation (q_sumsq non-null): q holds the raw projection, and the kernel applies the
  // across-heads RMSNorm (from per-128-column partial sums of squares, [Sq, qss_ld], blocks in
  // order) with q_gamma [heads*128] and, if q_cos is given, the interleaved RoPE ([Sq, 64] tables).
  const float* q_sumsq;
  int64_t qss_ld;
  const float* q_gamma;
  const float* q_cos;
  const float* q_sin;
  float q_eps;
  int heads_per_group;  // attention_head_group_kernel: consecutive heads per workgroup (divides heads)
  float* row_sum;       // optional: each query's row sum of P, [heads][Sq] (wanmi_attention_exact)
  const float* q_rr;    // optional (with q_gamma): each query's across-heads 1/rms [Sq], in place of q_sumsq
};

// LDS tiles, a ring of kStages (tile t in slot t % kStages):
//   sK: [64 keys][128 d] bf16, 16-byte chunk index XOR (key & 15)
//   sV: [128 d][64 slots] bf16, 16-byte chunk index XOR f(d) = (d & 7) ^ ((d >> 3) & 1)
// One LDS cycle serves 16 lanes from 64 banks of 4 bytes: the K reads cover 16 keys (one 256-byte
// row each, 16 distinct chunks); the V^T reads cover 16 d-rows of 128 bytes, two rows per bank
// cycle, and f gives the eight even and the eight odd rows eight distinct chunks.
__device__ __forceinline__ int sk_off(int key, int chunk) { return key * 256 + ((chunk ^ (key & 15)) << 4); }
__device__ __forceinline__ int sv_off(int d, int chunk) { return d * 128 + ((chunk ^ ((d & 7) ^ ((d >> 3) & 1))) << 4); }
constexpr int kTileK = BKV * 256;      // bytes of one K tile
constexpr int kTileV = 128 * BKV * 2;  // bytes of one V^T tile
constexpr int kLoadsPerTile = 4;       // direct-to-LDS instructions per wave per tile (2 K + 2 V)

// Logits of one 32-key half (keys 32 i .. 32 i + 31 of the LDS tile) against the wave's 32 queries,
// in log2 units and already shifted by the bound: S^T = -c2 + K (s log2e Q)^T. The chain starts from
// `negc` (every register -c2 of the lane's query), so the softmax needs no per-element scale or
// subtraction. 8 MFMAs over d, K fragments read ahead of the chain.
__device__ __forceinline__ f32x16 qk_half(const uint8_t* cK, int i, const bf16x8 (&qf)[8], const f32x16& negc,
                                          int col, int hq) {
  bf16x8 kf[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) kf[t] = *reinterpret_cast<const bf16x8*>(cK + sk_off(i * 32 + col, 2 * t + hq));
  f32x16 s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0], qf[0], negc, 0, 0, 0);
#pragma unroll
  for (int t = 1; t < 8; ++t) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t], qf[t], s, 0, 0, 0);
  return s;
}

// P = exp2(S) for one half of shifted log2 logits, added to the lane's row sum and packed (bf16) as
// the two 16-key B operands of O^T += V^T P^T. Accumulator register r of lane l holds key
// 8 (r >> 2) + 4 (l >> 5) + (r & 3) of the half. kMask: keys at half positions >= `valid` get P = 0.
// kSumBf16: the row sum adds the bf16 P that the P V product multiplies (two per v_dot2 against
// (1, 1)), as the reference's [V | 1] column does (attention_const_max.py:454); otherwise it adds the
// fp32 P. Measured against fp64 attention on MI355X (S = 32760, 3 heads): self-attention 2.958e-3
// rms relative error either way, cross-attention over 512 keys 2.927e-3 (bf16 sum) vs 2.939e-3 (fp32
// sum); the bf16 sum costs self-attention 1.3% (17.09 vs 16.87 ms) and cross-attention nothing, so
// only the short-key instantiation uses it.
template <bool kMask, bool kSumBf16>
__device__ __forceinline__ void softmax_half(const f32x16& s, int hq, int valid, float& lsum, bf16x8 (&pf)[2]) {
#pragma clang fp contract(off)
  float p[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float x = __builtin_amdgcn_exp2f(s[r]);
    if constexpr (kMask) x = (r >> 2) * 8 + hq * 4 + (r & 3) < valid ? x : 0.0f;
    p[r] = x;
    if constexpr (!kSumBf16) lsum = lsum + x;
  }
  [[maybe_unused]] const bf16x2_t ones = {(__bf16)1.0f, (__bf16)1.0f};
  [[maybe_unused]] float part[2] = {0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = pack_bf16x2(p[8 * u + 2 * j], p[8 * u + 2 * j + 1]);
      if constexpr (kSumBf16)
        part[u] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[j]), ones, part[u], false);
    }
    pf[u] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
  }
  if constexpr (kSumBf16) lsum = lsum + (part[0] + part[1]);
}

// O^T += V^T P^T for one 32-key half (16-key groups 2 i, 2 i + 1 of the LDS tile): 8 MFMAs in four
// independent accumulator chains.
__device__ __forceinline__ void pv_half(const uint8_t* cV, int i, const bf16x8 (&pf)[2], f32x16 (&acc_o)[4], int col,
                                        int hq) {
  bf16x8 vf[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      vf[u][dt] = *reinterpret_cast<const bf16x8*>(cV + sv_off(dt * 32 + col, 2 * (2 * i + u) + hq));
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[u][dt], pf[u], acc_o[dt], 0, 0, 0);
}

// One step of the per-wave software pipeline over 32-key halves: the QK^T MFMAs of half h (K from
// cK, half i_cur) are independent of the softmax of half h-1 (s_prev), so the two streams interleave
// on the matrix and vector pipes; then half h-1's P V MFMAs (V from cV, half i_prev).
template <bool kMask, bool kSumBf16>
__device__ __forceinline__ void pipeline_step(const uint8_t* cK, int i_cur, const uint8_t* cV, int i_prev,
                                              const bf16x8 (&qf)[8], const f32x16& negc, f32x16& s_prev,
                                              f32x16 (&acc_o)[4], float& lsum, int col, int hq, int valid_prev) {
  const f32x16 s_cur = qk_half(cK, i_cur, qf, negc, col, hq);
  bf16x8 pf[2];
  softmax_half<kMask, kSumBf16>(s_prev, hq, valid_prev, lsum, pf);
  pv_half(cV, i_prev, pf, acc_o, col, hq);
  s_prev = s_cur;
}

// kShortKV: a separate instantiation for short key sequences (cross-attention over text tokens) so
// the two uses can be specialized and profiled apart; it sums the bf16 P (see softmax_half).
// kRebaseK: one head of K spans more than 2 GiB (the fused QKV layout, row stride 15360, at 720p), so
// the K descriptor is rebuilt at each tile's first key; otherwise one descriptor covers the head and
// the tile's offset travels in the wave-uniform soffset.
template <bool kShortKV, bool kRebaseK>
__global__ __launch_bounds__(kThreads) void attention_const_max_kernel(AttnArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) uint8_t sK[kStages][kTileK];
  __shared__ __attribute__((aligned(16))) uint8_t sV[kStages][kTileV];
  __shared__ __attribute__((aligned(16))) float sgam[kWaves][256];  // each wave's copy of the head's gamma

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups go to the 8 XCDs round-robin by linear index. With the heads a multiple of 8, XCD x
  // takes heads x * heads/8 .. + heads/8 - 1 whole, query block after query block, so that all of
  // its CUs stream the same head's K/V tiles through its L2 instead of every XCD fetching every head
  // (the same (head, query block) pairs, each computed as before).
  int hb = blockIdx.y, qb = blockIdx.x;
  if ((gridDim.y & 7) == 0) {
    const int nq = (int)gridDim.x;
    const int L = (int)blockIdx.x + (int)blockIdx.y * nq;
    const int k = L >> 3;
    hb = (L & 7) * (int)(gridDim.y >> 3) + k / nq;
    qb = k % nq;
  }
  const int h = hb;
  const int64_t q0 = (int64_t)qb * BQ + wave * 32;
  const int col = lane & 31;  // this lane's query within the wave's 32
  const int hq = lane >> 5;

  // Keys >= Sk fall outside the K descriptor's extent and read as zero. V^T ([128][vt_ld] per head,
  // vt_ld >= Sk rounded up to 64) always fits one descriptor, and every tile lies inside it.
  const uint16_t* k_head = a.k + h * a.k_hs;
  const u32x4 r_k_head = buffer_rsrc(k_head, kRebaseK ? 0u : (uint32_t)(((a.Sk - 1) * a.k_ss + 128) * 2));
  const u32x4 r_v = buffer_rsrc(a.vt + (int64_t)h * 128 * a.vt_ld, (uint32_t)(128 * a.vt_ld * 2));
  // DMA lane mapping: each wave fills 8 K rows (4 per 1 KiB instruction) and 16 V^T rows (8 per
  // instruction); lane l lands in physical chunk l & 15 (K) / l & 7 (V) of its row and fetches the
  // logical chunk the XOR swizzle assigns to that slot. The loads are issued through inline asm
  // (invisible to the compiler's wait-count pass, which would otherwise wait for the prefetches
  // before every LDS read); the loop waits for them itself.
  const int k_row = lane >> 4, k_pc = lane & 15;
  const int v_row = lane >> 3, v_pc = lane & 7;
  auto issue_tile_k = [&](int kt) {
    const int b = kt % kStages;
    const int64_t kbase = (int64_t)kt * BKV;
    // The tile's key offset stays in the per-lane offset (soffset is not range-checked), so that
    // keys >= Sk of the last tile read as zero.
    u32x4 r_k = r_k_head;
    int64_t key0 = kbase;
    if constexpr (kRebaseK) {
      const int64_t kvalid = a.Sk - kbase < BKV ? a.Sk - kbase : BKV;
      r_k = buffer_rsrc(k_head + kbase * a.k_ss, (uint32_t)(((kvalid - 1) * a.k_ss + 128) * 2));
      key0 = 0;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = wave * 8 + i * 4 + k_row;
      const int c = k_pc ^ (key & 15);
      lds_dma_b128_hot(r_k, (uint32_t)(((key0 + key) * a.k_ss + c * 8) * 2), lds_addr(sK[b] + (wave * 8 + i * 4) * 256));
    }
  };
  auto issue_tile_v = [&](int kt) {
    const int b = kt % kStages;
    const int64_t kbase = (int64_t)kt * BKV;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int d = wave * 16 + i * 8 + v_row;
      const int c = v_pc ^ (d & 7) ^ ((d >> 3) & 1);
      lds_dma_b128_hot(r_v, (uint32_t)((d * a.vt_ld + c * 8) * 2), (uint32_t)(kbase * 2),
                       lds_addr(sV[b] + (wave * 16 + i * 8) * 128));
    }
  };
  auto issue_tile = [&](int kt) {
    issue_tile_k(kt);
    issue_tile_v(kt);
  };
  const int ntiles = (int)((a.Sk + BKV - 1) / BKV);
  // The first three tiles go out before anything else, so their latency overlaps the Q loads.
  issue_tile(0);
  if (ntiles > 1) issue_tile(1);
  if (ntiles > 2) issue_tile(2);

  // ---- Q fragments (B operand): lane holds d = 16t + 8hq .. +7 of query q0 + col, t = 0..7 ----
  // Q through a descriptor based at the wave's first query; rows >= Sq read as zero.
  const int64_t qvalid = a.Sq - q0 < 32 ? (a.Sq - q0 > 0 ? a.Sq - q0 : 0) : 32;
  const __amdgpu_buffer_rsrc_t r_q =
      attn_rsrc(a.q + h * a.q_hs + (qvalid > 0 ? q0 * a.q_ss : 0), qvalid > 0 ? ((qvalid - 1) * a.q_ss + 128) * 2 : 0);
  // fused Q preparation: the query's across-heads 1/rms from its partial sums, in block order.
  // Every load of the prologue (Q, gamma, cos/sin, the partial sums) is issued before any of them is
  // used: issued per fragment and used at once, the loads were eight dependent memory round trips
  // (about 9 us per workgroup, 40% of a cross-attention launch).
  const bool qprep = a.q_sumsq != nullptr || a.q_rr != nullptr;
  const bool qrope = qprep && a.q_cos != nullptr;
  // The head's gamma (128 floats, the same for every query) goes to LDS, one copy per wave so that no
  // barrier is needed before the wave reads it; read per lane from L2 it was 16 loads of 1 KiB per
  // wave through the texture unit, more than the wave's Q itself.
  if (qprep) lds_dma_b128(buffer_rsrc(a.q_gamma + h * 128, 128 * 4), (uint32_t)lane * 16, lds_addr(sgam[wave]));
  const __amdgpu_buffer_rsrc_t r_cs =
      attn_rsrc(qrope ? a.q_cos + (qvalid > 0 ? q0 * 64 : 0) : nullptr, qrope && qvalid > 0 ? qvalid * 64 * 4 : 0);
  const __amdgpu_buffer_rsrc_t r_sn =
      attn_rsrc(qrope ? a.q_sin + (qvalid > 0 ? q0 * 64 : 0) : nullptr, qrope && qvalid > 0 ? qvalid * 64 * 4 : 0);
  u32x4 qv[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    qv[t] = __builtin_amdgcn_raw_buffer_load_b128(r_q, (uint32_t)((col * a.q_ss + 16 * t + 8 * hq) * 2), 0, 0);
  if (qprep) {
    // the RoPE tables only when there is a rotation (the cross-attention query has none)
    u32x4 cv[8], sv[8];
    if (qrope) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        cv[t] = __builtin_amdgcn_raw_buffer_load_b128(r_cs, (uint32_t)((col * 64 + 8 * t + 4 * hq) * 4), 0, 0);
        sv[t] = __builtin_amdgcn_raw_buffer_load_b128(r_sn, (uint32_t)((col * 64 + 8 * t + 4 * hq) * 4), 0, 0);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) cv[t] = sv[t] = u32x4{0u, 0u, 0u, 0u};
    }
    float rr;
    if (a.q_rr != nullptr) {
      // the query's 1/rms, computed once per token by the K pass from the same partials, in the same
      // order, as the branch below (rows past Sq read as zero)
      const __amdgpu_buffer_rsrc_t r_rr = attn_rsrc(a.q_rr + (qvalid > 0 ? q0 : 0), qvalid * 4);
      rr = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_rr, (uint32_t)col * 4, 0, 0));
    } else {
    const __amdgpu_buffer_rsrc_t r_ss = attn_rsrc(a.q_sumsq + (qvalid > 0 ? q0 * a.qss_ld : 0),
                                                  qvalid > 0 ? ((qvalid - 1) * a.qss_ld + a.heads) * 4 : 0);
    float ss = 0.0f;
    if (a.heads <= 40) {
      // Five unconditional loads per lane: the lanes of half hq read blocks 20 hq .. 20 hq + 19 of
      // their query's partials, and a lane swap with lane ^ 32 (which holds the same query's other
      // twenty) gives every lane all forty: v_permlane32_swap of x with itself returns the lower
      // half's value first and the upper half's second in every lane. Blocks past `heads` (another
      // row's partials, or zeros past the extent) are masked to zero and add exactly nothing, so
      // the sum is the block-ordered one.
      u32x4 pv[5];
#pragma unroll
      for (int i = 0; i < 5; ++i)
        pv[i] = __builtin_amdgcn_raw_buffer_load_b128(r_ss, (uint32_t)((col * a.qss_ld + 20 * hq + 4 * i) * 4), 0, 0);
      float lo[20], hi[20];
#pragma unroll
      for (int i = 0; i < 5; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const auto r = __builtin_amdgcn_permlane32_swap(pv[i][j], pv[i][j], false, false);
          lo[4 * i + j] = __uint_as_float(r[0]);
          hi[4 * i + j] = __uint_as_float(r[1]);
        }
#pragma unroll
      for (int b = 0; b < 20; ++b) ss = ss + (b < a.heads ? lo[b] : 0.0f);
#pragma unroll
      for (int b = 0; b < 20; ++b) ss = ss + (20 + b < a.heads ? hi[b] : 0.0f);
    } else {
      for (int b4 = 0; b4 < a.heads; b4 += 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r_ss, (uint32_t)((col * a.qss_ld + b4) * 4), 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = ss + __uint_as_float(v[j]);
      }
    }
    rr = (float)(1.0 / sqrt((double)(ss / (float)(a.heads * 128)) + (double)a.q_eps));
    }
    // every load of the prologue is in (the math below needs them all), the gamma copy included
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    const float4* gl = reinterpret_cast<const float4*>(sgam[wave]);
    // x_hat = bf16((x rrms) gamma), then the pair rotation (a cos - b sin, a sin + b cos) -> bf16:
    // the same operations, in the same order, as the separate Q/K preparation pass
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 ga = gl[4 * t + 2 * hq], gb = gl[4 * t + 2 * hq + 1];
      const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float a0 = (bf16_lo(qv[t][j]) * rr) * gv[2 * j];
        float b0 = (bf16_hi(qv[t][j]) * rr) * gv[2 * j + 1];
        if (qrope) {
          round_bf16_pair(a0, b0);
          const float c = __uint_as_float(cv[t][j]), sn = __uint_as_float(sv[t][j]);
          const float ac = a0 * c, bs = b0 * sn, as = a0 * sn, bc = b0 * c;
          a0 = ac - bs;
          b0 = as + bc;
        }
        qv[t][j] = pack_bf16x2(a0, b0);
      }
    }
  }
  bf16x8 qf[8];
  float qn2 = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bf16_lo(qv[t][j]), hi = bf16_hi(qv[t][j]);
      qn2 = qn2 + lo * lo;
      qn2 = qn2 + hi * hi;
    }
    // the MFMA operand is Q pre-scaled by s log2(e) and rounded to bf16 (the reference pre-scales Q
    // by s before its QK^T as well), so the logits come out in log2 units
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(bf16_lo(qv[t][j]) * a.scale_log2, bf16_hi(qv[t][j]) * a.scale_log2);
    qf[t] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
  }
  qn2 = qn2 + __shfl_xor(qn2, 32, 64);
  // c_i in log2 units: s * ||q_i|| * max||k|| * log2(e), from the unscaled bf16 Q
  const float c2 = a.scale_log2 * sqrtf(qn2) * a.kmax[h];
  f32x16 negc;
#pragma unroll
  for (int r = 0; r < 16; ++r) negc[r] = -c2;

  f32x16 acc_o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[i][r] = 0.0f;
  float lsum = 0.0f;

  // Pipeline over 32-key halves h = 2t + i: step h computes S(h) and the softmax and P V of h-1.
  // Tile t is read by steps 2t .. 2t+2, so when every wave has passed the barrier at the top of tile
  // t, tile t-2's slot is free and tile t+2 is loaded into it (two tiles of prefetch, one barrier per
  // tile). The Q loads were issued after tiles 0-2, so the compiler's waits for them also cover
  // tile 0; the explicit waits below cover the rest.
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  __syncthreads();
  f32x16 s_prev = qk_half(sK[0], 0, qf, negc, col, hq);
  const int sk_rem = (int)(a.Sk - (int64_t)(ntiles - 1) * BKV);  // keys in the last tile (1..64)
  if (ntiles == 1)
    pipeline_step<true, kShortKV>(sK[0], 1, sV[0], 0, qf, negc, s_prev, acc_o, lsum, col, hq, sk_rem);
  else
    pipeline_step<false, kShortKV>(sK[0], 1, sV[0], 0, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
  // Tile t of the steady state (1 <= t < ntiles - 1): outstanding loads are tiles t and t+1 (four
  // per wave each); wait for tile t, publish it, refill tile t-2's slot with tile t+2, then the two
  // pipeline steps of t (`slot` = t % kStages). Tile t+2's K goes out after the barrier and its V^T
  // between the two steps, so that the eight waves' loads reach the texture unit in two bursts
  // rather than one that every wave waits behind. Wave priorities: the two waves of a SIMD (w and
  // w + 4) start the tile together and the older, favoured by the arbiter, gets ahead, then idles
  // at the next barrier while the younger finishes alone. So the first step runs at priority 1 and
  // the older wave drops to 0 for the second while the younger stays at 1: a wave still in its
  // first step wins over one in its second, and the younger wins their second steps, which keeps
  // the pair together, one's exps beside the other's MFMAs. Loads and results are those of the
  // unpartitioned tile (bit-identical).
  auto steady_tile = [&](int t, int slot) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kLoadsPerTile));
    __syncthreads();
    if (t + 2 < ntiles) issue_tile_k(t + 2);
    const int prev = (slot + kStages - 1) % kStages;
    __builtin_amdgcn_s_setprio(1);
    pipeline_step<false, kShortKV>(sK[slot], 0, sV[prev], 1, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
    if (wave < 4) __builtin_amdgcn_s_setprio(0);
    if (t + 2 < ntiles) issue_tile_v(t + 2);
    pipeline_step<false, kShortKV>(sK[slot], 1, sV[slot], 0, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
    __builtin_amdgcn_s_setprio(0);
  };
  for (int t = 1; t < ntiles - 1; ++t) steady_tile(t, t % kStages);
  if (ntiles > 1) {
    const int tl = ntiles - 1;
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    const uint8_t* kc = sK[tl % kStages];
    pipeline_step<false, kShortKV>(kc, 0, sV[(tl - 1) % kStages], 1, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
    pipeline_step<true, kShortKV>(kc, 1, sV[tl % kStages], 0, qf, negc, s_prev, acc_o, lsum, col, hq, sk_rem);
  }
  {  // drain: softmax and P V of the last half
    bf16x8 pf[2];
    softmax_half<true, kShortKV>(s_prev, hq, sk_rem - 32, lsum, pf);
    pv_half(sV[(ntiles - 1) % kStages], 1, pf, acc_o, col, hq);
  }

  // ---- normalize and store ----
  lsum = lsum + __shfl_xor(lsum, 32, 64);
  const float inv = 1.0f / fmaxf(lsum, kSumFloor);
  const int64_t qi = q0 + col;
  const bool qok = qi < a.Sq;
  if (a.row_sum != nullptr && qok && hq == 0) a.row_sum[(int64_t)h * a.Sq + qi] = lsum;
  if (a.out_mode == WANMI_ATTN_OUT_TOKEN) {
    uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + h * a.o_hs + qi * a.o_ss;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = dt * 32 + gi * 8 + hq * 4;
        const float v0 = acc_o[dt][gi * 4] * inv, v1 = acc_o[dt][gi * 4 + 1] * inv;
        const float v2 = acc_o[dt][gi * 4 + 2] * inv, v3 = acc_o[dt][gi * 4 + 3] * inv;
        if (qok) *reinterpret_cast<uint2*>(out + d) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
      }
  } else if (a.out_mode == WANMI_ATTN_OUT_DMAJOR) {
    uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + h * a.o_hs + qi;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dt * 32 + (r >> 2) * 8 + hq * 4 + (r & 3);
        if (qok) out[d * a.o_ds] = (uint16_t)(pack_bf16x2(acc_o[dt][r] * inv, 0.0f) & 0xFFFFu);
      }
  } else {  // MX codes, token-major; a 32-wide block of d is one d tile, split between lane and lane^32
    // Each wave's 32 query rows (128 code bytes each) are staged in LDS and written as whole rows,
    // 16 bytes per lane; written straight from the accumulator layout every store instruction would
    // touch 32 rows with 4 bytes each. The staging slot is that of tile ntiles - 3 (or one never
    // filled), which no wave reads after the last tile's barrier; 16-byte chunks are XOR-swizzled by
    // the row so that the writes and the row reads spread over the banks. A query's four scale bytes
    // (d tiles 0-3) go out as one word.
    uint8_t* stg = (wave < 4 ? sK[(ntiles + 1) % kStages] : sV[(ntiles + 1) % kStages]) + (wave & 3) * 4096;
    uint32_t sw = 0;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      // bf16 pairs; the block's largest exponent field is that of the largest (bits & 0x7fff)
      uint32_t pp[8];
      u16x2_t mag = {0, 0};
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        pp[r / 2] = pack_bf16x2(acc_o[dt][r] * inv, acc_o[dt][r + 1] * inv);
        mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2_t, pp[r / 2] & 0x7FFF7FFFu));
      }
      int e = (int)(max(mag[0], mag[1]) >> 7);
      e = max_with_lane_xor32(e);
      const int sx = max(e - 7, 0);
      const float sc = __uint_as_float((uint32_t)sx << 23);
      sw |= (uint32_t)sx << (8 * dt);
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int d = dt * 32 + gi * 8 + hq * 4;
        const uint32_t c4 = cvt_e4m3x4_scaled(pp[2 * gi], pp[2 * gi + 1], sc);
        *reinterpret_cast<uint32_t*>(stg + col * 128 + ((((d >> 4) ^ (col & 7)) << 4) | (d & 15))) = c4;
      }
    }
    // the MX rows and scales non-temporal, as the GEMMs' outputs (cross-attention 443.6 -> 429.7 us
    // with the caches flushed between launches)
    if (qok && hq == 0) __builtin_nontemporal_store(sw, reinterpret_cast<uint32_t*>(a.out_scales + qi * a.os_ss + h * 4));
    uint8_t* out = reinterpret_cast<uint8_t*>(a.out) + h * a.o_hs;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int qr = it * 8 + (lane >> 3), ch = lane & 7;
      const uint4 v = *reinterpret_cast<const uint4*>(stg + qr * 128 + ((ch ^ (qr & 7)) << 4));
      const int64_t qg = q0 + qr;
      if (qg < a.Sq) __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&v), reinterpret_cast<u32x4*>(out + qg * a.o_ss + ch * 16));
    }
  }
}

// Several heads per workgroup, for short key sequences (cross-attention over the text tokens): with
// 8 key tiles per head, a workgroup that owned one head spent about as long in its prologue (Q, its
// norm inputs and the first K/V tiles, all waited on before the first MFMA) as in its key loop.
// Here one workgroup walks `heads_per_group` consecutive heads of its 256 queries. The tiles of its
// heads form one sequence g = hl * ntiles + kt through the same LDS ring, so the next head's first
// K/V tiles load while the current head finishes; the next head's Q (and gamma) load during the
// current head's drain and output; the queries' across-heads 1/rms, the same for every head, is
// computed once. Per head, the math is that of attention_const_max_kernel<true, false> (the bf16
// row sum of the short-key instantiation) in the same order, so the results are bit-identical.
// Requires ntiles >= 3, no RoPE on Q, K of one head within one descriptor (the host checks).
__global__ __launch_bounds__(kThreads) void attention_head_group_kernel(AttnArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) uint8_t sK[kStages][kTileK];
  __shared__ __attribute__((aligned(16))) uint8_t sV[kStages][kTileV];
  __shared__ __attribute__((aligned(16))) float sgam[kWaves][256];  // each wave's copy of the head's gamma
  __shared__ __attribute__((aligned(16))) uint8_t sStg[4][4096];    // MX output staging of waves 4-7

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hpw = a.heads_per_group;
  const int h_first = blockIdx.y * hpw;
  const int64_t q0 = (int64_t)blockIdx.x * BQ + wave * 32;
  const int col = lane & 31;
  const int hq = lane >> 5;
  const int ntiles = (int)((a.Sk + BKV - 1) / BKV);

  const int k_row = lane >> 4, k_pc = lane & 15;
  const int v_row = lane >> 3, v_pc = lane & 7;
  // Tile kt of the group's head hl into slot (hl * ntiles + kt) % kStages; same lane mapping and
  // descriptors as attention_const_max_kernel, built per tile from the head.
  auto issue_tile = [&](int hl, int kt, int part = 0) {  // part: 0 both, 1 K only, 2 V^T only
    const int b = (hl * ntiles + kt) % kStages;
    const int hd = h_first + hl;
    const u32x4 r_k = buffer_rsrc(a.k + hd * a.k_hs, (uint32_t)(((a.Sk - 1) * a.k_ss + 128) * 2));
    const u32x4 r_v = buffer_rsrc(a.vt + (int64_t)hd * 128 * a.vt_ld, (uint32_t)(128 * a.vt_ld * 2));
    const int64_t kbase = (int64_t)kt * BKV;
    if (part != 2) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int key = wave * 8 + i * 4 + k_row;
        const int c = k_pc ^ (key & 15);
        lds_dma_b128_hot(r_k, (uint32_t)(((kbase + key) * a.k_ss + c * 8) * 2), lds_addr(sK[b] + (wave * 8 + i * 4) * 256));
      }
    }
    if (part == 1) return;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int d = wave * 16 + i * 8 + v_row;
      const int c = v_pc ^ (d & 7) ^ ((d >> 3) & 1);
      lds_dma_b128_hot(r_v, (uint32_t)((d * a.vt_ld + c * 8) * 2), (uint32_t)(kbase * 2),
                       lds_addr(sV[b] + (wave * 16 + i * 8) * 128));
    }
  };
  // tile g + 2 of tile g = (hl, kt), if the group has one (ntiles >= 3: at most one wrap)
  auto issue_ahead = [&](int hl, int kt, int part = 0) {
    int kt2 = kt + 2, hl2 = hl;
    if (kt2 >= ntiles) {
      kt2 -= ntiles;
      ++hl2;
    }
    if (hl2 < hpw) issue_tile(hl2, kt2, part);
  };
  issue_tile(0, 0);
  issue_tile(0, 1);
  issue_tile(0, 2);

  const int64_t qvalid = a.Sq - q0 < 32 ? (a.Sq - q0 > 0 ? a.Sq - q0 : 0) : 32;
  // The wave's 32 query rows of head hd, 256 bytes each. Load t covers rows 8 (t & 3) .. + 7, the
  // 128-byte half t >> 2 of each (lane l: row 8 (t & 3) + (l >> 3), 16-byte chunk l & 7), so one
  // instruction touches eight cache lines; gathered straight into the MFMA's lane layout (lane l
  // holds query l & 31) each touched 32, and the kernel ran 7% longer (at 32760 queries over 512
  // keys). rearrange_q below moves the rows into the lane layout through LDS.
  auto issue_q = [&](int hd, u32x4 (&qv)[8]) {
    const __amdgpu_buffer_rsrc_t r_q = attn_rsrc(a.q + hd * a.q_hs + (qvalid > 0 ? q0 * a.q_ss : 0),
                                                 qvalid > 0 ? ((qvalid - 1) * a.q_ss + 128) * 2 : 0);
    // the lane's part of the offset in one register, recomputed per call (held across the head
    // loop, eight per-lane offsets were spilled and their reloads waited for the K/V loads in
    // flight); the row group and half as the scalar offset
    int l = lane;
    asm volatile("" : "+v"(l));
    const uint32_t voff = (uint32_t)(((l >> 3) * a.q_ss + 8 * (l & 7)) * 2);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      qv[t] = __builtin_amdgcn_raw_buffer_load_b128(r_q, voff, (uint32_t)((8 * (t & 3) * a.q_ss + 64 * (t >> 2)) * 2), 0);
  };
  // The loaded rows into the B-operand layout of the QK^T MFMAs: qv[t] = the 16 bytes of row
  // `col`, k-step t, half hq (row bytes 32 t + 16 hq). One 128-byte half of all 32 rows at a time
  // goes through `qs`, 4 KiB of LDS private to the wave, held as [row][8 chunks] with chunk
  // c ^ ((row >> 1) & 7), which keeps both the writes (two rows of eight chunks per 16 lanes) and the
  // reads (sixteen rows of one chunk) free of bank conflicts. A wave's LDS operations complete in
  // order, so the second half's writes cannot overtake the first half's reads.
  auto rearrange_q = [&](uint8_t* qs, u32x4 (&qv)[8]) {
    int l = lane;
    asm volatile("" : "+v"(l));  // addresses from the lane id per call, as in issue_q
    // write t: row 8 t + (l >> 3), chunk l & 7, whose swizzle (row >> 1) & 7 = 4 (t & 1) | (l >> 4)
    const int wsw = (l & 7) ^ (l >> 4);
    uint8_t* w0 = qs + (l >> 3) * 128 + (wsw << 4);
    uint8_t* w1 = qs + (l >> 3) * 128 + ((wsw ^ 4) << 4);
    // read t: row l & 31, chunk 2 t + (l >> 5)
    const uint8_t* rb = qs + (l & 31) * 128;
    const int rsw = ((l & 31) >> 1) & 7, h = l >> 5;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int t = 0; t < 4; ++t) *reinterpret_cast<u32x4*>((t & 1 ? w1 : w0) + t * 1024) = qv[4 * hf + t];
#pragma unroll
      for (int t = 0; t < 4; ++t) qv[4 * hf + t] = *reinterpret_cast<const u32x4*>(rb + ((((2 * t) | h) ^ rsw) << 4));
    }
  };
  const bool qprep = a.q_sumsq != nullptr || a.q_rr != nullptr;
  auto issue_gamma = [&](int hd) {
    if (qprep) lds_dma_b128(buffer_rsrc(a.q_gamma + hd * 128, 128 * 4), (uint32_t)lane * 16, lds_addr(sgam[wave]));
  };
  issue_gamma(h_first);
  u32x4 qv[8];
  issue_q(h_first, qv);
  // the queries' across-heads 1/rms, from the partial sums in block order (as in
  // attention_const_max_kernel: lane halves read twenty blocks each and swap)
  float rr = 0.0f;
  if (qprep && a.q_rr != nullptr) {
    const __amdgpu_buffer_rsrc_t r_rr = attn_rsrc(a.q_rr + (qvalid > 0 ? q0 : 0), qvalid * 4);
    rr = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_rr, (uint32_t)col * 4, 0, 0));
  } else if (qprep) {
    const __amdgpu_buffer_rsrc_t r_ss = attn_rsrc(a.q_sumsq + (qvalid > 0 ? q0 * a.qss_ld : 0),
                                                  qvalid > 0 ? ((qvalid - 1) * a.qss_ld + a.heads) * 4 : 0);
    float ss = 0.0f;
    if (a.heads <= 40) {
      u32x4 pv[5];
#pragma unroll
      for (int i = 0; i < 5; ++i)
        pv[i] = __builtin_amdgcn_raw_buffer_load_b128(r_ss, (uint32_t)((col * a.qss_ld + 20 * hq + 4 * i) * 4), 0, 0);
      float lo[20], hi[20];
#pragma unroll
      for (int i = 0; i < 5; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const auto r = __builtin_amdgcn_permlane32_swap(pv[i][j], pv[i][j], false, false);
          lo[4 * i + j] = __uint_as_float(r[0]);
          hi[4 * i + j] = __uint_as_float(r[1]);
        }
#pragma unroll
      for (int b = 0; b < 20; ++b) ss = ss + (b < a.heads ? lo[b] : 0.0f);
#pragma unroll
      for (int b = 0; b < 20; ++b) ss = ss + (20 + b < a.heads ? hi[b] : 0.0f);
    } else {
      for (int b4 = 0; b4 < a.heads; b4 += 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r_ss, (uint32_t)((col * a.qss_ld + b4) * 4), 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = ss + __uint_as_float(v[j]);
      }
    }
    rr = (float)(1.0 / sqrt((double)(ss / (float)(a.heads * 128)) + (double)a.q_eps));
  }
  const int sk_rem = (int)(a.Sk - (int64_t)(ntiles - 1) * BKV);

  for (int hl = 0; hl < hpw; ++hl) {
    const int h = h_first + hl;
    const int g0 = hl * ntiles;
    // Loop-invariant per-lane values passed through an empty asm per head: otherwise the compiler
    // hoists every lane's 64-bit output offsets out of the head loop and spills them.
    int64_t o_ss = a.o_ss, o_ds = a.o_ds, os_ss = a.os_ss;
    asm volatile("" : "+s"(o_ss), "+s"(o_ds), "+s"(os_ss));
    // This head's Q and gamma are in once every outstanding load is (tiles g0 and g0 + 1 were
    // issued before them).
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    // Q through the wave's MX staging area (free here: the previous head's staging was read back
    // above, in this wave's LDS order). Waves 0-3 use the K half of a ring slot that no load in
    // flight targets and that no wave reads until this head's first barrier: slot 3 in the first
    // head (tiles 0-2 are in slots 0-2, tile 3 goes out after the barrier of tile 1); later, the slot
    // of tile g0 + 2 (tile g0 - 2's K was read before the barrier of tile g0 - 1; tile g0 + 2 is
    // issued after this head's first barrier).
    rearrange_q(wave < 4 ? sK[hl == 0 ? kStages - 1 : (g0 + 2) % kStages] + wave * 4096 : sStg[wave & 3], qv);
    if (qprep) {
      const float4* gl = reinterpret_cast<const float4*>(sgam[wave]);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float4 ga = gl[4 * t + 2 * hq], gb = gl[4 * t + 2 * hq + 1];
        const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // one rounding to bf16: the pack is the reference's rounding after the norm
          qv[t][j] = pack_bf16x2((bf16_lo(qv[t][j]) * rr) * gv[2 * j], (bf16_hi(qv[t][j]) * rr) * gv[2 * j + 1]);
        }
      }
    }
    bf16x8 qf[8];
    float qn2 = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_lo(qv[t][j]), hi = bf16_hi(qv[t][j]);
        qn2 = qn2 + lo * lo;
        qn2 = qn2 + hi * hi;
      }
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(bf16_lo(qv[t][j]) * a.scale_log2, bf16_hi(qv[t][j]) * a.scale_log2);
      qf[t] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
    }
    qn2 = qn2 + __shfl_xor(qn2, 32, 64);
    const float c2 = a.scale_log2 * sqrtf(qn2) * a.kmax[h];
    f32x16 negc;
#pragma unroll
    for (int r = 0; r < 16; ++r) negc[r] = -c2;
    f32x16 acc_o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[i][r] = 0.0f;
    float lsum = 0.0f;

    // The head's first barrier: after it, the slot of tile g0 + 2 (tile g0 - 2's) is free.
    __syncthreads();
    if (hl > 0) issue_tile(hl, 2);
    const int s0 = g0 % kStages;
    f32x16 s_prev = qk_half(sK[s0], 0, qf, negc, col, hq);
    pipeline_step<false, true>(sK[s0], 1, sV[s0], 0, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
    // steady tiles: outstanding are tiles g and g + 1 (four loads per wave each); as in
    // attention_const_max_kernel, tile g + 2's K goes out after the barrier and its V^T between the
    // steps, and the first step runs at wave priority 1
    for (int t = 1; t < ntiles - 1; ++t) {
      const int slot = (g0 + t) % kStages;
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kLoadsPerTile));
      __syncthreads();
      issue_ahead(hl, t, 1);
      const int prev = (slot + kStages - 1) % kStages;
      __builtin_amdgcn_s_setprio(1);
      pipeline_step<false, true>(sK[slot], 0, sV[prev], 1, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
      __builtin_amdgcn_s_setprio(0);
      issue_ahead(hl, t, 2);
      pipeline_step<false, true>(sK[slot], 1, sV[slot], 0, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
    }
    // the last tile: the next head's tile 0 is outstanding behind it, unless this head is the last
    const int g_last = g0 + ntiles - 1;
    if (hl + 1 < hpw)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kLoadsPerTile));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    issue_ahead(hl, ntiles - 1);
    {
      const uint8_t* kc = sK[g_last % kStages];
      pipeline_step<false, true>(kc, 0, sV[(g_last - 1) % kStages], 1, qf, negc, s_prev, acc_o, lsum, col, hq, 32);
      pipeline_step<true, true>(kc, 1, sV[g_last % kStages], 0, qf, negc, s_prev, acc_o, lsum, col, hq, sk_rem);
    }
    // the next head's Q and gamma load while this head drains and writes its output
    if (hl + 1 < hpw) {
      issue_q(h + 1, qv);
      issue_gamma(h + 1);
    }
    {
      bf16x8 pf[2];
      softmax_half<true, true>(s_prev, hq, sk_rem - 32, lsum, pf);
      pv_half(sV[g_last % kStages], 1, pf, acc_o, col, hq);
    }

    lsum = lsum + __shfl_xor(lsum, 32, 64);
    const float inv = 1.0f / fmaxf(lsum, kSumFloor);
    const int64_t qi = q0 + col;
    const bool qok = qi < a.Sq;
    if (a.row_sum != nullptr && qok && hq == 0) a.row_sum[(int64_t)h * a.Sq + qi] = lsum;
    if (a.out_mode == WANMI_ATTN_OUT_TOKEN) {
      uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + h * a.o_hs + qi * o_ss;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = dt * 32 + gi * 8 + hq * 4;
          const float v0 = acc_o[dt][gi * 4] * inv, v1 = acc_o[dt][gi * 4 + 1] * inv;
          const float v2 = acc_o[dt][gi * 4 + 2] * inv, v3 = acc_o[dt][gi * 4 + 3] * inv;
          if (qok) *reinterpret_cast<uint2*>(out + d) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
        }
    } else if (a.out_mode == WANMI_ATTN_OUT_DMAJOR) {
      uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + h * a.o_hs + qi;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = dt * 32 + (r >> 2) * 8 + hq * 4 + (r & 3);
          if (qok) out[d * o_ds] = (uint16_t)(pack_bf16x2(acc_o[dt][r] * inv, 0.0f) & 0xFFFFu);
        }
    } else {
      // MX rows staged as in attention_const_max_kernel. The staging area must be one that no wave
      // reads after the last tile's barrier and that no load in flight writes: waves 0-3 use the K
      // half of tile g_last - 1's slot (that K was read within tile g_last - 1; the slot's V is
      // still read in tile g_last's first step, and the next head's tiles g_last + 1 and + 2 are in
      // the two other slots; tile g_last + 3 goes into this slot only after the next head's first
      // barrier, which every wave reaches after reading its staging back), waves 4-7 use sStg.
      uint8_t* stg = wave < 4 ? sK[(g_last + kStages - 1) % kStages] + wave * 4096 : sStg[wave & 3];
      uint32_t sw = 0;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        // bf16 pairs; the block's largest exponent field is that of the largest (bits & 0x7fff)
        uint32_t pp[8];
        u16x2_t mag = {0, 0};
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          pp[r / 2] = pack_bf16x2(acc_o[dt][r] * inv, acc_o[dt][r + 1] * inv);
          mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2_t, pp[r / 2] & 0x7FFF7FFFu));
        }
        int e = (int)(max(mag[0], mag[1]) >> 7);
        e = max_with_lane_xor32(e);
        const int sx = max(e - 7, 0);
        const float sc = __uint_as_float((uint32_t)sx << 23);
        sw |= (uint32_t)sx << (8 * dt);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = dt * 32 + gi * 8 + hq * 4;
          const uint32_t c4 = cvt_e4m3x4_scaled(pp[2 * gi], pp[2 * gi + 1], sc);
          *reinterpret_cast<uint32_t*>(stg + col * 128 + ((((d >> 4) ^ (col & 7)) << 4) | (d & 15))) = c4;
        }
      }
      if (qok && hq == 0) __builtin_nontemporal_store(sw, reinterpret_cast<uint32_t*>(a.out_scales + qi * os_ss + h * 4));
      uint8_t* out = reinterpret_cast<uint8_t*>(a.out) + h * a.o_hs;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int qr = it * 8 + (lane >> 3), ch = lane & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(stg + qr * 128 + ((ch ^ (qr & 7)) << 4));
        const int64_t qg = q0 + qr;
        if (qg < a.Sq) __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&v), reinterpret_cast<u32x4*>(out + qg * o_ss + ch * 16));
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Exact-softmax rescue for the constant-max kernels. The bound c_i = s ||q_i|| max_j ||k_j|| can
// exceed the row's true largest logit by so much that every P = exp(s q_i.k_j - c_i) underflows and
// the row sum collapses (c_i - max_j s q_i.k_j beyond about 87): the row then comes out as zero,
// where a running-max flash attention (the reference's attention_cte) gives the softmax. While the
// row sum is at least 2^-96 its largest P is at least 2^-113 for any Sk <= 2^17, a normal float, and
// the P that flush to zero (each below 2^-126) carry less than 2^-13 of the sum: the row is
// accurate. Rows below that (or NaN) are recomputed here, one wave per 64 rows of a head, each
// flagged row in two passes over the keys in fp32: the true max m = max_j s q.k_j, then
// sum_j exp(s q.k_j - m) v_j / sum_j exp(s q.k_j - m). V is read from V^T, whose 16-key groups hold
// key (r & 3) | ((r & 4) << 1) | ((r & 8) >> 1) in slot r (the order wanmi_transpose_heads writes,
// an involution). Only the token-major and d-major bf16 outputs are rewritten.
// ------------------------------------------------------------------------------------------------
constexpr float kRescueSum = 0x1p-96f;

__device__ __forceinline__ int vt_slot_key(int r) { return (r & 3) | ((r & 4) << 1) | ((r & 8) >> 1); }

// s q.k_j for key j of head h: q (already scaled by s) in LDS as 128 floats
__device__ __forceinline__ float rescue_logit(const AttnArgs& a, int h, int64_t j, const float* sq) {
  const uint16_t* kp = a.k + h * a.k_hs + j * a.k_ss;
  float dot = 0.0f;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const uint4 v = *reinterpret_cast<const uint4*>(kp + 8 * c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      dot = fmaf(bf16_lo(w[t]), sq[8 * c + 2 * t], dot);
      dot = fmaf(bf16_hi(w[t]), sq[8 * c + 2 * t + 1], dot);
    }
  }
  return dot;
}

__global__ __launch_bounds__(64) void attention_rescue_kernel(AttnArgs a) {
  __shared__ float sq[128];
  __shared__ float sp[64];
  const int lane = threadIdx.x;
  const int h = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  bool flag = false;
  if (r0 + lane < a.Sq) {
    const float rs = a.row_sum[(int64_t)h * a.Sq + r0 + lane];
    flag = !(rs >= kRescueSum);
  }
  uint64_t pending = __ballot(flag);
  while (pending) {
    const int i = __builtin_ctzll(pending);
    pending &= pending - 1;
    const int64_t qi = r0 + i;
    const uint32_t qw = *reinterpret_cast<const uint32_t*>(a.q + h * a.q_hs + qi * a.q_ss + 2 * lane);
    __syncthreads();  // the previous row is done with sq and sp
    sq[2 * lane] = bf16_lo(qw) * a.scale;
    sq[2 * lane + 1] = bf16_hi(qw) * a.scale;
    __syncthreads();
    float m = -__builtin_inff();
    for (int64_t j = lane; j < a.Sk; j += 64) m = fmaxf(m, rescue_logit(a, h, j, sq));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float o0 = 0.0f, o1 = 0.0f, l = 0.0f;
    const uint16_t* v0row = a.vt + ((int64_t)h * 128 + 2 * lane) * a.vt_ld;
    const uint16_t* v1row = v0row + a.vt_ld;
    for (int64_t j0 = 0; j0 < a.Sk; j0 += 64) {
      const int64_t j = j0 + lane;
      const float p = j < a.Sk ? __expf(rescue_logit(a, h, j, sq) - m) : 0.0f;
      l += p;
      __syncthreads();
      sp[lane] = p;
      __syncthreads();
      // slots j0 .. j0 + 63 of this lane's two V^T rows (vt_ld is a multiple of 64 and >= Sk, so
      // the chunk lies inside the row; keys past Sk have p = 0)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint4 x0 = *reinterpret_cast<const uint4*>(v0row + j0 + 8 * c);
        const uint4 x1 = *reinterpret_cast<const uint4*>(v1row + j0 + 8 * c);
        const uint32_t w0[4] = {x0.x, x0.y, x0.z, x0.w}, w1[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int s0 = 8 * c + 2 * t;  // slot within the chunk
          const float pa = sp[(s0 & ~15) | vt_slot_key(s0 & 15)];
          const float pb = sp[((s0 + 1) & ~15) | vt_slot_key((s0 + 1) & 15)];
          o0 = fmaf(pa, bf16_lo(w0[t]), o0);
          o0 = fmaf(pb, bf16_hi(w0[t]), o0);
          o1 = fmaf(pa, bf16_lo(w1[t]), o1);
          o1 = fmaf(pb, bf16_hi(w1[t]), o1);
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) l += __shfl_xor(l, o, 64);
    const float inv = 1.0f / l;  // l >= 1: the max term is exp(0)
    const uint32_t packed = pack_bf16x2(o0 * inv, o1 * inv);
    uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + h * a.o_hs;
    if (a.out_mode == WANMI_ATTN_OUT_TOKEN) {
      *reinterpret_cast<uint32_t*>(out + qi * a.o_ss + 2 * lane) = packed;
    } else {
      out[qi + (2 * lane) * a.o_ds] = (uint16_t)(packed & 0xFFFFu);
      out[qi + (2 * lane + 1) * a.o_ds] = (uint16_t)(packed >> 16);
    }
  }
}

// max over tokens of the per-head L2 norm of a [S, heads, 128] (strided) bf16 tensor. A token's
// head is 16 lanes (one DPP row, 16 bytes each); a wave takes 4 consecutive tokens per step through a
// descriptor based at its first token (the extent ends at the last valid row, so rows past S read as
// zero and cannot raise the maximum) and issues the loads of 4 steps before reducing any (16 KiB per
// wave in flight); the row sums use DPP moves, no LDS round trips.
__global__ __launch_bounds__(256) void head_max_norm_kernel(const uint16_t* x, int64_t hs, int64_t ss, int64_t S,
                                                            int heads, float* out) {
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint16_t* xh = x + h * hs;
  const uint32_t loff = (uint32_t)(((lane >> 4) * ss + (lane & 15) * 8) * 2);
  float mx = 0.0f;  // max of ||x||^2 (the root taken once at the end: monotone, correctly rounded)
  const int64_t step = (int64_t)gridDim.x * 16;
  for (int64_t wb = (int64_t)blockIdx.x * 16 + wave * 4; wb < S; wb += 4 * step) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t b = wb + u * step;
      const int64_t rows = S - b < 4 ? (S - b > 0 ? S - b : 0) : 4;
      const __amdgpu_buffer_rsrc_t r = attn_rsrc(rows > 0 ? xh + b * ss : xh, rows > 0 ? ((rows - 1) * ss + 128) * 2 : 0);
      v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, loff, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float n2 = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_lo(v[u][j]), hi = bf16_hi(v[u][j]);
        n2 += lo * lo + hi * hi;
      }
      n2 = n2 + dpp_f32<0xB1>(n2);   // quad_perm(1,0,3,2): xor 1
      n2 = n2 + dpp_f32<0x4E>(n2);   // quad_perm(2,3,0,1): xor 2
      n2 = n2 + dpp_f32<0x141>(n2);  // row_half_mirror: xor 4 on uniform quads
      n2 = n2 + dpp_f32<0x140>(n2);  // row_mirror: xor 8 on uniform 8-lane groups
      mx = fmaxf(mx, n2);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (lane == 0) atomicMax(reinterpret_cast<unsigned int*>(out) + h, __float_as_uint(sqrtf(mx)));
}

// The same maximum when a token's heads are contiguous (head stride 128, heads a multiple of 4, at
// most 40): a wave reads whole token rows (heads x 256 bytes, 1 KiB = 4 heads per instruction, all
// loads of two tokens in flight) instead of one head's 256 bytes per token row, so the reads are
// sequential; lane group l >> 4 of chunk c holds head 4 c + (l >> 4). Each wave keeps per-head maxima
// of ||x||^2 in registers; the workgroup reduces them through LDS and issues one atomic per head.
constexpr int kHmnRowWaves = 4;
__global__ __launch_bounds__(256) void head_max_norm_rows_kernel(const uint16_t* x, int64_t ss, int64_t S, int heads,
                                                                 float* out) {
  __shared__ float smax[kHmnRowWaves][40];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nch = heads / 4;
  float kmx[10];
#pragma unroll
  for (int c = 0; c < 10; ++c) kmx[c] = 0.0f;
  const int64_t stride = (int64_t)gridDim.x * kHmnRowWaves;
  for (int64_t t = (int64_t)blockIdx.x * kHmnRowWaves + wave; t < S; t += 2 * stride) {
    u32x4 v[2][10];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t tt = t + u * stride;
      // a second token past S: an empty extent, its loads read zero
      const __amdgpu_buffer_rsrc_t r = attn_rsrc(tt < S ? x + tt * ss : x, tt < S ? heads * 256 : 0);
#pragma unroll
      for (int c = 0; c < 10; ++c)
        v[u][c] = c < nch ? __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, c * 1024, 0) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < 10; ++c) {
        float n2 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = bf16_lo(v[u][c][j]), hi = bf16_hi(v[u][c][j]);
          n2 += lo * lo + hi * hi;
        }
        n2 = n2 + dpp_f32<0xB1>(n2);   // xor 1
        n2 = n2 + dpp_f32<0x4E>(n2);   // xor 2
        n2 = n2 + dpp_f32<0x141>(n2);  // xor 4 on uniform quads
        n2 = n2 + dpp_f32<0x140>(n2);  // xor 8 on uniform 8-lane groups
        kmx[c] = fmaxf(kmx[c], n2);
      }
  }
  if ((lane & 15) == 0) {
#pragma unroll
    for (int c = 0; c < 10; ++c)
      if (c < nch) smax[wave][4 * c + (lane >> 4)] = kmx[c];
  }
  __syncthreads();
  const int hd = threadIdx.x;
  if (hd < heads) {
    float m = smax[0][hd];
#pragma unroll
    for (int w = 1; w < kHmnRowWaves; ++w) m = fmaxf(m, smax[w][hd]);
    atomicMax(reinterpret_cast<unsigned int*>(out) + hd, __float_as_uint(sqrtf(m)));
  }
}

__global__ void attn_zero_kernel(float* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

}  // namespace wanmi

extern "C" int wanmi_head_max_norm(const void* x, int64_t head_stride, int64_t token_stride, int64_t S,
                                   int heads, float* out, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(S >= 0 && heads > 0 && heads <= 65535, WANMI_ERR_ARG, "wanmi_head_max_norm: bad S/heads");
  WANMI_REQUIRE(out, WANMI_ERR_ARG, "wanmi_head_max_norm: out must not be null");
  WANMI_REQUIRE(head_stride % 8 == 0 && token_stride % 8 == 0, WANMI_ERR_ARG,
                "wanmi_head_max_norm: strides must be multiples of 8 elements");
  WANMI_REQUIRE(S <= 1 || token_stride >= 128, WANMI_ERR_ARG,
                "wanmi_head_max_norm: token_stride=%lld must be >= 128 (tokens' head rows may not overlap)",
                (long long)token_stride);
  WANMI_REQUIRE((3 * token_stride + 128) * 2 < (1LL << 31), WANMI_ERR_UNSUPPORTED,
                "wanmi_head_max_norm: token_stride too large");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(attn_zero_kernel, dim3((heads + 255) / 256), dim3(256), 0, s, out, heads);
  int st = check_launch("wanmi_head_max_norm(zero)");
  if (st || S == 0) return st;
  WANMI_REQUIRE(x && ((uintptr_t)x % 16) == 0, WANMI_ERR_ARG, "wanmi_head_max_norm: x must be 16-byte aligned");
  if (head_stride == 128 && heads % 4 == 0 && heads <= 40 && token_stride >= heads * 128) {
    // heads contiguous within a token: whole rows per wave (two tokens per step, so 8 per workgroup)
    const int64_t blocks = min((S + 2 * kHmnRowWaves - 1) / (2 * kHmnRowWaves), (int64_t)1024);
    hipLaunchKernelGGL(head_max_norm_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const uint16_t*>(x), token_stride, S, heads, out);
    return check_launch("wanmi_head_max_norm");
  }
  const int64_t blocks = min((S + 15) / 16, (int64_t)256);
  hipLaunchKernelGGL(head_max_norm_kernel, dim3((unsigned)blocks, (unsigned)heads), dim3(256), 0, s,
                     static_cast<const uint16_t*>(x), head_stride, token_stride, S, heads, out);
  return check_launch("wanmi_head_max_norm");
}

namespace wanmi {
struct QPrep {
  const float* rr = nullptr;  // per-query 1/rms (in place of sumsq)
  const float* sumsq = nullptr;
  int64_t ld = 0;
  const float* gamma = nullptr;
  const float* cos = nullptr;
  const float* sin = nullptr;
  float eps = 0.0f;
};

static int attention_impl(const void* q, int64_t q_head_stride, int64_t q_token_stride, const void* k,
                          int64_t k_head_stride, int64_t k_token_stride, const void* vt, int64_t vt_ld,
                          const float* kmax, int64_t Sq, int64_t Sk, int heads, int head_dim, float scale,
                          int out_mode, void* out, int64_t o_head_stride, int64_t o_token_stride,
                          int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride, const QPrep& qp,
                          void* stream, float* row_sum = nullptr) {
  WANMI_REQUIRE(head_dim == 128, WANMI_ERR_UNSUPPORTED, "wanmi_attention_const_max: head_dim must be 128, got %d",
                head_dim);
  WANMI_REQUIRE(Sq >= 0 && Sk > 0 && heads > 0 && heads <= 65535, WANMI_ERR_ARG,
                "wanmi_attention_const_max: bad sizes Sq=%lld Sk=%lld heads=%d", (long long)Sq, (long long)Sk, heads);
  WANMI_REQUIRE(out_mode >= WANMI_ATTN_OUT_TOKEN && out_mode <= WANMI_ATTN_OUT_MX, WANMI_ERR_ARG,
                "wanmi_attention_const_max: unknown out_mode %d", out_mode);
  WANMI_REQUIRE(vt_ld >= Sk && vt_ld % 64 == 0, WANMI_ERR_ARG,
                "wanmi_attention_const_max: vt_ld=%lld must be >= Sk and a multiple of 64", (long long)vt_ld);
  WANMI_REQUIRE(q_token_stride % 8 == 0 && k_token_stride % 8 == 0 && q_head_stride % 8 == 0 && k_head_stride % 8 == 0,
                WANMI_ERR_ARG, "wanmi_attention_const_max: q/k strides must be multiples of 8 elements");
  WANMI_REQUIRE(!(scale <= 0.0f), WANMI_ERR_ARG, "wanmi_attention_const_max: scale must be > 0");
  if (Sq == 0) return WANMI_OK;
  WANMI_REQUIRE(q && k && vt && kmax && out, WANMI_ERR_ARG, "wanmi_attention_const_max: null pointer");
  WANMI_REQUIRE(out_mode != WANMI_ATTN_OUT_MX || out_scales, WANMI_ERR_ARG,
                "wanmi_attention_const_max: MX output needs out_scales");
  // MX rows are written 16 bytes at a time and a query's four scale bytes as one word
  WANMI_REQUIRE(out_mode != WANMI_ATTN_OUT_MX ||
                    (((uintptr_t)out % 16) == 0 && o_head_stride % 16 == 0 && o_token_stride % 16 == 0 &&
                     ((uintptr_t)out_scales % 4) == 0 && os_token_stride % 4 == 0),
                WANMI_ERR_ARG, "wanmi_attention_const_max: MX output needs 16-byte aligned rows and 4-byte aligned scales");
  // descriptors cover one wave's 32 queries, one 64-key tile, one head of V^T
  WANMI_REQUIRE((31 * q_token_stride + 128) * 2 < (1LL << 31) && (63 * k_token_stride + 128) * 2 < (1LL << 31) &&
                    128 * vt_ld * 2 < (1LL << 31),
                WANMI_ERR_UNSUPPORTED, "wanmi_attention_const_max: strides too large for 32-bit buffer offsets");
  WANMI_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)vt % 16) == 0,
                WANMI_ERR_ARG, "wanmi_attention_const_max: q/k/vt must be 16-byte aligned");
  AttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_hs = q_head_stride;
  a.q_ss = q_token_stride;
  a.k = static_cast<const uint16_t*>(k);
  a.k_hs = k_head_stride;
  a.k_ss = k_token_stride;
  a.vt = static_cast<const uint16_t*>(vt);
  a.vt_ld = vt_ld;
  a.kmax = kmax;
  a.Sq = Sq;
  a.Sk = Sk;
  a.heads = heads;
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out_mode = out_mode;
  a.out = out;
  a.o_hs = o_head_stride;
  a.o_ss = o_token_stride;
  a.o_ds = o_d_stride;
  a.out_scales = out_scales;
  a.os_ss = os_token_stride;
  a.q_sumsq = qp.sumsq;
  a.q_rr = qp.rr;
  a.qss_ld = qp.ld;
  a.q_gamma = qp.gamma;
  a.q_cos = qp.cos;
  a.q_sin = qp.sin;
  a.q_eps = qp.eps;
  a.row_sum = row_sum;
  const dim3 grid((unsigned)((Sq + BQ - 1) / BQ), (unsigned)heads);
  const bool rebase_k = ((Sk - 1) * k_token_stride + 128) * 2 >= (1LL << 31);
  // Short key sequences of three tiles or more with queries that take no RoPE (cross-attention):
  // several heads per workgroup (cross_heads_per_group; one head per workgroup when `heads` has no
  // divisor from 2 up).
  int hpw = 1;
  if (Sk <= 1024 && Sk > 2 * BKV && qp.cos == nullptr && !rebase_k) {
    const int cus = device_cu_count();
    hpw = cross_heads_per_group((int64_t)grid.x, heads, cus > 0 ? cus : 256);
  }
  a.heads_per_group = hpw;
  if (hpw > 1)
    hipLaunchKernelGGL(attention_head_group_kernel, dim3(grid.x, (unsigned)(heads / hpw)), dim3(kThreads), 0,
                       (hipStream_t)stream, a);
  else if (Sk <= 1024)
    hipLaunchKernelGGL(HIP_KERNEL_NAME(attention_const_max_kernel<true, false>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, a);
  else if (!rebase_k)
    hipLaunchKernelGGL(HIP_KERNEL_NAME(attention_const_max_kernel<false, false>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(HIP_KERNEL_NAME(attention_const_max_kernel<false, true>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, a);
  return check_launch("wanmi_attention_const_max");
}
}  // namespace wanmi

extern "C" int wanmi_attention_const_max(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                         const void* k, int64_t k_head_stride, int64_t k_token_stride,
                                         const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq,
                                         int64_t Sk, int heads, int head_dim, float scale, int out_mode,
                                         void* out, int64_t o_head_stride, int64_t o_token_stride,
                                         int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride,
                                         void* stream) {
  wanmi::clear_error();
  return wanmi::attention_impl(q, q_head_stride, q_token_stride, k, k_head_stride, k_token_stride, vt, vt_ld, kmax, Sq,
                               Sk, heads, head_dim, scale, out_mode, out, o_head_stride, o_token_stride, o_d_stride,
                               out_scales, os_token_stride, wanmi::QPrep{}, stream);
}

extern "C" int wanmi_attention_const_max_qrr(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                             const void* k, int64_t k_head_stride, int64_t k_token_stride,
                                             const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq,
                                             int64_t Sk, int heads, int head_dim, float scale, int out_mode,
                                             void* out, int64_t o_head_stride, int64_t o_token_stride,
                                             int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride,
                                             const float* q_rr, const float* q_gamma, const float* q_cos,
                                             const float* q_sin, void* stream) {
  using namespace wanmi;
  clear_error();
  // (no queries: an empty q_rr may have no storage)
  WANMI_REQUIRE((Sq == 0 || q_rr) && q_gamma, WANMI_ERR_ARG,
                "wanmi_attention_const_max_qrr: q_rr and q_gamma are required");
  WANMI_REQUIRE((q_cos == nullptr) == (q_sin == nullptr), WANMI_ERR_ARG,
                "wanmi_attention_const_max_qrr: q_cos and q_sin must both be given or both be null");
  WANMI_REQUIRE(((uintptr_t)q_rr % 4) == 0 && ((uintptr_t)q_gamma % 16) == 0 &&
                    (!q_cos || (((uintptr_t)q_cos % 16) == 0 && ((uintptr_t)q_sin % 16) == 0)),
                WANMI_ERR_ARG, "wanmi_attention_const_max_qrr: q_rr must be 4-byte, q_gamma, q_cos, q_sin 16-byte aligned");
  QPrep qp;
  qp.rr = q_rr;
  qp.gamma = q_gamma;
  qp.cos = q_cos;
  qp.sin = q_sin;
  return attention_impl(q, q_head_stride, q_token_stride, k, k_head_stride, k_token_stride, vt, vt_ld, kmax, Sq, Sk,
                        heads, head_dim, scale, out_mode, out, o_head_stride, o_token_stride, o_d_stride, out_scales,
                        os_token_stride, qp, stream);
}

extern "C" int wanmi_attention_const_max_qprep(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                               const void* k, int64_t k_head_stride, int64_t k_token_stride,
                                               const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq,
                                               int64_t Sk, int heads, int head_dim, float scale, int out_mode,
                                               void* out, int64_t o_head_stride, int64_t o_token_stride,
                                               int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride,
                                               const float* q_sumsq, int64_t q_sumsq_ld, const float* q_gamma,
                                               const float* q_cos, const float* q_sin, float q_eps, void* stream) {
  using namespace wanmi;
  clear_error();
  // (no queries: an empty q_sumsq may have no storage)
  WANMI_REQUIRE((Sq == 0 || q_sumsq) && q_gamma, WANMI_ERR_ARG,
                "wanmi_attention_const_max_qprep: q_sumsq and q_gamma are required");
  WANMI_REQUIRE((q_cos == nullptr) == (q_sin == nullptr), WANMI_ERR_ARG,
                "wanmi_attention_const_max_qprep: q_cos and q_sin must both be given or both be null");
  WANMI_REQUIRE(heads % 4 == 0 && q_sumsq_ld >= heads && q_sumsq_ld % 4 == 0, WANMI_ERR_ARG,
                "wanmi_attention_const_max_qprep: need heads %% 4 == 0 and q_sumsq_ld >= heads, a multiple of 4 "
                "(heads=%d, ld=%lld)", heads, (long long)q_sumsq_ld);
  WANMI_REQUIRE(!(q_eps < 0.0f), WANMI_ERR_ARG, "wanmi_attention_const_max_qprep: eps must be >= 0");
  WANMI_REQUIRE(((uintptr_t)q_sumsq % 16) == 0 && ((uintptr_t)q_gamma % 16) == 0 &&
                    (!q_cos || (((uintptr_t)q_cos % 16) == 0 && ((uintptr_t)q_sin % 16) == 0)),
                WANMI_ERR_ARG, "wanmi_attention_const_max_qprep: q_sumsq, q_gamma, q_cos, q_sin must be 16-byte aligned");
  WANMI_REQUIRE((31 * q_sumsq_ld + heads) * 4 < (1LL << 31), WANMI_ERR_UNSUPPORTED,
                "wanmi_attention_const_max_qprep: q_sumsq_ld too large");
  QPrep qp;
  qp.sumsq = q_sumsq;
  qp.ld = q_sumsq_ld;
  qp.gamma = q_gamma;
  qp.cos = q_cos;
  qp.sin = q_sin;
  qp.eps = q_eps;
  return attention_impl(q, q_head_stride, q_token_stride, k, k_head_stride, k_token_stride, vt, vt_ld, kmax, Sq, Sk,
                        heads, head_dim, scale, out_mode, out, o_head_stride, o_token_stride, o_d_stride, out_scales,
                        os_token_stride, qp, stream);
}

namespace wanmi {
// Row sums of the allocation-free exact attention (wanmi_attention_exact_noalloc): one fp32 per
// (head, query), at most kNoAllocRowSums = 4M of them (16 MiB, held on every GPU the library runs
// on until the process ends). In host code `scratch` names a host-side stand-in, not a device
// address; the device copy's address comes from hipGetSymbolAddress, once per device.
constexpr int64_t kNoAllocRowSums = int64_t(1) << 22;
static __device__ __align__(256) float scratch[kNoAllocRowSums];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static float* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch`, looked up at the first call on the device (with it current).
static int scratch_for_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  WANMI_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices, WANMI_ERR_HIP,
                "wanmi_attention_exact_noalloc: no current device (%s)", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    WANMI_REQUIRE(e == hipSuccess && ptr != nullptr, WANMI_ERR_HIP,
                  "wanmi_attention_exact_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return WANMI_OK;
}
}  // namespace wanmi

extern "C" int wanmi_attention_exact(const void* q, int64_t q_head_stride, int64_t q_token_stride, const void* k,
                                     int64_t k_head_stride, int64_t k_token_stride, const void* vt, int64_t vt_ld,
                                     const float* kmax, int64_t Sq, int64_t Sk, int heads, int head_dim, float scale,
                                     int out_mode, void* out, int64_t o_head_stride, int64_t o_token_stride,
                                     int64_t o_d_stride, float* row_sum, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(out_mode == WANMI_ATTN_OUT_TOKEN || out_mode == WANMI_ATTN_OUT_DMAJOR, WANMI_ERR_ARG,
                "wanmi_attention_exact: out_mode %d must be token-major or d-major bf16", out_mode);
  WANMI_REQUIRE((Sq == 0 || row_sum) && ((uintptr_t)row_sum % 4) == 0, WANMI_ERR_ARG,
                "wanmi_attention_exact: row_sum must be a 4-byte aligned [heads][Sq] buffer");
  WANMI_REQUIRE(out_mode != WANMI_ATTN_OUT_TOKEN || (((uintptr_t)out % 4) == 0 && o_head_stride % 2 == 0 &&
                                                     o_token_stride % 2 == 0),
                WANMI_ERR_ARG, "wanmi_attention_exact: token-major output rows must be 4-byte aligned");
  WANMI_REQUIRE(vt_ld % 64 == 0 && ((uintptr_t)vt % 16) == 0 && ((uintptr_t)k % 16) == 0 &&
                    k_token_stride % 8 == 0 && k_head_stride % 8 == 0 && ((uintptr_t)q % 4) == 0 &&
                    q_token_stride % 2 == 0 && q_head_stride % 2 == 0,
                WANMI_ERR_ARG, "wanmi_attention_exact: misaligned q/k/vt");
  int st = attention_impl(q, q_head_stride, q_token_stride, k, k_head_stride, k_token_stride, vt, vt_ld, kmax, Sq, Sk,
                          heads, head_dim, scale, out_mode, out, o_head_stride, o_token_stride, o_d_stride, nullptr, 0,
                          QPrep{}, stream, row_sum);
  if (st != WANMI_OK || Sq == 0) return st;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_hs = q_head_stride;
  a.q_ss = q_token_stride;
  a.k = static_cast<const uint16_t*>(k);
  a.k_hs = k_head_stride;
  a.k_ss = k_token_stride;
  a.vt = static_cast<const uint16_t*>(vt);
  a.vt_ld = vt_ld;
  a.Sq = Sq;
  a.Sk = Sk;
  a.heads = heads;
  a.scale = scale;
  a.out_mode = out_mode;
  a.out = out;
  a.o_hs = o_head_stride;
  a.o_ss = o_token_stride;
  a.o_ds = o_d_stride;
  a.row_sum = row_sum;
  hipLaunchKernelGGL(attention_rescue_kernel, dim3((unsigned)((Sq + 63) / 64), (unsigned)heads), dim3(64), 0,
                     (hipStream_t)stream, a);
  return check_launch("wanmi_attention_exact(rescue)");
}

extern "C" int wanmi_attention_exact_noalloc(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                             const void* k, int64_t k_head_stride, int64_t k_token_stride,
                                             const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq, int64_t Sk,
                                             int heads, int head_dim, float scale, int out_mode, void* out,
                                             int64_t o_head_stride, int64_t o_token_stride, int64_t o_d_stride,
                                             void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(heads > 0 && Sq >= 0 && (int64_t)heads * Sq <= kNoAllocRowSums, WANMI_ERR_ARG,
                "wanmi_attention_exact_noalloc: heads * Sq = %lld row sums exceed the %lld the library holds",
                (long long)heads * (long long)Sq, (long long)kNoAllocRowSums);
  float* row_sum = nullptr;
  const int st = scratch_for_current_device(&row_sum);
  if (st != WANMI_OK) return st;
  return wanmi_attention_exact(q, q_head_stride, q_token_stride, k, k_head_stride, k_token_stride, vt, vt_ld, kmax,
                               Sq, Sk, heads, head_dim, scale, out_mode, out, o_head_stride, o_token_stride, o_d_stride,
                               row_sum, stream);
}
