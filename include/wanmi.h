/*
 * wanmi.h - C ABI of the gfx950 (MI355X) Wan2.2 DiT-block hot-path library (libwanmi.so).
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise; the caller owns every buffer.
 *     No entry point allocates device memory except where a comment says so.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream). Work is enqueued
 *     asynchronously on that stream; nothing synchronizes.
 *   - bf16 tensors are passed as void* (raw 16-bit storage), e4m3fn codes and e8m0 scales as
 *     uint8_t*, fp32 vectors as float*.
 *   - Return value: WANMI_OK (0) or a negative WANMI_ERR_* code; wanmi_last_error() then returns a
 *     message for the calling thread.
 *
 * The reference these entry points replace is the Trainium plugin reecedantin/vllm-omni-neuron;
 * each declaration cites the reference interface it stands in for.
 */
#ifndef WANMI_H_
#define WANMI_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WANMI_ABI_VERSION 3

#define WANMI_OK 0
#define WANMI_ERR_ARG (-1)         /* bad pointer / size / enum argument */
#define WANMI_ERR_UNSUPPORTED (-2) /* valid request this build does not support */
#define WANMI_ERR_HIP (-3)         /* HIP runtime error while launching */

/* Normalization selector (reference NormType: LAYER_NORM / RMS_NORM / NO_NORM,
 * vllm_omni_neuron/kernels/nkilib/core/utils/common_types.py). */
#define WANMI_NORM_NONE 0
#define WANMI_NORM_LAYER 1
#define WANMI_NORM_RMS 2

/* Output quantization selector (reference QuantizationType NONE / ROW, plus MX). */
#define WANMI_QUANT_NONE 0 /* bf16 [T,H] */
#define WANMI_QUANT_MX 1   /* e4m3fn codes [T,H] + e8m0 scales [T,H/32], shared exponent = max - 7 */
#define WANMI_QUANT_ROW 2  /* packed [T,H+4]: e4m3fn codes then the row's fp32 dequant scale */

int wanmi_abi_version(void);
const char* wanmi_last_error(void);

/*
 * Fused adaptive LayerNorm + quantization, one HBM pass per row.
 *   x = hidden                                   (residual == NULL)
 *   x = bf16(residual + gate * hidden)           (residual != NULL; gate may be NULL -> plain add;
 *                                                 written to residual_out)
 *   y = bf16(Norm(x) * mul + add)                (mul / add may be NULL)
 *   out = y (bf16) | MX(y) | ROW(y)
 * hidden, residual, residual_out: bf16 [T,H]; gate, mul, add: fp32 [H].
 * out: bf16 [T,H] (NONE), e4m3fn [T,H] (MX, with scales [T,H/32]) or uint8 [T,H+4] (ROW).
 * Row statistics are fp32 sums in one fixed order (each of 64 lanes sums its columns 512c + 8l .. 8l+7
 * of every 512-column chunk c in sequence, then an xor butterfly over the lanes; two-pass mean and
 * variance; rstd = fp32(1 / sqrt(fp64(var) + eps))), so the bits do not depend on the launch.
 * Requires H % 32 == 0 and H <= 16384.
 * Replaces adaln_quant_kernel (vllm_omni_neuron/kernels/nkilib/experimental/norm/adaln_quant.py:117)
 * as launched by adaln_modulate (vllm_omni_neuron/diffusion/quantization/adaln_kernels.py:87).
 */
int wanmi_adaln_quant(const void* hidden, const void* residual, const float* gate, const float* mul,
                      const float* add, int64_t T, int64_t H, float eps, int norm_type,
                      int quant_type, void* out, uint8_t* scales, void* residual_out, void* stream);

/* Epilogue selector of wanmi_mxfp8_gemm. */
#define WANMI_EPI_BF16 0             /* out = bf16(acc * rs * cs + bias) */
#define WANMI_EPI_GELU_MX 1          /* out, out_scales = MX(bf16(gelu_tanh(acc * rs * cs + bias))) */
#define WANMI_EPI_GELU_BF16 2        /* out = bf16(gelu_tanh(acc * rs * cs + bias)) */
#define WANMI_EPI_GATED_RESIDUAL 3   /* out = bf16(residual + bf16(acc * rs * cs + bias) * gate) */

/*
 * MXFP8 block-scaled GEMM with fused epilogue:
 *   acc[m,n] = sum_k A[m,k] 2^(a_scales[m,k/32]-127) * W[n,k] 2^(w_scales[n,k/32]-127)   (fp32)
 * a_codes: e4m3fn [M, lda] (row stride lda >= K, lda % 16 == 0); a_scales: e8m0 [M, K/32];
 * w_codes: e4m3fn [N, K] (the weight transposed, K-contiguous); w_scales: e8m0 [N, K/32];
 * row_scale [M], col_scale [N], bias [N], gate [N]: fp32, each optional except as the epilogue
 * needs (row/col scales give the reference's ROW_MX dequant with neutral 127 block scales);
 * out: bf16 or e4m3fn [M, ldo]; out_scales: e8m0 [M, N/32] (GELU_MX); residual: bf16 [M, ldo].
 * Requires N % 256 == 0, K % 128 == 0, 256 * K and 256 * lda below 2^31, M * ldo below 2^32 and
 * ldo below 2^22 (32-bit buffer offsets).
 * Replaces the ROW_MX projection kernels behind row_mx_qkv_proj / row_mx_o_proj / row_mx_mlp
 * (vllm_omni_neuron/diffusion/quantization/row_mx_kernels.py:48-198): _qkv_cte_mx_impl
 * (kernels/nkilib/core/qkv/qkv_cte.py:2725) and mlp_cte_mx (kernels/nkilib/core/mlp/mlp_cte/mx/).
 */
int wanmi_mxfp8_gemm(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                     const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                     const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda, int epilogue,
                     void* out, int64_t ldo, uint8_t* out_scales, const void* residual,
                     const float* gate, void* stream);

/*
 * wanmi_mxfp8_gemm with the bf16 epilogue, which also writes per-row partial sums of squares of
 * the bf16 outputs: row_sumsq[m * (N/128) + b] = sum over the 128 columns of block b of out[m, c]^2
 * (fp32), for the blocks of columns [0, sumsq_cols) (sumsq_cols % 128 == 0). The across-heads
 * RMSNorm of the projected Q then needs no pass over Q: the attention kernel's Q load sums the
 * row's partials (wanmi_attention_const_max_qprep). Replaces the sum of squares the reference's
 * QKV kernel takes from its bf16 output tile (kernels/nkilib/core/qkv/qkv_cte.py:3781-3801).
 */
int wanmi_mxfp8_gemm_rowsumsq(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                              const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                              const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda,
                              void* out, int64_t ldo, float* row_sumsq, int64_t sumsq_cols,
                              void* stream);

/* Channel pairs the RoPE rotation of wanmi_qk_rmsnorm_rope acts on, within each head of 128. */
#define WANMI_ROTATE_INTERLEAVED 0 /* pair i = channels (2i, 2i+1): Wan's apply_rotary_emb_wan */
#define WANMI_ROTATE_HALVES 1      /* pair i = channels (i, i+64): rotate-half on channels de-interleaved
                                      per head (the reference's fused QKV kernel layout) */

/*
 * The fused [Q | K | V] projection in the attention's layouts: wanmi_mxfp8_gemm with the bf16
 * epilogue on the columns [0, vt_col0) -- Q and K, into out (ldo >= vt_col0), with optional per-row
 * partial sums of squares of the columns [0, sumsq_cols) in row_sumsq [M, vt_col0/128] as
 * wanmi_mxfp8_gemm_rowsumsq writes them -- while the columns [vt_col0, N) -- V -- go to vt as V^T
 * [(N - vt_col0)/128 heads][128][vt_ld] bf16 in the key order of wanmi_transpose_heads (inside each
 * group of 16 keys: 0-3, 8-11, 4-7, 12-15), zero for tokens M .. vt_ld - 1. vt_col0 and N - vt_col0
 * are multiples of 256; M > 0; M <= vt_ld <= M rounded up to 256 (the V launch writes every token
 * column of the 256-token tiles it covers, zeros past M), vt_ld % 64 == 0. Two launches on `stream` (Q|K, then V, whose
 * MFMAs take the token operand first so that four consecutive tokens of a feature are lane-local).
 * Replaces the QKV kernel of row_mx_qkv_proj (vllm_omni_neuron/diffusion/quantization/
 * row_mx_kernels.py:48-111, kernels/nkilib/core/qkv/qkv_cte.py:2725) together with the V transpose
 * the reference's attention kernels do internally (ring_attention_const_max_fwd.py:1180-1220).
 */
int wanmi_mxfp8_gemm_qkv(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                         const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                         const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda, void* out,
                         int64_t ldo, float* row_sumsq, int64_t sumsq_cols, void* vt, int64_t vt_col0,
                         int64_t vt_ld, void* stream);

/*
 * Across-heads RMSNorm + optional 3D RoPE, in place on a bf16 [S, heads*128] slab (row stride ld
 * elements):  x = bf16(x * rrms * gamma), rrms = 1/sqrt(mean_row(x^2) + eps); then per pair (a, b)
 * of each head (rope_pairs selects which channels pair): (a, b) -> bf16(a cos - b sin),
 * bf16(a sin + b cos) with cos_tab / sin_tab fp32 [S, 64] (angle i of pair i; both NULL = no RoPE).
 * gamma: fp32 [heads*128] in the slab's channel order.
 * maxnorm (optional, fp32 [heads]) receives max over tokens of each head's L2 norm of the output.
 * Replaces DistributedRMSNorm + apply_rotary_emb_wan (vllm_omni_neuron/diffusion/models/wan2_2/
 * wan2_2_transformer.py:879-893, diffusion/layers/rope.py:8-34) and the fused across-heads norm +
 * RoPE epilogue of the QKV kernel (kernels/nkilib/core/qkv/qkv_cte.py:3781-3990).
 */
int wanmi_qk_rmsnorm_rope(void* x, int64_t S, int64_t ld, int heads, const float* gamma,
                          const float* cos_tab, const float* sin_tab, int rope_pairs, float eps,
                          float* maxnorm, void* stream);

/*
 * wanmi_qk_rmsnorm_rope that also writes the queries' across-heads 1/rms for the attention's fused Q
 * preparation: q_rr[t] = 1 / sqrt(sum_b q_sumsq[t * q_sumsq_ld + b] / (q_heads * 128) + q_eps), the
 * sum taken in fp32 over the blocks b = 0 .. q_heads-1 in order and the root in fp64 (exactly what
 * wanmi_attention_const_max_qprep computes from the same partials). The K pass runs between the QKV
 * projection and the attention anyway; computed here once per token, the 1/rms costs the attention
 * one load per query (wanmi_attention_const_max_qrr) instead of q_heads per head. Replaces the same
 * reference interfaces as wanmi_qk_rmsnorm_rope.
 */
int wanmi_qk_rmsnorm_rope_qrr(void* x, int64_t S, int64_t ld, int heads, const float* gamma, const float* cos_tab,
                              const float* sin_tab, int rope_pairs, float eps, float* maxnorm, const float* q_sumsq,
                              int64_t q_sumsq_ld, int q_heads, float q_eps, float* q_rr, void* stream);

/* Table layouts of wanmi_rope_tables (per token s, fp32). */
#define WANMI_ROPE_PAIRS 0       /* [S, head_dim/2]: angle i of pair i (the kernels' own tables) */
#define WANMI_ROPE_INTERLEAVED 1 /* [S, head_dim]: each angle twice, (c0, c0, c1, c1, ...) -- the
                                    reference's freqs_cos / freqs_sin [1, S, 1, head_dim] */
#define WANMI_ROPE_ROTATE_HALF 2 /* [S, head_dim]: cat([base, base]) -- the rotate-half caches */

/*
 * Wan 3D rotary tables for a latent patch grid (frames, height, width), S = frames*height*width
 * tokens in raster order: the head's pairs split into time / height / width axes of
 * head_dim - 2*(2*(head_dim/6)), 2*(head_dim/6), 2*(head_dim/6) channels; pair j of an axis of dim d
 * at position p has the angle p / theta^(2j/d) (fp64), written as fp32 cos and sin.
 * frames, height, width <= max_seq_len (the reference's table length). cos_out / sin_out as the
 * layout says. Replaces WanRotaryPosEmbed (vllm_omni_neuron/diffusion/layers/rope.py:37-114), called
 * once per forward at diffusion/models/wan2_2/wan2_2_transformer.py:1757; the rotate-half layout is
 * _rope_rotate_half_caches (diffusion/quantization/row_mx_modules.py:51-76).
 */
int wanmi_rope_tables(int64_t frames, int64_t height, int64_t width, int head_dim, int64_t max_seq_len,
                      double theta, int layout, float* cos_out, float* sin_out, void* stream);

/*
 * V bf16, element (s, h, d) at v[s*ld + h*head_stride + d] (token-major: head_stride = 128;
 * head-major [heads, S, 128]: ld = 128, head_stride = S*128) -> V^T [heads, 128, S_pad] bf16, keys stored inside each
 * group of 16 in the order (0-3, 8-11, 4-7, 12-15), zero for keys >= S. S_pad % 64 == 0.
 * The layout the attention kernel's PV product reads; no reference counterpart (the reference's
 * attention kernels transpose internally, ring_attention_const_max_fwd.py:1180-1220).
 */
int wanmi_transpose_heads(const void* v, int64_t S, int64_t ld, int64_t head_stride, int heads,
                          void* vt, int64_t S_pad, void* stream);

/*
 * out[h] = max over tokens s of ||x[h, s, :128]||_2 for a strided bf16 tensor (element (h, s, d) at
 * x[h*head_stride + s*token_stride + d]). The key-norm input of the constant-max bound
 * (ring_attention_const_max_fwd.py:296-360, all_reduce(max) at 1198-1205).
 */
int wanmi_head_max_norm(const void* x, int64_t head_stride, int64_t token_stride, int64_t S,
                        int heads, float* out, void* stream);

/* Output layouts of wanmi_attention_const_max. */
#define WANMI_ATTN_OUT_TOKEN 0  /* bf16, element (h, s, d) at out[h*o_head + s*o_token + d] */
#define WANMI_ATTN_OUT_DMAJOR 1 /* bf16, element (h, s, d) at out[h*o_head + d*o_d + s] ([B,N,D,S]) */
#define WANMI_ATTN_OUT_MX 2     /* e4m3fn codes at out[h*o_head + s*o_token + d] (bytes) and e8m0
                                   scales at out_scales[s*os_token + h*4 + d/32]; out, o_head and
                                   o_token multiples of 16, out_scales and os_token multiples of 4 */

/*
 * Non-causal constant-max attention, head_dim 128, bf16 inputs, fp32 accumulation:
 *   o_i = sum_j exp(s q_i.k_j - c_i) v_j / max(sum_j exp(s q_i.k_j - c_i), 1e-37),
 *   c_i = s ||q_i|| kmax[h]   (kmax[h] >= max_j ||k_j||, e.g. from wanmi_head_max_norm)
 * q, k: element (h, s, d) at x[h*head_stride + s*token_stride + d]; vt: [heads, 128, vt_ld] from
 * wanmi_transpose_heads (vt_ld % 64 == 0, >= Sk).
 * Replaces ring_attention_const_max_fwd on one device (vllm_omni_neuron/kernels/nkilib/
 * experimental/attention/ring_attention_const_max_fwd.py:959) and the flash attention behind
 * _nki_attend / wan_cp_self_attention (diffusion/models/wan2_2/wan2_2_transformer.py:653, 806).
 */
int wanmi_attention_const_max(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                              const void* k, int64_t k_head_stride, int64_t k_token_stride,
                              const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq,
                              int64_t Sk, int heads, int head_dim, float scale, int out_mode,
                              void* out, int64_t o_head_stride, int64_t o_token_stride,
                              int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride,
                              void* stream);

/*
 * wanmi_attention_const_max with the Q preparation fused into the kernel's Q load: q holds the raw
 * projection, and each query is normalized across heads, then optionally rotated, before use:
 *   q_hat = bf16(bf16(q * rrms * q_gamma) rotated),  rrms = 1/sqrt(sum_b q_sumsq[s, b] / (heads*128) + q_eps)
 * q_sumsq: [Sq, q_sumsq_ld] fp32 per-128-column partial sums of squares of the row (heads blocks,
 * summed in block order; from wanmi_mxfp8_gemm_rowsumsq); q_gamma: fp32 [heads*128]; q_cos, q_sin:
 * fp32 [Sq, 64] pair tables or both NULL (no RoPE). heads % 4 == 0.
 * Replaces DistributedRMSNorm + apply_rotary_emb_wan on Q (vllm_omni_neuron/diffusion/models/
 * wan2_2/wan2_2_transformer.py:879-893, diffusion/layers/rope.py:8-34) and the normalize-and-rotate
 * epilogue of the reference's QKV kernel (kernels/nkilib/core/qkv/qkv_cte.py:3870-3990).
 */
int wanmi_attention_const_max_qprep(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                    const void* k, int64_t k_head_stride, int64_t k_token_stride,
                                    const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq,
                                    int64_t Sk, int heads, int head_dim, float scale, int out_mode,
                                    void* out, int64_t o_head_stride, int64_t o_token_stride,
                                    int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride,
                                    const float* q_sumsq, int64_t q_sumsq_ld, const float* q_gamma,
                                    const float* q_cos, const float* q_sin, float q_eps, void* stream);

/*
 * wanmi_attention_const_max_qprep with each query's across-heads 1/rms given, q_rr [Sq] fp32, in place
 * of the partial sums (as wanmi_qk_rmsnorm_rope_qrr computes it from them: the same operations in the
 * same order, so the result is bit-identical to passing the partials). The Q load then reads one
 * float per query instead of `heads` partial sums for every head. Replaces the same reference
 * interfaces as wanmi_attention_const_max_qprep.
 */
int wanmi_attention_const_max_qrr(const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                  const void* k, int64_t k_head_stride, int64_t k_token_stride,
                                  const void* vt, int64_t vt_ld, const float* kmax, int64_t Sq,
                                  int64_t Sk, int heads, int head_dim, float scale, int out_mode,
                                  void* out, int64_t o_head_stride, int64_t o_token_stride,
                                  int64_t o_d_stride, uint8_t* out_scales, int64_t os_token_stride,
                                  const float* q_rr, const float* q_gamma, const float* q_cos,
                                  const float* q_sin, void* stream);

/*
 * Exact-softmax attention for the drop-ins of a running-max flash attention: the reference's
 * registered attention_cte op and _nki_attend (vllm_omni_neuron/diffusion/models/wan2_2/
 * wan2_2_transformer.py:83-108, 165-171, 653-674), which wan_cp_self_attention runs on one device
 * (806-847). Runs wanmi_attention_const_max (arguments as there; out_mode TOKEN or DMAJOR only, the
 * bf16 layouts those drop-ins return) writing every query's row sum of P to row_sum [heads][Sq] fp32,
 * then recomputes every row whose sum is below 2^-96 (the constant-max bound exceeded the row's
 * largest logit by so much that its P underflowed, or the sum is NaN) with the row's true max, in
 * fp32: o = sum_j exp(s q.k_j - m) v_j / sum_j exp(s q.k_j - m), m = max_j s q.k_j. Rows at or above
 * 2^-96 keep the constant-max result, which is then within bf16 rounding of the softmax. Two
 * launches on `stream`; row_sum is scratch the caller owns (its contents on return are the
 * constant-max row sums).
 */
int wanmi_attention_exact(const void* q, int64_t q_head_stride, int64_t q_token_stride, const void* k,
                          int64_t k_head_stride, int64_t k_token_stride, const void* vt, int64_t vt_ld,
                          const float* kmax, int64_t Sq, int64_t Sk, int heads, int head_dim, float scale,
                          int out_mode, void* out, int64_t o_head_stride, int64_t o_token_stride,
                          int64_t o_d_stride, float* row_sum, void* stream);

/*
 * wanmi_attention_exact without the row_sum workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It
 * has no counterpart in the reference. The row sums live in a static device array of the library,
 * 4M floats (16 MiB) on every GPU the library runs on, held until the process ends: heads * Sq
 * must be at most 4194304 (WANMI_ERR_ARG otherwise). The array's device address is looked up once
 * per device at the first call on it. Nothing is allocated or freed here. Every call on one GPU
 * shares that GPU's array and leaves the last call's row sums in it, so calls that overlap on one
 * GPU (different streams, or threads without ordering) race; calls in order on one stream do not.
 * Arguments and results are those of wanmi_attention_exact.
 */
int wanmi_attention_exact_noalloc(const void* q, int64_t q_head_stride, int64_t q_token_stride, const void* k,
                                  int64_t k_head_stride, int64_t k_token_stride, const void* vt, int64_t vt_ld,
                                  const float* kmax, int64_t Sq, int64_t Sk, int heads, int head_dim, float scale,
                                  int out_mode, void* out, int64_t o_head_stride, int64_t o_token_stride,
                                  int64_t o_d_stride, void* stream);

/*
 * wanmi_qk_rmsnorm_rope with the result written to `out` instead of back into x: element (token t,
 * head h, d) at out[t*out_token_stride + h*out_head_stride + d] (strides multiples of 8 elements,
 * out 16-byte aligned, heads <= 40). For the head-major NBSd result of the reference's projection
 * (qkv_cte.py output_layout NBSd, row_mx_modules.py:478-507), written in the normalization pass
 * instead of by a separate transposing copy. Bits as the in-place form.
 */
int wanmi_qk_rmsnorm_rope_to(const void* x, int64_t S, int64_t ld, int heads, const float* gamma, const float* cos_tab,
                             const float* sin_tab, int rope_pairs, float eps, void* out, int64_t out_token_stride,
                             int64_t out_head_stride, void* stream);

/*
 * d-major bf16 attention output -> token-major MX activation, one pass: x holds element (b, n, d, s)
 * at x[b*b_stride + n*h_stride + d*d_stride + s] (d < 128); codes [B*S, heads*128] e4m3fn and scales
 * [B*S, heads*4] e8m0 (one per 32 consecutive channels, the adaLN kernel's MX rule), the layout
 * wanmi_mxfp8_gemm takes as its activation. Replaces the in-kernel quantization of the reference's
 * ROW_MX o-projection input (row_mx_kernels.py:114-138, fed d-major by wan2_2_transformer.py:815-836).
 * Needs S a multiple of 8, strides multiples of 8 elements with d_stride >= S, 16-byte aligned x and
 * codes (WANMI_ERR_UNSUPPORTED otherwise).
 */
int wanmi_dmajor_to_mx(const void* x, int64_t B, int heads, int64_t S, int64_t b_stride, int64_t h_stride,
                       int64_t d_stride, void* codes, uint8_t* scales, void* stream);

/*
 * Streaming device-to-device copy of `bytes` (a multiple of 16; src and dst 16-byte aligned, not
 * overlapping) on `stream`: 16-byte loads, eight per thread in flight before its non-temporal
 * stores, one 32 KiB chunk per workgroup. Measurement infrastructure with no counterpart in the
 * reference: the practical HBM streaming rate the memory-bound kernels (adaLN + quantization, the
 * K normalization pass) are compared against.
 */
int wanmi_hbm_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

/*
 * Streaming read-2-write-1 pass (measurement infrastructure, no counterpart in the reference):
 * reads `src_bytes` (a multiple of 32768) and writes src_bytes / 2 to dst. Chunk k of 32 KiB is
 * read as 2048 16-byte words w[0..2047] in the order thread t of 256 reads w[256 i + t], i < 8;
 * output chunk k (16 KiB) holds, in 16-byte slot 256 i + t (i < 4), w[256 (2 i) + t] xor
 * w[256 (2 i + 1) + t]. Same load and store form as the copy; its rate is the HBM ceiling for the
 * adaLN + MX pass's 2:1 read/write mix.
 */
int wanmi_hbm_stream_fold(const void* src, void* dst, int64_t src_bytes, void* stream);

/*
 * Element-wise fp32 -> e4m3fn conversion exactly as the kernels perform it (round to nearest even,
 * hardware conversion; inputs must satisfy |x| < 464). Test hook for the conversion's known-answer
 * tests; it has no counterpart in the reference (which relies on torch's float8_e4m3fn cast,
 * adaln_quant_torch.py:35).
 */
int wanmi_e4m3_encode(const float* in, uint8_t* out, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WANMI_H_ */
