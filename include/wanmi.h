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

#define WANMI_ABI_VERSION 1

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
 * Statistics are exact fixed-grid sums in fp64, so results do not depend on the reduction order.
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
 * Requires N % 256 == 0, K % 128 == 0.
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
