"""MX (per-32 e8m0) and ROW (per-row fp32) FP8 quantization -- oracle, test infrastructure only.

MX rule, restated from ``_mx_dequant`` (vllm_omni_neuron/kernels/nkilib/experimental/norm/
adaln_quant_torch.py:151-175), which mirrors ``reference_mx_dequant``
(kernels/nkilib/core/rmsnorm/rmsnorm_mx_prefill_torch.py:214-246) and the MLP intermediate
quantizer ``_mx_quantize`` (kernels/nkilib/core/mlp/mlp_torch.py:252-271):

    per row, per block of 32 contiguous values along the last dim:
      E    = max_i ((bits_f32(y_i) >> 23) & 0xFF)
      s    = clip(E - 7, 0, 255)                        (the e8m0 byte; 7 = e4m3fn max exponent)
      code = RNE_e4m3fn(clip(y_i * 2^(127 - s), -448, 448))

ROW rule, restated from the ROW branch of ``adaln_quant_torch_ref`` (adaln_quant_torch.py:131-142)
and the packed layout the QKV kernel reads (qkv_cte.py:3671-3682, tail width qkv_cte_utils.py:49):

    amax = max_i |y_i|;  dq = max(amax / 448, 1e-6)  (fp32);  code = RNE_e4m3fn(y_i / dq)  (fp32 div)
    packed row = [codes (H bytes) | little-endian bytes of fp32 dq]
"""

from __future__ import annotations

import numpy as np

from .fp8 import E4M3_MAX, e4m3_decode, e4m3_encode, e8m0_value, exp_field

MX_BLOCK = 32
FP8_MAX_EXP = 7  # adaln_quant_torch.py:31
MIN_DEQUANT_SCALE = np.float32(1e-6)  # adaln_quant_torch.py:30


def mx_quantize(y: np.ndarray):
    """y [..., K] (fp32 values; K % 32 == 0) -> (codes uint8 [..., K], scales uint8 [..., K/32])."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    K = y.shape[-1]
    if K % MX_BLOCK:
        raise ValueError(f"MX last dim {K} must be a multiple of {MX_BLOCK}")
    blocks = y.reshape(*y.shape[:-1], K // MX_BLOCK, MX_BLOCK)
    emax = exp_field(blocks).max(axis=-1)
    s = np.clip(emax - FP8_MAX_EXP, 0, 255)
    # y * 2^(127 - s) is exact in fp32: a power-of-two scaling whose results stay below 2^8
    scaled = blocks * np.ldexp(np.float32(1.0), (127 - s)[..., None]).astype(np.float32)
    scaled = np.clip(scaled, np.float32(-E4M3_MAX), np.float32(E4M3_MAX))
    codes = e4m3_encode(scaled).reshape(y.shape)
    return codes, s.astype(np.uint8)


def mx_dequantize(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """(codes [..., K], scales [..., K/32]) -> fp64 values code * 2^(s - 127)."""
    vals = e4m3_decode(codes).astype(np.float64)
    f = np.repeat(e8m0_value(scales), MX_BLOCK, axis=-1)
    return vals * f


def row_quantize(y: np.ndarray):
    """y [..., H] fp32 -> (codes uint8 [..., H], dq fp32 [..., 1])."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    amax = np.abs(y).max(axis=-1, keepdims=True)
    dq = np.maximum(amax / np.float32(E4M3_MAX), MIN_DEQUANT_SCALE).astype(np.float32)
    q = np.clip((y / dq).astype(np.float32), -E4M3_MAX, E4M3_MAX)
    return e4m3_encode(q), dq


def row_pack(codes: np.ndarray, dq: np.ndarray) -> np.ndarray:
    """Packed ``[..., H + 4]`` bytes: codes then the 4 little-endian bytes of the fp32 dq."""
    tail = np.ascontiguousarray(dq.astype("<f4")).view(np.uint8).reshape(*dq.shape[:-1], 4)
    return np.concatenate([codes, tail], axis=-1)


def row_unpack(packed: np.ndarray):
    """Inverse of :func:`row_pack`: -> (codes [..., H], dq fp32 [..., 1])."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    codes = packed[..., :-4]
    dq = np.ascontiguousarray(packed[..., -4:]).view("<f4").astype(np.float32)
    return codes, dq
