"""MXFP8 projections, GELU-tanh and the MLP -- oracle, test infrastructure only.

Restates the ROW_MX / MX projection arithmetic of the reference in fp64:

- ``_mlp_ref_standard`` (vllm_omni_neuron/kernels/nkilib/core/mlp/mlp_torch.py:401-599):
  ``up = (x * in_scale) @ (W_up * w_scale) + b_up``; ``g = GELU_tanh(up)``; ``(codes, s) = MX(g)``
  (mlp_torch.py:252-271, 586-594); ``out = (codes * 2^(s-127)) @ (W_down * w_scale) + b_down``.
  The MLP is composed from these pieces in ``block.mxfp8_block`` and in the tests.
- the QKV / o-proj ROW_MX epilogue ``psum * row_scale * col_scale + bias``
  (kernels/nkilib/core/qkv/qkv_cte.py:3996-4021).

With MX operands every dequantized value is exact in fp64, so the product here is the exact sum
the hardware approximates in fp32.
"""

from __future__ import annotations

import numpy as np
import torch

from . import mx as mx_mod
from .fp8 import bf16_round


def dequant_mx(codes: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(mx_mod.mx_dequantize(codes, scales))


def mx_gemm(a_codes, a_scales, w_codes, w_scales, bias=None, row_scale=None, col_scale=None):
    """fp64 ``A_deq @ W_deq^T * row_scale * col_scale + bias``; W stored ``[N, K]`` (K-contiguous)."""
    a = dequant_mx(a_codes, a_scales)
    w = dequant_mx(w_codes, w_scales)
    y = a @ w.T
    if row_scale is not None:
        y = y * torch.as_tensor(np.asarray(row_scale, np.float64)).reshape(-1, 1)
    if col_scale is not None:
        y = y * torch.as_tensor(np.asarray(col_scale, np.float64)).reshape(1, -1)
    if bias is not None:
        y = y + torch.as_tensor(np.asarray(bias, np.float64)).reshape(1, -1)
    return y


def abs_gemm(a_codes, a_scales, w_codes, w_scales):
    """``|A_deq| @ |W_deq|^T``: the magnitude scale of fp32 accumulation error per output."""
    a = dequant_mx(a_codes, a_scales).abs()
    w = dequant_mx(w_codes, w_scales).abs()
    return a @ w.T


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """GELU with the tanh approximation (torch ``F.gelu(approximate="tanh")``, mlp_torch.py:172)."""
    return torch.nn.functional.gelu(x, approximate="tanh")


def quantize_weight(w_kn: np.ndarray):
    """Reference-layout weight ``[K, N]`` (``x @ W``) -> MX ``(codes [N, K], scales [N, K/32])``
    quantized along K from bf16 values, the layout the GEMM consumes."""
    wt = bf16_round(np.ascontiguousarray(np.asarray(w_kn, np.float32).T))
    return mx_mod.mx_quantize(wt)
