"""Canonical fused adaLN + quantization -- oracle, test infrastructure only.

Restates ``_eager_adaln`` (vllm_omni_neuron/diffusion/quantization/adaln_kernels.py:51-84) with a
fixed, order-independent definition of the row statistics so that a GPU result can be compared bit
for bit:

    x = h                                     or  x = bf16(fl32(h * gate) + res)   (adaln_kernels.py:58-66)
    E = max biased fp32 exponent over the row
    LayerNorm (two-pass, fp64, on an exact fixed grid):
        S1 = sum rint(x * 2^(165-E)),            mu64  = (S1 * 2^(E-165)) / H
        S2 = sum rint((x - mu64)^2 * 2^(289-2E)), var64 = (S2 * 2^(2E-289)) / H
        mu = fp32(mu64), rstd = fp32(1 / sqrt(var64 + eps))
        xh = fl32(fl32(x - mu) * rstd)
    RMSNorm: S = sum rint(x^2 * 2^(291-2E)); rrms = fp32(1/sqrt(S*2^(2E-291)/H + eps)); xh = fl32(x*rrms)
    y = bf16(fl32(fl32(xh * mul) + add))      (mul / add optional, fp32, no FMA)

Every rounded term is an integer of magnitude < 2^39 and H <= 16384, so each sum is exact in fp64.
``F.layer_norm``'s own fp32 reduction order is not reproducible off the CPU it ran on; the distance
from this definition to the eager path is measured in the tests (bf16 ulps of y).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import mx as mx_mod
from .fp8 import bf16_round, exp_field


def _row_exp_max(x: np.ndarray) -> np.ndarray:
    return exp_field(x).max(axis=-1, keepdims=True)


def layer_norm_stats(x: np.ndarray, eps: float):
    """x fp32 [..., H] -> (mu fp32 [..., 1], rstd fp32 [..., 1]) per the fixed-grid definition."""
    H = x.shape[-1]
    E = _row_exp_max(x)
    xd = x.astype(np.float64)
    s1 = np.rint(np.ldexp(xd, 165 - E)).sum(axis=-1, keepdims=True)
    mu64 = np.ldexp(s1, E - 165) / np.float64(H)
    d = xd - mu64
    s2 = np.rint(np.ldexp(d * d, 289 - 2 * E)).sum(axis=-1, keepdims=True)
    var64 = np.ldexp(s2, 2 * E - 289) / np.float64(H)
    rstd64 = 1.0 / np.sqrt(var64 + np.float64(np.float32(eps)))
    return mu64.astype(np.float32), rstd64.astype(np.float32)


def rms_norm_stat(x: np.ndarray, eps: float) -> np.ndarray:
    """x fp32 [..., H] -> rrms fp32 [..., 1]."""
    H = x.shape[-1]
    E = _row_exp_max(x)
    xd = x.astype(np.float64)
    s = np.rint(np.ldexp(xd * xd, 291 - 2 * E)).sum(axis=-1, keepdims=True)
    ms64 = np.ldexp(s, 2 * E - 291) / np.float64(H)
    return (1.0 / np.sqrt(ms64 + np.float64(np.float32(eps)))).astype(np.float32)


def adaln_y(hidden, mul=None, add=None, *, eps=1e-6, norm_type="layer_norm", residual=None, gate=None):
    """Modulated bf16 activation (as fp32) and the bf16 residual sum (or None).

    hidden / residual: fp32 arrays holding bf16 values, [..., H]; mul / add / gate: fp32 [H] or None.
    """
    x = np.ascontiguousarray(hidden, dtype=np.float32)
    res_out = None
    if residual is not None:
        if gate is not None:
            x = (x * np.asarray(gate, np.float32)).astype(np.float32)
        x = (x + np.asarray(residual, np.float32)).astype(np.float32)
        res_out = bf16_round(x)
        x = res_out
    if norm_type == "layer_norm":
        mu, rstd = layer_norm_stats(x, eps)
        xh = ((x - mu).astype(np.float32) * rstd).astype(np.float32)
    elif norm_type == "rms_norm":
        xh = (x * rms_norm_stat(x, eps)).astype(np.float32)
    elif norm_type == "none":
        xh = x
    else:
        raise ValueError(f"unsupported norm_type {norm_type!r}")
    t = xh
    if mul is not None:
        t = (t * np.asarray(mul, np.float32)).astype(np.float32)
    if add is not None:
        t = (t + np.asarray(add, np.float32)).astype(np.float32)
    return bf16_round(t), res_out


def adaln_quant(hidden, mul=None, add=None, *, eps=1e-6, norm_type="layer_norm", quant="none",
                residual=None, gate=None):
    """Canonical fused adaLN + quantization.

    Returns a dict: ``y`` (bf16 values as fp32), ``residual_out`` (or None), and for quant="mx"
    ``codes``/``scales``; for quant="row" ``packed`` ([..., H+4] uint8), ``codes`` and ``dq``.
    """
    y, res_out = adaln_y(hidden, mul, add, eps=eps, norm_type=norm_type, residual=residual, gate=gate)
    out = {"y": y, "residual_out": res_out}
    if quant == "mx":
        out["codes"], out["scales"] = mx_mod.mx_quantize(y)
    elif quant == "row":
        codes, dq = mx_mod.row_quantize(y)
        out["codes"], out["dq"] = codes, dq
        out["packed"] = mx_mod.row_pack(codes, dq)
    elif quant != "none":
        raise ValueError(f"unsupported quant {quant!r}")
    return out


def eager_adaln_y(hidden, mul=None, add=None, *, eps=1e-6, norm_type="layer_norm", residual=None, gate=None):
    """The reference's unfused path in torch on the CPU (``_eager_adaln``, adaln_kernels.py:51-84),
    quant="none": returns bf16 ``y`` as fp32 numpy. Used only to measure the canonical definition's
    distance from ``F.layer_norm``."""
    h = torch.from_numpy(np.ascontiguousarray(hidden, np.float32)).to(torch.bfloat16)
    x = h.float()
    if residual is not None:
        r = torch.from_numpy(np.ascontiguousarray(residual, np.float32)).to(torch.bfloat16)
        if gate is not None:
            x = x * torch.from_numpy(np.asarray(gate, np.float32))
        x = (x + r.float()).to(torch.bfloat16).float()
    if norm_type == "layer_norm":
        norm = F.layer_norm(x, (x.shape[-1],), None, None, eps)
    elif norm_type == "rms_norm":
        norm = x / torch.sqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    else:
        norm = x
    if mul is not None:
        norm = norm * torch.from_numpy(np.asarray(mul, np.float32))
    if add is not None:
        norm = norm + torch.from_numpy(np.asarray(add, np.float32))
    return norm.to(torch.bfloat16).float().numpy()
