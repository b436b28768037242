"""Canonical fused adaLN + quantization -- oracle, test infrastructure only.

Restates ``_eager_adaln`` (vllm_omni_neuron/diffusion/quantization/adaln_kernels.py:51-84) with a
fixed definition of the row statistics so that a GPU result can be compared bit for bit:

    x = h                                     or  x = bf16(fl32(h * gate) + res)   (adaln_kernels.py:58-66)
    Summation order (fp32): the row is cut into chunks of 512 columns; "lane" l (0..63) owns
    columns c*512 + 8l .. 8l+7 of every chunk c and adds its values sequentially (chunk by chunk,
    column order inside a chunk); the 64 lane sums then combine in an xor butterfly with offsets
    1, 2, 4, 8, 16, 32 (v_l <- v_l + v_(l^o)).
    LayerNorm (two-pass): mu = S1 / H,  S1 = sum x
                          var = S2 / H, S2 = sum fl(fl(x - mu)^2),  rstd = fp32(1/sqrt(fp64(var) + eps))
                          xh = fl32(fl32(x - mu) * rstd)
    RMSNorm:  ms = S / H, S = sum fl(x^2), rrms = fp32(1/sqrt(fp64(ms) + eps)), xh = fl32(x * rrms)
    y = bf16(fl32(fl32(xh * mul) + add))      (mul / add optional, fp32, no FMA)

``F.layer_norm``'s own fp32 reduction order is not reproducible off the CPU it ran on; the distance
from this definition to the eager path is measured in the tests (bf16 ulps of y).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import mx as mx_mod
from .fp8 import bf16_round, exp_field


def _lane_major(x: np.ndarray) -> np.ndarray:
    """[T, H] -> [T, 64, NCH*8]: each lane's columns in its summation order (zero padded)."""
    T, H = x.shape
    nch = -(-H // 512)
    xp = np.zeros((T, nch * 512), np.float32)
    xp[:, :H] = x
    return xp.reshape(T, nch, 64, 8).transpose(0, 2, 1, 3).reshape(T, 64, nch * 8)


def _valid_lane_major(T: int, H: int) -> np.ndarray:
    return _lane_major(np.ones((1, H), np.float32))[0] > 0


def _ordered_sum(terms: np.ndarray) -> np.ndarray:
    """[T, 64, n] fp32 -> [T, 1]: sequential per-lane fp32 sums, then the xor butterfly."""
    acc = np.zeros(terms.shape[:2], np.float32)
    for i in range(terms.shape[2]):
        acc = (acc + terms[:, :, i]).astype(np.float32)
    lanes = np.arange(64)
    for o in (1, 2, 4, 8, 16, 32):
        acc = (acc + acc[:, lanes ^ o]).astype(np.float32)
    return acc[:, :1]


def layer_norm_stats(x: np.ndarray, eps: float):
    """x fp32 [T, H] -> (mu fp32 [T, 1], rstd fp32 [T, 1]) in the canonical order."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    T, H = x.shape
    lm = _lane_major(x)
    mu = (_ordered_sum(lm) / np.float32(H)).astype(np.float32)
    d = (lm - mu[:, :, None]).astype(np.float32)
    with np.errstate(over="ignore"):  # fp32 squares of extreme rows overflow to inf, as on the GPU
        q = (d * d).astype(np.float32)
    q = np.where(_valid_lane_major(T, H)[None], q, np.float32(0.0))
    var = (_ordered_sum(q) / np.float32(H)).astype(np.float32)
    rstd = (1.0 / np.sqrt(var.astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)
    return mu, rstd


def rms_norm_stat(x: np.ndarray, eps: float) -> np.ndarray:
    """x fp32 [T, H] -> rrms fp32 [T, 1] in the canonical order."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    H = x.shape[-1]
    lm = _lane_major(x)
    ms = (_ordered_sum((lm * lm).astype(np.float32)) / np.float32(H)).astype(np.float32)
    return (1.0 / np.sqrt(ms.astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)


def adaln_y(hidden, mul=None, add=None, *, eps=1e-6, norm_type="layer_norm", residual=None, gate=None):
    """Modulated bf16 activation (as fp32) and the bf16 residual sum (or None).

    hidden / residual: fp32 arrays holding bf16 values, [..., H]; mul / add / gate: fp32 [H] or None.
    """
    shape = np.shape(hidden)
    x = np.ascontiguousarray(hidden, dtype=np.float32).reshape(-1, shape[-1])
    if residual is not None:
        residual = np.asarray(residual, np.float32).reshape(-1, shape[-1])
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
    y = bf16_round(t).reshape(shape)
    return y, (None if res_out is None else res_out.reshape(shape))


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
