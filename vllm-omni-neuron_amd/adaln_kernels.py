"""Fused adaptive LayerNorm (+ FP8 quantization) entry point for the Wan DiT, on gfx950.

Drop-in for ``adaln_modulate`` (vllm_omni_neuron/diffusion/quantization/adaln_kernels.py:87-201):
same argument list, same ``[B, S, H]`` / ``[T, H]`` handling, same per-batch loop over
``[B, 1, H]`` modulation vectors, same ``(residual_out, modulated)`` return when a residual is fused.
Differences, all deliberate:

- ``quant="mx"`` is supported (the reference raises NotImplementedError for it,
  adaln_kernels.py:36-40) and returns an :class:`MXTensor` (e4m3fn codes + e8m0 scales per 32).
- ``quant="row"`` returns the reference's packed ``[..., H + 4]`` layout (float8_e4m3fn codes
  followed by the 4 bytes of the row's fp32 dequant scale).
- There is no eager fallback: the reference's capability gate (``_can_use_adaln_kernel``) returns
  False off-device and runs ``_eager_adaln`` on the host; here a CPU tensor is an error.
- mul / add / gate stay fp32 (``_eager_adaln`` semantics, adaln_kernels.py:58-76).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .common_types import DtypeMode, MXTensor, NormType, QuantizationType

_MAX_HIDDEN = 16384
_SUPPORTED_NORMS = ("layer_norm", "rms_norm", "none")
_SUPPORTED_QUANTS = ("none", "row", "mx")


def _validate(hidden: torch.Tensor, norm_type: str, quant: str, ocp: bool) -> None:
    if quant not in _SUPPORTED_QUANTS:
        raise ValueError(f"unsupported quant {quant!r}")
    if norm_type not in _SUPPORTED_NORMS:
        raise ValueError(f"unsupported norm_type {norm_type!r}")
    if not ocp:
        raise NotImplementedError("only OCP e4m3fn FP8 (ocp=True) is produced on gfx950")
    if hidden.dim() < 2:
        raise ValueError(f"hidden must be [B, S, H] or [T, H], got {tuple(hidden.shape)}")
    if hidden.dtype != torch.bfloat16:
        raise ValueError(f"hidden must be bfloat16, got {hidden.dtype}")
    H = hidden.shape[-1]
    if H > _MAX_HIDDEN or H % 32:
        raise ValueError(f"hidden size {H} must be a multiple of 32 and <= {_MAX_HIDDEN}")


def _row(vec: torch.Tensor | None, b: int, H: int) -> torch.Tensor | None:
    """[B, 1, H] (per batch) or [H] / [1, H] (shared) -> contiguous fp32 [H] for batch ``b``."""
    if vec is None:
        return None
    v = vec[b] if vec.dim() == 3 else vec
    return v.reshape(H).to(torch.float32).contiguous()


def adaln_quant_2d(
    x: torch.Tensor,
    mul: torch.Tensor | None,
    add: torch.Tensor | None,
    *,
    eps: float,
    norm_type: str,
    quant: str,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
):
    """One launch over a contiguous bf16 ``[T, H]``; mul/add/gate are fp32 ``[H]`` or None.

    Returns ``out`` or ``(residual_out, out)`` with ``out`` a bf16 tensor, an :class:`MXTensor` or a
    packed ``[T, H + 4]`` float8_e4m3fn tensor.
    """
    lib = _lib.load()
    _lib.require_gpu(x, mul, add, residual, gate, what="adaln_modulate")
    T, H = x.shape
    x = x.contiguous()
    if residual is not None:
        residual = residual.contiguous()
        if residual.shape != x.shape or residual.dtype != torch.bfloat16:
            raise ValueError("residual must be bf16 and match hidden's shape")
    dev = x.device
    scales = None
    if quant == "none":
        out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    elif quant == "mx":
        out = torch.empty((T, H), dtype=torch.uint8, device=dev)
        scales = torch.empty((T, H // 32), dtype=torch.uint8, device=dev)
    else:
        out = torch.empty((T, H + 4), dtype=torch.uint8, device=dev)
    residual_out = torch.empty_like(x) if residual is not None else None
    status = lib.wanmi_adaln_quant(
        _lib.ptr(x),
        _lib.ptr(residual),
        _lib.ptr(gate if residual is not None else None),
        _lib.ptr(mul),
        _lib.ptr(add),
        T,
        H,
        float(eps),
        _lib.NORM[norm_type],
        _lib.QUANT[quant],
        _lib.ptr(out),
        _lib.ptr(scales),
        _lib.ptr(residual_out),
        _lib.stream_of(x),
    )
    _lib.check(status, "wanmi_adaln_quant")
    if quant == "mx":
        out = MXTensor(out.view(torch.float8_e4m3fn), scales)
    elif quant == "row":
        out = out.view(torch.float8_e4m3fn)
    return out if residual is None else (residual_out, out)


def adaln_modulate(
    hidden: torch.Tensor,
    mul: torch.Tensor | None = None,
    add: torch.Tensor | None = None,
    *,
    eps: float,
    norm_type: str = "layer_norm",
    quant: str = "none",
    ocp: bool = True,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
):
    """Fused ``Quantize(Norm(residual + gate * hidden) * mul + add)`` on the GPU.

    ``hidden`` is ``[B, S, H]`` or ``[T, H]`` bf16; ``mul`` / ``add`` / ``gate`` are ``[B, 1, H]``
    (per batch), ``[H]`` / ``[1, H]`` (shared) or None. Without ``residual`` returns the modulated
    tensor; with it returns ``(residual_out, modulated)`` where ``residual_out`` is the bf16
    ``residual + gate * hidden`` (the block's carried residual).
    """
    _validate(hidden, norm_type, quant, ocp)
    have_residual = residual is not None
    hidden_3d = hidden.unsqueeze(0) if hidden.dim() == 2 else hidden
    residual_3d = None
    if have_residual:
        residual_3d = residual.unsqueeze(0) if residual.dim() == 2 else residual
    B, H = hidden_3d.shape[0], hidden_3d.shape[-1]
    lead = hidden_3d.shape[1:-1]

    outs, res_outs = [], []
    for b in range(B):
        x2 = hidden_3d[b].reshape(-1, H)
        r2 = residual_3d[b].reshape(-1, H) if have_residual else None
        res = adaln_quant_2d(
            x2,
            _row(mul, b, H),
            _row(add, b, H),
            eps=eps,
            norm_type=norm_type,
            quant=quant,
            residual=r2,
            gate=_row(gate, b, H) if have_residual else None,
        )
        if have_residual:
            res_outs.append(res[0])
            res = res[1]
        outs.append(res)

    def _stack(parts, width_fn):
        if len(parts) == 1:  # B == 1: a view, no copy
            return parts[0].reshape(1, *lead, width_fn(parts[0]))
        return torch.stack([p.reshape(*lead, width_fn(p)) for p in parts], dim=0)

    if quant == "mx":
        out = MXTensor(
            _stack([o.codes for o in outs], lambda p: p.shape[-1]),
            _stack([o.scales for o in outs], lambda p: p.shape[-1]),
        )
        if hidden.dim() == 2:
            out = MXTensor(out.codes[0], out.scales[0])
    else:
        out = _stack(outs, lambda p: p.shape[-1])
        if hidden.dim() == 2:
            out = out[0]
    if not have_residual:
        return out
    residual_out = _stack(res_outs, lambda p: p.shape[-1])
    if hidden.dim() == 2:
        residual_out = residual_out[0]
    return residual_out, out


@dataclass(frozen=True)
class AdaLNQuantKernelArgs:
    """Configuration of :func:`adaln_quant_kernel` (the reference's dataclass of the same name,
    adaln_quant.py:70-114, with the same fields, defaults and checks)."""

    norm_type: NormType = NormType.LAYER_NORM
    quantization_type: QuantizationType = QuantizationType.NONE
    eps: float = 1e-6
    lower_bound: float = 0.0

    def __post_init__(self):
        if self.norm_type not in (NormType.LAYER_NORM, NormType.RMS_NORM, NormType.NO_NORM):
            raise ValueError(f"{self.norm_type.name} normalization is not supported")
        if self.quantization_type not in (QuantizationType.NONE, QuantizationType.ROW, QuantizationType.MX):
            raise ValueError(f"{self.quantization_type.name} quantization is not supported")
        if not self.lower_bound >= 0:
            raise ValueError(f"Lower bound must be non-negative but got {self.lower_bound}")
        if not self.eps >= 0:
            raise ValueError(f"Epsilon must be non-negative but got {self.eps}")

    def has_lower_bound(self) -> bool:
        return self.lower_bound is not None and self.lower_bound > 0.000001


def _vector(vec: torch.Tensor | None, name: str, H: int) -> torch.Tensor | None:
    """A per-hidden vector ``[H]`` or ``[1, H]`` (any float dtype) -> contiguous fp32 ``[H]``."""
    if vec is None:
        return None
    if vec.dim() not in (1, 2):
        raise ValueError(f"Rank of {name} must be 1 or 2 but got {vec.dim()}")
    if vec.shape[-1] != H:
        raise ValueError(f"{name} vector length must equal {H} but got {vec.shape[-1]}")
    if vec.dim() == 2 and vec.shape[0] > 1:
        raise ValueError(f"{name} first dimension {vec.shape[0]} must be at most 1")
    return vec.reshape(H).to(torch.float32).contiguous()


def adaln_quant_kernel(
    hidden: torch.Tensor,
    kargs: AdaLNQuantKernelArgs,
    mul: torch.Tensor | None = None,
    add: torch.Tensor | None = None,
    dtype_mode: DtypeMode = DtypeMode.NON_OCP,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
):
    """Kernel-level drop-in for ``adaln_quant_kernel`` (vllm_omni_neuron/kernels/nkilib/experimental/
    norm/adaln_quant.py:117-234), as ``adaln_modulate`` launches it per batch element
    (adaln_kernels.py:150-201): ``[..., H]`` bf16 ``hidden`` (rank >= 2, all leading dims are rows),
    ``mul`` / ``add`` / ``gate`` ``[H]`` or ``[1, H]``. Returns the modulated ``[..., H]`` bf16, or
    ``[..., H + 4]`` float8_e4m3fn for ROW (codes, then the row's fp32 dequant scale); with
    ``residual``, ``(residual_out, modulated)`` where ``residual_out = bf16(residual + gate *
    hidden)``. One launch of the fused kernel.

    As in the reference, MX quantization is not produced here (the caller's MX path is
    ``adaln_modulate(quant="mx")``) and ``gate`` requires ``residual``. gfx950 FP8 is the OCP e4m3fn
    format, so ROW output needs ``dtype_mode`` OCP or AUTO (the reference's default NON_OCP is its
    e4m3 with max 240), and the ROW clip bound (``lower_bound`` > 0) is not implemented: both raise
    NotImplementedError. mul / add are consumed as given (the reference's bridge rounds them to the
    hidden dtype before this call).
    """
    if not isinstance(kargs, AdaLNQuantKernelArgs):
        raise TypeError("kargs must be an AdaLNQuantKernelArgs")
    if kargs.quantization_type == QuantizationType.MX:
        raise NotImplementedError("MX quantization is not implemented in adaln_quant_kernel; the caller must use "
                                  "adaln_modulate(quant='mx').")
    row = kargs.quantization_type == QuantizationType.ROW
    if row and dtype_mode == DtypeMode.NON_OCP:
        raise NotImplementedError("NON_OCP e4m3 (max 240) is not an FP8 format of gfx950; use DtypeMode.OCP")
    if row and kargs.has_lower_bound():
        raise NotImplementedError("the ROW clip bound (lower_bound > 0) is not implemented")
    if hidden.dim() < 2:
        raise ValueError(f"Rank of hidden must be at least 2 but got {hidden.dim()}")
    if hidden.dtype != torch.bfloat16:
        raise ValueError(f"hidden must be bfloat16, got {hidden.dtype}")
    H = hidden.shape[-1]
    if H > _MAX_HIDDEN or H % 32:
        raise ValueError(f"hidden size {H} must be a multiple of 32 and <= {_MAX_HIDDEN}")
    if gate is not None and residual is None:
        raise ValueError("gate requires residual (gate scales the sub-layer output before the residual add)")
    if residual is not None and (residual.shape != hidden.shape or residual.dtype != torch.bfloat16):
        raise ValueError(f"residual must be bf16 {tuple(hidden.shape)}, got {residual.dtype} {tuple(residual.shape)}")
    res = adaln_quant_2d(
        hidden.reshape(-1, H),
        _vector(mul, "mul", H),
        _vector(add, "add", H),
        eps=kargs.eps,
        norm_type=kargs.norm_type.value,
        quant="row" if row else "none",
        residual=None if residual is None else residual.reshape(-1, H),
        gate=_vector(gate, "gate", H),
    )
    lead = hidden.shape[:-1]
    if residual is None:
        return res.view(*lead, res.shape[-1])
    return res[0].view(*lead, H), res[1].view(*lead, res[1].shape[-1])
