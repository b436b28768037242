"""Boundary vocabulary shared by the ops: the reference's enums plus the MX tensor pair.

The enum members mirror vllm_omni_neuron/kernels/nkilib/core/utils/common_types.py (NormType,
QuantizationType, DtypeMode, QKVOutputLayout) so call sites read the same; only the members the Wan DiT
path uses are kept.
"""

from __future__ import annotations

import enum
from typing import NamedTuple

import torch


class NormType(enum.Enum):
    NO_NORM = "none"
    LAYER_NORM = "layer_norm"
    RMS_NORM = "rms_norm"
    RMS_NORM_ACROSS_HEADS = "rms_norm_across_heads"


class QuantizationType(enum.Enum):
    NONE = "none"
    ROW = "row"
    MX = "mx"
    ROW_MX = "row_mx"


class DtypeMode(enum.Enum):
    """FP8 e4m3 variant of a ROW-quantized output: NON_OCP (max 240), OCP (e4m3fn, max 448), AUTO
    (what the hardware supports: OCP on gfx950)."""

    NON_OCP = "non_ocp"
    OCP = "ocp"
    AUTO = "auto"


class QKVOutputLayout(enum.Enum):
    BSD = "bsd"  # [B, S, (nq + 2 nkv) * d]
    NBSd = "nbsd"  # [N, B, S, d]


class ActFnType(enum.Enum):
    """MLP activation (reference ActFnType); Wan's FFN uses the tanh-approximated GELU."""

    SiLU = "silu"
    GELU = "gelu"
    GELU_Tanh_Approx = "gelu_tanh_approx"
    Swish = "swish"
    ReLU = "relu"
    SquaredReLU = "squared_relu"


class MLPGateUpWeightLayout(enum.Enum):
    """How the reference lays out the MLP up/gate weight for its kernel. Here every weight is an
    :class:`MXWeight` or a packed ``[K/4, N, 4]`` tensor; the member only documents the caller's
    intent and is accepted for signature compatibility."""

    CONTIGUOUS = "contiguous"
    H_X4_INNERMOST = "h_x4_innermost"


class ComputationMode(enum.Enum):
    """Reference MLP dispatch mode: context encoding (PREFILL) or token generation (DECODE)."""

    AUTO = "auto"
    PREFILL = "prefill"
    DECODE = "decode"


class QKNormConfig(NamedTuple):
    """Across-heads RMSNorm applied to Q and/or K before RoPE (reference QKNormConfig)."""

    q_norm: NormType | None
    k_norm: NormType | None
    eps: float = 1e-6


class MXTensor(NamedTuple):
    """An MXFP8 activation: e4m3fn codes [..., K] and one e8m0 scale per 32 codes [..., K/32].

    Element ``i`` of a row dequantizes to ``codes[i] * 2**(scales[i // 32] - 127)``.
    """

    codes: torch.Tensor  # torch.float8_e4m3fn
    scales: torch.Tensor  # torch.uint8

    @property
    def shape(self):
        return self.codes.shape

    def dequantize(self, dtype=torch.float32) -> torch.Tensor:
        f = torch.exp2(self.scales.to(torch.float32) - 127.0)
        f = f.repeat_interleave(32, dim=-1)
        return (self.codes.to(torch.float32) * f).to(dtype)
