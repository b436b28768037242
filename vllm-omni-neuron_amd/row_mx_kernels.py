"""MXFP8 projection entry points for the Wan DiT on gfx950.

Drop-ins for the reference's ROW_MX projection launchers
(vllm_omni_neuron/diffusion/quantization/row_mx_kernels.py):

- :func:`row_quantize_packed` (row_mx_kernels.py:12-45): bf16 rows to the packed ROW layout.
- :func:`row_mx_mlp` (row_mx_kernels.py:141-198): gate-less GELU-tanh MLP, up projection with the
  GELU + MX re-quantization fused in its epilogue, then the down projection.
- :func:`row_mx_qkv_proj` (row_mx_kernels.py:48-111) and :func:`row_mx_o_proj` (114-138) are in
  :mod:`.attention_ops` next to the Q/K normalization they fuse with.

Weights live in the GEMM's own layout, an :class:`MXWeight`: the reference-layout ``[K, N]``
weight (``x @ W``) transposed to ``[N, K]`` and MX-quantized along K (one e8m0 scale per 32),
produced once by :func:`quantize_weight_mx` -- the counterpart of the reference's offline weight
packers (row_mx_loaders.py), which lay FP8 weights out for Neuron SBUF instead.

Activations are :class:`MXTensor` (what ``adaln_modulate(quant="mx")`` returns) or the reference's
packed ROW layout ``[..., K + 4]``; the latter is split into codes, neutral block scales and a
per-row fp32 scale applied in the epilogue (ROW_MX semantics, qkv_cte.py:3996-4021).
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib
from .adaln_kernels import adaln_quant_2d
from .common_types import MXTensor

EPILOGUES = {"bf16": 0, "gelu_mx": 1, "gelu_bf16": 2, "gated_residual": 3}
_NEUTRAL_SCALE = 127


class MXWeight(NamedTuple):
    """A projection weight in GEMM layout: ``codes [N, K]`` e4m3fn, ``scales [N, K/32]`` e8m0,
    an optional per-output-channel fp32 ``col_scale [N]`` (ROW_MX dequant) and fp32 ``bias [N]``.

    ``rope_pairs`` says how the Q/K output channels of a fused QKV weight pair up for RoPE:
    ``"interleaved"`` (Wan's natural order, pairs (2i, 2i+1)) or ``"halves"`` (channels
    de-interleaved per head as the reference's loader stores them, pairs (i, i+64))."""

    codes: torch.Tensor
    scales: torch.Tensor
    col_scale: torch.Tensor | None = None
    bias: torch.Tensor | None = None
    rope_pairs: str = "interleaved"

    @property
    def out_features(self) -> int:
        return self.codes.shape[0]

    @property
    def in_features(self) -> int:
        return self.codes.shape[1]


def quantize_weight_mx(weight_kn: torch.Tensor, bias: torch.Tensor | None = None) -> MXWeight:
    """Reference-layout weight ``[K, N]`` (bf16, on the GPU) -> :class:`MXWeight` ``[N, K]``.

    The transpose is a one-time layout change; the quantization runs the adaLN kernel with no
    normalization and MX output, i.e. exactly the activation quantizer, along K.
    """
    if weight_kn.dim() != 2:
        raise ValueError("weight must be [K, N]")
    wt = weight_kn.to(torch.bfloat16).t().contiguous()
    q = adaln_quant_2d(wt, None, None, eps=0.0, norm_type="none", quant="mx")
    b = None if bias is None else bias.reshape(-1).to(torch.float32).contiguous()
    return MXWeight(q.codes, q.scales, None, b)


def packed_weight_to_mx(weight: torch.Tensor, weight_scales: torch.Tensor | None = None,
                        bias: torch.Tensor | None = None, *, rope_pairs: str = "halves") -> MXWeight:
    """The reference's packed ROW_MX projection weight ``[K/4, N, 4]`` float8_e4m3fn (four
    consecutive contraction values innermost, row_mx_modules.py:299-301; ``[H, I]`` packed by
    ``packed_fused_qkv_weight_loader``, row_mx_loaders.py:219-246) -> :class:`MXWeight`.

    The codes are kept as they are (``[N, K]``, K-contiguous), the block scales are neutral (2^0)
    and ``weight_scales`` (``[1, N]``, the checkpoint scalars expanded per channel) becomes the
    per-channel ``col_scale`` of the epilogue -- the ROW_MX dequant ``psum * r_s * c_n``
    (qkv_cte.py:3996-4021). The reference loader de-interleaves the Q/K channels of the fused
    self-attention weight per head (row_mx_loaders.py:26-71), hence ``rope_pairs="halves"``."""
    if weight.dim() != 3 or weight.shape[-1] != 4:
        raise ValueError(f"packed weight must be [K/4, N, 4], got {list(weight.shape)}")
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise ValueError(f"packed weight must be float8_e4m3fn, got {weight.dtype}")
    if rope_pairs not in ("interleaved", "halves"):
        raise ValueError(f"unknown rope_pairs {rope_pairs!r}")
    K4, N, _ = weight.shape
    K = 4 * K4
    if K % 32:
        raise ValueError(f"contraction {K} must be a multiple of 32")
    codes = weight.view(torch.uint8).permute(1, 0, 2).reshape(N, K).contiguous()
    scales = torch.full((N, K // 32), _NEUTRAL_SCALE, dtype=torch.uint8, device=weight.device)
    w = MXWeight(codes.view(torch.float8_e4m3fn), scales, None, None, rope_pairs)
    return _with(w, weight_scales, bias)


def _split_row_packed(packed: torch.Tensor):
    """Reference ROW-packed ``[T, K + 4]`` -> (codes [T, K], neutral scales, row scale [T])."""
    raw = packed.view(torch.uint8)
    K = raw.shape[-1] - 4
    codes = raw[:, :K].contiguous()
    row_scale = raw[:, K:].contiguous().view(torch.float32).reshape(-1)
    scales = torch.full((raw.shape[0], K // 32), _NEUTRAL_SCALE, dtype=torch.uint8, device=raw.device)
    return codes, scales, row_scale


def _as_mx_2d(x):
    """MXTensor / ROW-packed tensor of any leading shape -> (codes2d, scales2d, row_scale, lead)."""
    if isinstance(x, MXTensor):
        if x.codes.dtype not in (torch.float8_e4m3fn, torch.uint8):
            raise ValueError(f"MX codes must be float8_e4m3fn, got {x.codes.dtype}")
        K = x.codes.shape[-1]
        if K % 32:
            raise ValueError(f"MX activation width {K} must be a multiple of 32")
        lead = x.codes.shape[:-1]
        codes = x.codes.reshape(-1, K).view(torch.uint8)
        _lib.expect(x.scales, "activation scales", dtype=torch.uint8, shape=(*lead, K // 32), contiguous=False)
        scales = x.scales.reshape(-1, K // 32)
        if codes.stride(1) != 1 or scales.stride(1) != 1:
            raise ValueError("MX codes and scales must have unit stride along the last dimension")
        return codes, scales, None, lead
    if not isinstance(x, torch.Tensor) or x.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise ValueError("the activation must be an MXTensor or a ROW-packed float8_e4m3fn tensor [..., K + 4]")
    if x.shape[-1] < 36 or (x.shape[-1] - 4) % 32:
        raise ValueError(f"ROW-packed width {x.shape[-1]} must be K + 4 with K a multiple of 32")
    lead = x.shape[:-1]
    codes, scales, row_scale = _split_row_packed(x.reshape(-1, x.shape[-1]))
    return codes, scales, row_scale, lead


def _check_weight(weight: MXWeight, what: str = "weight") -> None:
    if not isinstance(weight, MXWeight):
        raise ValueError(f"{what} must be an MXWeight (see quantize_weight_mx / packed_weight_to_mx)")
    N, K = weight.codes.shape if weight.codes.dim() == 2 else (None, None)
    if N is None or weight.codes.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise ValueError(f"{what}.codes must be float8_e4m3fn [N, K], got {weight.codes.dtype} "
                         f"{list(weight.codes.shape)}")
    if not weight.codes.is_contiguous():
        raise ValueError(f"{what}.codes must be contiguous")
    _lib.expect(weight.scales, f"{what}.scales", dtype=torch.uint8, shape=(N, K // 32))
    _lib.expect(weight.col_scale, f"{what}.col_scale", dtype=torch.float32, shape=(N,), optional=True)
    _lib.expect(weight.bias, f"{what}.bias", dtype=torch.float32, shape=(N,), optional=True)


def mxfp8_linear(
    x,
    weight: MXWeight,
    *,
    epilogue: str = "bf16",
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    row_sumsq: torch.Tensor | None = None,
    sumsq_cols: int = 0,
):
    """``epilogue(x @ W^T * row_scale * col_scale + bias)`` on the MXFP8 GEMM kernel.

    ``x``: :class:`MXTensor` ``[..., K]`` or ROW-packed ``[..., K + 4]``. Returns bf16 ``[..., N]``,
    or an :class:`MXTensor` for ``epilogue="gelu_mx"``. ``gated_residual`` computes
    ``bf16(residual + bf16(y) * gate)`` with ``residual`` bf16 ``[..., N]`` and ``gate`` fp32 ``[N]``.
    ``row_sumsq`` (bf16 epilogue only): fp32 ``[M, N/128]`` receiving, for the column blocks of
    ``[0, sumsq_cols)``, each row's sum of squares of the bf16 outputs of the block (the input of the
    across-heads RMSNorm fused into the attention's Q load).
    """
    if epilogue not in EPILOGUES:
        raise ValueError(f"unknown epilogue {epilogue!r}")
    lib = _lib.load()
    _check_weight(weight)
    codes, scales, row_scale, lead = _as_mx_2d(x)
    M, K = codes.shape
    N = weight.out_features
    if weight.in_features != K:
        raise ValueError(f"activation K={K} does not match weight K={weight.in_features}")
    res2 = None
    if epilogue == "gated_residual":
        if residual is None or gate is None:
            raise ValueError("gated_residual needs residual and gate")
        _lib.expect(residual, "residual", dtype=torch.bfloat16, contiguous=False)
        if residual.numel() != M * N:
            raise ValueError(f"residual must hold [{M}, {N}] elements, got {list(residual.shape)}")
        res2 = residual.reshape(M, N).contiguous()
        _lib.expect(gate, "gate", dtype=torch.float32, contiguous=False)
        if gate.numel() != N:
            raise ValueError(f"gate must hold {N} elements, got {gate.numel()}")
        gate = gate.reshape(N).contiguous()
    elif residual is not None or gate is not None:
        raise ValueError("residual and gate belong to the gated_residual epilogue")
    if out is not None:
        want = torch.uint8 if epilogue == "gelu_mx" else torch.bfloat16
        _lib.expect(out, "out", dtype=want, shape=(M, N), contiguous=False, row_contiguous=True)
        if out.stride(0) % 16 or (epilogue == "gated_residual" and out.stride(0) != N):
            raise ValueError("out must have a row stride that is a multiple of 16 (N for gated_residual)")
    if row_sumsq is not None:
        if epilogue != "bf16":
            raise ValueError("row_sumsq needs the bf16 epilogue")
        _lib.expect(row_sumsq, "row_sumsq", dtype=torch.float32, shape=(M, N // 128))
    _lib.require_gpu(codes, scales, row_scale, weight.codes, weight.scales, weight.col_scale, weight.bias, res2,
                     gate, out, row_sumsq, what="mxfp8_linear")
    dev = codes.device
    out_scales = None
    if epilogue == "gelu_mx":
        out = torch.empty((M, N), dtype=torch.uint8, device=dev) if out is None else out
        out_scales = torch.empty((M, N // 32), dtype=torch.uint8, device=dev)
    else:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev) if out is None else out
    if row_sumsq is not None:
        status = lib.wanmi_mxfp8_gemm_rowsumsq(
            _lib.ptr(codes), _lib.ptr(scales), _lib.ptr(weight.codes), _lib.ptr(weight.scales), _lib.ptr(row_scale),
            _lib.ptr(weight.col_scale), _lib.ptr(weight.bias), M, N, K, codes.stride(0), _lib.ptr(out), out.stride(0),
            _lib.ptr(row_sumsq), int(sumsq_cols), _lib.stream_of(codes),
        )
        _lib.check(status, "wanmi_mxfp8_gemm_rowsumsq")
        return out.reshape(*lead, N)
    status = lib.wanmi_mxfp8_gemm(
        _lib.ptr(codes),
        _lib.ptr(scales),
        _lib.ptr(weight.codes),
        _lib.ptr(weight.scales),
        _lib.ptr(row_scale),
        _lib.ptr(weight.col_scale),
        _lib.ptr(weight.bias),
        M,
        N,
        K,
        codes.stride(0),
        EPILOGUES[epilogue],
        _lib.ptr(out),
        out.stride(0),
        _lib.ptr(out_scales),
        _lib.ptr(res2),
        _lib.ptr(gate if epilogue == "gated_residual" else None),
        _lib.stream_of(codes),
    )
    _lib.check(status, "wanmi_mxfp8_gemm")
    if epilogue == "gelu_mx":
        return MXTensor(out.view(torch.float8_e4m3fn).reshape(*lead, N), out_scales.reshape(*lead, N // 32))
    return out.reshape(*lead, N)


def mxfp8_qkv_linear(x, weight: MXWeight, *, vt_col0: int, row_sumsq: torch.Tensor | None = None,
                     sumsq_cols: int = 0, head_dim: int = 128):
    """The fused ``[Q | K | V]`` projection in the attention's layouts: returns ``(qk, vt)`` with
    ``qk`` bf16 ``[M, vt_col0]`` (the columns before ``vt_col0``, token-major) and ``vt`` bf16
    ``[(N - vt_col0) / 128, 128, S_pad]`` (the V columns transposed per head into the attention
    kernel's key order, S_pad = M rounded up to 64, zero past M). ``row_sumsq``: fp32
    ``[M, vt_col0/128]`` receiving the per-128-column sums of squares of the bf16 outputs for the
    blocks of ``[0, sumsq_cols)``, as in :func:`mxfp8_linear`."""
    lib = _lib.load()
    _check_weight(weight)
    codes, scales, row_scale, lead = _as_mx_2d(x)
    M, K = codes.shape
    N = weight.out_features
    if weight.in_features != K:
        raise ValueError(f"activation K={K} does not match weight K={weight.in_features}")
    if vt_col0 <= 0 or vt_col0 >= N or vt_col0 % 256 or (N - vt_col0) % 256:
        raise ValueError(f"vt_col0={vt_col0} and N - vt_col0 must be multiples of 256 (N={N})")
    if row_sumsq is not None:
        _lib.expect(row_sumsq, "row_sumsq", dtype=torch.float32, shape=(M, vt_col0 // 128))
    _lib.require_gpu(codes, scales, row_scale, weight.codes, weight.scales, weight.col_scale, weight.bias, row_sumsq,
                     what="mxfp8_qkv_linear")
    dev = codes.device
    s_pad = (max(M, 1) + 63) // 64 * 64
    qk = torch.empty((M, vt_col0), dtype=torch.bfloat16, device=dev)
    if M == 0:  # no tokens: nothing to project, V^T is all padding
        return qk.reshape(*lead, vt_col0), torch.zeros(((N - vt_col0) // head_dim, head_dim, s_pad),
                                                       dtype=torch.bfloat16, device=dev)
    vt = torch.empty(((N - vt_col0) // head_dim, head_dim, s_pad), dtype=torch.bfloat16, device=dev)
    status = lib.wanmi_mxfp8_gemm_qkv(
        _lib.ptr(codes), _lib.ptr(scales), _lib.ptr(weight.codes), _lib.ptr(weight.scales), _lib.ptr(row_scale),
        _lib.ptr(weight.col_scale), _lib.ptr(weight.bias), M, N, K, codes.stride(0), _lib.ptr(qk), qk.stride(0),
        _lib.ptr(row_sumsq), int(sumsq_cols) if row_sumsq is not None else 0, _lib.ptr(vt), vt_col0, s_pad,
        _lib.stream_of(codes),
    )
    _lib.check(status, "wanmi_mxfp8_gemm_qkv")
    return qk.reshape(*lead, vt_col0), vt


def row_quantize_packed(hidden: torch.Tensor) -> torch.Tensor:
    """bf16 rows ``[T, H]`` or ``[B, T, H]`` -> ROW-packed ``[..., H + 4]`` float8_e4m3fn bytes: each
    row's e4m3 codes, then the 4 little-endian bytes of its fp32 dequant scale
    ``max(amax / 448, 1e-6)`` (codes = RNE(y / scale)), the layout the ROW_MX projections read.

    Drop-in for the reference's ``row_quantize_packed`` (row_mx_kernels.py:12-45: nkilib's
    rmsnorm_quant with NO_NORM, ROW quantization, no clip bound), which the model runs once per
    generation on the text context before every block's cross-attention K/V projection
    (wan2_2_transformer.py:1686-1691, row_mx_modules.py:509-542). Here it is one launch of the fused
    adaLN kernel in its NO_NORM / ROW mode, whose rule is the ROW branch of adaln_quant_torch.py:
    131-142 (the vendored ROW path that mirrors rmsnorm_quant, adaln_quant.py:472-530). H must be a
    multiple of 32 (at most 16384).
    """
    if hidden.dim() not in (2, 3):
        raise ValueError(f"row_quantize_packed expects [T, H] or [B, T, H], got {tuple(hidden.shape)}")
    if hidden.dtype != torch.bfloat16:
        raise ValueError(f"row_quantize_packed expects bf16 rows, got {hidden.dtype}")
    H = hidden.shape[-1]
    packed = adaln_quant_2d(hidden.reshape(-1, H), None, None, eps=1e-6, norm_type="none", quant="row")
    return packed.view(*hidden.shape[:-1], H + 4)


def row_mx_mlp(
    packed_hidden,
    up_weight: MXWeight,
    down_weight: MXWeight,
    up_w_scale: torch.Tensor | None = None,
    down_w_scale: torch.Tensor | None = None,
    up_bias: torch.Tensor | None = None,
    down_bias: torch.Tensor | None = None,
):
    """Wan's gate-less GELU-tanh MLP: ``down(MX(GELU_tanh(up(x) + b_up))) + b_down``.

    Same argument order as the reference (row_mx_kernels.py:141-149). ``packed_hidden`` is the
    ROW-packed ``[..., H + 4]`` activation of ``adaln_modulate(quant="row")`` or an :class:`MXTensor`.
    ``*_w_scale`` are the per-output-channel fp32 dequant scales of the ROW_MX recipe (``[N]``,
    ``[1, N]``, or the reference's partition-expanded ``[P, N]`` whose rows are equal; row 0 is used);
    biases override the weights' own. Returns bf16 ``[..., H]``.
    """
    up = _with(up_weight, up_w_scale, up_bias)
    down = _with(down_weight, down_w_scale, down_bias)
    inter = mxfp8_linear(packed_hidden, up, epilogue="gelu_mx")
    return mxfp8_linear(inter, down, epilogue="bf16")


def _channel_vector(t: torch.Tensor | None, n: int, what: str) -> torch.Tensor | None:
    """A per-output-channel fp32 vector given as ``[n]``, ``[1, n]`` or ``[P, n]`` (rows equal; the
    reference expands its scalar scales over partitions) -> contiguous fp32 ``[n]``."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or t.dim() == 0 or t.shape[-1] != n:
        raise ValueError(f"{what} must be [{n}], [1, {n}] or [P, {n}], got "
                         f"{list(t.shape) if isinstance(t, torch.Tensor) else type(t).__name__}")
    if not t.is_floating_point():
        raise ValueError(f"{what} must be floating point, got {t.dtype}")
    return t.reshape(-1, n)[0].to(torch.float32).contiguous()


def _with(w: MXWeight, col_scale, bias) -> MXWeight:
    _check_weight(w)
    n = w.out_features
    cs = w.col_scale if col_scale is None else _channel_vector(col_scale, n, "weight scale")
    b = w.bias if bias is None else _channel_vector(bias, n, "bias")
    return MXWeight(w.codes, w.scales, cs, b, w.rope_pairs)
