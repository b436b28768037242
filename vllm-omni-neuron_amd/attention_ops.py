"""Wan attention on gfx950: QK normalization + RoPE, constant-max attention, and the projections
around it.

Drop-ins for the reference's attention-side op boundary:

- :func:`wan_cp_self_attention` (vllm_omni_neuron/diffusion/models/wan2_2/wan2_2_transformer.py:
  806-847): token-major ``[B, S, N, D]`` q/k/v -> d-major ``[B, N, D, S]``. One GPU: ``cp_size`` must
  be 1 (the reference's ring over a context-parallel group is the multi-GPU variant).
- :func:`_nki_attend` (wan2_2_transformer.py:653-674): ``[B, N, S, D]`` -> ``[B, N, D, S]``.
- :func:`ring_attention_const_max_fwd` (kernels/nkilib/experimental/attention/
  ring_attention_const_max_fwd.py:959): token-major ``[b, S, h, d]`` -> ``[b, h, S, d]``.
- :func:`row_mx_qkv_proj` (diffusion/quantization/row_mx_kernels.py:48-111): fused projection +
  across-heads QK RMSNorm + RoPE.
- :func:`row_mx_o_proj` (row_mx_kernels.py:114-138): d-major attention -> ``[B, S, H]``.

All attention here is the constant-max form (exact softmax by shift invariance, no running max):
``c_i = s ||q_i|| max_j ||k_j||`` with the key norms taken over the whole key sequence on the GPU.
"""

from __future__ import annotations

from typing import NamedTuple

import math

import torch

from . import _lib
from .adaln_kernels import adaln_quant_2d
from .common_types import MXTensor, NormType, QKVOutputLayout
from .row_mx_kernels import MXWeight, _with, mxfp8_linear  # noqa: F401

HEAD_DIM = 128
OUT_TOKEN, OUT_DMAJOR, OUT_MX = 0, 1, 2


def _pad64(n: int) -> int:
    return (n + 63) // 64 * 64


def rope_pair_tables(cos: torch.Tensor, sin: torch.Tensor):
    """Wan interleaved tables ``[..., S, (1,) 128]`` -> one angle per pair, fp32 ``[S, 64]``
    (``cos[..., 0::2]``, ``sin[..., 1::2]`` exactly as ``apply_rotary_emb_wan`` reads them)."""
    c = cos.reshape(-1, cos.shape[-1])[:, 0::2]
    s = sin.reshape(-1, sin.shape[-1])[:, 1::2]
    return c.to(torch.float32).contiguous(), s.to(torch.float32).contiguous()


_ROTATE = {"interleaved": 0, "halves": 1}


def _check_rope_tables(cos, sin, S: int, what: str) -> None:
    """cos / sin: both None, or fp32 contiguous ``[S, 64]`` pair tables for the S rows."""
    if (cos is None) != (sin is None):
        raise ValueError(f"{what}: cos and sin must both be given or both be None")
    if cos is not None:
        _lib.expect(cos, f"{what}: cos", dtype=torch.float32, shape=(S, HEAD_DIM // 2))
        _lib.expect(sin, f"{what}: sin", dtype=torch.float32, shape=(S, HEAD_DIM // 2))


def qk_rmsnorm_rope_(x: torch.Tensor, gamma: torch.Tensor, *, cos=None, sin=None, eps: float = 1e-6,
                     want_max: bool = False, rope_pairs: str = "interleaved", q_sumsq: torch.Tensor | None = None,
                     q_rr: torch.Tensor | None = None, q_eps: float | None = None):
    """In place on a bf16 ``[S, heads*128]`` view (unit column stride): across-heads RMSNorm * gamma,
    then RoPE with pair tables ``cos``/``sin`` fp32 ``[S, 64]`` when given, on the channel pairs
    ``rope_pairs`` names (``"interleaved"``: (2i, 2i+1); ``"halves"``: (i, i+64), the rotate-half
    order of de-interleaved channels). Returns the per-head max norm ``[heads]`` (fp32) when
    ``want_max``.

    ``q_sumsq`` (fp32 ``[S, >= heads]``, the QKV GEMM's per-128-column partial sums of squares of Q)
    with ``q_rr`` (fp32 ``[S]``, written): also the queries' across-heads 1/rms, for the attention's
    fused Q preparation (``QPrep(rr=q_rr)``), with ``q_eps`` (default ``eps``)."""
    lib = _lib.load()
    if rope_pairs not in _ROTATE:
        raise ValueError(f"unknown rope_pairs {rope_pairs!r}")
    if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.stride(1) != 1 or x.dtype != torch.bfloat16:
        raise ValueError("x must be a bf16 [S, heads*128] view with unit column stride")
    S, W = x.shape
    if W % (4 * HEAD_DIM):
        raise ValueError(f"x width {W} must be a multiple of {4 * HEAD_DIM} (heads a multiple of 4)")
    if x.stride(0) % 8 or x.data_ptr() % 16:
        raise ValueError("x rows must be 16-byte aligned")
    heads = W // HEAD_DIM
    if not isinstance(gamma, torch.Tensor) or gamma.numel() != W or not gamma.is_floating_point():
        raise ValueError(f"gamma must be a floating-point tensor of {W} elements")
    _check_rope_tables(cos, sin, S, "qk_rmsnorm_rope")
    _lib.require_gpu(x, gamma, cos, sin, what="qk_rmsnorm_rope")
    gamma = gamma.reshape(W).to(torch.float32).contiguous()
    kmax = torch.empty(heads, dtype=torch.float32, device=x.device) if want_max else None
    if (q_sumsq is None) != (q_rr is None):
        raise ValueError("q_sumsq and q_rr go together")
    if q_rr is not None:
        _lib.expect(q_sumsq, "q_sumsq", dtype=torch.float32, shape=(S, None), contiguous=False, row_contiguous=True)
        if q_sumsq.shape[1] < heads:
            raise ValueError(f"q_sumsq needs at least {heads} partial sums per row")
        _lib.expect(q_rr, "q_rr", dtype=torch.float32, shape=(S,))
        _lib.require_gpu(q_sumsq, q_rr, x, what="qk_rmsnorm_rope")
        st = lib.wanmi_qk_rmsnorm_rope_qrr(
            _lib.ptr(x), S, x.stride(0), heads, _lib.ptr(gamma), _lib.ptr(cos), _lib.ptr(sin), _ROTATE[rope_pairs],
            float(eps), _lib.ptr(kmax), _lib.ptr(q_sumsq), q_sumsq.stride(0), heads,
            float(eps if q_eps is None else q_eps), _lib.ptr(q_rr), _lib.stream_of(x),
        )
        _lib.check(st, "wanmi_qk_rmsnorm_rope_qrr")
        return kmax
    st = lib.wanmi_qk_rmsnorm_rope(
        _lib.ptr(x), S, x.stride(0), heads, _lib.ptr(gamma), _lib.ptr(cos), _lib.ptr(sin), _ROTATE[rope_pairs],
        float(eps), _lib.ptr(kmax), _lib.stream_of(x),
    )
    _lib.check(st, "wanmi_qk_rmsnorm_rope")
    return kmax


def qk_rmsnorm_rope_to(x: torch.Tensor, out: torch.Tensor, gamma: torch.Tensor, *, cos=None, sin=None,
                       eps: float = 1e-6, rope_pairs: str = "interleaved") -> torch.Tensor:
    """:func:`qk_rmsnorm_rope_` with the result written to ``out`` instead of back into ``x``: ``out``
    a bf16 ``[S, heads, 128]`` view with unit d stride and any token / head strides (the head-major
    ``[heads, S, 128]`` layout as ``.permute(1, 0, 2)``, for instance), at most 40 heads. Same bits."""
    lib = _lib.load()
    if rope_pairs not in _ROTATE:
        raise ValueError(f"unknown rope_pairs {rope_pairs!r}")
    if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.stride(1) != 1 or x.dtype != torch.bfloat16:
        raise ValueError("x must be a bf16 [S, heads*128] view with unit column stride")
    S, W = x.shape
    if W % (4 * HEAD_DIM) or W > 40 * HEAD_DIM:
        raise ValueError(f"x width {W} must be a multiple of {4 * HEAD_DIM}, at most {40 * HEAD_DIM}")
    if x.stride(0) % 8 or x.data_ptr() % 16:
        raise ValueError("x rows must be 16-byte aligned")
    heads = W // HEAD_DIM
    if not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or tuple(out.shape) != (S, heads, HEAD_DIM) \
            or out.stride(2) != 1 or out.stride(0) % 8 or out.stride(1) % 8 or out.data_ptr() % 16:
        raise ValueError(f"out must be a bf16 [{S}, {heads}, {HEAD_DIM}] view with unit d stride, 16-byte aligned rows")
    if not isinstance(gamma, torch.Tensor) or gamma.numel() != W or not gamma.is_floating_point():
        raise ValueError(f"gamma must be a floating-point tensor of {W} elements")
    _check_rope_tables(cos, sin, S, "qk_rmsnorm_rope_to")
    _lib.require_gpu(x, out, gamma, cos, sin, what="qk_rmsnorm_rope_to")
    gamma = gamma.reshape(W).to(torch.float32).contiguous()
    st = lib.wanmi_qk_rmsnorm_rope_to(
        _lib.ptr(x), S, x.stride(0), heads, _lib.ptr(gamma), _lib.ptr(cos), _lib.ptr(sin), _ROTATE[rope_pairs],
        float(eps), _lib.ptr(out), out.stride(0), out.stride(1), _lib.stream_of(x),
    )
    _lib.check(st, "wanmi_qk_rmsnorm_rope_to")
    return out


def transpose_heads(v: torch.Tensor):
    """bf16 ``[S, N, 128]`` (any strides with unit d stride) -> V^T ``[N, 128, S_pad]`` in the
    attention kernel's key order; returns ``(vt, S_pad)``."""
    lib = _lib.load()
    _lib.require_gpu(v, what="transpose_heads")
    if v.dim() != 3 or v.shape[-1] != HEAD_DIM or v.stride(2) != 1:
        raise ValueError("v must be [S, N, 128] with unit d stride")
    S, N, _ = v.shape
    S_pad = _pad64(max(S, 1))
    vt = torch.empty((N, HEAD_DIM, S_pad), dtype=torch.bfloat16, device=v.device)
    st = lib.wanmi_transpose_heads(_lib.ptr(v), S, v.stride(0), v.stride(1), N, _lib.ptr(vt), S_pad, _lib.stream_of(v))
    _lib.check(st, "wanmi_transpose_heads")
    return vt, S_pad


def head_max_norm(k: torch.Tensor) -> torch.Tensor:
    """bf16 ``[S, N, 128]`` (unit d stride) -> fp32 ``[N]``: max over tokens of each head's norm."""
    lib = _lib.load()
    _lib.require_gpu(k, what="head_max_norm")
    S, N, _ = k.shape
    out = torch.empty(N, dtype=torch.float32, device=k.device)
    st = lib.wanmi_head_max_norm(_lib.ptr(k), k.stride(1), k.stride(0), S, N, _lib.ptr(out), _lib.stream_of(k))
    _lib.check(st, "wanmi_head_max_norm")
    return out


class QPrep(NamedTuple):
    """Q preparation fused into the attention's Q load: ``sumsq`` fp32 ``[Sq, >= N]`` per-128-column
    partial sums of squares of the raw q rows (from ``mxfp8_linear(..., row_sumsq=...)``), ``gamma``
    fp32 ``[N*128]`` (the across-heads RMSNorm weight), optional RoPE pair tables ``cos``/``sin``
    fp32 ``[Sq, 64]``, and the norm's ``eps``. ``rr`` (fp32 ``[Sq]``): each query's 1/rms already
    computed from those partials (``qk_rmsnorm_rope_(..., q_sumsq=, q_rr=)``); given, ``sumsq`` and
    ``eps`` are not used and the Q load reads one float per query."""

    sumsq: torch.Tensor | None
    gamma: torch.Tensor
    cos: torch.Tensor | None = None
    sin: torch.Tensor | None = None
    eps: float = 1e-6
    rr: torch.Tensor | None = None


def attention_core(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, kmax: torch.Tensor, scale: float,
                   out_mode: int = OUT_TOKEN, out: torch.Tensor | None = None, q_prep: QPrep | None = None,
                   exact: bool = False):
    """Constant-max attention on ``[S, N, 128]`` views q (Sq) and k (Sk), V^T from
    :func:`transpose_heads`. Returns token-major bf16 ``[Sq, N*128]``, d-major bf16
    ``[N, 128, Sq]`` or an :class:`MXTensor` ``[Sq, N*128]``. With ``q_prep`` q is the raw
    projection and the kernel applies the across-heads RMSNorm (and RoPE) to it on load, exactly as
    :func:`qk_rmsnorm_rope_` would in a separate pass.

    ``exact``: the semantics of a running-max softmax for any inputs (``wanmi_attention_exact``):
    rows whose constant-max row sum underflowed (the bound exceeded the row's largest logit by more
    than about 87) are recomputed with the row's true max. Token-major and d-major outputs only,
    without ``q_prep``. The constant-max reference kernels (the ring attention and the block's own
    path) do not do this."""
    lib = _lib.load()
    if exact and (q_prep is not None or out_mode == OUT_MX):
        raise ValueError("exact attention produces token-major or d-major bf16 output from prepared q")
    if q.dim() != 3 or k.dim() != 3 or q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise ValueError("q, k must be bf16 [S, N, 128] views")
    Sq, N, D = q.shape
    Sk = k.shape[0]
    if D != HEAD_DIM or k.shape[1:] != (N, D) or q.stride(2) != 1 or k.stride(2) != 1:
        raise ValueError("q, k must be [S, N, 128] with unit d stride and matching heads")
    _lib.expect(vt, "vt", dtype=torch.bfloat16, shape=(N, D, None))
    if vt.shape[-1] < Sk or vt.shape[-1] % 64:
        raise ValueError(f"vt must be [N, 128, S_pad] with S_pad >= {Sk} a multiple of 64 (transpose_heads)")
    _lib.expect(kmax, "kmax", dtype=torch.float32, shape=(N,))
    if out is not None:
        if out_mode == OUT_TOKEN:
            _lib.expect(out, "out", dtype=torch.bfloat16, shape=(Sq, N * D), contiguous=False, row_contiguous=True)
        elif out_mode == OUT_DMAJOR:
            _lib.expect(out, "out", dtype=torch.bfloat16, shape=(N, D, Sq), contiguous=False, row_contiguous=True)
        else:
            _lib.expect(out, "out", dtype=torch.uint8, shape=(Sq, N * D), contiguous=False, row_contiguous=True)
    if out_mode not in (OUT_TOKEN, OUT_DMAJOR, OUT_MX):
        raise ValueError(f"unknown out_mode {out_mode}")
    if q_prep is not None:
        if q_prep.rr is not None:
            _lib.expect(q_prep.rr, "q_prep.rr", dtype=torch.float32, shape=(Sq,))
        else:
            _lib.expect(q_prep.sumsq, "q_prep.sumsq", dtype=torch.float32, shape=(Sq, None), contiguous=False,
                        row_contiguous=True)
            if q_prep.sumsq.shape[1] < N:
                raise ValueError(f"q_prep.sumsq needs at least {N} partial sums per row")
        if not isinstance(q_prep.gamma, torch.Tensor) or q_prep.gamma.numel() != N * D:
            raise ValueError(f"q_prep.gamma must hold {N * D} elements")
        _check_rope_tables(q_prep.cos, q_prep.sin, Sq, "attention q_prep")
        _lib.require_gpu(q_prep.sumsq, q_prep.rr, q_prep.gamma, q_prep.cos, q_prep.sin, what="attention")
    _lib.require_gpu(q, k, vt, kmax, out, what="attention")
    dev = q.device
    scales = None
    if out_mode == OUT_TOKEN:
        out = torch.empty((Sq, N * D), dtype=torch.bfloat16, device=dev) if out is None else out
        o_hs, o_ss, o_ds = D, out.stride(0), 1
    elif out_mode == OUT_DMAJOR:
        out = torch.empty((N, D, Sq), dtype=torch.bfloat16, device=dev) if out is None else out
        o_hs, o_ss, o_ds = out.stride(0), 1, out.stride(1)
    else:
        out = torch.empty((Sq, N * D), dtype=torch.uint8, device=dev) if out is None else out
        scales = torch.empty((Sq, N * D // 32), dtype=torch.uint8, device=dev)
        o_hs, o_ss, o_ds = D, out.stride(0), 1
    common = (
        _lib.ptr(q), q.stride(1), q.stride(0), _lib.ptr(k), k.stride(1), k.stride(0), _lib.ptr(vt),
        vt.shape[-1], _lib.ptr(kmax), Sq, Sk, N, D, float(scale), out_mode, _lib.ptr(out), o_hs, o_ss, o_ds,
        _lib.ptr(scales), 0 if scales is None else scales.stride(0),
    )
    if exact:
        row_sum = torch.empty((N, Sq), dtype=torch.float32, device=dev)
        st = lib.wanmi_attention_exact(*common[:-2], _lib.ptr(row_sum), _lib.stream_of(q))
        _lib.check(st, "wanmi_attention_exact")
    elif q_prep is None:
        st = lib.wanmi_attention_const_max(*common, _lib.stream_of(q))
        _lib.check(st, "wanmi_attention_const_max")
    elif q_prep.rr is not None:
        gamma = q_prep.gamma.reshape(-1).to(torch.float32).contiguous()
        st = lib.wanmi_attention_const_max_qrr(
            *common, _lib.ptr(q_prep.rr), _lib.ptr(gamma), _lib.ptr(q_prep.cos), _lib.ptr(q_prep.sin),
            _lib.stream_of(q),
        )
        _lib.check(st, "wanmi_attention_const_max_qrr")
    else:
        ss = q_prep.sumsq
        gamma = q_prep.gamma.reshape(-1).to(torch.float32).contiguous()
        st = lib.wanmi_attention_const_max_qprep(
            *common, _lib.ptr(ss), ss.stride(0), _lib.ptr(gamma), _lib.ptr(q_prep.cos), _lib.ptr(q_prep.sin),
            float(q_prep.eps), _lib.stream_of(q),
        )
        _lib.check(st, "wanmi_attention_const_max_qprep")
    if out_mode == OUT_MX:
        return MXTensor(out.view(torch.float8_e4m3fn), scales)
    return out


def _attend_bsnd(q, k, v, scale, out_mode, exact):
    """One batch element: q [Sq, N, D], k/v [Sk, N, D] (unit d stride). ``exact``: running-max
    softmax semantics (rows whose constant-max sum underflowed are recomputed, see attention_core)."""
    vt, _ = transpose_heads(v)
    return attention_core(q, k, vt, head_max_norm(k), scale, out_mode, exact=exact)


def wan_cp_self_attention(query, key, value, scale, cp_size=1, cp_group=None, cp_replica_groups=None):
    """Token-major ``[B, S, N, D]`` q/k/v (already normalized and rotated) -> d-major
    ``[B, N, D, S]`` (the layout the o-projection consumes)."""
    if cp_size != 1:
        raise NotImplementedError("context-parallel attention spans several GPUs; this build runs on one")
    outs = [_attend_bsnd(query[b], key[b], value[b], scale, OUT_DMAJOR, True) for b in range(query.shape[0])]
    return torch.stack(outs, dim=0) if len(outs) > 1 else outs[0].unsqueeze(0)


def _nki_attend(query, key, value, scale):
    """Non-causal attention over ``[B, N, S, D]`` q/k/v -> d-major ``[B, N, D, S_q]``."""
    outs = [
        _attend_bsnd(query[b].transpose(0, 1), key[b].transpose(0, 1), value[b].transpose(0, 1), scale, OUT_DMAJOR,
                     True)
        for b in range(query.shape[0])
    ]
    return torch.stack(outs, dim=0) if len(outs) > 1 else outs[0].unsqueeze(0)


def attention_cte(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """The reference's registered attention op ``wan_transformer::attention_cte``
    (wan2_2_transformer.py:165-171, launching ``_wan_attention_kernel`` 83-108): ``[BN, S_q, 128]``
    q already multiplied by the softmax scale, ``[BN, S_k, 128]`` k and v, non-causal, unit scale,
    d-major ``[BN, 128, S_q]`` out. Each of the BN rows is one head of the constant-max kernel."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3 or q.shape[0] != k.shape[0] or k.shape != v.shape:
        raise ValueError(f"attention_cte expects [BN, S, 128] q/k/v, got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    return _attend_bsnd(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), 1.0, OUT_DMAJOR, True)


def register_torch_ops() -> bool:
    """Registers :func:`attention_cte` as the functional torch op ``wan_transformer::attention_cte``
    (``mutates_args=()``, as the reference's ``nki_op`` registration, lite_compat.py:88-95), with a
    fake implementation for shape propagation. Returns False, registering nothing, when an op of
    that name already exists in the process."""
    if hasattr(torch.ops, "wan_transformer") and hasattr(torch.ops.wan_transformer, "attention_cte"):
        return False
    op = torch.library.custom_op("wan_transformer::attention_cte", attention_cte, mutates_args=())

    @op.register_fake
    def _(q, k, v):
        return q.new_empty((q.shape[0], q.shape[2], q.shape[1]))

    return True


def ring_attention_const_max_fwd(q, k, v, replica_groups=None, num_workers=1, softmax_scale=None,
                                 training=False, lse_dtype=None, kv_prefetch_depth=2):
    """Token-major ``[b, S, h, d]`` q/k/v -> ``[b, h, S, d]`` with the constant-max softmax.

    One GPU holds the whole sequence, so the ring has a single member (``num_workers`` must be 1)
    and ``kv_prefetch_depth`` has nothing to prefetch. ``training=True`` (log-sum-exp output) is not
    part of the inference path and is rejected.
    """
    if num_workers != 1 or replica_groups:
        raise NotImplementedError("a multi-member ring spans several GPUs; this build runs on one")
    if training:
        raise NotImplementedError("the log-sum-exp output (training=True) is not produced")
    if q.shape[-1] != HEAD_DIM:
        raise ValueError(f"head_dim must be 128, got {q.shape[-1]}")
    scale = softmax_scale or 1.0 / math.sqrt(q.shape[-1])
    outs = []
    for b in range(q.shape[0]):
        o = _attend_bsnd(q[b], k[b], v[b], scale, OUT_TOKEN, False)  # [S, h*d], the ring kernel's constant max
        outs.append(o.view(q.shape[1], q.shape[2], HEAD_DIM).transpose(0, 1))
    return torch.stack(outs, dim=0)


def _base_angles(cache: torch.Tensor, B: int, S: int, what: str) -> list[torch.Tensor]:
    """Rotate-half cache ``[B, S, 128]`` (or ``[S, 128]``, ``[1, S, 128]``) = ``cat([base, base])``
    (row_mx_modules.py:51-76) -> per batch element the fp32 ``[S, 64]`` base angles."""
    if not isinstance(cache, torch.Tensor) or cache.shape[-1] != HEAD_DIM or cache.dim() not in (2, 3):
        raise ValueError(f"{what} must be [B, S, {HEAD_DIM}] (rotate-half cache)")
    c = cache if cache.dim() == 3 else cache.unsqueeze(0)
    if c.shape[1] != S or c.shape[0] not in (1, B):
        raise ValueError(f"{what} must be [{B}, {S}, {HEAD_DIM}], got {list(cache.shape)}")
    return [c[min(b, c.shape[0] - 1), :, : HEAD_DIM // 2].to(torch.float32).contiguous() for b in range(B)]


def _norm_kind(kind, what: str) -> bool:
    """True for the across-heads RMSNorm, False for none; anything else is not on the Wan path."""
    if kind is None or kind == NormType.NO_NORM:
        return False
    if kind == NormType.RMS_NORM_ACROSS_HEADS:
        return True
    raise NotImplementedError(f"{what}={kind} is not supported (the Wan path uses RMS_NORM_ACROSS_HEADS)")


def row_mx_qkv_proj(
    packed_hidden,
    weight,
    weight_scales: torch.Tensor | None = None,
    bias: torch.Tensor | None = None,
    *,
    num_heads: int,
    head_dim: int,
    num_kv_heads: int = 0,
    fused_rope: bool = False,
    cos_cache: torch.Tensor | None = None,
    sin_cache: torch.Tensor | None = None,
    qk_norm_pre_rope=None,
    qk_norm_pre_rope_q_gamma: torch.Tensor | None = None,
    qk_norm_pre_rope_k_gamma: torch.Tensor | None = None,
    norm_eps: float = 1e-6,
    replica_groups=None,
    output_layout=None,
):
    """Fused ``[Q | K | V]`` projection with the across-heads QK RMSNorm and RoPE applied to Q/K.

    ``packed_hidden``: the ROW-packed ``[B, S, H + 4]`` activation (``adaln_modulate(quant="row")``)
    or an :class:`MXTensor`. ``weight``: the reference's packed ``[H/4, I, 4]`` float8_e4m3fn weight
    (Q/K channels de-interleaved per head, as its loader stores them) or an :class:`MXWeight`;
    ``weight_scales`` ``[1, I]`` and ``bias`` ``[1, I]`` as the reference passes them.
    ``cos_cache``/``sin_cache`` are the rotate-half caches ``[B, S, head_dim]`` (``cat([base,
    base])``, row_mx_modules.py:51-76). RoPE rotates the channel pairs of the weight's order: the
    halves (i, i+64) for the reference's de-interleaved weight (rotate-half, as its kernel does),
    Wan's interleaved pairs for an :class:`MXWeight` in natural order (``rope_pairs``). Either way
    Q.K equals Wan's interleaved RoPE. Returns bf16 ``[B, S, (nq + 2 nkv) * d]`` (BSD) or
    ``[nq + 2 nkv, B, S, d]`` (NBSd), in the weight's channel order.
    """
    from .row_mx_kernels import packed_weight_to_mx

    if head_dim != HEAD_DIM:
        raise NotImplementedError(f"head_dim must be {HEAD_DIM}, got {head_dim}")
    if replica_groups:
        raise NotImplementedError("tensor-parallel replica groups span several GPUs")
    if output_layout not in (None, QKVOutputLayout.BSD, QKVOutputLayout.NBSd):
        raise ValueError(f"unknown output_layout {output_layout}")
    w = packed_weight_to_mx(weight, weight_scales, bias) if isinstance(weight, torch.Tensor) else _with(
        weight, weight_scales, bias)
    nq, nkv = num_heads, num_kv_heads
    width = (nq + 2 * nkv) * head_dim
    if w.out_features != width:
        raise ValueError(f"weight has {w.out_features} output channels, expected (num_heads + 2 num_kv_heads) "
                         f"* head_dim = {width}")
    norm = qk_norm_pre_rope
    eps = norm.eps if norm is not None else norm_eps
    norm_q = _norm_kind(norm.q_norm if norm is not None else None, "q_norm")
    norm_k = nkv > 0 and _norm_kind(norm.k_norm if norm is not None else None, "k_norm")
    if norm_q and qk_norm_pre_rope_q_gamma is None:
        raise ValueError("the Q norm needs qk_norm_pre_rope_q_gamma")
    if norm_k and qk_norm_pre_rope_k_gamma is None:
        raise ValueError("the K norm needs qk_norm_pre_rope_k_gamma")
    if fused_rope and not (norm_q and (nkv == 0 or norm_k)):
        # the rotation rides on the norm pass; the Wan self-attention always normalizes both
        raise NotImplementedError("fused RoPE is applied together with the across-heads Q and K norms")

    y = mxfp8_linear(packed_hidden, w)
    lead = y.shape[:-1]
    B, S = (1, lead[0]) if len(lead) == 1 else (math.prod(lead[:-1]), lead[-1])
    y2 = y.reshape(B * S, width)
    cos = sin = [None] * B
    if fused_rope:
        if cos_cache is None or sin_cache is None:
            raise ValueError("fused_rope needs cos_cache and sin_cache")
        cos = _base_angles(cos_cache, B, S, "cos_cache")
        sin = _base_angles(sin_cache, B, S, "sin_cache")
    nbsd = output_layout == QKVOutputLayout.NBSd
    # NBSd: the norm passes write their heads straight into the head-major result (up to 40 heads a
    # pass); the other heads are copied there
    out = torch.empty(width // head_dim, B, S, head_dim, dtype=y.dtype, device=y.device) if nbsd else None
    direct = [False, False]
    for b in range(B):  # the caches may differ per batch element; the norm is per row
        rows = y2[b * S : (b + 1) * S]
        for i, (on, h0, nh, gam) in enumerate(((norm_q, 0, nq, qk_norm_pre_rope_q_gamma),
                                               (norm_k, nq, nkv, qk_norm_pre_rope_k_gamma))):
            if not on:
                continue
            part = rows[:, h0 * head_dim : (h0 + nh) * head_dim]
            if nbsd and nh <= 40:
                qk_rmsnorm_rope_to(part, out[h0 : h0 + nh, b].permute(1, 0, 2), gam, cos=cos[b], sin=sin[b], eps=eps,
                                   rope_pairs=w.rope_pairs)
                direct[i] = True
            else:
                qk_rmsnorm_rope_(part, gam, cos=cos[b], sin=sin[b], eps=eps, rope_pairs=w.rope_pairs)
    if not nbsd:
        return y
    heads_all = y.reshape(B, S, width // head_dim, head_dim)
    done = [(0, nq)] if direct[0] else []
    done += [(nq, nq + nkv)] if direct[1] else []
    start = 0
    for lo, hi in done + [(width // head_dim, width // head_dim)]:
        if lo > start:  # heads not written by a norm pass
            out[start:lo].copy_(heads_all[:, :, start:lo].permute(2, 0, 1, 3))
        start = hi
    return out.reshape(width // head_dim, *lead, head_dim)


def row_mx_o_proj(attention: torch.Tensor, weight: MXWeight, weight_scales: torch.Tensor | None = None,
                  bias: torch.Tensor | None = None) -> torch.Tensor:
    """d-major bf16 attention ``[B, N, D, S]`` -> ``[B, S, H]``: the activation is MX-quantized along
    N*D (the reference's kernel quantizes it internally) and projected with the MXFP8 GEMM.
    ``weight_scales`` ``[P, H]`` / ``[1, H]`` / ``[H]`` (the reference expands its scalar scale over
    partitions, row_mx_modules.py:243-250) and ``bias`` ``[1, H]`` override the weight's own."""
    if not isinstance(attention, torch.Tensor) or attention.dim() != 4 or attention.dtype != torch.bfloat16:
        raise ValueError("attention must be bf16 [B, N, D, S]")
    w = _with(weight, weight_scales, bias)
    B, N, D, S = attention.shape
    if N * D != w.in_features:
        raise ValueError(f"attention has N*D = {N * D} channels, the weight contracts {w.in_features}")
    xq = dmajor_to_mx(attention)
    y = mxfp8_linear(xq, w)
    return y.reshape(B, S, -1)


def dmajor_to_mx(attention: torch.Tensor) -> MXTensor:
    """d-major bf16 ``[B, N, 128, S]`` -> the token-major MX activation ``[B*S, N*128]`` (codes + one
    e8m0 scale per 32 channels), in one pass (``wanmi_dmajor_to_mx``) when the token axis is
    contiguous with S and the strides multiples of 8; otherwise a transposing copy and the adaLN
    kernel's NO_NORM / MX mode, which give the same bits."""
    if not isinstance(attention, torch.Tensor) or attention.dim() != 4 or attention.dtype != torch.bfloat16:
        raise ValueError("attention must be bf16 [B, N, D, S]")
    B, N, D, S = attention.shape
    if D != HEAD_DIM:
        raise NotImplementedError(f"head_dim {D} (only {HEAD_DIM} is built)")
    lib = _lib.load()
    _lib.require_gpu(attention, what="dmajor_to_mx")
    bs, hs, ds, ss = attention.stride()
    if (B * S == 0 or ss != 1 or S % 8 or ds < S or bs % 8 or hs % 8 or ds % 8
            or attention.data_ptr() % 16):
        x = attention.permute(0, 3, 1, 2).reshape(B * S, N * D).contiguous()
        return adaln_quant_2d(x, None, None, eps=0.0, norm_type="none", quant="mx")
    codes = torch.empty(B * S, N * D, dtype=torch.uint8, device=attention.device)
    scales = torch.empty(B * S, N * D // 32, dtype=torch.uint8, device=attention.device)
    _lib.check(lib.wanmi_dmajor_to_mx(_lib.ptr(attention), B, N, S, bs, hs, ds, _lib.ptr(codes), _lib.ptr(scales),
                                      _lib.stream_of(attention)), "wanmi_dmajor_to_mx")
    return MXTensor(codes.view(torch.float8_e4m3fn), scales)
