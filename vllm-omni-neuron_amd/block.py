"""The Wan2.2 DiT transformer block and the 40-block forward on the gfx950 kernels.

Follows ``WanTransformerBlock.forward`` (vllm_omni_neuron/diffusion/models/wan2_2/
wan2_2_transformer.py:1428-1513) with every projection in MXFP8 and attention in bf16:

    e = scale_shift_table + temb                     -> shift, scale, gate, c_shift, c_scale, c_gate
    a1 = MX(LN(h) * (1 + scale) + shift)              adaLN kernel
    q, k, V^T = a1 @ Wqkv + b                         MXFP8 GEMM (+ per-row sums of q^2 per 128 columns;
                                                      V written transposed for the attention)
    k = RoPE(RMS_heads(k) g_k), max||k||              prep kernel
    o1 = MX(attention(RoPE(RMS_heads(q) g_q), k, v))  constant-max attention, Q prepared on load, MX out
    h1 = h + gate * (o1 @ Wo + b);  a2 = MX(LN_affine(h1))          GEMM (gated residual) + adaLN
    o2 = MX(attention(RMS_heads(a2 @ Wq2 + b) g_q2, K2, V2))    GEMM (+ sums of q2^2) + cross-attention
    h2 = h1 + (o2 @ Wo2 + b);  a3 = MX(LN(h2) * (1 + c_scale) + c_shift)    GEMM (residual) + adaLN
    h3 = h2 + c_gate * (MX(GELU_tanh(a3 @ Wup + b)) @ Wdown + b)     GEMM (GELU+MX) + GEMM (gated residual)

Every residual add runs in the epilogue of the GEMM that produces the branch, as
``bf16(residual + bf16(y) * gate)`` (fp32 product, then the sum; gate 1 for the cross-attention
branch): the reference does the first two adds in its adaLN kernel (adaln_kernels.py:58-66 for the
eager form) with the same fp32 product and sum of the bf16 branch output, so the results are the
same bits, and the bf16 branch output never makes a round trip through HBM.

The cross-attention K/V depend only on the text context, so -- as in the reference
(``forward_and_cache_cross_attention_kv``, wan2_2_transformer.py:1675-1725) -- they are projected once
per generation by :func:`project_cross_kv` and reused by every step. The 40-block loop is
``WanTransformer3DModel.forward``'s (wan2_2_transformer.py:1818-1825).
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import attention_ops as ops
from .adaln_kernels import adaln_quant_2d
from .rope import rope_tables
from .row_mx_kernels import MXWeight, mxfp8_linear, mxfp8_qkv_linear, quantize_weight_mx

DIM, HEADS, HEAD_DIM, FFN = 5120, 40, 128, 13824


class BlockWeights(NamedTuple):
    scale_shift_table: torch.Tensor  # fp32 [6, DIM]
    qkv: MXWeight  # [3*DIM, DIM]
    norm_q: torch.Tensor  # fp32 [DIM]
    norm_k: torch.Tensor
    o: MXWeight
    norm2_weight: torch.Tensor  # fp32 [DIM] (affine LayerNorm of the cross-attention input)
    norm2_bias: torch.Tensor
    q2: MXWeight
    k2: MXWeight
    v2: MXWeight
    norm_q2: torch.Tensor
    norm_k2: torch.Tensor
    o2: MXWeight
    up: MXWeight  # [FFN, DIM]
    down: MXWeight  # [DIM, FFN]


class CrossKV(NamedTuple):
    k: torch.Tensor  # bf16 [S_txt, HEADS, 128], normalized
    vt: torch.Tensor  # bf16 [HEADS, 128, S_pad]
    kmax: torch.Tensor  # fp32 [HEADS]


def random_block_weights(device, generator=None, std: float = 0.02, dim: int = DIM, ffn: int = FFN,
                         heads: int = HEADS, qk_gamma_mean: float = 0.0, keep_raw: bool = True):
    """Random-init block (weights N(0, std) in bf16, quantized to MX on the GPU). Returns the GEMM
    layout weights and (``keep_raw``) the bf16 reference-layout tensors they came from (``x @ W``)."""

    def rnd(*shape):
        return (torch.randn(*shape, device=device, generator=generator) * std).to(torch.bfloat16)

    def vec(n, mean=0.0):
        return (mean + torch.randn(n, device=device, generator=generator) * std).float()

    raw = {
        "scale_shift_table": vec(6 * dim).view(6, dim),
        "qkv_w": rnd(dim, 3 * dim), "qkv_b": vec(3 * dim),
        "norm_q": vec(dim, qk_gamma_mean), "norm_k": vec(dim, qk_gamma_mean),
        "o_w": rnd(dim, dim), "o_b": vec(dim),
        "norm2_weight": vec(dim), "norm2_bias": vec(dim),
        "q2_w": rnd(dim, dim), "q2_b": vec(dim),
        "k2_w": rnd(dim, dim), "k2_b": vec(dim),
        "v2_w": rnd(dim, dim), "v2_b": vec(dim),
        "norm_q2": vec(dim, qk_gamma_mean), "norm_k2": vec(dim, qk_gamma_mean),
        "o2_w": rnd(dim, dim), "o2_b": vec(dim),
        "up_w": rnd(dim, ffn), "up_b": vec(ffn),
        "down_w": rnd(ffn, dim), "down_b": vec(dim),
    }
    q = lambda n: quantize_weight_mx(raw[n + "_w"], raw[n + "_b"])  # noqa: E731
    w = BlockWeights(
        raw["scale_shift_table"], q("qkv"), raw["norm_q"], raw["norm_k"], q("o"), raw["norm2_weight"],
        raw["norm2_bias"], q("q2"), q("k2"), q("v2"), raw["norm_q2"], raw["norm_k2"], q("o2"), q("up"), q("down"),
    )
    return w, (raw if keep_raw else None)


def project_cross_kv(w: BlockWeights, context: torch.Tensor, eps: float = 1e-6) -> CrossKV:
    """Text context ``[S_txt, DIM]`` bf16 -> normalized K, V^T and the key-norm bound (once per
    generation; the reference row-packs the context once and projects K/V per expert)."""
    ctx = adaln_quant_2d(context.contiguous(), None, None, eps=0.0, norm_type="none", quant="mx")
    k = mxfp8_linear(ctx, w.k2)
    kmax = ops.qk_rmsnorm_rope_(k, w.norm_k2, eps=eps, want_max=True)
    v = mxfp8_linear(ctx, w.v2)
    heads = k.shape[1] // HEAD_DIM
    vt, _ = ops.transpose_heads(v.view(-1, heads, HEAD_DIM))
    return CrossKV(k.view(-1, heads, HEAD_DIM), vt, kmax)


_ONES: dict = {}


def _ones(n: int, device) -> torch.Tensor:
    """fp32 ones [n] on ``device`` (the gate of the ungated residual add), made once per device."""
    key = (torch.device(device), n)
    if key not in _ONES:
        _ONES[key] = torch.ones(n, dtype=torch.float32, device=device)
    return _ONES[key]


def modulation(tables: torch.Tensor, temb: torch.Tensor) -> torch.Tensor:
    """``e = scale_shift_table + temb`` (wan2_2_transformer.py:1454-1456) for a stack of blocks'
    tables ``[B, 6, DIM]`` at once, as the rows the block uses: fp32 ``[B, 6, DIM]`` holding
    shift, 1 + scale, gate, c_shift, 1 + c_scale, c_gate (each row contiguous)."""
    e = tables.float() + temb.reshape(1, 6, -1).float()
    e[:, 1] += 1.0
    e[:, 4] += 1.0
    return e


def block_forward(w: BlockWeights, h: torch.Tensor, temb: torch.Tensor, rope, cross: CrossKV,
                  eps: float = 1e-6, timer=None, mod: torch.Tensor | None = None) -> torch.Tensor:
    """One block on ``h`` bf16 ``[S, DIM]``; ``temb`` ``[6, DIM]`` (or ``[1, 6, DIM]``); ``rope`` is
    ``(cos, sin)`` pair tables ``[S, 64]``. ``timer(name, fn)`` optionally wraps each kernel launch.
    ``mod``: this block's rows of :func:`modulation` when the caller computed them for all blocks."""
    run = timer or (lambda name, fn: fn())
    S, dim = h.shape
    heads = dim // HEAD_DIM
    scale = HEAD_DIM**-0.5
    if mod is None:
        mod = modulation(w.scale_shift_table[None], temb)[0]
    shift, one_p_sc, gate, c_shift, one_p_csc, c_gate = (mod[i] for i in range(6))
    cos, sin = rope

    a1 = run("adaln", lambda: adaln_quant_2d(h, one_p_sc, shift, eps=eps, norm_type="layer_norm", quant="mx"))
    # The QKV GEMM writes Q and K token-major, V already transposed per head for the attention (V^T),
    # and the Q rows' sums of squares per 128 columns; the attention normalizes and rotates Q as it
    # loads it. K is prepared in a pass of its own: the key-norm bound needs max ||k|| over all keys
    # before the attention starts.
    q_ss = torch.empty((S, 2 * dim // 128), dtype=torch.float32, device=h.device)
    qk, vt = run("gemm_qkv", lambda: mxfp8_qkv_linear(a1, w.qkv, vt_col0=2 * dim, row_sumsq=q_ss, sumsq_cols=dim))
    # the K pass also reduces each query's partial sums to its 1/rms, once per token
    q_rr = torch.empty(S, dtype=torch.float32, device=h.device)
    kmax = run("qk_prep", lambda: ops.qk_rmsnorm_rope_(qk[:, dim:], w.norm_k, cos=cos, sin=sin, eps=eps, want_max=True,
                                                        q_sumsq=q_ss, q_rr=q_rr))
    q = qk[:, :dim].view(S, heads, HEAD_DIM)
    k = qk[:, dim:].view(S, heads, HEAD_DIM)
    o1 = run("self_attention", lambda: ops.attention_core(q, k, vt, kmax, scale, ops.OUT_MX,
                                                         q_prep=ops.QPrep(None, w.norm_q, cos, sin, eps, rr=q_rr)))
    h1 = run("gemm_o", lambda: mxfp8_linear(o1, w.o, epilogue="gated_residual", residual=h, gate=gate))
    a2 = run("adaln", lambda: adaln_quant_2d(h1, w.norm2_weight, w.norm2_bias, eps=eps, norm_type="layer_norm",
                                             quant="mx"))
    q2_ss = torch.empty((S, dim // 128), dtype=torch.float32, device=h.device)
    q2 = run("gemm_q2", lambda: mxfp8_linear(a2, w.q2, row_sumsq=q2_ss, sumsq_cols=dim))
    o2 = run("cross_attention", lambda: ops.attention_core(q2.view(S, heads, HEAD_DIM), cross.k, cross.vt, cross.kmax,
                                                          scale, ops.OUT_MX, q_prep=ops.QPrep(q2_ss, w.norm_q2, eps=eps)))
    h2 = run("gemm_o2", lambda: mxfp8_linear(o2, w.o2, epilogue="gated_residual", residual=h1, gate=_ones(dim, h.device)))
    a3 = run("adaln", lambda: adaln_quant_2d(h2, one_p_csc, c_shift, eps=eps, norm_type="layer_norm", quant="mx"))
    inter = run("gemm_up", lambda: mxfp8_linear(a3, w.up, epilogue="gelu_mx"))
    return run("gemm_down", lambda: mxfp8_linear(inter, w.down, epilogue="gated_residual", residual=h2, gate=c_gate))


def dit_forward(blocks, h: torch.Tensor, temb: torch.Tensor, rope, crosses, eps: float = 1e-6, timer=None,
                tables: torch.Tensor | None = None):
    """The 40-block loop of one DiT forward (one CFG branch), cross-attention K/V cached. ``rope``
    is either the ``(cos, sin)`` pair tables ``[S, 64]`` or the latent patch grid ``(F, H, W)``; given
    the grid, the tables are built here, once per forward, as the reference's forward calls its
    rotary embedding (wan2_2_transformer.py:1757). The modulation rows of every block are formed in
    one batched op up front; ``tables`` optionally holds the blocks' stacked ``scale_shift_table``
    ``[B, 6, DIM]`` (built here otherwise)."""
    run = timer or (lambda name, fn: fn())
    if len(rope) == 3 and all(isinstance(v, int) for v in rope):
        grid = tuple(rope)
        if grid[0] * grid[1] * grid[2] != h.shape[0]:
            raise ValueError(f"grid {grid} holds {grid[0] * grid[1] * grid[2]} tokens, h has {h.shape[0]}")
        rope = run("rope_tables", lambda: rope_tables(grid, device=h.device))
    if tables is None:
        tables = torch.stack([w.scale_shift_table for w in blocks])
    mods = modulation(tables, temb)
    for i, (w, cross) in enumerate(zip(blocks, crosses)):
        h = block_forward(w, h, temb, rope, cross, eps, timer, mod=mods[i])
    return h
