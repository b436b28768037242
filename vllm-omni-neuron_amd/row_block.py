"""The reference's own FP8 block recipe -- ROW activations -- composed from the drop-ins.

``WanTransformerBlock.forward`` (vllm_omni_neuron/diffusion/models/wan2_2/wan2_2_transformer.py:
1428-1513) with its FP8 leaves: ``_leaf_quant`` returns ``"row"`` for every FP8 leaf (T:1423-1426),
so each adaLN site row-packs its output (``[.., H + 4]``: e4m3 codes and the row's fp32 dequant
scale) and the leaves consume that packed activation:

    packed = adaln_modulate(h, 1 + scale, shift, quant="row")                       T:1458-1465
    attn1 = WanSelfAttentionFP8.forward(packed, rotary_emb)                          row_mx_modules.py:340-404
          = row_mx_o_proj(wan_cp_self_attention(split(row_mx_qkv_proj(packed, fused norm + RoPE))))
    h1, packed = adaln_modulate(attn1, norm2.w, norm2.b, quant="row", residual=h, gate=gate)   T:1480-1488
    attn2 = WanCrossAttentionFP8.forward(packed, K/V cache)                          row_mx_modules.py:478-495
          = row_mx_o_proj(_nki_attend(row_mx_qkv_proj(packed, Q norm, NBSd).transpose(0, 1), K, V))
    h2, packed = adaln_modulate(attn2, 1 + c_scale, c_shift, quant="row", residual=h1)       T:1497-1505
    out = (h2 + row_mx_mlp(packed) * c_gate)                                          T:1508-1512, 679-708

with the weights in the forms the reference's loaders produce: per-tensor FP8 checkpoint weights
(``scale = amax / 448``) packed ``[K/4, N, 4]``, the checkpoint scalars expanded per output channel
(``_expand_per_tensor_scales_to_channels``, row_mx_loaders.py:115-140), the fused QKV weight, bias and
the Q/K norm gammas de-interleaved per head (row_mx_loaders.py:26-71, 194-243) so that the fused
rotate-half RoPE reproduces Wan's interleaved RoPE; the rotate-half caches are ``cat([base, base])``
of the interleaved tables (row_mx_modules.py:51-76). Each packed weight is converted once to the
GEMM's layout (:func:`packed_weight_to_mx`), as a model would at load time.

Each step calls the drop-in the reference module calls, in the same order, with one fusion: the
FFN's down projection carries the block's last gated add in its epilogue. ``row_mx_mlp`` followed by
the framework add computes ``bf16(h2 + bf16(ffn) * c_gate)`` (fp32 product, then the sum); the GEMM's
gated-residual epilogue computes exactly that, so the bits are the same and one launch and a round
trip of the FFN output through HBM are saved.

This path exists to run the reference's recipe as it is; the block of :mod:`.block` is the faster
MX-activation path (per-32 block scales, fused Q preparation, V^T written by the QKV GEMM).
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from .adaln_kernels import adaln_modulate
from .attention_ops import _nki_attend, row_mx_o_proj, row_mx_qkv_proj, wan_cp_self_attention
from .block import DIM, FFN, HEAD_DIM, modulation
from .common_types import NormType, QKNormConfig, QKVOutputLayout
from .rope import rope_tables
from .row_mx_kernels import MXWeight, mxfp8_linear, packed_weight_to_mx, row_quantize_packed

FP8_MAX = 448.0


class RowBlockWeights(NamedTuple):
    """One block's parameters in the reference's ROW_MX module forms (converted once to the GEMM's
    layout): per-channel-scaled FP8 projections with their biases, de-interleaved self-attention Q/K
    channels and gammas, natural-order cross-attention projections."""

    scale_shift_table: torch.Tensor  # fp32 [6, dim]
    qkv: MXWeight  # [3 dim, dim], Q/K channels de-interleaved per head (rope_pairs "halves")
    norm_q: torch.Tensor  # fp32 [1, dim], de-interleaved
    norm_k: torch.Tensor
    o: MXWeight
    norm2_weight: torch.Tensor
    norm2_bias: torch.Tensor
    q2: MXWeight
    k2: MXWeight
    v2: MXWeight
    norm_q2: torch.Tensor  # fp32 [1, dim]
    norm_k2: torch.Tensor
    o2: MXWeight
    up: MXWeight
    down: MXWeight


def deinterleave_perm(head_dim: int = HEAD_DIM) -> torch.Tensor:
    """Per-head channel order ``[0, 2, .., d-2, 1, 3, .., d-1]``: rotate-half RoPE on channels in
    this order equals Wan's interleaved RoPE on the original ones (row_mx_loaders.py:26-39)."""
    idx = torch.arange(head_dim // 2)
    return torch.cat([2 * idx, 2 * idx + 1])


def deinterleave_columns(n_heads: int, head_dim: int = HEAD_DIM) -> torch.Tensor:
    """Column index that de-interleaves every head of an ``n_heads * head_dim`` block."""
    return (torch.arange(n_heads)[:, None] * head_dim + deinterleave_perm(head_dim)[None]).reshape(-1)


def per_tensor_fp8(w_kn: torch.Tensor):
    """A reference-layout weight ``[K, N]`` as the FP8 checkpoint stores it: e4m3fn codes of
    ``w / s`` and the scalar ``s = amax / 448``."""
    s = w_kn.float().abs().max().clamp_min(1e-30) / FP8_MAX
    return (w_kn.float() / s).to(torch.float8_e4m3fn), s.reshape(1)


def pack_x4(codes_kn: torch.Tensor) -> torch.Tensor:
    """FP8 ``[K, N]`` -> the reference's packed ``[K/4, N, 4]`` (four consecutive contraction values
    innermost, row_mx_modules.py:299-301)."""
    K, N = codes_kn.shape
    return codes_kn.view(torch.uint8).reshape(K // 4, 4, N).permute(0, 2, 1).contiguous().view(torch.float8_e4m3fn)


def row_block_weights(raw: dict, heads: int | None = None):
    """The bf16 reference-layout tensors of one block (``x @ W``, as :func:`block.random_block_weights`
    returns with ``keep_raw``) -> (:class:`RowBlockWeights`, natural-order checkpoint form).

    Every projection is quantized per tensor as the FP8 checkpoint stores it (the fused QKV weight as
    its three Q, K, V tensors with three scalars), packed ``[K/4, N, 4]`` (Q/K de-interleaved for the
    self-attention) and converted once with :func:`packed_weight_to_mx`. The second value maps each
    projection name to ``(codes [K, N] e4m3fn, per-channel scale [N])`` in natural channel order, the
    checkpoint's own content (for checks)."""
    dim = raw["qkv_w"].shape[0]
    heads = heads or dim // HEAD_DIM
    dev = raw["qkv_w"].device
    ckpt = {}

    def quant(name, w_kn):
        codes, s = per_tensor_fp8(w_kn)
        ckpt[name] = (codes, s.expand(w_kn.shape[1]).contiguous())
        return codes, s

    parts = [quant(f"qkv_{p}", raw["qkv_w"][:, i * dim : (i + 1) * dim]) for i, p in enumerate("qkv")]
    codes = torch.cat([c for c, _ in parts], dim=1)
    scale = torch.cat([s.expand(dim) for _, s in parts])
    ckpt["qkv"] = (codes, scale)
    cols = deinterleave_columns(heads).to(dev)
    order = torch.cat([cols, dim + cols, torch.arange(2 * dim, 3 * dim, device=dev)])
    qkv = packed_weight_to_mx(pack_x4(codes.view(torch.uint8)[:, order].contiguous().view(torch.float8_e4m3fn)),
                              scale[order][None], raw["qkv_b"].float()[order][None], rope_pairs="halves")

    def proj(name):
        c, s = quant(name, raw[name + "_w"])
        return packed_weight_to_mx(pack_x4(c), s.expand(c.shape[1])[None], raw[name + "_b"].float()[None],
                                   rope_pairs="interleaved")

    w = RowBlockWeights(
        raw["scale_shift_table"].float().reshape(6, dim), qkv,
        raw["norm_q"].float()[cols][None].contiguous(), raw["norm_k"].float()[cols][None].contiguous(),
        proj("o"), raw["norm2_weight"].float(), raw["norm2_bias"].float(),
        proj("q2"), proj("k2"), proj("v2"), raw["norm_q2"].float()[None].contiguous(),
        raw["norm_k2"].float()[None].contiguous(), proj("o2"), proj("up"), proj("down"),
    )
    return w, ckpt


def project_cross_kv_row(w: RowBlockWeights, context: torch.Tensor, eps: float = 1e-6):
    """The text context ``[S_txt, dim]`` (or ``[1, S_txt, dim]``) bf16 -> the block's cached
    ``(key, value)``, each ``[1, N, S_txt, 128]``: ``row_quantize_packed`` once
    (wan2_2_transformer.py:1686-1691), then ``WanCrossAttentionFP8.project_kv``
    (row_mx_modules.py:509-542): K with the across-heads norm (its gamma in the Q slot), V plain,
    both NBSd, transposed to ``[B, N, S, D]``."""
    ctx = context if context.dim() == 3 else context.unsqueeze(0)
    packed = row_quantize_packed(ctx.contiguous())
    heads = w.k2.out_features // HEAD_DIM
    key = row_mx_qkv_proj(packed, w.k2, num_heads=heads, head_dim=HEAD_DIM,
                          qk_norm_pre_rope=QKNormConfig(NormType.RMS_NORM_ACROSS_HEADS, None, eps),
                          qk_norm_pre_rope_q_gamma=w.norm_k2, norm_eps=eps, output_layout=QKVOutputLayout.NBSd)
    value = row_mx_qkv_proj(packed, w.v2, num_heads=heads, head_dim=HEAD_DIM, output_layout=QKVOutputLayout.NBSd)
    return key.transpose(0, 1), value.transpose(0, 1)


def rotate_half_caches(grid, device):
    """``(cos_cache, sin_cache)`` fp32 ``[1, S, 128]``: ``cat([base, base])`` of the Wan tables of the
    latent grid (row_mx_modules.py:51-76, 358-366), built on the GPU."""
    cos, sin = rope_tables(grid, layout="rotate_half", device=device)
    return cos.unsqueeze(0), sin.unsqueeze(0)


def row_block_forward(w: RowBlockWeights, h: torch.Tensor, temb: torch.Tensor, caches, cross, eps: float = 1e-6,
                      timer=None, mod: torch.Tensor | None = None) -> torch.Tensor:
    """One block of the ROW recipe on ``h`` bf16 ``[S, dim]``; ``caches`` = rotate-half
    ``(cos, sin)`` ``[1, S, 128]``; ``cross`` = ``(key, value)`` from :func:`project_cross_kv_row`.
    ``timer(name, fn)`` optionally wraps each step."""
    run = timer or (lambda name, fn: fn())
    S, dim = h.shape
    heads = dim // HEAD_DIM
    scale = HEAD_DIM**-0.5
    if mod is None:
        mod = modulation(w.scale_shift_table[None], temb)[0]
    shift, one_p_sc, gate, c_shift, one_p_csc, c_gate = (mod[i] for i in range(6))
    cos_cache, sin_cache = caches
    x = h.unsqueeze(0)
    across = NormType.RMS_NORM_ACROSS_HEADS

    # self-attention (WanSelfAttentionFP8.forward)
    packed = run("adaln", lambda: adaln_modulate(x, one_p_sc, shift, eps=eps, norm_type="layer_norm", quant="row"))
    qkv = run("qkv_proj", lambda: row_mx_qkv_proj(
        packed, w.qkv, num_heads=heads, head_dim=HEAD_DIM, num_kv_heads=heads, fused_rope=True, cos_cache=cos_cache,
        sin_cache=sin_cache, qk_norm_pre_rope=QKNormConfig(across, across, eps), qk_norm_pre_rope_q_gamma=w.norm_q,
        qk_norm_pre_rope_k_gamma=w.norm_k, norm_eps=eps))
    q, k, v = (t.unflatten(2, (heads, HEAD_DIM)) for t in torch.tensor_split(qkv, 3, dim=-1))
    att = run("self_attention", lambda: wan_cp_self_attention(q, k, v, scale, 1, None, None))
    attn1 = run("o_proj", lambda: row_mx_o_proj(att, w.o))
    h1, packed = run("adaln", lambda: adaln_modulate(attn1, w.norm2_weight, w.norm2_bias, eps=eps, norm_type="layer_norm",
                                                     quant="row", residual=x, gate=gate))
    # cross-attention (WanCrossAttentionFP8: _project_query, _nki_attend on the cached K/V, o-proj)
    query = run("q2_proj", lambda: row_mx_qkv_proj(
        packed, w.q2, num_heads=heads, head_dim=HEAD_DIM, qk_norm_pre_rope=QKNormConfig(across, None, eps),
        qk_norm_pre_rope_q_gamma=w.norm_q2, norm_eps=eps, output_layout=QKVOutputLayout.NBSd))
    att2 = run("cross_attention", lambda: _nki_attend(query.transpose(0, 1), cross[0], cross[1], scale))
    attn2 = run("o2_proj", lambda: row_mx_o_proj(att2, w.o2))
    h2, packed = run("adaln", lambda: adaln_modulate(attn2, one_p_csc, c_shift, eps=eps, norm_type="layer_norm",
                                                     quant="row", residual=h1, gate=None))
    # FFN (WanFeedForwardFP8 -> row_mx_mlp) and the block's gated add, fused into the down projection
    packed2d = packed.reshape(S, dim + 4)
    inter = run("mlp_up", lambda: mxfp8_linear(packed2d, w.up, epilogue="gelu_mx"))
    return run("mlp_down", lambda: mxfp8_linear(inter, w.down, epilogue="gated_residual", residual=h2.reshape(S, dim),
                                                gate=c_gate))


def row_dit_forward(blocks, h: torch.Tensor, temb: torch.Tensor, grid, crosses, eps: float = 1e-6, timer=None,
                    tables: torch.Tensor | None = None) -> torch.Tensor:
    """The 40-block loop of the ROW recipe (one CFG branch, cross-attention K/V cached): the
    rotate-half caches are built once per forward from the latent grid (the reference builds its
    rotary tables once per forward, T:1757, and each FP8 self-attention derives the caches from
    them); the modulation rows of every block in one batched op."""
    run = timer or (lambda name, fn: fn())
    caches = run("rope_tables", lambda: rotate_half_caches(grid, h.device))
    if tables is None:
        tables = torch.stack([w.scale_shift_table for w in blocks])
    mods = modulation(tables, temb)
    for i, (w, cross) in enumerate(zip(blocks, crosses)):
        h = row_block_forward(w, h, temb, caches, cross, eps, timer, mod=mods[i])
    return h


__all__ = ["RowBlockWeights", "row_block_weights", "project_cross_kv_row", "row_block_forward", "row_dit_forward",
           "rotate_half_caches", "deinterleave_columns", "per_tensor_fp8", "pack_x4", "DIM", "FFN"]
