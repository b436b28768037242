"""The Wan transformer block composed from the oracle pieces -- test infrastructure only.

Three restatements of ``WanTransformerBlock.forward`` (vllm_omni_neuron/diffusion/models/wan2_2/
wan2_2_transformer.py:1428-1513):

- :func:`mxfp8_block`: the MXFP8 recipe at exactly the quantization points the GPU path uses
  (MX activations from the canonical adaLN, MX weights, bf16 projection outputs, bf16 q/k/v,
  MX attention output and GELU intermediate). GEMMs run in fp32 on dequantized operands (exact
  products; fp32 accumulation, far inside the bf16 tolerance); attention is exact softmax in fp64.
- :func:`row_mx_block`: the reference's own FP8 recipe, ROW activations at every adaLN site and
  per-tensor FP8 checkpoint weights with per-channel scales (the ROW_MX modules of
  row_mx_modules.py), MX re-quantization of the attention outputs and of the GELU intermediate.
- :func:`bf16_eager_block`: the reference's BF16 eager fallback chain -- ``_eager_adaln``
  (adaln_kernels.py:51-84), ``torch.matmul`` projections (wan2_2_transformer.py:1104),
  ``DistributedRMSNorm`` (879-893), ``apply_rotary_emb_wan`` (rope.py:8-34), ``_torch_attend``
  (640-650), ``_wan_o_proj`` fallback (244-254), ``_wan_mlp`` fallback (389-408) and the final gated
  add (1510-1512). This is the CPU path timed as the baseline, and the BF16 point the MXFP8 block's
  quantization error is reported against.

Weights come as the bf16 reference-layout dict of ``block.random_block_weights`` (``x @ W``) plus,
for the MXFP8 path, their MX codes/scales in GEMM layout (optionally with a per-output-channel
scale, the per-tensor FP8 checkpoint recipe).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import adaln as oadaln
from . import attention as oattn
from . import mx as omx
from . import rope as orope
from .fp8 import bf16_round

HEAD_DIM = 128


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


def _deq(codes, scales) -> torch.Tensor:
    return torch.from_numpy(omx.mx_dequantize(np.asarray(codes), np.asarray(scales)).astype(np.float32))


def _mx_of(y: torch.Tensor):
    return omx.mx_quantize(y.float().numpy())


def _proj(a_deq: torch.Tensor, wq) -> torch.Tensor:
    """fp32 ``A_deq @ W_deq^T``, times the per-output-channel scale when ``wq`` carries one.

    ``wq`` = (codes [N, K], scales [N, K/32]) for an MX weight, or (codes, scales, col_scale [N])
    for a per-tensor FP8 checkpoint weight loaded with neutral block scales: the ROW_MX weight
    dequant ``* c_i`` of qkv_cte.py:3996-4021 / row_mx_loaders.py:115-140, applied after the
    accumulation as the GPU epilogue applies it."""
    y = a_deq @ _deq(wq[0], wq[1]).T
    if len(wq) > 2 and wq[2] is not None:
        y = y * torch.as_tensor(np.asarray(wq[2], np.float32)).reshape(1, -1)
    return y


def _lin(a_codes, a_scales, wq, bias) -> torch.Tensor:
    """bf16(A_deq @ W_deq^T [* col_scale] + b), fp32 accumulation; ``wq`` as in :func:`_proj`."""
    y = _proj(_deq(a_codes, a_scales), wq) + bias.float()
    return _bf16(y)


def _attend(q, k, v, scale):
    """[S, N, D] bf16-valued tensors -> bf16-valued [S, N*D] via exact fp64 softmax attention."""
    o = oattn.torch_attend(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), scale, dtype=torch.float64)
    return _bf16(o.transpose(0, 1).reshape(q.shape[0], -1))


def _attend_kernel(q, k, v, scale):
    """As :func:`_attend`, with the reference attention kernel's rounding points
    (``const_max_kernel_attention``) instead of exact softmax."""
    o = oattn.const_max_kernel_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), scale)
    return _bf16(o.transpose(0, 1).reshape(q.shape[0], -1))


def mxfp8_block(raw, wq, h, temb, context, grid, eps=1e-6, attend=None):
    """MXFP8 block on CPU. ``raw``: bf16/fp32 reference tensors; ``wq``: name -> (codes, scales)
    numpy in GEMM layout; h [S, dim] bf16; temb [6, dim]; context [S_txt, dim] bf16; ``attend``:
    the attention of both sub-layers (default exact fp64 softmax, :func:`_attend`; or
    :func:`_attend_kernel`).
    Returns the intermediates (``a1_codes``/``a1_scales``, ``qkv``, ``attn1``, ``h1``, ``attn2``,
    ``h2``, ``inter``) and ``out``."""
    attend = attend or _attend
    S, dim = h.shape
    heads = dim // HEAD_DIM
    scale = HEAD_DIM**-0.5
    e = raw["scale_shift_table"].float() + temb.reshape(6, dim).float()
    shift, sc, gate, c_shift, c_sc, c_gate = (e[i] for i in range(6))
    cos, sin = orope.wan_rope(grid)
    hn = h.float().numpy()

    a1 = oadaln.adaln_quant(hn, (1 + sc).numpy(), shift.numpy(), eps=eps, quant="mx")
    qkv = _lin(a1["codes"], a1["scales"], wq["qkv"], raw["qkv_b"])
    q = orope.rms_norm_across_heads(qkv[:, :dim].to(torch.bfloat16), raw["norm_q"], eps).view(1, S, heads, HEAD_DIM)
    k = orope.rms_norm_across_heads(qkv[:, dim : 2 * dim].to(torch.bfloat16), raw["norm_k"], eps).view(1, S, heads, HEAD_DIM)
    q = orope.apply_rotary_emb_wan(q, cos[None, :, None], sin[None, :, None])[0]
    k = orope.apply_rotary_emb_wan(k, cos[None, :, None], sin[None, :, None])[0]
    v = qkv[:, 2 * dim :].to(torch.bfloat16).view(S, heads, HEAD_DIM)
    o1 = attend(q, k, v, scale)
    o1c, o1s = _mx_of(o1)
    attn1 = _lin(o1c, o1s, wq["o"], raw["o_b"])

    r2 = oadaln.adaln_quant(attn1.numpy(), raw["norm2_weight"].numpy(), raw["norm2_bias"].numpy(), eps=eps,
                            quant="mx", residual=hn, gate=gate.numpy())
    h1 = torch.from_numpy(r2["residual_out"])
    q2 = _lin(r2["codes"], r2["scales"], wq["q2"], raw["q2_b"])
    q2 = orope.rms_norm_across_heads(q2.to(torch.bfloat16), raw["norm_q2"], eps).view(S, heads, HEAD_DIM)
    cc, cs = _mx_of(context.float())
    k2 = orope.rms_norm_across_heads(_lin(cc, cs, wq["k2"], raw["k2_b"]).to(torch.bfloat16), raw["norm_k2"], eps)
    v2 = _lin(cc, cs, wq["v2"], raw["v2_b"]).to(torch.bfloat16)
    St = context.shape[0]
    o2 = attend(q2, k2.view(St, heads, HEAD_DIM), v2.view(St, heads, HEAD_DIM), scale)
    o2c, o2s = _mx_of(o2)
    attn2 = _lin(o2c, o2s, wq["o2"], raw["o2_b"])

    r3 = oadaln.adaln_quant(attn2.numpy(), (1 + c_sc).numpy(), c_shift.numpy(), eps=eps, quant="mx",
                            residual=h1.numpy(), gate=None)
    h2 = torch.from_numpy(r3["residual_out"])
    up = _proj(_deq(r3["codes"], r3["scales"]), wq["up"]) + raw["up_b"].float()
    g = torch.from_numpy(bf16_round(F.gelu(up, approximate="tanh").numpy()))
    gc, gs = _mx_of(g)
    ffn = _lin(gc, gs, wq["down"], raw["down_b"])
    out = _bf16(h2 + ffn * c_gate)
    return {"a1_codes": a1["codes"], "a1_scales": a1["scales"], "qkv": qkv, "attn1": attn1, "h1": h1,
            "attn2": attn2, "h2": h2, "inter": g, "out": out}


def _row_lin(codes, dq, ck, bias) -> torch.Tensor:
    """The ROW_MX projection of a ROW-quantized activation (codes [T, K] uint8, per-row dq [T, 1])
    with a per-tensor FP8 checkpoint weight ``ck = (codes [K, N] e4m3fn, per-channel scale [N])``:
    ``bf16((codes . W_codes) * dq * c + b)`` (qkv_cte.py:3996-4021), fp32 accumulation."""
    a = torch.from_numpy(omx.e4m3_decode(np.asarray(codes)).astype(np.float32))
    y = (a @ ck[0].float()) * torch.as_tensor(np.asarray(dq, np.float32)).reshape(-1, 1) * ck[1].float().reshape(1, -1)
    return _bf16(y + bias.float())


def _mx_lin(a_codes, a_scales, ck, bias) -> torch.Tensor:
    """An MX activation against a per-tensor FP8 checkpoint weight: ``bf16((A_deq . W_codes) * c + b)``."""
    y = (_deq(a_codes, a_scales) @ ck[0].float()) * ck[1].float().reshape(1, -1)
    return _bf16(y + bias.float())


def row_mx_block(raw, ckpt, h, temb, context, grid, eps=1e-6, attend=None):
    """The reference's FP8 recipe with ROW activations (``_leaf_quant`` = "row", T:1423-1426), in
    natural channel order, on CPU: every adaLN site row-quantizes (per-row ``amax / 448`` scale),
    the projections are ROW_MX (codes x FP8 checkpoint codes x row scale x channel scale + bias),
    the o-projections MX-quantize their attention input (row_mx_o_proj), the FFN up projection is
    followed by GELU-tanh, bf16 and MX (mlp_torch.py:586-594), and the block ends with the gated add
    (T:1508-1512). ``ckpt``: projection name (``qkv``, ``o``, ``q2``, ``k2``, ``v2``, ``o2``, ``up``,
    ``down``) -> (codes [K, N] e4m3fn, per-channel scale [N]); ``raw`` as :func:`mxfp8_block`.
    Returns the intermediates (``a1_packed``, ``qkv``, ``attn1``, ``h1``, ``attn2``, ``h2``,
    ``inter``) and ``out``."""
    attend = attend or _attend
    S, dim = h.shape
    heads = dim // HEAD_DIM
    scale = HEAD_DIM**-0.5
    e = raw["scale_shift_table"].float() + temb.reshape(6, dim).float()
    shift, sc, gate, c_shift, c_sc, c_gate = (e[i] for i in range(6))
    cos, sin = orope.wan_rope(grid)
    hn = h.float().numpy()

    a1 = oadaln.adaln_quant(hn, (1 + sc).numpy(), shift.numpy(), eps=eps, quant="row")
    qkv = _row_lin(a1["codes"], a1["dq"], ckpt["qkv"], raw["qkv_b"])
    q = orope.rms_norm_across_heads(qkv[:, :dim].to(torch.bfloat16), raw["norm_q"], eps).view(1, S, heads, HEAD_DIM)
    k = orope.rms_norm_across_heads(qkv[:, dim : 2 * dim].to(torch.bfloat16), raw["norm_k"], eps).view(1, S, heads, HEAD_DIM)
    q = orope.apply_rotary_emb_wan(q, cos[None, :, None], sin[None, :, None])[0]
    k = orope.apply_rotary_emb_wan(k, cos[None, :, None], sin[None, :, None])[0]
    v = qkv[:, 2 * dim :].to(torch.bfloat16).view(S, heads, HEAD_DIM)
    o1 = attend(q, k, v, scale)
    o1c, o1s = _mx_of(o1)
    attn1 = _mx_lin(o1c, o1s, ckpt["o"], raw["o_b"])

    r2 = oadaln.adaln_quant(attn1.numpy(), raw["norm2_weight"].numpy(), raw["norm2_bias"].numpy(), eps=eps,
                            quant="row", residual=hn, gate=gate.numpy())
    h1 = torch.from_numpy(r2["residual_out"])
    q2 = _row_lin(r2["codes"], r2["dq"], ckpt["q2"], raw["q2_b"])
    q2 = orope.rms_norm_across_heads(q2.to(torch.bfloat16), raw["norm_q2"], eps).view(S, heads, HEAD_DIM)
    cc, cdq = omx.row_quantize(context.float().numpy())
    k2 = orope.rms_norm_across_heads(_row_lin(cc, cdq, ckpt["k2"], raw["k2_b"]).to(torch.bfloat16), raw["norm_k2"], eps)
    v2 = _row_lin(cc, cdq, ckpt["v2"], raw["v2_b"]).to(torch.bfloat16)
    St = context.shape[0]
    o2 = attend(q2, k2.view(St, heads, HEAD_DIM), v2.view(St, heads, HEAD_DIM), scale)
    o2c, o2s = _mx_of(o2)
    attn2 = _mx_lin(o2c, o2s, ckpt["o2"], raw["o2_b"])

    r3 = oadaln.adaln_quant(attn2.numpy(), (1 + c_sc).numpy(), c_shift.numpy(), eps=eps, quant="row",
                            residual=h1.numpy(), gate=None)
    h2 = torch.from_numpy(r3["residual_out"])
    a3 = torch.from_numpy(omx.e4m3_decode(r3["codes"]).astype(np.float32))
    up = (a3 @ ckpt["up"][0].float()) * torch.from_numpy(r3["dq"]).reshape(-1, 1) * ckpt["up"][1].float() \
        + raw["up_b"].float()
    g = torch.from_numpy(bf16_round(F.gelu(up, approximate="tanh").numpy()))
    gc, gs = _mx_of(g)
    ffn = _mx_lin(gc, gs, ckpt["down"], raw["down_b"])
    out = _bf16(h2 + ffn * c_gate)
    return {"a1_packed": a1["packed"], "qkv": qkv, "attn1": attn1, "h1": h1, "attn2": attn2, "h2": h2, "inter": g,
            "out": out}


def bf16_eager_block(raw, h, temb, context, grid, eps=1e-6):
    """The reference's BF16 eager fallback block, in torch on the CPU (bf16 tensors)."""
    bf = torch.bfloat16
    S, dim = h.shape
    heads = dim // HEAD_DIM
    scale = HEAD_DIM**-0.5
    W = {k: (v.to(bf) if v.dim() == 2 and k.endswith("_w") else v) for k, v in raw.items()}
    e = raw["scale_shift_table"].float()[None] + temb.reshape(1, 6, dim).float()
    shift, sc, gate, c_shift, c_sc, c_gate = e.chunk(6, dim=1)
    cos, sin = orope.wan_rope(grid)
    hb = h.to(bf)[None]

    def eager_adaln(x, mul, add, residual=None, g=None):
        xf = x.float()
        res_out = None
        if residual is not None:
            if g is not None:
                xf = xf * g.float()
            xf = xf + residual.float()
            res_out = xf.type_as(residual)
            xf = res_out.float()
        n = F.layer_norm(xf, (xf.shape[-1],), None, None, eps)
        if mul is not None:
            n = n * mul.float()
        if add is not None:
            n = n + add.float()
        y = n.type_as(x)
        return y if residual is None else (res_out, y)

    def rms(x, w):
        return orope.rms_norm_across_heads(x, w, eps)

    def attend(q, k, v):  # [B, N, S, D] -> d-major [B, N, D, S] (_torch_attend + transpose)
        sc_ = torch.matmul(q.float() * scale, k.float().transpose(-2, -1))
        return torch.matmul(torch.softmax(sc_, dim=-1), v.float()).to(q.dtype).transpose(2, 3)

    def o_proj(active, w, b):  # _wan_o_proj torch fallback
        B, N, D, S_ = active.shape
        return torch.matmul(active.reshape(B, N * D, S_).transpose(1, 2), w) + b.to(bf)

    nh = eager_adaln(hb, 1 + sc, shift)
    qkv = torch.matmul(nh, W["qkv_w"]) + raw["qkv_b"].to(bf)
    q, k, v = torch.tensor_split(qkv, [dim, 2 * dim], dim=-1)
    q = rms(q, raw["norm_q"]).unflatten(2, (heads, HEAD_DIM))
    k = rms(k, raw["norm_k"]).unflatten(2, (heads, HEAD_DIM))
    v = v.unflatten(2, (heads, HEAD_DIM))
    q = orope.apply_rotary_emb_wan(q, cos[None, :, None], sin[None, :, None])
    k = orope.apply_rotary_emb_wan(k, cos[None, :, None], sin[None, :, None])
    a1 = o_proj(attend(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)), W["o_w"], raw["o_b"])
    h1, nh = eager_adaln(a1, raw["norm2_weight"], raw["norm2_bias"], residual=hb, g=gate)
    q2 = rms(torch.matmul(nh, W["q2_w"]) + raw["q2_b"].to(bf), raw["norm_q2"]).unflatten(2, (heads, HEAD_DIM))
    ctx = context.to(bf)[None]
    k2 = rms(torch.matmul(ctx, W["k2_w"]) + raw["k2_b"].to(bf), raw["norm_k2"]).unflatten(2, (heads, HEAD_DIM))
    v2 = (torch.matmul(ctx, W["v2_w"]) + raw["v2_b"].to(bf)).unflatten(2, (heads, HEAD_DIM))
    a2 = o_proj(attend(q2.transpose(1, 2), k2.transpose(1, 2), v2.transpose(1, 2)), W["o2_w"], raw["o2_b"])
    h2, nh = eager_adaln(a2, 1 + c_sc, c_shift, residual=h1)
    up = F.gelu(torch.matmul(nh, W["up_w"]) + raw["up_b"].to(bf), approximate="tanh")
    ffn = torch.matmul(up, W["down_w"]) + raw["down_b"].to(bf)
    return (h2.float() + ffn.float() * c_gate).type_as(h2)[0]
