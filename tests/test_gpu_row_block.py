"""GPU parity of the reference's own FP8 block recipe: ROW activations, composed from the drop-ins.

``row_block.row_block_forward`` runs ``WanTransformerBlock.forward`` with its FP8 leaves
(wan2_2_transformer.py:1428-1513, ``_leaf_quant`` = "row") through ``adaln_modulate(quant="row")``,
``row_mx_qkv_proj`` (fused across-heads norm + rotate-half RoPE on de-interleaved Q/K channels),
``wan_cp_self_attention``, ``row_mx_o_proj``, the cross-attention leaf on cached K/V (``_nki_attend``)
and ``row_mx_mlp``, on per-tensor FP8 checkpoint weights with per-channel scales, exactly as
row_mx_modules.py:340-404, 478-546 and 679-708 call them.

Workload: the single-block configuration (dim 5120, 40 heads x 128, FFN 13824, 1x30x52 latent grid
= 1560 tokens, 512 text tokens, weights N(0, 0.02), q/k gammas N(1, 0.02), activations and
modulation N(0, 1), seeded).

1. Stage-wise, every step recomputed from the GPU's own inputs to it: the adaLN sites' ROW-packed
   bytes and bf16 residuals bit-exact against the oracle; projections (ROW_MX: codes x FP8 weight
   codes x row scale x channel scale + bias) and the norm/RoPE after them in fp64 on the GPU, the
   attention outputs against fp64 softmax over every key: max|err|/max|ref| <= 2e-2, cosine >=
   0.999 (the projection and attention bars of the other tests); the GELU intermediate's MX codes
   at least 99.7% identical to the MX quantization of the fp64 GELU (the FFN floor of the MX block).
   The oracle's computations are in natural channel order; the Q/K outputs are compared after the
   same per-head de-interleave the GPU weights carry.
2. End to end against ``oracle.block.row_mx_block`` from the same block input, with the bars of the
   MX block test relative to the noise floor measured here (the oracle with the reference attention
   kernel's rounding points against the exact oracle).
"""

import numpy as np
import pytest
import torch

from oracle import adaln as oadaln
from oracle import block as oblock
from oracle import mx as omx
from oracle import rope as orope

pytestmark = pytest.mark.gpu

GRID = (1, 30, 52)
HD = 128


def _metrics(got, ref):
    got, ref = got.double().flatten().cpu(), ref.double().flatten().cpu()
    rel = float((got - ref).abs().max() / ref.abs().max())
    rms = float((got - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt())
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=0))
    return rel, rms, cos


class Fails(list):
    def close(self, got, ref, what, bar=(2e-2, 0.999)):
        rel, _, cos = _metrics(got, ref)
        print(f"{what}: rel_err {rel:.2e} cos {cos:.6f}", flush=True)
        if not (rel <= bar[0] and cos >= bar[1]):
            self.append((what, rel, cos))

    def exact(self, got, ref, what):
        same = np.array_equal(np.asarray(got), np.asarray(ref))
        print(f"{what}: bit-exact {same}", flush=True)
        if not same:
            self.append((what, "not bit-exact"))


def _row_proj(packed, ck, bias):
    """fp64 ROW_MX projection on the GPU of a ROW-packed [T, K + 4] activation with a checkpoint
    weight (codes [K, N] e4m3fn, per-channel scale [N]), natural channel order, rounded to bf16."""
    raw = packed.reshape(-1, packed.shape[-1]).view(torch.uint8)
    K = raw.shape[-1] - 4
    a = raw[:, :K].contiguous().view(torch.float8_e4m3fn).double()
    dq = raw[:, K:].contiguous().view(torch.float32).double()
    y = (a @ ck[0].double()) * dq * ck[1].double() + bias.double()
    return y.to(torch.bfloat16)


def _mx_proj(codes, scales, ck, bias):
    """fp64 projection of an MX activation (codes [T, K], e8m0 scales [T, K/32]) with a checkpoint
    weight, rounded to bf16."""
    v = codes.view(torch.float8_e4m3fn).double()
    s = torch.exp2(scales.double() - 127.0)
    a = (v.view(v.shape[0], -1, 32) * s.unsqueeze(-1)).view(v.shape)
    return ((a @ ck[0].double()) * ck[1].double() + bias.double()).to(torch.bfloat16)


def _attend(q, k, v, scale):
    """fp64 softmax attention, q [Sq, N, D], k/v [Sk, N, D] -> d-major [N, D, Sq]."""
    out = []
    for h in range(q.shape[1]):
        p = torch.softmax((q[:, h].double() * scale) @ k[:, h].double().T, dim=-1)
        out.append((p @ v[:, h].double()).T)
    return torch.stack(out)


def _mx_of_dmajor(att):
    """d-major bf16 [1, N, D, S] -> the MX codes/scales of its token-major [S, N*D] rows, as
    row_mx_o_proj quantizes its activation (oracle MX rule, on the CPU)."""
    x = att[0].permute(2, 0, 1).reshape(att.shape[-1], -1).float().cpu().numpy()
    c, s = omx.mx_quantize(x)
    return torch.from_numpy(c).to(att.device), torch.from_numpy(s).to(att.device)


def test_row_recipe_block(pkg, dev):
    blk, rb = pkg.block, pkg.row_block
    g = torch.Generator(device=dev).manual_seed(606)
    _, raw = blk.random_block_weights(dev, g, qk_gamma_mean=1.0)
    w, ck = rb.row_block_weights(raw)
    gc = torch.Generator().manual_seed(607)
    dim = raw["qkv_w"].shape[0]
    heads = dim // HD
    S = GRID[0] * GRID[1] * GRID[2]
    h = torch.randn(S, dim, generator=gc).to(torch.bfloat16)
    temb = torch.randn(6, dim, generator=gc)
    ctx = torch.randn(512, dim, generator=gc).to(torch.bfloat16)
    hd, td, cd = h.to(dev), temb.to(dev), ctx.to(dev)
    e = (raw["scale_shift_table"].float() + td.float()).cpu()
    shift, sc, gate, c_shift, c_sc, c_gate = (e[i] for i in range(6))
    fails = Fails()

    # ---- the cached text K/V (row_quantize_packed + project_kv) ----
    key, value = rb.project_cross_kv_row(w, cd)
    assert key.shape == value.shape == (1, heads, 512, HD)
    cpk = pkg.row_quantize_packed(cd[None])
    fails.exact(cpk.view(torch.uint8).cpu().numpy()[0],
                omx.row_pack(*omx.row_quantize(ctx.float().numpy())), "context row pack")
    k_lin = _row_proj(cpk, ck["k2"], raw["k2_b"])
    k_ref = orope.rms_norm_across_heads(k_lin.cpu(), raw["norm_k2"].cpu(), 1e-6).view(512, heads, HD)
    fails.close(key[0].permute(1, 0, 2).cpu(), k_ref, "cross K")
    fails.close(value[0].permute(1, 0, 2).cpu(), _row_proj(cpk, ck["v2"], raw["v2_b"]).cpu().view(512, heads, HD), "cross V")

    # ---- one block, every step's output kept ----
    snap = {}

    def timer(name, fn):
        r = fn()
        if isinstance(r, tuple):
            parts = [x.clone() for x in r]
            keep = type(r)(*parts) if hasattr(r, "_fields") else tuple(parts)
        else:
            keep = r.clone() if isinstance(r, torch.Tensor) else r
        snap.setdefault(name, []).append(keep)
        return r

    caches = rb.rotate_half_caches(GRID, dev)
    out = rb.row_block_forward(w, hd, td, caches, (key, value), timer=timer)
    assert out.shape == (S, dim) and out.dtype == torch.bfloat16
    a1 = snap["adaln"][0]
    h1, a2 = snap["adaln"][1]
    h2, a3 = snap["adaln"][2]

    # adaLN 1: ROW-packed bytes
    r1 = oadaln.adaln_quant(h.float().numpy(), (1 + sc).numpy(), shift.numpy(), eps=1e-6, quant="row")
    fails.exact(a1.view(torch.uint8).cpu().numpy()[0], r1["packed"], "adaLN 1 (ROW packed)")

    # fused QKV projection + across-heads norm + RoPE, de-interleaved Q/K channels
    cols = rb.deinterleave_columns(heads)
    order = torch.cat([cols, dim + cols, torch.arange(2 * dim, 3 * dim)])
    lin = _row_proj(a1, ck["qkv"], raw["qkv_b"]).cpu()
    cos, sin = orope.wan_rope(GRID)
    q = orope.rms_norm_across_heads(lin[:, :dim], raw["norm_q"].cpu(), 1e-6).view(1, S, heads, HD)
    k = orope.rms_norm_across_heads(lin[:, dim : 2 * dim], raw["norm_k"].cpu(), 1e-6).view(1, S, heads, HD)
    q = orope.apply_rotary_emb_wan(q, cos[None, :, None], sin[None, :, None]).view(S, dim)
    k = orope.apply_rotary_emb_wan(k, cos[None, :, None], sin[None, :, None]).view(S, dim)
    qkv_ref = torch.cat([q, k, lin[:, 2 * dim :].float()], dim=1)[:, order]
    qkv = snap["qkv_proj"][0][0].cpu()
    for name, sl in (("Q", slice(0, dim)), ("K", slice(dim, 2 * dim)), ("V", slice(2 * dim, 3 * dim))):
        fails.close(qkv[:, sl], qkv_ref[:, sl], f"qkv_proj {name}")

    # self-attention (d-major) from the GPU's q, k, v
    qg, kg, vg = (snap["qkv_proj"][0][0][:, i * dim : (i + 1) * dim].view(S, heads, HD) for i in range(3))
    att = snap["self_attention"][0]
    fails.close(att[0], _attend(qg, kg, vg, HD**-0.5), "self-attention")
    # o-projection from the GPU's attention
    oc, os_ = _mx_of_dmajor(att)
    attn1 = snap["o_proj"][0]
    fails.close(attn1[0], _mx_proj(oc, os_, ck["o"], raw["o_b"]), "o_proj")

    # adaLN 2 (gated residual, affine LayerNorm) from the GPU's o-projection
    r2 = oadaln.adaln_quant(attn1[0].float().cpu().numpy(), raw["norm2_weight"].cpu().numpy(),
                            raw["norm2_bias"].cpu().numpy(), eps=1e-6, quant="row", residual=h.float().numpy(),
                            gate=gate.numpy())
    fails.exact(h1[0].float().cpu().numpy(), r2["residual_out"], "adaLN 2 residual")
    fails.exact(a2.view(torch.uint8).cpu().numpy()[0], r2["packed"], "adaLN 2 (ROW packed)")

    # cross-attention query (NBSd), attention on the cached K/V, o2
    q2 = snap["q2_proj"][0]
    q2_ref = orope.rms_norm_across_heads(_row_proj(a2, ck["q2"], raw["q2_b"]).cpu(), raw["norm_q2"].cpu(), 1e-6)
    fails.close(q2[:, 0].permute(1, 0, 2).reshape(S, dim).cpu(), q2_ref, "q2_proj")
    att2 = snap["cross_attention"][0]
    fails.close(att2[0], _attend(q2[:, 0].permute(1, 0, 2), key[0].permute(1, 0, 2), value[0].permute(1, 0, 2),
                                 HD**-0.5), "cross-attention")
    oc2, os2 = _mx_of_dmajor(att2)
    attn2 = snap["o2_proj"][0]
    fails.close(attn2[0], _mx_proj(oc2, os2, ck["o2"], raw["o2_b"]), "o2_proj")

    # adaLN 3 (ungated residual)
    r3 = oadaln.adaln_quant(attn2[0].float().cpu().numpy(), (1 + c_sc).numpy(), c_shift.numpy(), eps=1e-6,
                            quant="row", residual=h1[0].float().cpu().numpy(), gate=None)
    fails.exact(h2[0].float().cpu().numpy(), r3["residual_out"], "adaLN 3 residual")
    fails.exact(a3.view(torch.uint8).cpu().numpy()[0], r3["packed"], "adaLN 3 (ROW packed)")

    # FFN: up (GELU + MX) from the GPU's packed activation, down with the gated residual
    inter = snap["mlp_up"][0]
    raw3 = a3.reshape(S, dim + 4).view(torch.uint8)
    a3v = raw3[:, :dim].contiguous().view(torch.float8_e4m3fn).double()
    a3dq = raw3[:, dim:].contiguous().view(torch.float32).double()
    up = (a3v @ ck["up"][0].double()) * a3dq * ck["up"][1].double() + raw["up_b"].double()
    gel = torch.nn.functional.gelu(up, approximate="tanh").to(torch.bfloat16).float().cpu().numpy()
    rc, rs = omx.mx_quantize(gel)
    same = float((inter.codes.view(torch.uint8).cpu().numpy() == rc).mean())
    print(f"mlp_up GELU+MX: identical codes {same:.4f}", flush=True)
    if same < 0.997:
        fails.append(("mlp_up codes", same))
    down = _mx_proj(inter.codes.view(torch.uint8), inter.scales, ck["down"], raw["down_b"])
    out_ref = (h2[0].float() + down.float() * c_gate.to(dev)).to(torch.bfloat16)
    fails.close(out, out_ref, "mlp_down + gated residual")
    assert not fails, fails

    # ---- end to end against the oracle ROW block, relative to the measured noise floor ----
    ck_cpu = {n: (c.cpu(), s.cpu()) for n, (c, s) in ck.items() if n in ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down")}
    raw_cpu = {n: t.cpu() for n, t in raw.items()}
    exact = oblock.row_mx_block(raw_cpu, ck_cpu, h, temb, ctx, GRID)["out"]
    kern = oblock.row_mx_block(raw_cpu, ck_cpu, h, temb, ctx, GRID, attend=oblock._attend_kernel)["out"]
    got = out.cpu()
    m_gpu = _metrics(got.float() - h.float(), exact.float() - h.float())
    m_floor = _metrics(kern.float() - h.float(), exact.float() - h.float())
    print(f"update, GPU vs exact oracle: max rel {m_gpu[0]:.2e} rms rel {m_gpu[1]:.2e} cos {m_gpu[2]:.6f}")
    print(f"update, reference kernel numerics vs exact: max rel {m_floor[0]:.2e} rms rel {m_floor[1]:.2e} "
          f"cos {m_floor[2]:.6f}")
    rel, rms, cosv = _metrics(got, exact)
    print(f"output, GPU vs exact oracle: max rel {rel:.2e} rms rel {rms:.2e} cos {cosv:.6f}")
    assert cosv >= 0.999 and rms <= 3e-2 and rel <= 6e-2, (rel, rms, cosv)
    n_rel, n_rms, n_cos = m_floor
    g_rel, g_rms, g_cos = m_gpu
    assert g_rms <= 1.25 * n_rms and g_rel <= 1.5 * n_rel and 1 - g_cos <= 1.5 * (1 - n_cos), (m_gpu, m_floor)


def test_row_dit_forward_matches_blocks(pkg, dev):
    """The ROW recipe's block loop (rotate-half caches built once per forward) equals block-by-block
    calls bit for bit, over two blocks at a reduced width (dim 1024, 8 heads, FFN 2816)."""
    blk, rb = pkg.block, pkg.row_block
    g = torch.Generator(device=dev).manual_seed(17)
    made = [blk.random_block_weights(dev, g, dim=1024, ffn=2816, heads=8, qk_gamma_mean=1.0) for _ in range(2)]
    ws = [rb.row_block_weights(raw)[0] for _, raw in made]
    grid = (2, 10, 12)
    S = grid[0] * grid[1] * grid[2]
    h = torch.randn(S, 1024, device=dev, generator=g).to(torch.bfloat16)
    temb = torch.randn(6, 1024, device=dev, generator=g)
    ctx = torch.randn(77, 1024, device=dev, generator=g).to(torch.bfloat16)
    crosses = [rb.project_cross_kv_row(w, ctx) for w in ws]
    caches = rb.rotate_half_caches(grid, dev)
    x = h
    for w, cr in zip(ws, crosses):
        x = rb.row_block_forward(w, x, temb, caches, cr)
    assert torch.equal(rb.row_dit_forward(ws, h, temb, grid, crosses), x)
    assert torch.isfinite(x.float()).all()
