"""Pin the composed block oracle (CPU only).

``oracle.block`` holds two independent restatements of ``WanTransformerBlock.forward``
(wan2_2_transformer.py:1428-1513): the MXFP8 recipe at the GPU path's quantization points
(``mxfp8_block``, built from the pinned adaLN / MX / GEMM / RoPE / attention oracles) and the
reference's BF16 eager chain (``bf16_eager_block``: ``F.layer_norm``, ``torch.matmul``,
``torch.softmax``). They share no code beyond the RoPE tables and the across-heads RMSNorm, so a
slip in the order of operations of either (a modulation row used at the wrong site, a gate on the
wrong residual, a missing bias) separates them far beyond the MXFP8 quantization error that
separates them otherwise. The planted slips below, made in the oracle's inputs, show the margin.

Shape: dim 256 (2 heads of 128), FFN 512, a 1x4x6 latent grid (24 tokens), 16 text tokens;
weights N(0, 0.02), q/k gammas N(1, 0.02), activations and modulation N(0, 1), seeded.
"""

import torch

from oracle import block as ob
from oracle import gemm as og

DIM, FFN, GRID, ST = 256, 512, (1, 4, 6), 16
NAMES = ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down")


def _setup(seed=5):
    g = torch.Generator().manual_seed(seed)

    def rnd(*s):
        return (torch.randn(*s, generator=g) * 0.02).to(torch.bfloat16)

    def vec(n, m=0.0):
        return (m + torch.randn(n, generator=g) * 0.02).float()

    raw = {"scale_shift_table": vec(6 * DIM).view(6, DIM), "qkv_w": rnd(DIM, 3 * DIM), "qkv_b": vec(3 * DIM),
           "norm_q": vec(DIM, 1.0), "norm_k": vec(DIM, 1.0), "o_w": rnd(DIM, DIM), "o_b": vec(DIM),
           "norm2_weight": vec(DIM, 1.0), "norm2_bias": vec(DIM), "q2_w": rnd(DIM, DIM), "q2_b": vec(DIM),
           "k2_w": rnd(DIM, DIM), "k2_b": vec(DIM), "v2_w": rnd(DIM, DIM), "v2_b": vec(DIM),
           "norm_q2": vec(DIM, 1.0), "norm_k2": vec(DIM, 1.0), "o2_w": rnd(DIM, DIM), "o2_b": vec(DIM),
           "up_w": rnd(DIM, FFN), "up_b": vec(FFN), "down_w": rnd(FFN, DIM), "down_b": vec(DIM)}
    wq = {n: og.quantize_weight(raw[n + "_w"].float().numpy()) for n in NAMES}
    S = GRID[0] * GRID[1] * GRID[2]
    h = torch.randn(S, DIM, generator=g).to(torch.bfloat16)
    temb = torch.randn(6, DIM, generator=g)
    ctx = torch.randn(ST, DIM, generator=g).to(torch.bfloat16)
    return raw, wq, h, temb, ctx


def _cos_update(a, b, h):
    a, b = (a.double() - h.double()).flatten(), (b.double() - h.double()).flatten()
    return float(torch.nn.functional.cosine_similarity(a, b, dim=0))


def test_mxfp8_block_agrees_with_the_eager_block():
    raw, wq, h, temb, ctx = _setup()
    eager = ob.bf16_eager_block(raw, h, temb, ctx, GRID)
    mx = ob.mxfp8_block(raw, wq, h, temb, ctx, GRID)["out"]
    kern = ob.mxfp8_block(raw, wq, h, temb, ctx, GRID, attend=ob._attend_kernel)["out"]
    c = _cos_update(mx, eager, h)
    assert c >= 0.995, c
    assert _cos_update(kern, eager, h) >= 0.995
    # the intermediates the GPU stages are checked against have the documented shapes
    r = ob.mxfp8_block(raw, wq, h, temb, ctx, GRID)
    assert r["qkv"].shape == (h.shape[0], 3 * DIM) and r["inter"].shape == (h.shape[0], FFN)


def test_planted_composition_slips_are_far_outside_the_quantization_gap():
    raw, wq, h, temb, ctx = _setup()
    eager = ob.bf16_eager_block(raw, h, temb, ctx, GRID)
    base = _cos_update(ob.mxfp8_block(raw, wq, h, temb, ctx, GRID)["out"], eager, h)
    slips = {
        # shift and scale of the first adaLN site swapped
        "shift<->scale": temb[[1, 0, 2, 3, 4, 5]],
        # the self-attention gate applied to the FFN residual and vice versa
        "gate<->c_gate": temb[[0, 1, 5, 3, 4, 2]],
        # cross-attention modulation rows used at the FFN site
        "c_shift<->shift": temb[[3, 1, 2, 0, 4, 5]],
    }
    for name, t in slips.items():
        raw_t = dict(raw)
        c = _cos_update(ob.mxfp8_block(raw_t, wq, h, t, ctx, GRID)["out"], eager, h)
        assert c < base - 0.05, (name, c, base)


def _checkpoint(raw):
    """Per-tensor FP8 checkpoint weights (codes [K, N] e4m3fn of w / s, s = amax / 448, expanded per
    channel), the fused QKV as its three Q, K, V tensors with three scalars."""
    def quant(w):
        s = w.float().abs().max() / 448.0
        return (w.float() / s).to(torch.float8_e4m3fn), s

    ck = {}
    parts = [quant(raw["qkv_w"][:, i * DIM : (i + 1) * DIM]) for i in range(3)]
    ck["qkv"] = (torch.cat([c for c, _ in parts], 1), torch.cat([s.expand(DIM) for _, s in parts]))
    for n in NAMES[1:]:
        c, s = quant(raw[n + "_w"])
        ck[n] = (c, s.expand(c.shape[1]))
    return ck


def test_row_recipe_block_agrees_with_the_eager_block():
    """The ROW recipe (``row_mx_block``: ROW activations, per-tensor FP8 weights with per-channel
    scales) against the independent BF16 eager chain: its update agrees within the quantization gap
    (per-row activation scales lose more than per-32 block scales, so the bar is lower than the MX
    recipe's), and the planted composition slips fall far below it."""
    raw, _, h, temb, ctx = _setup()
    ck = _checkpoint(raw)
    eager = ob.bf16_eager_block(raw, h, temb, ctx, GRID)
    r = ob.row_mx_block(raw, ck, h, temb, ctx, GRID)
    base = _cos_update(r["out"], eager, h)
    assert base >= 0.995, base
    assert r["a1_packed"].shape == (h.shape[0], DIM + 4) and r["inter"].shape == (h.shape[0], FFN)
    for name, t in {"shift<->scale": temb[[1, 0, 2, 3, 4, 5]], "gate<->c_gate": temb[[0, 1, 5, 3, 4, 2]],
                    "c_shift<->shift": temb[[3, 1, 2, 0, 4, 5]]}.items():
        c = _cos_update(ob.row_mx_block(raw, ck, h, t, ctx, GRID)["out"], eager, h)
        assert c < base - 0.05, (name, c, base)
    # a dropped channel scale (the weight codes taken as the weights) is far off as well
    bad = {n: (c, torch.ones_like(s)) for n, (c, s) in ck.items()}
    c = _cos_update(ob.row_mx_block(raw, bad, h, temb, ctx, GRID)["out"], eager, h)
    assert c < base - 0.05, c
