"""GPU parity of one Wan2.2-A14B-shaped block (MXFP8 projections, bf16 attention).

Workload (the single-block configuration): dim 5120, 40 heads x 128, FFN 13824 GELU-tanh,
RMSNorm on q/k (eps 1e-6), 3D RoPE over a 1x30x52 latent grid (1560 tokens), cross-attention to
512 text tokens. Weights N(0, 0.02) except the q/k RMSNorm gammas, N(1, 0.02) (with N(0, 0.02)
gammas q and k are ~0 and attention degenerates to a plain average); activations N(0, 1);
6x5120 timestep modulation N(0, 1). All seeded.

Two levels of checking:
1. stage-wise: every kernel stage of the block is re-computed by the oracle from the GPU's own
   inputs to that stage. adaLN stages (codes, scales, bf16 residual) must be bit-exact; bf16 stage
   outputs (GEMMs, norm/RoPE) must meet max|err|/max|ref| <= 2e-2 and cosine >= 0.999; MX stage
   outputs (attention, GELU) are compared with the oracle's MX quantization of its own bf16 result:
   at least 98.5% (self-attention), 91% (cross-attention over 512 keys) and 99.7% (GELU) of the
   codes identical, and no fewer than the reference attention kernel's own numerics reach (less
   0.01), every element within one e4m3 step plus 2^-7 of its 32-block max, cosine >= 0.999.
   Measured: GPU 99.3%, 92.5%, 99.86%; the reference kernel's rounding points (bf16 P, bf16
   pre-scaled Q, fp16 shifted scores; ``oracle.attention.const_max_kernel_attention``) on the same
   stage inputs keep 99.1% (self) and 90.2% (cross) of the exact oracle's codes. Over 512 text keys
   a bf16 rounding of P or of the pre-scaled Q moves outputs across e4m3 boundaries most often.
2. end to end: the oracle's MXFP8 block from the same block inputs vs the GPU block output:
   cosine >= 0.999, relative RMS error <= 3e-2 and max|err|/max|ref| <= 6e-2, and relative to
   the noise floor measured in the same test: the oracle block run with the reference kernel's
   attention numerics against the exact oracle block (measured max 3.5e-2, RMS 2.4e-2, cosine
   0.99972; the GPU: 3.2e-2, 2.3e-2, 0.99973). The GPU may be no further from the exact oracle
   than 1.25x that RMS, 1.5x that max error and 1.5x that cosine deficit. The floor is this large
   because the block is chaotic at the rounding level: each of its five MX requantization points
   turns a one-ulp difference into a full e4m3 step for elements near a boundary (moving 0.1% of
   the input elements by one bf16 ulp moves the oracle's own output by max 4.4e-2, RMS 2.3e-2).
   The stage-wise checks pin every kernel at the single-stage bars. The BF16 eager reference block
   is reported (the gap is the MXFP8 quantization error), with only a loose cosine asserted.
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


FAILS = []


def _close(got, ref, what, bar=(2e-2, 0.999)):
    got, ref = got.double().flatten(), ref.double().flatten()
    rel = float((got - ref).abs().max() / ref.abs().max())
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=0))
    print(f"{what}: rel_err {rel:.2e} cos {cos:.6f}")
    if not (rel <= bar[0] and cos >= bar[1]):
        FAILS.append((what, rel, cos))


def _e2e_metrics(got, ref):
    got, ref = got.double().flatten(), ref.double().flatten()
    rel = float((got - ref).abs().max() / ref.abs().max())
    rms = float((got - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt())
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=0))
    return rel, rms, cos


def _close_e2e(got, ref, what, noise=None):
    """Absolute bars, and with ``noise`` (the metrics of the reference kernel's numerics against the
    same exact oracle) bars relative to it: the GPU may sit no further from the exact oracle than
    the reference's own attention numerics do, with a margin (1.25x RMS, 1.5x max error, 1.5x the
    cosine deficit)."""
    rel, rms, cos = _e2e_metrics(got, ref)
    print(f"{what}: max rel_err {rel:.2e} rms rel_err {rms:.2e} cos {cos:.6f}")
    assert cos >= 0.999 and rms <= 3e-2 and rel <= 6e-2, (what, rel, rms, cos)
    if noise is not None:
        n_rel, n_rms, n_cos = noise
        assert rms <= 1.25 * n_rms and rel <= 1.5 * n_rel and 1 - cos <= 1.5 * (1 - n_cos), (what, (rel, rms, cos), noise)


def _mx_close(got_mx, ref_bf16, what, min_same, kernel_bf16=None):
    """GPU MX output vs MX(oracle bf16 output): codes mostly identical; every element within one
    e4m3 step of itself plus 2^-7 of its 32-block's max (bf16-level absolute error of the stage).
    ``kernel_bf16``: the same stage through the reference attention kernel's rounding points; the
    share of its MX codes identical to the exact oracle's is printed beside the GPU's."""
    rc, rs = omx.mx_quantize(ref_bf16.float().numpy())
    gc, gs = _mx_np(got_mx)
    g = omx.mx_dequantize(gc, gs)
    r = omx.mx_dequantize(rc, rs)
    same = float((gc == rc).mean())
    if kernel_bf16 is not None:
        kc, _ = omx.mx_quantize(kernel_bf16.float().numpy())
        same_k = float((kc == rc).mean())
        print(f"{what}: reference kernel numerics vs exact: identical codes {same_k:.4f}")
        min_same = max(min_same, same_k - 0.01)
    bmax = np.repeat(np.abs(r).reshape(*r.shape[:-1], -1, 32).max(axis=-1), 32, axis=-1)
    tol = 2.0**-3 * np.maximum(np.abs(g), np.abs(r)) + 2.0**-7 * bmax + 1e-30
    worst = float((np.abs(g - r) / tol).max())
    cos = float(np.dot(g.ravel(), r.ravel()) / (np.linalg.norm(g) * np.linalg.norm(r)))
    print(f"{what}: identical codes {same:.4f}, max |diff|/tol {worst:.2f}, cos {cos:.6f}")
    if not (same >= min_same and worst <= 1.0 and cos >= 0.999):
        FAILS.append((what, same, worst, cos))


def _np8(t):
    return t.view(torch.uint8).cpu().numpy()


def _mx_np(m):
    return _np8(m.codes), m.scales.cpu().numpy()


def _deq(m):
    return torch.from_numpy(omx.mx_dequantize(*_mx_np(m)))


@pytest.fixture(scope="module")
def run(pkg, dev):
    blk = pkg.block
    g = torch.Generator(device=dev).manual_seed(1234)
    w, raw = blk.random_block_weights(dev, g, qk_gamma_mean=1.0)
    S = GRID[0] * GRID[1] * GRID[2]
    gc = torch.Generator().manual_seed(99)
    h = torch.randn(S, 5120, generator=gc).to(torch.bfloat16)
    temb = torch.randn(6, 5120, generator=gc)
    ctx = torch.randn(512, 5120, generator=gc).to(torch.bfloat16)
    cos, sin = orope.wan_rope(GRID)
    rope = pkg.rope_tables(GRID, device=dev)
    cross = blk.project_cross_kv(w, ctx.to(dev))
    snap, live = {}, {}

    def timer(name, fn):
        r = fn()
        # snapshot (the Q|K buffer is normalized in place right after its GEMM) and keep the live object
        if isinstance(r, tuple) and all(isinstance(x, torch.Tensor) for x in r):
            parts = [x.clone() for x in r]
            c = type(r)(*parts) if hasattr(r, "_fields") else tuple(parts)
        else:
            c = r.clone() if isinstance(r, torch.Tensor) else r
        snap.setdefault(name, []).append(c)
        live.setdefault(name, []).append(r)
        return r

    out = blk.block_forward(w, h.to(dev), temb.to(dev), rope, cross, timer=timer).cpu()
    raw_c = {k: v.cpu() for k, v in raw.items()}
    names = ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down")
    wq = {n: (_np8(getattr(w, n).codes), getattr(w, n).scales.cpu().numpy()) for n in names}
    return dict(w=w, raw=raw_c, wq=wq, h=h, temb=temb, ctx=ctx, cross=cross, snap=snap, live=live, out=out, S=S,
                cos=cos, sin=sin)


def test_block_stagewise(pkg, dev, run):
    r = run
    raw, wq, snap, live, S = r["raw"], r["wq"], r["snap"], r["live"], r["S"]
    e = raw["scale_shift_table"].float() + r["temb"].float()
    shift, sc, gate, c_shift, c_sc, c_gate = (e[i] for i in range(6))
    heads, D, dim = 40, 128, 5120
    s = D**-0.5

    # adaLN 1 (bit-exact)
    a1 = snap["adaln"][0]
    ref = oadaln.adaln_quant(r["h"].float().numpy(), (1 + sc).numpy(), shift.numpy(), quant="mx")
    np.testing.assert_array_equal(_np8(a1.codes), ref["codes"])
    np.testing.assert_array_equal(a1.scales.cpu().numpy(), ref["scales"])
    # QKV projection from the GPU's a1: Q|K token-major, V written transposed (V^T)
    qk_pre, vt = (t.cpu() for t in snap["gemm_qkv"][0])
    order = [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    S_pad = vt.shape[-1]
    slot_key = torch.tensor([16 * (i // 16) + order[i % 16] for i in range(S_pad)])
    v_tok = torch.empty(S_pad, heads, D, dtype=torch.bfloat16)
    v_tok[slot_key] = vt.permute(2, 0, 1)
    assert not bool(v_tok[S:].float().any()), "V^T past the last token must be zero"
    qkv_pre = torch.cat([qk_pre.float(), v_tok[:S].reshape(S, dim).float()], dim=1)
    _close(qkv_pre, oblock._lin(*_mx_np(a1), wq["qkv"], raw["qkv_b"]), "qkv projection (V as V^T)")
    # Q/K RMSNorm + RoPE from the GPU's projection: K in place (its own pass), Q inside the attention
    qkv_post = live["gemm_qkv"][0][0].cpu()
    refn = {}
    for part, gname in ((0, "norm_q"), (1, "norm_k")):
        x = qkv_pre[:, part * dim : (part + 1) * dim].to(torch.bfloat16)
        rn = orope.rms_norm_across_heads(x, raw[gname]).view(1, S, heads, D)
        refn[gname] = orope.apply_rotary_emb_wan(rn, r["cos"][None, :, None], r["sin"][None, :, None]).view(S, dim)
    _close(qkv_post[:, dim : 2 * dim], refn["norm_k"], "norm_k + RoPE")
    assert torch.equal(qkv_post[:, :dim], qk_pre[:, :dim]), "Q must stay the raw projection"
    # self-attention from the GPU's raw q (normalized + rotated on load), k, v, against the oracle's
    # attention over the oracle-prepared q
    k = qkv_post[:, dim : 2 * dim].view(S, heads, D)
    v = v_tok[:S]
    o1 = snap["self_attention"][0]
    qn = refn["norm_q"].to(torch.bfloat16).view(S, heads, D)
    _mx_close(o1, oblock._attend(qn, k, v, s), "self-attention with Q RMSNorm+RoPE on load (MX out)", 0.985,
              kernel_bf16=oblock._attend_kernel(qn, k, v, s))
    # o-proj with the gated residual in its epilogue, from the GPU's MX attention output:
    # h1 = bf16(h + bf16(o1 @ Wo + b) * gate)
    h1 = snap["gemm_o"][0].cpu()
    attn1_ref = oblock._lin(*_mx_np(o1), wq["o"], raw["o_b"])
    h1_ref = oadaln.adaln_quant(attn1_ref.numpy(), None, None, norm_type="none", residual=r["h"].float().numpy(),
                                gate=gate.numpy())["residual_out"]
    _close(h1, torch.from_numpy(h1_ref), "o-proj + gated residual")
    # ... and bit for bit what the GEMM's plain output followed by adaLN's residual add gives (the
    # branch itself is not compared after the fact: one bf16 ulp of the sum is several percent of a
    # small branch)
    attn1_gpu = pkg.mxfp8_linear(live["self_attention"][0], r["w"].o)
    h1_two = pkg.adaln_kernels.adaln_quant_2d(attn1_gpu, None, None, eps=0.0, norm_type="none", quant="none",
                                              residual=r["h"].to(dev), gate=gate.to(dev))[0]
    assert torch.equal(h1_two.cpu(), h1), "fused o-proj residual differs from the two-kernel path"
    # adaLN 2 (bit-exact)
    a2 = snap["adaln"][1]
    ref = oadaln.adaln_quant(h1.float().numpy(), raw["norm2_weight"].numpy(), raw["norm2_bias"].numpy(), quant="mx")
    np.testing.assert_array_equal(_np8(a2.codes), ref["codes"])
    np.testing.assert_array_equal(a2.scales.cpu().numpy(), ref["scales"])
    # cross-attention query projection + RMSNorm
    q2_pre = snap["gemm_q2"][0].cpu()
    _close(q2_pre, oblock._lin(*_mx_np(a2), wq["q2"], raw["q2_b"]), "cross q projection")
    q2 = orope.rms_norm_across_heads(q2_pre.to(torch.bfloat16), raw["norm_q2"])
    # cached cross K/V vs the oracle's projection of the same context
    cc, cs = omx.mx_quantize(r["ctx"].float().numpy())
    k2 = orope.rms_norm_across_heads(oblock._lin(cc, cs, wq["k2"], raw["k2_b"]).to(torch.bfloat16), raw["norm_k2"])
    v2 = oblock._lin(cc, cs, wq["v2"], raw["v2_b"])
    _close(r["cross"].k.cpu().reshape(512, dim), k2, "cross K (projected once)")
    vt = r["cross"].vt.cpu()[:, :, :512]
    order = [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    slot_key = torch.tensor([16 * (i // 16) + order[i % 16] for i in range(512)])
    v_gpu = torch.empty(512, heads, D, dtype=torch.bfloat16)
    v_gpu[slot_key] = vt.permute(2, 0, 1)
    _close(v_gpu.reshape(512, dim), v2, "cross V (projected once)")
    # cross-attention from the GPU's q2 and cached K/V
    o2 = snap["cross_attention"][0]
    _mx_close(o2, oblock._attend(q2.view(S, heads, D), r["cross"].k.cpu(), v_gpu, s), "cross-attention (MX out)", 0.91,
              kernel_bf16=oblock._attend_kernel(q2.view(S, heads, D), r["cross"].k.cpu(), v_gpu, s))
    # cross o-proj with the residual in its epilogue: h2 = bf16(h1 + bf16(o2 @ Wo2 + b))
    h2 = snap["gemm_o2"][0].cpu()
    attn2_ref = oblock._lin(*_mx_np(o2), wq["o2"], raw["o2_b"])
    h2_ref = oadaln.adaln_quant(attn2_ref.numpy(), None, None, norm_type="none", residual=h1.float().numpy(),
                                gate=None)["residual_out"]
    _close(h2, torch.from_numpy(h2_ref), "cross o-proj + residual")
    attn2_gpu = pkg.mxfp8_linear(live["cross_attention"][0], r["w"].o2)
    h2_two = pkg.adaln_kernels.adaln_quant_2d(attn2_gpu, None, None, eps=0.0, norm_type="none", quant="none",
                                              residual=h1.to(dev), gate=None)[0]
    assert torch.equal(h2_two.cpu(), h2), "fused cross o-proj residual differs from the two-kernel path"
    # adaLN 3 (bit-exact)
    a3 = snap["adaln"][2]
    ref = oadaln.adaln_quant(h2.float().numpy(), (1 + c_sc).numpy(), c_shift.numpy(), quant="mx")
    np.testing.assert_array_equal(_np8(a3.codes), ref["codes"])
    # FFN up + GELU + MX from the GPU's a3
    inter = snap["gemm_up"][0]
    up = oblock._deq(*_mx_np(a3)) @ oblock._deq(*wq["up"]).T + raw["up_b"].float()
    _mx_close(inter, torch.nn.functional.gelu(up, approximate="tanh").to(torch.bfloat16), "FFN up + GELU (MX out)", 0.997)
    # down projection + gated residual from the GPU's MX intermediate
    ffn = oblock._lin(*_mx_np(inter), wq["down"], raw["down_b"])
    ref_out = (h2.float().cpu() + ffn * c_gate).to(torch.bfloat16).float()
    _close(r["out"], ref_out, "FFN down + gated residual")
    _close(r["out"] - h2.float().cpu(), ref_out - h2.float().cpu(), "FFN branch (out - h2)")
    assert not FAILS, FAILS


def test_block_end_to_end(run):
    r = run
    ref = oblock.mxfp8_block(r["raw"], r["wq"], r["h"], r["temb"], r["ctx"], GRID)
    refk = oblock.mxfp8_block(r["raw"], r["wq"], r["h"], r["temb"], r["ctx"], GRID, attend=oblock._attend_kernel)
    hf = r["h"].float()
    n_out, n_upd = _e2e_metrics(refk["out"], ref["out"]), _e2e_metrics(refk["out"] - hf, ref["out"] - hf)
    print("reference kernel numerics vs exact oracle block: output max rel {:.2e} rms {:.2e} cos {:.6f}".format(*n_out))
    print("reference kernel numerics vs exact oracle block: update max rel {:.2e} rms {:.2e} cos {:.6f}".format(*n_upd))
    _close_e2e(r["out"], ref["out"], "block output vs MXFP8 oracle block", noise=n_out)
    _close_e2e(r["out"] - hf, ref["out"] - hf, "block update (out - h) vs oracle", noise=n_upd)
    _close_e2e(r["out"], refk["out"], "block output vs oracle block with the kernel's attention numerics")
    eager = oblock.bf16_eager_block(r["raw"], r["h"], r["temb"], r["ctx"], GRID).float()
    cos_e = float(torch.nn.functional.cosine_similarity(r["out"].double().flatten(), eager.double().flatten(), dim=0))
    d_e = float(torch.nn.functional.cosine_similarity((r["out"] - r["h"].float()).double().flatten(),
                                                      (eager - r["h"].float()).double().flatten(), dim=0))
    print(f"vs BF16 eager reference block: cos(out) {cos_e:.6f}, cos(out - h) {d_e:.6f} (MXFP8 quantization budget)")
    assert cos_e >= 0.99
