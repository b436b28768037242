"""GPU: a block loaded from a ComfyUI FP8-scaled checkpoint runs on the MXFP8 kernels.

The checkpoint is synthetic but in the real file format (per-tensor absmax e4m3 weights with scalar
F32 scales, F16 biases / norms / modulation; see comfy_ckpt.py), at reduced width: dim 512
(4 heads x 128; the Q/K norm kernel takes a multiple of 4 heads), FFN 1024, 1 layer. Loaded
through ``ComfyFp8Checkpoint`` the weights keep their checkpoint codes, neutral e8m0 block scales
and a per-channel ``col_scale``: the reference's ROW_MX recipe (row_mx_loaders.py:115-140,
194-260; qkv_cte.py:3996-4021).

1. Every projection on MX activations against the oracle's fp64 product of the dequantized
   operands times the per-channel scale, plus bias: max|err|/max|ref| <= 2e-2, cosine >= 0.999
   (the GEMM bar).
2. The whole block on those weights against the oracle's MXFP8 block given the same codes, block
   scales and per-channel scales: the end-to-end bars of test_gpu_block.py (cosine >= 0.999,
   relative RMS <= 3e-2, max relative <= 6e-2).
"""

import numpy as np
import pytest
import torch

from comfy_ckpt import write_checkpoint
from oracle import block as oblock
from oracle import gemm as ogemm
from oracle import mx as omx
from oracle import rope as orope

pytestmark = pytest.mark.gpu

DIM, FFN, GRID, S_TXT = 512, 1024, (1, 4, 8), 16


@pytest.fixture(scope="module")
def loaded(pkg, dev, tmp_path_factory):
    path = tmp_path_factory.mktemp("ckpt") / "wan_fp8_scaled.safetensors"
    write_checkpoint(path, num_layers=1, dim=DIM, ffn=FFN, seed=11)
    f = pkg.comfy_fp8_checkpoint.ComfyFp8Checkpoint(str(path), num_layers=1)
    host = f.host_block(0)
    w = pkg.comfy_fp8_checkpoint.block_weights_from_host(host, dev)
    return host, w


def _np8(t):
    return t.view(torch.uint8).cpu().numpy()


def _close(got, ref, what, rel_bar=2e-2, cos_bar=0.999):
    got, ref = got.double().flatten(), ref.double().flatten()
    rel = float((got - ref).abs().max() / ref.abs().max())
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=0))
    print(f"{what}: rel_err {rel:.2e} cos {cos:.6f}")
    assert rel <= rel_bar and cos >= cos_bar, (what, rel, cos)


def test_checkpoint_projections(pkg, dev, loaded):
    host, w = loaded
    g = torch.Generator().manual_seed(5)
    for name in ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down"):
        mw = getattr(w, name)
        assert torch.equal(mw.codes.cpu(), host[name].codes)
        assert bool((mw.scales == 127).all())
        x = torch.randn(200, mw.in_features, generator=g).to(torch.bfloat16)
        xa = pkg.adaln_kernels.adaln_quant_2d(x.to(dev), None, None, eps=0.0, norm_type="none", quant="mx")
        y = pkg.mxfp8_linear(xa, mw).cpu()
        ref = ogemm.mx_gemm(_np8(xa.codes), xa.scales.cpu().numpy(), host[name].codes.numpy(),
                            mw.scales.cpu().numpy(), bias=host[name].bias.numpy(),
                            col_scale=host[name].col_scale.numpy())
        _close(y, ref, f"checkpoint {name} projection")


def test_checkpoint_block_end_to_end(pkg, dev, loaded):
    host, w = loaded
    blk = pkg.block
    S = GRID[0] * GRID[1] * GRID[2]
    gc = torch.Generator().manual_seed(21)
    h = torch.randn(S, DIM, generator=gc).to(torch.bfloat16)
    temb = torch.randn(6, DIM, generator=gc)
    ctx = torch.randn(S_TXT, DIM, generator=gc).to(torch.bfloat16)
    cos, sin = orope.wan_rope(GRID)
    rope = pkg.attention_ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    cross = blk.project_cross_kv(w, ctx.to(dev))
    out = blk.block_forward(w, h.to(dev), temb.to(dev), rope, cross).cpu()
    assert bool(torch.isfinite(out.float()).all())

    raw = {k: host[k] for k in ("scale_shift_table", "norm_q", "norm_k", "norm2_weight", "norm2_bias", "norm_q2",
                                "norm_k2")}
    wq = {}
    for name in ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down"):
        p = host[name]
        raw[f"{name}_b"] = p.bias
        wq[name] = (p.codes.numpy(), np.full((p.codes.shape[0], p.codes.shape[1] // 32), 127, np.uint8),
                    p.col_scale.numpy())
    ref = oblock.mxfp8_block(raw, wq, h, temb, ctx, GRID)["out"]
    for got, want, what in ((out, ref, "block output"), (out - h.float(), ref - h.float(), "block update (out - h)")):
        got, want = got.double().flatten(), want.double().flatten()
        rel = float((got - want).abs().max() / want.abs().max())
        rms = float((got - want).pow(2).mean().sqrt() / want.pow(2).mean().sqrt())
        c = float(torch.nn.functional.cosine_similarity(got, want, dim=0))
        print(f"checkpoint {what} vs MXFP8 oracle block: max rel {rel:.2e} rms rel {rms:.2e} cos {c:.6f}")
        assert c >= 0.999 and rms <= 3e-2 and rel <= 6e-2, (what, rel, rms, c)


def test_checkpoint_mx_scales_are_neutral(loaded):
    """The block scales the loader writes are e8m0 127 = 2^0, so the oracle's MX dequant of the codes
    equals the plain e4m3 value."""
    host, w = loaded
    codes = host["o"].codes.numpy()
    deq = omx.mx_dequantize(codes, w.o.scales.cpu().numpy())
    assert np.array_equal(deq, torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy())
