"""Three chained Wan blocks (the DiT forward's loop) against the chained MXFP8 oracle.

Workload: the single-block shape (1x30x52 = 1560 tokens, 512 text tokens, dim 5120, 40 heads x 128,
FFN 13824), three blocks with their own random N(0, 0.02) weights (q/k gammas N(1, 0.02)) and
their own cached cross-attention K/V, as ``WanTransformer3DModel.forward`` runs them
(wan2_2_transformer.py:1806-1825: the cross K/V cache is built once per block, then each block
takes the previous one's output). RoPE tables come from the package's own builder.

1. ``dit_forward`` equals block-by-block ``block_forward`` bit for bit.
2. Every block, from the GPU's own input to it, passes the stage-wise checks on every token row
   (``blockcheck``: adaLN bit-exact, GEMMs per element against fp64, attentions against fp64).
3. The GPU chain against the oracle's chain from the same latent. The two are different MXFP8
   pipelines whose requantization points (attention outputs, GELU) round slightly different
   values, so they drift apart by the quantization noise; the bars below are the measured noise
   of this workload with a margin (see the module constants), while a defect in any stage moves
   the update (out - h) by far more.
"""

import pytest
import torch

import blockcheck
from oracle import block as oblock

pytestmark = pytest.mark.gpu

GRID = (1, 30, 52)
S, DIM, NBLK = 1560, 5120, 3
# end-to-end bars against the chained oracle (measured values in the assertion messages)
COS_OUT, COS_UPDATE, RMS_UPDATE = 0.999, 0.999, 4e-2


def _metrics(got, ref):
    got, ref = got.double().flatten(), ref.double().flatten()
    rel = float((got - ref).abs().max() / ref.abs().max())
    rms = float((got - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt())
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=0))
    return rel, rms, cos


def test_three_block_chain(pkg, dev):
    blk = pkg.block
    g = torch.Generator(device=dev).manual_seed(4321)
    made = [blk.random_block_weights(dev, g, qk_gamma_mean=1.0) for _ in range(NBLK)]
    blocks = [w for w, _ in made]
    gc = torch.Generator().manual_seed(77)
    h0 = torch.randn(S, DIM, generator=gc).to(torch.bfloat16)
    temb = torch.randn(6, DIM, generator=gc)
    ctx = torch.randn(512, DIM, generator=gc).to(torch.bfloat16)
    rope = pkg.rope_tables(GRID, device=dev)
    crosses = [blk.project_cross_kv(w, ctx.to(dev)) for w in blocks]
    td = temb.to(dev)

    fails = blockcheck.Failures()
    h = h0.to(dev)
    ins = []
    for i, (w, cr) in enumerate(zip(blocks, crosses)):
        ins.append(h)
        print(f"block {i}", flush=True)
        h, _ = blockcheck.check_block_rows(pkg, w, h, td, rope, cr, torch.arange(S), GRID, fails=fails)
    assert not fails, fails
    assert torch.equal(blk.dit_forward(blocks, h0.to(dev), td, rope, crosses), h)

    # the oracle's chain from the same latent
    ref = h0
    for i, (w, raw) in enumerate(made):
        raw_c = {k: v.cpu() for k, v in raw.items()}
        names = ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down")
        wq = {n: (getattr(w, n).codes.view(torch.uint8).cpu().numpy(), getattr(w, n).scales.cpu().numpy())
              for n in names}
        ref = oblock.mxfp8_block(raw_c, wq, ref, temb, ctx, GRID)["out"].to(torch.bfloat16)
        print(f"oracle block {i} done", flush=True)
    got = h.cpu()
    m_out = _metrics(got, ref)
    m_upd = _metrics(got.float() - h0.float(), ref.float() - h0.float())
    print(f"chain output: max rel {m_out[0]:.2e} rms rel {m_out[1]:.2e} cos {m_out[2]:.6f}")
    print(f"chain update (out - h0): max rel {m_upd[0]:.2e} rms rel {m_upd[1]:.2e} cos {m_upd[2]:.6f}")
    assert m_out[2] >= COS_OUT, m_out
    assert m_upd[2] >= COS_UPDATE and m_upd[1] <= RMS_UPDATE, m_upd
