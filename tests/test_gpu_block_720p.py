"""One Wan2.2-A14B block at the 720p step's sequence length, stage by stage.

Workload: the 720p step's latent grid 21x45x80 = 75600 tokens, 512 text tokens, dim 5120, 40
heads x 128, FFN 13824, random N(0, 0.02) weights (q/k RMSNorm gammas N(1, 0.02)), seeded N(0, 1)
latent, text context and timestep modulation. One head of K in the fused QKV output spans more
than 2 GiB here, so the attention runs its rebased-descriptor instantiation. Every stage of
``block_forward`` is checked on 128 token rows (the first 32, the last 32 and 64 spread between)
from the GPU's own inputs to that stage (see ``blockcheck``): adaLN bit-exact, GEMMs per element
against fp64 products, K norm + RoPE against the oracle, both attentions against fp64 softmax
over every key.
"""

import pytest
import torch

import blockcheck

pytestmark = pytest.mark.gpu

GRID = (21, 45, 80)
S, DIM = 21 * 45 * 80, 5120


def test_block_720p_stagewise(pkg, dev):
    blk = pkg.block
    g = torch.Generator(device=dev).manual_seed(720)
    w, _ = blk.random_block_weights(dev, g, qk_gamma_mean=1.0, keep_raw=False)
    h = torch.randn(S, DIM, generator=g, device=dev).to(torch.bfloat16)
    temb = torch.randn(6, DIM, generator=g, device=dev)
    ctx = torch.randn(512, DIM, generator=g, device=dev).to(torch.bfloat16)
    rope = pkg.rope_tables(GRID, device=dev)
    cross = blk.project_cross_kv(w, ctx)
    gc = torch.Generator().manual_seed(7)
    rows = torch.cat([torch.arange(32), 32 + torch.randperm(S - 64, generator=gc)[:64], torch.arange(S - 32, S)])
    print(f"720p block: S={S}, rows checked: {rows.numel()}", flush=True)
    out, fails = blockcheck.check_block_rows(pkg, w, h, temb, rope, cross, rows, GRID)
    assert not fails, fails
    assert bool(torch.isfinite(out.float()).all())
