"""The Wan 3D RoPE tables built on the GPU, and the rotate-half pairing of the Q/K pass.

``rope_tables`` / ``WanRotaryPosEmbed`` must reproduce the oracle's restatement of
``WanRotaryPosEmbed`` (rope.py:37-114; fp64 angles, fp32 cos/sin) bit for bit for the three grids
of the workloads -- the single block (1x30x52), the 480p step (21x30x52) and the 720p step
(21x45x80) -- in all three layouts. The oracle's tables are pinned by the closed-form angle test.

The Q/K pass with ``rope_pairs="halves"`` on channels de-interleaved per head must give exactly the
bits of the interleaved pass on the natural channels, permuted the same way (the equivalence the
reference's fused QKV kernel relies on, row_mx_loaders.py:26-39).
"""

import pytest
import torch

from oracle import rope as orope

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("grid", [(1, 30, 52), (21, 30, 52), (21, 45, 80)])
def test_tables_bit_exact(pkg, dev, grid):
    cos, sin = orope.wan_rope(grid)  # interleaved [S, 128] fp32
    for layout, ref_c, ref_s in [
        ("interleaved", cos, sin),
        ("pairs", *orope.base_angles(cos, sin)),
        ("rotate_half", torch.cat([cos[:, 0::2]] * 2, -1), torch.cat([sin[:, 1::2]] * 2, -1)),
    ]:
        c, s = pkg.rope_tables(grid, layout=layout, device=dev)
        assert torch.equal(c.cpu(), ref_c), (grid, layout)
        assert torch.equal(s.cpu(), ref_s), (grid, layout)


def test_module_forward_matches_reference_shapes(pkg, dev):
    rope = pkg.WanRotaryPosEmbed(128, (1, 2, 2), 1024)
    hs = torch.empty(1, 16, 21, 60, 104, device=dev)  # latent video -> 21 x 30 x 52 patches
    c, s = rope(hs)
    assert c.shape == (1, 32760, 1, 128) and c.dtype == torch.float32 and c.device == hs.device
    ref_c, ref_s = orope.wan_rope((21, 30, 52))
    assert torch.equal(c[0, :, 0].cpu(), ref_c) and torch.equal(s[0, :, 0].cpu(), ref_s)
    pc, ps = rope.pair_tables((21, 30, 52), dev)
    assert torch.equal(pc, c[0, :, 0, 0::2]) and torch.equal(ps, s[0, :, 0, 1::2])
    with pytest.raises(ValueError):
        pkg.rope_tables((1, 1, 2000), device=dev)


def _perm_cols(Nh, dev):
    perm = torch.cat([torch.arange(0, 128, 2), torch.arange(1, 128, 2)]).to(dev)
    return (torch.arange(Nh, device=dev)[:, None] * 128 + perm[None]).reshape(-1)


def test_rotate_half_pairs_equal_interleaved_on_permuted_channels(pkg, dev):
    """Bit for bit on inputs whose sums of squares are exact in fp32 (multiples of 2^-3 up to 1,
    so the row sums do not depend on the order in which the permuted lanes add them). The per-head
    key-norm maxima sum squares of the rotated outputs, whose order the permutation changes, so
    they agree to fp32 rounding."""
    ops = pkg.attention_ops
    S, Nh = 1560, 40
    g = torch.Generator(device=dev).manual_seed(5)
    x = (torch.randint(-8, 9, (S, Nh * 128), generator=g, device=dev).float() / 8).to(torch.bfloat16)
    gamma = 1.0 + 0.1 * torch.randn(Nh * 128, generator=g, device=dev)
    c, s = pkg.rope_tables((1, 30, 52), device=dev)
    cols = _perm_cols(Nh, dev)
    a = x.clone()
    ka = ops.qk_rmsnorm_rope_(a, gamma, cos=c, sin=s, want_max=True)
    b = x[:, cols].contiguous()
    kb = ops.qk_rmsnorm_rope_(b, gamma[cols], cos=c, sin=s, want_max=True, rope_pairs="halves")
    assert torch.equal(b, a[:, cols])
    assert bool(((ka - kb).abs() <= 1e-6 * ka).all())


def test_rotate_half_pairs_against_the_oracle(pkg, dev):
    """Random inputs: the halves pass against the oracle's rotate-half statement on the
    de-interleaved channels (row_mx_modules.py:51-76), within one bf16 rounding."""
    ops = pkg.attention_ops
    S, Nh = 1560, 40
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(S, Nh * 128, generator=g, device=dev).to(torch.bfloat16)
    gamma = 1.0 + 0.1 * torch.randn(Nh * 128, generator=g, device=dev)
    c, s = pkg.rope_tables((1, 30, 52), device=dev)
    cols = _perm_cols(Nh, dev)
    b = x[:, cols].contiguous()
    ops.qk_rmsnorm_rope_(b, gamma[cols], cos=c, sin=s, rope_pairs="halves")
    xn = orope.rms_norm_across_heads(x.cpu()[:, cols.cpu()], gamma.cpu()[cols.cpu()])
    cc, ss = c.cpu(), s.cpu()
    ref = orope.apply_rotate_half(xn.view(S, Nh, 128), torch.cat([cc, cc], -1)[:, None],
                                  torch.cat([ss, ss], -1)[:, None]).float()
    got = b.cpu().float().view(S, Nh, 128)
    err = (got - ref).abs()
    assert float(err.max()) <= 2.0**-7 * float(ref.abs().max())
    assert float((err > 0).float().mean()) < 1e-3
