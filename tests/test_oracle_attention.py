"""Pin the attention / RoPE oracle (CPU only).

- exact attention vs a brute-force loop on tiny shapes;
- constant-max attention equals exact softmax attention and is invariant to the subtracted
  constant; a fully underflowed row hits the 1e-37 sum floor and returns zeros;
- Wan RoPE: angles match the closed form theta^(-2i/dim) * position per axis, the rotation preserves
  norms, and interleaved RoPE equals rotate-half RoPE on de-interleaved channels (the equivalence
  the reference's fused QKV path relies on, row_mx_loaders.py:26-39, row_mx_modules.py:51-76).
"""

import math

import torch

from oracle import attention as oa
from oracle import rope as orope


def test_torch_attend_matches_brute_force():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(3, 5, 4, generator=g, dtype=torch.float64) for _ in range(3))
    out = oa.torch_attend(q, k, v, 0.5, dtype=torch.float64)
    for b in range(3):
        for i in range(5):
            w = [math.exp(0.5 * float(q[b, i] @ k[b, j])) for j in range(5)]
            z = sum(w)
            ref = sum(w[j] / z * v[b, j] for j in range(5))
            assert torch.allclose(out[b, i], ref, atol=1e-12)


def test_const_max_equals_softmax_and_is_shift_invariant():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, 3, 64, 128, generator=g)
    k = torch.randn(2, 3, 80, 128, generator=g)
    v = torch.randn(2, 3, 80, 128, generator=g)
    s = 128**-0.5
    ref = oa.torch_attend(q, k, v, s, dtype=torch.float64)
    cm = oa.const_max_attention(q, k, v, s)
    assert torch.allclose(cm, ref, atol=1e-10)
    c = oa.const_max_bound(q, k, s)
    assert torch.allclose(oa.const_max_attention(q, k, v, s, c=c + 7.0), ref, atol=1e-10)
    # the bound really bounds every score
    scores = (q.double() @ k.double().transpose(-2, -1)) * s
    assert bool((scores <= c + 1e-9).all())


def test_const_max_underflow_clamp():
    q = torch.ones(1, 4, 128)
    k = torch.ones(1, 6, 128)
    v = torch.randn(1, 6, 128)
    out = oa.const_max_attention(q, k, v, 1.0, c=torch.full((1, 4, 1), 1e4, dtype=torch.float64))
    assert bool((out == 0).all())


def test_wan_rope_closed_form():
    cos, sin = orope.wan_rope((3, 4, 5))
    assert cos.shape == (60, 128)
    # token (f=2, h=1, w=3); axis dims t/h/w = 44/42/42, interleaved duplicates
    tok = 2 * 20 + 1 * 5 + 3
    for lane, (pos, base, dim) in {0: (2, 0, 44), 10: (2, 0, 44), 44: (1, 44, 42), 50: (1, 44, 42),
                                   86: (3, 86, 42), 127: (3, 86, 42)}.items():
        i = (lane - base) // 2
        ang = pos * 10000.0 ** (-2 * i / dim)
        assert abs(float(cos[tok, lane]) - math.cos(ang)) < 1e-6
        assert abs(float(sin[tok, lane]) - math.sin(ang)) < 1e-6
        assert cos[tok, lane - (lane - base) % 2] == cos[tok, lane - (lane - base) % 2 + 1]


def test_rope_preserves_norm_and_matches_rotate_half():
    g = torch.Generator().manual_seed(2)
    cos, sin = orope.wan_rope((2, 3, 4))
    x = torch.randn(1, 24, 5, 128, generator=g, dtype=torch.float64)
    c4, s4 = cos.double()[None, :, None, :], sin.double()[None, :, None, :]
    y = orope.apply_rotary_emb_wan(x, c4, s4)
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), atol=1e-10)
    perm = orope.deinterleave_perm(128)
    bc, bs = orope.base_angles(c4, s4)
    y_rh = orope.apply_rotate_half(x[..., perm], torch.cat([bc, bc], -1), torch.cat([bs, bs], -1))
    assert torch.allclose(y_rh.to(torch.float64), y[..., perm], atol=1e-6)


def test_rms_norm_across_heads():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 512, generator=g).to(torch.bfloat16)
    w = torch.ones(512)
    y = orope.rms_norm_across_heads(x, w).float()
    assert torch.allclose(y.pow(2).mean(dim=-1), torch.ones(7), atol=2e-2)
