"""Pin the attention / RoPE oracle (CPU only).

- exact attention vs a brute-force loop on tiny shapes;
- constant-max attention equals exact softmax attention and is invariant to the subtracted
  constant; a fully underflowed row hits the 1e-37 sum floor and returns zeros;
- the reference kernel's rounding points (``const_max_kernel_attention``): identical keys give the
  exact mean of V whatever the rounding; a two-key case whose bf16 P is known by hand
  (exp(-1.09765625) = 0.33365... rounds to 0.333984375) checks that both the numerator and the
  row sum use the rounded P; on random data the result stays within bf16-level error of exact
  attention;
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


def test_kernel_numerics_identical_keys_give_the_mean():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(5, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 128, generator=g).to(torch.bfloat16).expand(7, 128)
    v = torch.randn(7, 128, generator=g).to(torch.bfloat16)
    out = oa.const_max_kernel_attention(q, k, v, 128**-0.5)
    assert torch.allclose(out, v.double().mean(dim=0).expand(5, 128), atol=1e-12)


def test_kernel_numerics_round_p_in_both_sums():
    # q = (1, 0), keys (2, 0) and (0.90234375, 1), scale 1: c = 1 * 1 * max(2, 1.347) = 2, scores 2
    # and 0.90234375, shifted 0 and -1.09765625 (exact in fp16), P = 1 and bf16(0.3336521...) =
    # 0.333984375. With V = I the output is (1, p) / (1 + p) for that rounded p.
    q = torch.tensor([[1.0, 0.0]]).to(torch.bfloat16)
    k = torch.tensor([[2.0, 0.0], [0.90234375, 1.0]]).to(torch.bfloat16)
    v = torch.eye(2).to(torch.bfloat16)
    out = oa.const_max_kernel_attention(q, k, v, 1.0)
    p = 0.333984375
    assert math.exp(-1.09765625) != p
    assert torch.allclose(out, torch.tensor([[1.0 / (1 + p), p / (1 + p)]], dtype=torch.float64), atol=1e-12)


def test_kernel_numerics_close_to_exact_attention():
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(2, 48, 128, generator=g).to(torch.bfloat16) for _ in range(3))
    s = 128**-0.5
    ref = oa.torch_attend(q, k, v, s, dtype=torch.float64)
    out = oa.const_max_kernel_attention(q, k, v, s)
    err = (out - ref).abs().max()
    assert 0 < err <= 2.0**-7 * v.double().abs().max()


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


def test_rms_norm_across_heads_unit_mean_square():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 512, generator=g).to(torch.bfloat16)
    w = torch.ones(512)
    y = orope.rms_norm_across_heads(x, w).float()
    assert torch.allclose(y.pow(2).mean(dim=-1), torch.ones(7), atol=2e-2)


def test_rms_norm_is_across_heads_not_per_head():
    """Heads at very different scales: one RMS over the whole row (DistributedRMSNorm at tp=1,
    wan2_2_transformer.py:879-893) leaves their ratio intact; a per-head norm would make every
    head unit-RMS. Closed form for a row whose head h holds the constant a_h over 128 channels:
    y = a_h / sqrt(mean_h(a_h^2) + eps) * gamma."""
    a = [8.0, 0.25, -2.0, 0.0]  # bf16-exact head values
    x = torch.cat([torch.full((128,), v) for v in a])[None].to(torch.bfloat16)
    gamma = torch.cat([torch.full((128,), gv) for gv in (1.0, 2.0, 0.5, 3.0)])
    y = orope.rms_norm_across_heads(x, gamma).float()[0]
    rms = math.sqrt(sum(v * v for v in a) / 4 + 1e-6)
    for hd, (v, gv) in enumerate(zip(a, (1.0, 2.0, 0.5, 3.0))):
        want = v / rms * gv
        got = y[hd * 128 : (hd + 1) * 128]
        assert bool((got == got[0]).all())
        assert abs(float(got[0]) - want) <= 2.0**-8 * abs(want) + 1e-30, (hd, float(got[0]), want)
    # a per-head norm would give head 1 the value 2.0 (unit RMS times gamma 2); across heads it is
    # 0.25 / 4.14 * 2 = 0.12
    assert float(y[128]) < 0.2


def test_rms_norm_eps_inside_the_root():
    """A constant row c with c^2 comparable to eps: y = c / sqrt(c^2 + eps) * gamma. Dropping eps
    gives 1.0 and adding it outside the root (c / (|c| + eps)) gives 0.999; the closed form is
    1 / sqrt(2) = 0.7071 here."""
    c = 2.0**-10  # c^2 = 2^-20 ~ 9.5e-7 ~ eps
    eps = 2.0**-20
    x = torch.full((1, 256), c).to(torch.bfloat16)
    y = orope.rms_norm_across_heads(x, torch.ones(256), eps).float()
    assert abs(float(y[0, 0]) - 2.0**-0.5) <= 2.0**-8, float(y[0, 0])
    # eps as given (1e-6 in the Wan config) on a row of 1e-3: 1e-3 / sqrt(1e-6 + 1e-6)
    x = torch.full((1, 256), 1e-3).to(torch.bfloat16)
    y = orope.rms_norm_across_heads(x, torch.ones(256), 1e-6).float()
    xv = float(x[0, 0].float())
    assert abs(float(y[0, 0]) - xv / math.sqrt(xv * xv + 1e-6)) <= 2.0**-8
