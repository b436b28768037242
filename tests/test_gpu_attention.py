"""GPU parity of the Q/K preparation and constant-max attention kernels.

Tolerances (bf16 inputs, bf16 P, fp32 accumulation): attention outputs vs exact fp64 softmax
attention on the same bf16 inputs: max |err| / max |ref| <= 2e-2 and cosine >= 0.999 (the stated
bar), plus a per-element bound of 2^-6 * max|ref|. QK norm + RoPE vs the torch restatement: within
2 bf16 ulps elementwise (multiply by reciprocal vs divide, and order of the sum of squares).
MX output codes must equal the MX quantization of the kernel's own bf16 output, bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import mx as omx
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _check_attn(out, ref):
    out, ref = out.double(), ref.double()
    err = (out - ref).abs()
    m = ref.abs().max()
    cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0)
    assert err.max() / m <= 2e-2 and cos >= 0.999, (float(err.max() / m), float(cos))
    assert bool((err <= 2.0**-6 * m).all())


# key counts cover 1, 2, 3, 4, 5, 7 and 8 tiles of 64 (the K/V ring loads two tiles per barrier, so
# odd and even tile counts and a partial last tile take different paths). With 3 to 16 tiles and
# more than one head, a workgroup walks several heads (grids this small fit one round of the CUs,
# where two heads per group leave the most workgroups: 2 and 4 heads in groups of 2, 12 heads in six
# over a last tile of one key, 10 in five; 3 heads in one group of 3; larger groups in
# test_cross_attention_head_groups). With the heads a multiple of 8 the one-head-per-workgroup
# kernels place whole heads per XCD: 8 heads over 2 tiles (the short-key kernel) and 16 over 18
# tiles.
@pytest.mark.parametrize("Sq,Sk,N", [(1, 1, 1), (300, 200, 2), (129, 197, 3), (64, 512, 4), (96, 100, 2),
                                     (70, 150, 1), (40, 300, 1), (33, 448, 1), (1000, 129, 12), (513, 512, 10),
                                     (300, 100, 8), (200, 1100, 16)])
def test_attention_core_small(pkg, dev, Sq, Sk, N):
    ops = pkg.attention_ops
    q, k, v = _rand((Sq, N, 128), 1), _rand((Sk, N, 128), 2), _rand((Sk, N, 128), 3)
    s = 128**-0.5
    vt, _ = ops.transpose_heads(v.to(dev))
    kmax = ops.head_max_norm(k.to(dev))
    ref = oa.torch_attend(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), s, dtype=torch.float64)
    tok = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s, ops.OUT_TOKEN).cpu()
    _check_attn(tok.view(Sq, N, 128).transpose(0, 1), ref)
    dm = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s, ops.OUT_DMAJOR).cpu()
    _check_attn(dm.transpose(1, 2), ref)
    torch.testing.assert_close(dm.transpose(1, 2).contiguous(), tok.view(Sq, N, 128).transpose(0, 1).contiguous(), rtol=0, atol=0)
    mx = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s, ops.OUT_MX)
    codes, scales = omx.mx_quantize(tok.float().numpy())
    np.testing.assert_array_equal(mx.codes.view(torch.uint8).cpu().numpy(), codes)
    np.testing.assert_array_equal(mx.scales.cpu().numpy(), scales)


@pytest.mark.parametrize("S,N,layout", [(100, 3, "token"), (100, 8, "token"), (1560, 40, "qkv"), (77, 4, "head"),
                                         (64, 4, "token")])
def test_transpose_heads_layout(pkg, dev, S, N, layout):
    """V^T in the attention's key order, for per-head rows (3 heads, head-major) and the four-head
    form (heads contiguous in a token: token-major and the [Q | K | V] rows), with a partial last
    64-key tile."""
    v = _rand((S, N, 128), 5 + S + N)
    if layout == "token":
        vd = v.to(dev)
    elif layout == "qkv":
        vd = torch.zeros(S, 3, N, 128, dtype=torch.bfloat16, device=dev)
        vd[:, 2] = v.to(dev)
        vd = vd[:, 2]
    else:
        vd = v.to(dev).permute(1, 0, 2).contiguous().permute(1, 0, 2)
    vt, S_pad = pkg.attention_ops.transpose_heads(vd)
    assert S_pad == (S + 63) // 64 * 64
    order = [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    slot_key = torch.tensor([16 * (s // 16) + order[s % 16] for s in range(S_pad)])
    ref = torch.zeros(N, 128, S_pad, dtype=torch.bfloat16)
    vp = torch.cat([v, torch.zeros(S_pad - S, N, 128, dtype=torch.bfloat16)])
    ref[:] = vp[slot_key].permute(1, 2, 0)
    assert torch.equal(vt.cpu(), ref)


@pytest.mark.parametrize("S,N,layout", [(777, 5, "token"), (1, 3, "token"), (5, 4, "token"), (4099, 40, "qkv"),
                                         (300, 6, "head"), (32760, 40, "qkv")])
def test_head_max_norm(pkg, dev, S, N, layout):
    """max over tokens of each head's norm, for token-major, strided ([Q | K | V] rows) and
    head-major K, with the largest key planted in the last token, the first, and one in between."""
    k = _rand((S, N, 128), 6 + S, scale=2.0)
    k[-1, 0] *= 3.0
    k[0, N - 1] *= 3.0
    k[S // 2, N // 2] *= 3.0
    if layout == "token":
        kd = k.to(dev)
    elif layout == "qkv":
        kd = torch.zeros(S, 3, N, 128, dtype=torch.bfloat16, device=dev)
        kd[:, 1] = k.to(dev)
        kd = kd[:, 1]
    else:
        kd = k.to(dev).permute(1, 0, 2).contiguous().permute(1, 0, 2)
    got = pkg.attention_ops.head_max_norm(kd).cpu()
    ref = k.float().norm(dim=-1).amax(dim=0)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=0)


def _ulps(a, b):
    ia = a.view(torch.int16).int()
    ib = b.view(torch.int16).int()
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return (ia - ib).abs()


@pytest.mark.parametrize("with_rope", [True, False])
def test_qk_rmsnorm_rope(pkg, dev, with_rope):
    grid = (1, 30, 52)  # 1560 tokens, the single-block latent grid
    S, N = 1560, 40
    x = _rand((S, N * 128), 7, scale=3.0)
    g = torch.Generator().manual_seed(8)
    gamma = 1 + 0.02 * torch.randn(N * 128, generator=g)
    cos, sin = orope.wan_rope(grid)
    xd = x.to(dev).clone()
    c64, s64 = pkg.attention_ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    kmax = pkg.attention_ops.qk_rmsnorm_rope_(
        xd, gamma.to(dev), cos=c64 if with_rope else None, sin=s64 if with_rope else None, eps=1e-6, want_max=True
    )
    ref = orope.rms_norm_across_heads(x, gamma, 1e-6).view(1, S, N, 128)
    if with_rope:
        ref = orope.apply_rotary_emb_wan(ref, cos[None, :, None, :], sin[None, :, None, :])
    ref = ref.view(S, N * 128)
    got = xd.cpu()
    u = _ulps(got, ref)
    assert float((u > 0).float().mean()) < 0.02
    if not with_rope:
        assert int(u.max()) <= 2
    else:
        # a*cos - b*sin can cancel; bound by one bf16 ulp of the rotation-invariant pair magnitude
        pair = ref.float().view(S, -1, 2).norm(dim=-1, keepdim=True).expand(-1, -1, 2).reshape(S, -1)
        assert bool(((got.float() - ref.float()).abs() <= 2.0**-7 * pair + 1e-30).all())
    torch.testing.assert_close(kmax.cpu(), xd.cpu().float().view(S, N, 128).norm(dim=-1).amax(dim=0), rtol=1e-5, atol=0)


def test_const_max_shift_invariance_and_underflow(pkg, dev):
    ops = pkg.attention_ops
    q, k, v = _rand((256, 2, 128), 11), _rand((300, 2, 128), 12), _rand((300, 2, 128), 13)
    vt, _ = ops.transpose_heads(v.to(dev))
    kmax = ops.head_max_norm(k.to(dev))
    s = 128**-0.5
    a = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s).cpu().double()
    b = ops.attention_core(q.to(dev), k.to(dev), vt, kmax * 1.5, s).cpu().double()
    assert (a - b).abs().max() <= 2.0**-6 * a.abs().max()
    # a bound so loose that every probability underflows: the 1e-37 floor returns zeros
    z = ops.attention_core(q.to(dev), k.to(dev), vt, torch.full_like(kmax, 1e30), s).cpu()
    assert bool((z == 0).all())


def test_self_attention_full_length_rows(pkg, dev):
    """Full self-attention sequence (21x30x52 = 32760 tokens, 40 heads, normalized + RoPE'd q/k);
    96 query rows spread over heads and positions checked against exact fp64 attention."""
    ops = pkg.attention_ops
    S, N = 32760, 40
    gdev = torch.Generator(device=dev).manual_seed(21)
    qkv = torch.randn(S, 3 * N * 128, generator=gdev, device=dev).to(torch.bfloat16)
    gamma = torch.ones(N * 128, device=dev)
    cos, sin = orope.wan_rope((21, 30, 52))
    c64, s64 = ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    ops.qk_rmsnorm_rope_(qkv[:, : N * 128], gamma, cos=c64, sin=s64)
    kmax = ops.qk_rmsnorm_rope_(qkv[:, N * 128 : 2 * N * 128], gamma, cos=c64, sin=s64, want_max=True)
    q = qkv[:, : N * 128].view(S, N, 128)
    k = qkv[:, N * 128 : 2 * N * 128].view(S, N, 128)
    v = qkv[:, 2 * N * 128 :].view(S, N, 128)
    vt, _ = ops.transpose_heads(v)
    out = ops.attention_core(q, k, vt, kmax, 128**-0.5)
    rows = torch.tensor([0, 1, 127, 128, 5000, 16383, 32639, 32640, 32759] + list(range(9000, 9087, 1)))[:96]
    for h in (0, 17, 39):
        ref = oa.torch_attend(q[rows, h].cpu(), k[:, h].cpu(), v[:, h].cpu(), 128**-0.5, dtype=torch.float64)
        _check_attn(out.view(S, N, 128)[rows, h].cpu(), ref)


def test_self_attention_720p_rows(pkg, dev):
    """Self-attention of the 720p step: 81 frames at 1280x720 = a 21x45x80 latent grid, 75600
    tokens, 40 heads, normalized + RoPE'd q/k; 96 query rows over three heads (incl. the ragged last
    query block) against exact fp64 attention over all 75600 keys."""
    ops = pkg.attention_ops
    grid = (21, 45, 80)
    S, N = grid[0] * grid[1] * grid[2], 40
    gdev = torch.Generator(device=dev).manual_seed(22)
    qkv = torch.randn(S, 3 * N * 128, generator=gdev, device=dev).to(torch.bfloat16)
    gamma = torch.ones(N * 128, device=dev)
    cos, sin = orope.wan_rope(grid)
    c64, s64 = ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    ops.qk_rmsnorm_rope_(qkv[:, : N * 128], gamma, cos=c64, sin=s64)
    kmax = ops.qk_rmsnorm_rope_(qkv[:, N * 128 : 2 * N * 128], gamma, cos=c64, sin=s64, want_max=True)
    q = qkv[:, : N * 128].view(S, N, 128)
    k = qkv[:, N * 128 : 2 * N * 128].view(S, N, 128)
    v = qkv[:, 2 * N * 128 :].view(S, N, 128)
    vt, _ = ops.transpose_heads(v)
    out = ops.attention_core(q, k, vt, kmax, 128**-0.5)
    rows = torch.tensor([0, 1, 255, 256, 37800, 75263, 75264, 75599] + list(range(50000, 50088)))[:96]
    for h in (3, 20, 38):
        ref = oa.torch_attend(q[rows, h].cpu(), k[:, h].cpu(), v[:, h].cpu(), 128**-0.5, dtype=torch.float64)
        _check_attn(out.view(S, N, 128)[rows, h].cpu(), ref)


def test_cross_attention_full_shape_rows(pkg, dev):
    """Cross-attention of the step: 32760 video-token queries (normalized across heads, no RoPE) over
    512 text keys, 40 heads, through the short-key instantiation; 96 query rows over three heads
    (incl. the ragged last query block) against exact fp64 attention."""
    ops = pkg.attention_ops
    S, T, N = 32760, 512, 40
    gdev = torch.Generator(device=dev).manual_seed(23)
    q = torch.randn(S, N * 128, generator=gdev, device=dev).to(torch.bfloat16)
    k = torch.randn(T, N * 128, generator=gdev, device=dev).to(torch.bfloat16)
    v = torch.randn(T, N, 128, generator=gdev, device=dev).to(torch.bfloat16)
    gamma = torch.ones(N * 128, device=dev)
    ops.qk_rmsnorm_rope_(q, gamma)
    kmax = ops.qk_rmsnorm_rope_(k, gamma, want_max=True)
    q, k = q.view(S, N, 128), k.view(T, N, 128)
    vt, _ = ops.transpose_heads(v)
    out = ops.attention_core(q, k, vt, kmax, 128**-0.5)
    rows = torch.tensor([0, 1, 255, 256, 16000, 32511, 32512, 32759] + list(range(20000, 20088)))[:96]
    for h in (0, 21, 39):
        ref = oa.torch_attend(q[rows, h].cpu(), k[:, h].cpu(), v[:, h].cpu(), 128**-0.5, dtype=torch.float64)
        _check_attn(out.view(S, N, 128)[rows, h].cpu(), ref)


@pytest.mark.parametrize("Sq,N,hpw", [(16384, 12, 3), (16384, 20, 5), (32760, 8, 4)])
def test_cross_attention_head_groups(pkg, dev, Sq, N, hpw):
    """Head groups of 3, 4 and 5 over many workgroups (64 query blocks x 4 groups of 3 heads or
    4 x 5, 128 blocks x 2 groups of 4: one round of 256 CUs each), 512 keys: sampled query rows of
    every head group against exact fp64 attention, the d-major output equal to the token-major one
    and the MX output the MX quantization of it, bit for bit. The expected group size is the
    library's choice for an MI355X (256 CUs); on another CU count the same checks run at its
    choice."""
    ops = pkg.attention_ops
    Sk = 512
    g = torch.Generator().manual_seed(Sq + N)
    q = torch.randn(Sq, N, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(Sk, N, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(Sk, N, 128, generator=g).to(torch.bfloat16)
    s = 128**-0.5
    vt, _ = ops.transpose_heads(v.to(dev))
    kmax = ops.head_max_norm(k.to(dev))
    tok = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s, ops.OUT_TOKEN)
    dm = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s, ops.OUT_DMAJOR)
    mx = ops.attention_core(q.to(dev), k.to(dev), vt, kmax, s, ops.OUT_MX)
    tok = tok.cpu().view(Sq, N, 128)
    assert torch.equal(dm.cpu().permute(0, 2, 1).contiguous(), tok.permute(1, 0, 2).contiguous())
    codes, scales = omx.mx_quantize(tok.view(Sq, N * 128).float().numpy())
    np.testing.assert_array_equal(mx.codes.view(torch.uint8).cpu().numpy(), codes)
    np.testing.assert_array_equal(mx.scales.cpu().numpy(), scales)
    rows = torch.cat([torch.arange(0, 32), torch.randint(0, Sq, (32,), generator=g), torch.arange(Sq - 32, Sq)])
    for h0 in range(0, N, hpw):  # the first and last head of every group
        for h in sorted({h0, h0 + hpw - 1}):
            ref = oa.torch_attend(q[rows, h].unsqueeze(0), k[:, h].unsqueeze(0), v[:, h].unsqueeze(0), s,
                                  dtype=torch.float64)
            _check_attn(tok[rows, h].unsqueeze(0), ref)


@pytest.mark.parametrize("with_rope", [True, False])
def test_attention_with_q_prepared_on_load(pkg, dev, with_rope):
    """q raw, the across-heads RMSNorm (+ RoPE) applied in the attention's Q load from per-head
    partial sums of squares: against exact fp64 attention over the oracle-prepared q, and close to
    the separate-pass path (same operations; only the order of the row sum differs)."""
    ops = pkg.attention_ops
    Sq, Sk, N = 300, 200, 4
    grid = (1, 10, 30)
    g = torch.Generator().manual_seed(33)
    q = torch.randn(Sq, N * 128, generator=g).to(torch.bfloat16)
    k = torch.randn(Sk, N, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(Sk, N, 128, generator=g).to(torch.bfloat16)
    gamma = 1 + 0.1 * torch.randn(N * 128, generator=g)
    cos, sin = orope.wan_rope(grid)
    c64, s64 = ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    qd, kd = q.to(dev), k.to(dev)
    vt, _ = ops.transpose_heads(v.to(dev))
    kmax = ops.head_max_norm(kd)
    sumsq = q.float().pow(2).view(Sq, N, 128).sum(-1).to(dev)
    prep = ops.QPrep(sumsq, gamma.to(dev), c64 if with_rope else None, s64 if with_rope else None, 1e-6)
    out = ops.attention_core(qd.view(Sq, N, 128), kd, vt, kmax, 128**-0.5, q_prep=prep).cpu()
    qn = orope.rms_norm_across_heads(q, gamma).view(1, Sq, N, 128)
    if with_rope:
        qn = orope.apply_rotary_emb_wan(qn, cos[None, :, None], sin[None, :, None])
    qn = qn.view(Sq, N, 128).to(torch.bfloat16)
    for h in range(N):
        ref = oa.torch_attend(qn[:, h], k[:, h], v[:, h], 128**-0.5, dtype=torch.float64)
        _check_attn(out.view(Sq, N, 128)[:, h], ref)
    q2 = qd.clone()
    ops.qk_rmsnorm_rope_(q2, gamma.to(dev), cos=c64 if with_rope else None, sin=s64 if with_rope else None)
    two_pass = ops.attention_core(q2.view(Sq, N, 128), kd, vt, kmax, 128**-0.5).cpu()
    diff = (out.float() - two_pass.float()).abs().max() / two_pass.float().abs().max()
    assert diff <= 1e-2, diff


def test_dropins_match_reference_layouts(pkg, dev):
    ops = pkg.attention_ops
    B, N, S, D = 1, 4, 200, 128
    q, k, v = _rand((B, S, N, D), 31), _rand((B, S, N, D), 32), _rand((B, S, N, D), 33)
    s = D**-0.5
    ref = oa.torch_attend(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), s, dtype=torch.float64)  # [B,N,S,D]
    o1 = ops.wan_cp_self_attention(q.to(dev), k.to(dev), v.to(dev), s, 1, None, None).cpu()  # [B,N,D,S]
    _check_attn(o1.transpose(2, 3), ref)
    o2 = ops._nki_attend(q.transpose(1, 2).to(dev), k.transpose(1, 2).to(dev), v.transpose(1, 2).to(dev), s).cpu()
    _check_attn(o2.transpose(2, 3), ref)
    o3 = ops.ring_attention_const_max_fwd(q.to(dev), k.to(dev), v.to(dev), softmax_scale=s).cpu()  # [B,N,S,D]
    _check_attn(o3, ref)
    # the registered op as _nki_attend launches it (wan2_2_transformer.py:668-674): [BN, S, D] with
    # q pre-scaled, d-major [BN, D, S] out; 77 keys (a ragged last tile)
    qb, kb, vb = (t.transpose(1, 2).reshape(B * N, -1, D) for t in (q, k[:, :77], v[:, :77]))
    ref4 = oa.torch_attend(qb[None], kb[None], vb[None], s, dtype=torch.float64)[0]  # [BN, S, D]
    o4 = torch.ops.wan_transformer.attention_cte((qb.float() * s).to(torch.bfloat16).to(dev), kb.to(dev), vb.to(dev))
    assert o4.shape == (B * N, D, S)
    ref4s = oa.torch_attend(((qb.float() * s).to(torch.bfloat16))[None], kb[None], vb[None], 1.0, dtype=torch.float64)[0]
    _check_attn(o4.cpu().transpose(1, 2), ref4s)
    _check_attn(o4.cpu().transpose(1, 2), ref4)
    with pytest.raises(NotImplementedError):
        ops.wan_cp_self_attention(q.to(dev), k.to(dev), v.to(dev), s, 2, None, None)


def _loose_bound_case(B, N, Sq, Sk, seed):
    """Inputs whose constant-max bound c = s ||q|| max||k|| is far above many rows' largest logit:
    key 0 of every head has norm 400 along d = 0 while the other keys are N(0, 1); even query rows
    have norm ~100 orthogonal to d = 0 (their true largest logit is ~30 below... c ~ 3500: every P
    of the row underflows), odd rows lie along d = 0 (c equals their logit with key 0: no
    underflow). A constant-max kernel returns the even rows as zero."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, N, 128, generator=g) * 9.0
    q[:, 0::2, :, 0] = 0.0
    q[:, 1::2] = 0.05 * q[:, 1::2]
    q[:, 1::2, :, 0] = 50.0
    k = torch.randn(B, Sk, N, 128, generator=g)
    k[:, 0] = 0.0
    k[:, 0, :, 0] = 400.0
    v = torch.randn(B, Sk, N, 128, generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


@pytest.mark.parametrize("Sk", [500, 1900])
def test_exact_dropins_survive_a_loose_bound(pkg, dev, Sk):
    """The drop-ins of the reference's running-max attention (``_nki_attend``, the registered
    ``attention_cte`` op, ``wan_cp_self_attention``) give the softmax even where the constant-max
    bound exceeds a row's largest logit by thousands (every P of the row underflows): those rows are
    recomputed with the row's true max. 500 keys run the head-group kernel, 1900 the one-head kernel.
    Bars as the other attention tests, against fp64 softmax."""
    ops = pkg.attention_ops
    B, N, Sq = 1, 8, 150
    s = 128**-0.5
    q, k, v = _loose_bound_case(B, N, Sq, Sk, seed=Sk)
    ref = oa.torch_attend(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), s, dtype=torch.float64)
    assert float(ref[:, :, 0::2].abs().max()) > 0.1  # the underflowing rows are not zero in the softmax
    # the plain constant-max kernel indeed loses the even rows (what the rescue is for)
    vt, _ = ops.transpose_heads(v[0].to(dev))
    plain = ops.attention_core(q[0].to(dev), k[0].to(dev), vt, ops.head_max_norm(k[0].to(dev)), s).cpu()
    assert float(plain.view(Sq, N, 128)[0::2].float().abs().max()) == 0.0
    o1 = ops._nki_attend(q.transpose(1, 2).to(dev), k.transpose(1, 2).to(dev), v.transpose(1, 2).to(dev), s).cpu()
    _check_attn(o1.transpose(2, 3), ref)
    o2 = ops.wan_cp_self_attention(q.to(dev), k.to(dev), v.to(dev), s, 1, None, None).cpu()
    _check_attn(o2.transpose(2, 3), ref)
    qb, kb, vb = (t.transpose(1, 2).reshape(B * N, -1, 128) for t in (q, k, v))
    qs = (qb.float() * s).to(torch.bfloat16)
    o3 = torch.ops.wan_transformer.attention_cte(qs.to(dev), kb.to(dev), vb.to(dev)).cpu()
    ref3 = oa.torch_attend(qs[None], kb[None], vb[None], 1.0, dtype=torch.float64)[0]
    _check_attn(o3.transpose(1, 2), ref3)


@pytest.mark.parametrize("Sk,with_rope", [(1900, True), (512, False), (200, True)])
def test_query_rrms_from_the_k_pass_is_bit_identical(pkg, dev, Sk, with_rope):
    """The K pass's per-token Q 1/rms (``qk_rmsnorm_rope_(..., q_sumsq=, q_rr=)``) equals, bit for
    bit, the fp32 block-ordered sum of the partials with the root in fp64 (restated here on the
    CPU), and the attention reading it (``QPrep(rr=...)``) gives the same bits as the attention
    summing the partials itself -- the one-head kernel with RoPE (1900 keys), the head-group kernel
    without (512 keys, 40 heads), the short-key kernel (200 keys) -- in MX and token-major output.
    Sq = 1000 leaves a ragged last query block; partials with a stride wider than the heads."""
    ops = pkg.attention_ops
    Sq, N, grid = 1000, 40, (1, 20, 50)
    g = torch.Generator().manual_seed(Sk)
    q = torch.randn(Sq, N * 128, generator=g).to(torch.bfloat16)
    kslab = torch.randn(Sq, N * 128, generator=g).to(torch.bfloat16)
    k = torch.randn(Sk, N, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(Sk, N, 128, generator=g).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(N * 128, generator=g)).float()
    ss = torch.zeros(Sq, 2 * N)
    ss[:, :N] = q.float().pow(2).view(Sq, N, 128).sum(-1) * (1 + 0.01 * torch.rand(Sq, N, generator=g))
    cos, sin = orope.wan_rope(grid)
    c64, s64 = ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    c64, s64 = (c64, s64) if with_rope else (None, None)
    ssd = ss.to(dev)
    rr = torch.full((Sq,), float("nan"), device=dev)
    ops.qk_rmsnorm_rope_(kslab.to(dev), gamma.to(dev), cos=c64, sin=s64, eps=1e-6, q_sumsq=ssd, q_rr=rr)
    # the restatement: sequential fp32 sum over the 40 blocks, fp64 root
    acc = np.zeros(Sq, np.float32)
    for b in range(N):
        acc = (acc + ss[:, b].numpy()).astype(np.float32)
    want = (1.0 / np.sqrt((acc / np.float32(N * 128)).astype(np.float64) + np.float64(np.float32(1e-6)))).astype(np.float32)
    np.testing.assert_array_equal(rr.cpu().numpy(), want)
    qd, kd = q.to(dev).view(Sq, N, 128), k.to(dev)
    vt, _ = ops.transpose_heads(v.to(dev))
    kmax = ops.head_max_norm(kd)
    for mode in (ops.OUT_MX, ops.OUT_TOKEN):
        a = ops.attention_core(qd, kd, vt, kmax, 128**-0.5, mode, q_prep=ops.QPrep(ssd, gamma.to(dev), c64, s64, 1e-6))
        b = ops.attention_core(qd, kd, vt, kmax, 128**-0.5, mode, q_prep=ops.QPrep(None, gamma.to(dev), c64, s64,
                                                                                  rr=rr))
        if mode == ops.OUT_MX:
            assert torch.equal(a.codes.view(torch.uint8), b.codes.view(torch.uint8)) and torch.equal(a.scales, b.scales)
        else:
            assert torch.equal(a, b)
