"""Every query of the full self-attention of the DiT step against fp64 attention.

The row tests check 96 query rows of three heads against the oracle. Here all 32760 queries of
all 40 heads are checked against torch's fp64 softmax attention on the GPU. It runs in chunks of
4096 queries, on the same bf16 (normalized, RoPE'd) inputs the kernel reads. The GPU's fp64
result is not exact: on a slice it agrees with the oracle's CPU fp64 ``torch_attend`` to 1e-6 of
max |ref|, four orders below the bar, and the test asserts that. The bars are the attention
tests' own, per head: max |err| / max |ref| <= 2e-2, cosine >= 0.999, and every element within
2^-6 max |ref|.

The launch is repeated and must be bit-identical. The MX output mode (what the o-projection
consumes) is checked on every element against the kernel's own bf16 output, within e4m3
rounding: 2^-4 |y| plus half the subnormal step, 2^-10 of the block scale.
"""

import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope

pytestmark = pytest.mark.gpu

S, N, D = 32760, 40, 128
CHUNK = 4096


def _attend_fp64(q, k, v, scale):
    """Exact fp64 attention of one head: q [Sq, D], k/v [Sk, D] bf16 on the device."""
    kt = k.double().T.contiguous()
    vd = v.double()
    out = torch.empty(q.shape[0], D, dtype=torch.float64, device=q.device)
    for r0 in range(0, q.shape[0], CHUNK):
        s = (q[r0 : r0 + CHUNK].double() * scale) @ kt
        out[r0 : r0 + CHUNK] = torch.softmax(s, dim=-1) @ vd
    return out


def test_self_attention_full_shape_every_query(pkg, dev):
    ops = pkg.attention_ops
    scale = D**-0.5
    gdev = torch.Generator(device=dev).manual_seed(31)
    qkv = torch.randn(S, 3 * N * D, generator=gdev, device=dev).to(torch.bfloat16)
    gamma = 1.0 + 0.1 * torch.randn(N * D, generator=gdev, device=dev)
    cos, sin = orope.wan_rope((21, 30, 52))
    c64, s64 = ops.rope_pair_tables(cos.to(dev), sin.to(dev))
    ops.qk_rmsnorm_rope_(qkv[:, : N * D], gamma, cos=c64, sin=s64)
    kmax = ops.qk_rmsnorm_rope_(qkv[:, N * D : 2 * N * D], gamma, cos=c64, sin=s64, want_max=True)
    q = qkv[:, : N * D].view(S, N, D)
    k = qkv[:, N * D : 2 * N * D].view(S, N, D)
    v = qkv[:, 2 * N * D :].view(S, N, D)
    vt, _ = ops.transpose_heads(v)
    out = ops.attention_core(q, k, vt, kmax, scale)
    assert torch.equal(out, ops.attention_core(q, k, vt, kmax, scale))
    out = out.view(S, N, D)

    # the GPU fp64 reference agrees with the oracle's CPU one on a slice, far inside the bar
    rows = torch.tensor([0, 4095, 4096, 32759])
    ref_slice = oa.torch_attend(q[rows, 5].cpu(), k[:, 5].cpu(), v[:, 5].cpu(), scale, dtype=torch.float64)
    mine = _attend_fp64(q[rows.to(dev), 5], k[:, 5], v[:, 5], scale).cpu()
    assert (mine - ref_slice).abs().max() <= 1e-6 * ref_slice.abs().max()

    worst = []
    for h in range(N):
        ref = _attend_fp64(q[:, h], k[:, h], v[:, h], scale)
        o = out[:, h].double()
        err = (o - ref).abs()
        m = ref.abs().max()
        cosv = torch.nn.functional.cosine_similarity(o.flatten(), ref.flatten(), dim=0)
        rel = (err.max() / m).item()
        worst.append(rel)
        assert rel <= 2e-2 and cosv.item() >= 0.999, (h, rel, cosv.item())
        assert bool((err <= 2.0**-6 * m).all()), h
    assert max(worst) <= 2e-2

    y = out.reshape(S, N * D)
    mx = ops.attention_core(q, k, vt, kmax, scale, ops.OUT_MX)
    mx2 = ops.attention_core(q, k, vt, kmax, scale, ops.OUT_MX)
    assert torch.equal(mx.codes.view(torch.uint8), mx2.codes.view(torch.uint8))
    assert torch.equal(mx.scales, mx2.scales)
    sc = torch.exp2(mx.scales.double() - 127.0)
    dq = (mx.codes.view(torch.float8_e4m3fn).double().view(S, -1, 32) * sc.unsqueeze(-1)).view(S, N * D)
    yd = y.double()
    step = (sc * 2.0**-10).repeat_interleave(32, dim=1)
    assert bool(((dq - yd).abs() <= 2.0**-4 * yd.abs() + step).all())


def test_cross_attention_full_shape_every_query(pkg, dev):
    """Cross-attention of the step: 32760 queries over 512 text keys, 40 heads, across-heads
    RMSNorm on Q and K without RoPE (as for the text context); every query of every head against
    fp64 attention at the bars above, repeat bit-identical."""
    ops = pkg.attention_ops
    scale = D**-0.5
    Sk = 512
    gdev = torch.Generator(device=dev).manual_seed(32)
    q2d = torch.randn(S, N * D, generator=gdev, device=dev).to(torch.bfloat16)
    kv = torch.randn(Sk, 2 * N * D, generator=gdev, device=dev).to(torch.bfloat16)
    gamma = 1.0 + 0.1 * torch.randn(N * D, generator=gdev, device=dev)
    ops.qk_rmsnorm_rope_(q2d, gamma)
    kmax = ops.qk_rmsnorm_rope_(kv[:, : N * D], gamma, want_max=True)
    q = q2d.view(S, N, D)
    k = kv[:, : N * D].view(Sk, N, D)
    v = kv[:, N * D :].view(Sk, N, D)
    vt, _ = ops.transpose_heads(v)
    out = ops.attention_core(q, k, vt, kmax, scale)
    assert torch.equal(out, ops.attention_core(q, k, vt, kmax, scale))
    out = out.view(S, N, D)
    rows = torch.tensor([0, 255, 256, 32759])
    ref_slice = oa.torch_attend(q[rows, 7].cpu(), k[:, 7].cpu(), v[:, 7].cpu(), scale, dtype=torch.float64)
    mine = _attend_fp64(q[rows.to(dev), 7], k[:, 7], v[:, 7], scale).cpu()
    assert (mine - ref_slice).abs().max() <= 1e-6 * ref_slice.abs().max()
    for h in range(N):
        ref = _attend_fp64(q[:, h], k[:, h], v[:, h], scale)
        o = out[:, h].double()
        err = (o - ref).abs()
        m = ref.abs().max()
        cosv = torch.nn.functional.cosine_similarity(o.flatten(), ref.flatten(), dim=0)
        assert (err.max() / m).item() <= 2e-2 and cosv.item() >= 0.999, (h, (err.max() / m).item(), cosv.item())
        assert bool((err <= 2.0**-6 * m).all()), h


def _projected_q(pkg, dev, seed):
    """Raw Q as the block makes it: the MXFP8 GEMM of an MX activation, with the per-128-column
    sums of squares of its bf16 outputs written by the GEMM's epilogue."""
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn(S, N * D, generator=g, device=dev).to(torch.bfloat16)
    aq = pkg.adaln_modulate(a, eps=1e-6, quant="mx")
    w = (torch.randn(N * D, N * D, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wq = pkg.quantize_weight_mx(w, 0.1 * torch.randn(N * D, generator=g, device=dev))
    ss = torch.empty(S, N * D // 128, dtype=torch.float32, device=dev)
    q = pkg.mxfp8_linear(aq, wq, row_sumsq=ss, sumsq_cols=N * D)
    gamma = 1.0 + 0.1 * torch.randn(N * D, generator=g, device=dev)
    return q, ss, gamma


def _check_heads(out, q_ref, k, v, scale):
    for h in range(N):
        ref = _attend_fp64(q_ref[:, h], k[:, h], v[:, h], scale)
        o = out[:, h].double()
        err = (o - ref).abs()
        m = ref.abs().max()
        cosv = torch.nn.functional.cosine_similarity(o.flatten(), ref.flatten(), dim=0)
        assert (err.max() / m).item() <= 2e-2 and cosv.item() >= 0.999, (h, (err.max() / m).item(), cosv.item())
        assert bool((err <= 2.0**-6 * m).all()), h


@pytest.mark.parametrize("kind", ["self", "cross"])
def test_fused_q_prep_attention_full_shape(pkg, dev, kind):
    """The attention the block and the bench run: Q is the raw projection, normalized across heads
    from the GEMM's partial sums (and, for self-attention, rotated with the 21x30x52 tables built by
    the package) as the kernel loads it. Every query of all 40 heads against fp64 attention over
    the oracle's prepared Q (``DistributedRMSNorm`` + ``apply_rotary_emb_wan`` on the same raw q),
    at the bars above; repeat launches bit-identical, MX output within e4m3 rounding."""
    ops = pkg.attention_ops
    scale = D**-0.5
    q_raw, ss, gamma = _projected_q(pkg, dev, 41 if kind == "self" else 42)
    gdev = torch.Generator(device=dev).manual_seed(43)
    Sk = S if kind == "self" else 512
    kv = torch.randn(Sk, 2 * N * D, generator=gdev, device=dev).to(torch.bfloat16)
    gk = 1.0 + 0.1 * torch.randn(N * D, generator=gdev, device=dev)
    cos = sin = None
    if kind == "self":
        cos, sin = pkg.rope_tables((21, 30, 52), device=dev)
    kmax = ops.qk_rmsnorm_rope_(kv[:, : N * D], gk, cos=cos if kind == "self" else None,
                                sin=sin if kind == "self" else None, want_max=True)
    k = kv[:, : N * D].view(Sk, N, D)
    v = kv[:, N * D :].view(Sk, N, D)
    vt, _ = ops.transpose_heads(v)
    qp = ops.QPrep(ss, gamma, cos, sin, 1e-6)
    q = q_raw.view(S, N, D)
    out = ops.attention_core(q, k, vt, kmax, scale, q_prep=qp)
    assert torch.equal(out, ops.attention_core(q, k, vt, kmax, scale, q_prep=qp))
    mx = ops.attention_core(q, k, vt, kmax, scale, ops.OUT_MX, q_prep=qp)
    # the oracle's Q preparation of the same raw projection
    qn = orope.rms_norm_across_heads(q_raw.cpu(), gamma.cpu()).view(1, S, N, D)
    if kind == "self":
        ic, isn = orope.wan_rope((21, 30, 52))
        qn = orope.apply_rotary_emb_wan(qn, ic[None, :, None], isn[None, :, None])
    q_ref = qn[0].to(dev)
    out = out.view(S, N, D)
    _check_heads(out, q_ref, k, v, scale)
    y = out.reshape(S, N * D).double()
    sc = torch.exp2(mx.scales.double() - 127.0)
    dq = (mx.codes.view(torch.float8_e4m3fn).double().view(S, -1, 32) * sc.unsqueeze(-1)).view(S, N * D)
    step = (sc * 2.0**-10).repeat_interleave(32, dim=1)
    assert bool(((dq - y).abs() <= 2.0**-4 * y.abs() + step).all())
