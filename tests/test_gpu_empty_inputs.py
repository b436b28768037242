"""No tokens through the hot-path entry points: every one returns an empty result of the right shape
(or, for the key-norm pass, zero maxima) and launches nothing that reads its inputs. The reference's
torch paths return empty tensors for these shapes (an empty matmul, LayerNorm or softmax over zero
rows)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

D = 512


def _mx(pkg, dev, rows, k):
    x = torch.empty(rows, k, dtype=torch.bfloat16, device=dev)
    return pkg.adaln_modulate(x, eps=0.0, norm_type="none", quant="mx")


def _weight(pkg, dev, k, n):
    g = torch.Generator(device=dev).manual_seed(k + n)
    return pkg.quantize_weight_mx(torch.randn(k, n, device=dev, generator=g) * 0.02,
                                  torch.randn(n, device=dev, generator=g) * 0.1)


@pytest.mark.parametrize("K", [384, 512])  # the simple loop and the pipelined ring kernel
def test_gemm_epilogues_without_tokens(pkg, dev, K):
    xq = _mx(pkg, dev, 0, K)
    w = _weight(pkg, dev, K, D)
    assert pkg.mxfp8_linear(xq, w).shape == (0, D)
    y = pkg.mxfp8_linear(xq, w, epilogue="gelu_mx")
    assert y.codes.shape == (0, D) and y.scales.shape == (0, D // 32)
    r = pkg.mxfp8_linear(xq, w, epilogue="gated_residual",
                         residual=torch.empty(0, D, dtype=torch.bfloat16, device=dev),
                         gate=torch.ones(D, device=dev))
    assert r.shape == (0, D)
    ss = torch.empty(0, D // 128, device=dev)
    assert pkg.mxfp8_linear(xq, w, row_sumsq=ss, sumsq_cols=D).shape == (0, D)


def test_qkv_projection_without_tokens(pkg, dev):
    xq = _mx(pkg, dev, 0, D)
    w = _weight(pkg, dev, D, 3 * D)
    qk, vt = pkg.row_mx_kernels.mxfp8_qkv_linear(xq, w, vt_col0=2 * D)
    torch.cuda.synchronize()
    assert qk.shape == (0, 2 * D)
    assert vt.shape == (D // 128, 128, 64) and not bool(vt.any())  # all padding


def test_attention_without_queries(pkg, dev):
    ops = pkg.attention_ops
    g = torch.Generator(device=dev).manual_seed(3)
    N, Sk = 4, 100  # the fused Q preparation takes heads in fours
    k = torch.randn(Sk, N, 128, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(Sk, N, 128, device=dev, generator=g).to(torch.bfloat16)
    vt, _ = ops.transpose_heads(v)
    kmax = ops.head_max_norm(k)
    q = torch.empty(0, N, 128, dtype=torch.bfloat16, device=dev)
    s = 128**-0.5
    assert ops.attention_core(q, k, vt, kmax, s).numel() == 0
    mx = ops.attention_core(q, k, vt, kmax, s, ops.OUT_MX)
    assert mx.codes.numel() == 0 and mx.scales.numel() == 0
    # the exact drop-in form (its per-query row sums), and the fused Q preparation from partial sums
    # or from per-query 1/rms, all with no storage behind the empty per-query buffers
    assert ops.attention_core(q, k, vt, kmax, s, exact=True).numel() == 0
    gamma = torch.ones(N * 128, device=dev)
    prep = ops.QPrep(torch.empty(0, 4, device=dev), gamma)
    assert ops.attention_core(q, k, vt, kmax, s, ops.OUT_MX, q_prep=prep).codes.numel() == 0
    prep_rr = ops.QPrep(None, gamma, rr=torch.empty(0, device=dev))
    assert ops.attention_core(q, k, vt, kmax, s, ops.OUT_MX, q_prep=prep_rr).codes.numel() == 0


def test_key_norm_pass_without_tokens(pkg, dev):
    ops = pkg.attention_ops
    x = torch.empty(0, 4 * 128, dtype=torch.bfloat16, device=dev)
    gamma = torch.ones(4 * 128, device=dev)
    kmax = ops.qk_rmsnorm_rope_(x, gamma, eps=1e-6, want_max=True)
    torch.cuda.synchronize()
    assert kmax.shape == (4,) and not bool(kmax.any())
    # with the queries' 1/rms from their partial sums (none), and written to a head-major output
    kmax = ops.qk_rmsnorm_rope_(x, gamma, eps=1e-6, want_max=True, q_sumsq=torch.empty(0, 8, device=dev),
                                q_rr=torch.empty(0, device=dev))
    torch.cuda.synchronize()
    assert not bool(kmax.any())
    out = torch.empty(4, 0, 128, dtype=torch.bfloat16, device=dev).permute(1, 0, 2)
    assert ops.qk_rmsnorm_rope_to(x, out, gamma).shape == (0, 4, 128)


def test_dmajor_to_mx_without_tokens(pkg, dev):
    att = torch.empty(1, 4, 128, 0, dtype=torch.bfloat16, device=dev)
    out = pkg.attention_ops.dmajor_to_mx(att)
    assert out.codes.shape[0] == 0 and out.scales.shape[0] == 0
