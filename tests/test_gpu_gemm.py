"""GPU parity of the MXFP8 GEMM and its epilogues against the fp64 oracle.

Operands follow the GEMM workload: activations N(0,1) and weights N(0,0.02), both MX-quantized
along K by the max-7 rule. Tolerance (bf16 output, fp32 accumulate): every element within
2^-8 * |ref| + 2^-14 * (|A| @ |W|^T) (bf16 rounding plus the MFMA's fp32 accumulation,
whose internal adds are coarser than sequential IEEE fp32); plus the summary bar
max rel err <= 2e-2 and cosine >= 0.999. The GELU+MX epilogue's codes and scales must equal the
oracle's MX quantization of the kernel's own bf16 GELU output, bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import gemm as og
from oracle import mx as omx

pytestmark = pytest.mark.gpu


def _operands(pkg, dev, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(K, N, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1
    xq = pkg.adaln_modulate(x.to(dev), eps=0.0, norm_type="none", quant="mx")
    wq = pkg.quantize_weight_mx(w.to(dev), b.to(dev))
    a_codes = xq.codes.view(torch.uint8).cpu().numpy()
    a_scales = xq.scales.cpu().numpy()
    w_codes = wq.codes.view(torch.uint8).cpu().numpy()
    w_scales = wq.scales.cpu().numpy()
    return xq, wq, (a_codes, a_scales, w_codes, w_scales), b.numpy()


def _check(y, ref, absg):
    y = y.double()
    err = (y - ref).abs()
    bound = 2.0**-8 * ref.abs() + 2.0**-14 * absg + 1e-30
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item()}"
    rel = err.max() / ref.abs().max()
    cos = torch.nn.functional.cosine_similarity(y.flatten(), ref.flatten(), dim=0)
    assert rel <= 2e-2 and cos >= 0.999, (rel.item(), cos.item())


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (300, 512, 256), (257, 768, 640), (1560, 1280, 5120)])
def test_gemm_bf16(pkg, dev, M, N, K):
    xq, wq, ops, b = _operands(pkg, dev, M, N, K, seed=M + N + K)
    y = pkg.mxfp8_linear(xq, wq).cpu()
    ref = og.mx_gemm(*ops, bias=b)
    _check(y, ref, og.abs_gemm(*ops))


def test_weight_quantization_matches_oracle(pkg, dev):
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(640, 512, generator=g) * 0.02).to(torch.bfloat16)
    wq = pkg.quantize_weight_mx(w.to(dev))
    codes, scales = og.quantize_weight(w.float().numpy())
    np.testing.assert_array_equal(wq.codes.view(torch.uint8).cpu().numpy(), codes)
    np.testing.assert_array_equal(wq.scales.cpu().numpy(), scales)


def test_gemm_gelu_mx_epilogue(pkg, dev):
    M, N, K = 520, 1024, 1280
    xq, wq, ops, b = _operands(pkg, dev, M, N, K, seed=17)
    inter_bf16 = pkg.mxfp8_linear(xq, wq, epilogue="gelu_bf16").cpu()
    inter_mx = pkg.mxfp8_linear(xq, wq, epilogue="gelu_mx")
    ref = og.gelu_tanh(og.mx_gemm(*ops, bias=b))
    _check(inter_bf16, ref, og.abs_gemm(*ops) + 1e-3)
    codes, scales = omx.mx_quantize(inter_bf16.float().numpy())
    np.testing.assert_array_equal(inter_mx.scales.cpu().numpy(), scales)
    np.testing.assert_array_equal(inter_mx.codes.view(torch.uint8).cpu().numpy(), codes)


@pytest.mark.parametrize("K", [384, 512])  # the simple loop and the pipelined ring kernel
def test_gemm_gated_residual_epilogue(pkg, dev, K):
    """bf16(res + bf16(y) * gate) on every element; M = 300 leaves the second row tile with one
    partial and three empty 64-row halves (the residual rows past M read as zero)."""
    M, N = 300, 512
    xq, wq, ops, b = _operands(pkg, dev, M, N, K, seed=23)
    g = torch.Generator().manual_seed(24)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    gate = torch.randn(N, generator=g)
    y = pkg.mxfp8_linear(xq, wq, epilogue="gated_residual", residual=res.to(dev), gate=gate.to(dev)).cpu()
    lin = og.mx_gemm(*ops, bias=b)
    ref = res.double() + lin.to(torch.bfloat16).double() * gate.double()
    err = (y.double() - ref).abs()
    # bf16(lin) on the GPU may sit one bf16 ulp (<= 2^-7 relative) from the oracle's bf16(lin)
    bound = 2.0**-8 * ref.abs() + (2.0**-7 * lin.abs() + 2.0**-14 * og.abs_gemm(*ops)) * gate.abs().double()
    assert bool((err <= bound + 1e-30).all())


def test_gemm_row_mx_mode(pkg, dev):
    """Reference ROW_MX recipe: ROW-packed activation (per-row fp32 scale, neutral block scales)
    times per-channel-scaled weights, dequantized in the epilogue (qkv_cte.py:3996-4021)."""
    M, N, K = 200, 512, 384
    g = torch.Generator().manual_seed(31)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    packed = pkg.adaln_modulate(x.to(dev), eps=0.0, norm_type="none", quant="row")
    w = (torch.randn(K, N, generator=g) * 0.02).to(torch.bfloat16)
    wq = pkg.quantize_weight_mx(w.to(dev))
    col = (torch.rand(N, generator=g) + 0.5)
    wq = pkg.MXWeight(wq.codes, wq.scales, col.to(dev), None)
    y = pkg.mxfp8_linear(packed, wq).cpu()
    codes, dq = omx.row_unpack(packed.view(torch.uint8).cpu().numpy())
    a_scales = np.full((M, K // 32), 127, np.uint8)
    ops = (codes, a_scales, wq.codes.view(torch.uint8).cpu().numpy(), wq.scales.cpu().numpy())
    ref = og.mx_gemm(*ops, row_scale=dq[:, 0], col_scale=col.numpy())
    absg = og.abs_gemm(*ops) * torch.from_numpy(dq.astype(np.float64)) * col.double().reshape(1, -1)
    _check(y, ref, absg)


def test_gemm_full_qkv_shape_row_subset(pkg, dev):
    """Config-3 QKV shape [32760, 5120] x [5120, 15360]; 48 rows (incl. the ragged last tile)
    checked against the fp64 oracle."""
    M, N, K = 32760, 15360, 5120
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(K, N, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    xq = pkg.adaln_modulate(x, eps=0.0, norm_type="none", quant="mx")
    wq = pkg.quantize_weight_mx(w)
    y = pkg.mxfp8_linear(xq, wq)
    rows = torch.tensor([0, 1, 255, 256, 4097, 16000, 32511, 32512] + list(range(32720, 32760)), device=dev)
    ops = (
        xq.codes.view(torch.uint8)[rows].cpu().numpy(), xq.scales[rows].cpu().numpy(),
        wq.codes.view(torch.uint8).cpu().numpy(), wq.scales.cpu().numpy(),
    )
    _check(y[rows].cpu(), og.mx_gemm(*ops), og.abs_gemm(*ops))


def test_gemm_720p_qkv_shape_row_subset(pkg, dev):
    """QKV projection of the 720p step, [75600, 5120] x [5120, 15360] (the 15360-wide bf16 output is
    2.3 GB); 48 rows (incl. the ragged last tile) against the fp64 oracle."""
    M, N, K = 75600, 15360, 5120
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(K, N, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g, device=dev) * 0.1
    xq = pkg.adaln_modulate(x, eps=0.0, norm_type="none", quant="mx")
    del x
    wq = pkg.quantize_weight_mx(w, b)
    y = pkg.mxfp8_linear(xq, wq)
    rows = torch.tensor([0, 1, 255, 256, 37800, 75263, 75264, 75265] + list(range(75560, 75600)), device=dev)
    ops = (
        xq.codes.view(torch.uint8)[rows].cpu().numpy(), xq.scales[rows].cpu().numpy(),
        wq.codes.view(torch.uint8).cpu().numpy(), wq.scales.cpu().numpy(),
    )
    _check(y[rows].cpu(), og.mx_gemm(*ops, bias=b.cpu().numpy()), og.abs_gemm(*ops) + 1e-3)


def test_gemm_row_sumsq(pkg, dev):
    """bf16 epilogue with per-row partial sums of squares: out is bit-identical to the plain GEMM,
    row_sumsq[:, b] equals the fp64 sum of the squared bf16 outputs of column block b (to fp32
    summation error) for the blocks below sumsq_cols, and the other blocks are not written."""
    M, N, K = 300, 768, 640
    xq, wq, ops, b = _operands(pkg, dev, M, N, K, seed=5)
    y = pkg.mxfp8_linear(xq, wq)
    rs = torch.full((M, N // 128), float("nan"), device=dev)
    y2 = pkg.mxfp8_linear(xq, wq, row_sumsq=rs, sumsq_cols=512)
    assert torch.equal(y, y2)
    ref = y.double().cpu().pow(2).view(M, N // 128, 128).sum(-1)
    got = rs.cpu().double()
    assert torch.allclose(got[:, :4], ref[:, :4], rtol=2e-5, atol=0.0), (got[:, :4] - ref[:, :4]).abs().max()
    assert bool(torch.isnan(got[:, 4:]).all())
    with pytest.raises(ValueError, match="multiple of 128"):
        pkg.mxfp8_linear(xq, wq, row_sumsq=rs, sumsq_cols=100)


def test_gemm_rejects_unsupported_shapes(pkg, dev):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16).to(dev)
    xq = pkg.adaln_modulate(x, eps=0.0, norm_type="none", quant="mx")
    wq = pkg.quantize_weight_mx((torch.randn(256, 200, generator=g) * 0.02).to(torch.bfloat16).to(dev))
    with pytest.raises(NotImplementedError, match="multiple of 256"):
        pkg.mxfp8_linear(xq, wq)


def test_gemm_full_mlp_shapes_row_subset(pkg, dev):
    """MLP shapes of the GEMM workload: up [32760, 5120] x [5120, 13824] with the GELU-tanh epilogue
    (bf16 and MX outputs) and down [32760, 13824] x [13824, 5120] with the gated-residual epilogue;
    48 rows each (incl. the ragged last tile) against the fp64 oracle, MX codes bit-exact against
    the MX quantization of the kernel's own bf16 GELU output."""
    M, D, F = 32760, 5120, 13824
    g = torch.Generator(device=dev).manual_seed(11)
    rows = torch.tensor([0, 1, 255, 256, 4097, 16000, 32511, 32512] + list(range(32720, 32760)), device=dev)
    # up + GELU
    x = torch.randn(M, D, generator=g, device=dev).to(torch.bfloat16)
    w_up = (torch.randn(D, F, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    b_up = torch.randn(F, generator=g, device=dev) * 0.1
    xq = pkg.adaln_modulate(x, eps=0.0, norm_type="none", quant="mx")
    wq = pkg.quantize_weight_mx(w_up, b_up)
    y = pkg.mxfp8_linear(xq, wq, epilogue="gelu_bf16")[rows].cpu()
    y_mx = pkg.mxfp8_linear(xq, wq, epilogue="gelu_mx")
    ops = (
        xq.codes.view(torch.uint8)[rows].cpu().numpy(), xq.scales[rows].cpu().numpy(),
        wq.codes.view(torch.uint8).cpu().numpy(), wq.scales.cpu().numpy(),
    )
    _check(y, og.gelu_tanh(og.mx_gemm(*ops, bias=b_up.cpu().numpy())), og.abs_gemm(*ops) + 1e-3)
    codes, scales = omx.mx_quantize(y.float().numpy())
    np.testing.assert_array_equal(y_mx.scales[rows].cpu().numpy(), scales)
    np.testing.assert_array_equal(y_mx.codes.view(torch.uint8)[rows].cpu().numpy(), codes)
    del x, xq, w_up, wq, y_mx
    # down + gated residual
    h = torch.randn(M, F, generator=g, device=dev).to(torch.bfloat16)
    w_dn = (torch.randn(F, D, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    b_dn = torch.randn(D, generator=g, device=dev) * 0.1
    res = torch.randn(M, D, generator=g, device=dev).to(torch.bfloat16)
    gate = torch.randn(D, generator=g, device=dev)
    hq = pkg.adaln_modulate(h, eps=0.0, norm_type="none", quant="mx")
    wq = pkg.quantize_weight_mx(w_dn, b_dn)
    y = pkg.mxfp8_linear(hq, wq, epilogue="gated_residual", residual=res, gate=gate)[rows].cpu()
    ops = (
        hq.codes.view(torch.uint8)[rows].cpu().numpy(), hq.scales[rows].cpu().numpy(),
        wq.codes.view(torch.uint8).cpu().numpy(), wq.scales.cpu().numpy(),
    )
    lin = og.mx_gemm(*ops, bias=b_dn.cpu().numpy())
    gate_c = gate.cpu().double()
    ref = res[rows].cpu().double() + lin.to(torch.bfloat16).double() * gate_c
    err = (y.double() - ref).abs()
    bound = 2.0**-8 * ref.abs() + (2.0**-7 * lin.abs() + 2.0**-14 * og.abs_gemm(*ops)) * gate_c.abs()
    assert bool((err <= bound + 1e-30).all())


@pytest.mark.parametrize("K", [640, 1024])
@pytest.mark.parametrize("M", [300, 1560, 4100])
def test_qkv_projection_writes_v_transposed(pkg, dev, M, K):
    """``mxfp8_qkv_linear``: the Q|K columns bit-identical to the plain GEMM's, the Q sums of squares
    identical, and the V columns written as V^T in the attention's key order -- against
    ``transpose_heads`` of the plain GEMM's V (zero past the last token) within one bf16 rounding (its
    MFMAs take the operands in the other order, so the fp32 accumulation may round differently).
    K = 640 runs the simple-loop kernel, K = 1024 (a multiple of 512) the pipelined ring kernel."""
    dim = 1024
    xq, wq, _, _ = _operands(pkg, dev, M, 3 * dim, K, seed=M + K)
    ss_ref = torch.empty(M, 3 * dim // 128, device=dev)
    full = pkg.mxfp8_linear(xq, wq, row_sumsq=ss_ref, sumsq_cols=dim)
    ss = torch.full((M, 2 * dim // 128), float("nan"), device=dev)
    qk, vt = pkg.row_mx_kernels.mxfp8_qkv_linear(xq, wq, vt_col0=2 * dim, row_sumsq=ss, sumsq_cols=dim)
    assert qk.shape == (M, 2 * dim) and vt.shape == (dim // 128, 128, (M + 63) // 64 * 64)
    assert torch.equal(qk, full[:, : 2 * dim])
    vt_ref, _ = pkg.attention_ops.transpose_heads(full[:, 2 * dim :].view(M, dim // 128, 128))
    d = (vt.float() - vt_ref.float()).abs()
    assert bool((d <= 2.0**-8 * vt_ref.float().abs()).all()), float(d.max())
    assert float((d > 0).float().mean()) < 1e-3
    # slot r of a 16-key group holds key (r & 3) | ((r & 4) << 1) | ((r & 8) >> 1): the padding is
    # the slots whose key is >= M (not simply the slots >= M when M is not a multiple of 16)
    slots = torch.arange(vt.shape[-1])
    key = (slots & ~15) | (slots & 3) | ((slots & 4) << 1) | ((slots & 8) >> 1)
    assert not bool(vt[:, :, (key >= M).to(dev)].any()), "V^T padding past the last token must be zero"
    assert torch.equal(ss[:, : dim // 128], ss_ref[:, : dim // 128])
    assert bool(torch.isnan(ss[:, dim // 128 :]).all())
