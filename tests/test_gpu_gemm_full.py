"""Every element of the full-shape GEMMs of the DiT step (32760 tokens) against an fp64 product.

The row-subset tests compare 48 rows per shape with the numpy oracle. Here the whole output of
each projection shape of the step is compared, element by element, with the fp64 product of the
dequantized MX operands, computed by torch on the GPU in row chunks. Dequantized MX values are
exact in fp64. The GPU product is pinned to the oracle's CPU product on four rows, to 2^-20 of
|A| @ |W|^T, 64 times below the bound's accumulation term. The bound
is the row-subset tests' own: 2^-8 |ref| + 2^-14 (|A| @ |W|^T), plus max rel err <= 2e-2.

Each launch is also repeated and must be bit-identical. This catches tiles that read stale
offsets or stale LDS data, which a fixed row subset can miss.

The GELU+MX output is checked on every element against the kernel's own bf16 GELU output. e4m3
keeps 3 mantissa bits, so a decoded value lies within 2^-4 |y| of the value it encodes. Below the
normal range the step is 2^-9 of the block scale, so the error there is at most 2^-10 of it.
"""

import numpy as np
import pytest
import torch

from oracle import gemm as og
from oracle import mx as omx

pytestmark = pytest.mark.gpu

M, DIM, FFN = 32760, 5120, 13824
CHUNK = 8192


def _dq(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """MX codes [R, K] (e4m3) and e8m0 scales [R, K/32] -> fp64 [R, K] on the device."""
    v = codes.view(torch.float8_e4m3fn).to(torch.float64)
    s = torch.exp2(scales.to(torch.float64) - 127.0)
    return (v.view(v.shape[0], -1, 32) * s.unsqueeze(-1)).view(v.shape)


def _pin_dq(codes: torch.Tensor, scales: torch.Tensor) -> None:
    """The torch dequantization above equals the oracle's on a slice."""
    c = codes[:64].view(torch.uint8)
    s = scales[:64]
    np.testing.assert_array_equal(_dq(c, s).cpu().numpy(), omx.mx_dequantize(c.cpu().numpy(), s.cpu().numpy()))


def _operands(pkg, dev, K, N, seed, bias=True):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(K, N, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g, device=dev) * 0.1 if bias else None
    xq = pkg.adaln_modulate(x, eps=0.0, norm_type="none", quant="mx")
    del x
    wq = pkg.quantize_weight_mx(w, b)
    _pin_dq(xq.codes, xq.scales)
    _pin_dq(wq.codes, wq.scales)
    return g, xq, wq, b


def _chunks(xq, wq, b):
    """(rows, fp64 A·Wᵀ + b, fp64 |A|·|W|ᵀ) per chunk of CHUNK rows."""
    wd = _dq(wq.codes, wq.scales)
    wt, wat = wd.T.contiguous(), wd.abs().T.contiguous()
    del wd
    for r0 in range(0, M, CHUNK):
        r1 = min(M, r0 + CHUNK)
        a = _dq(xq.codes[r0:r1], xq.scales[r0:r1])
        lin = a @ wt
        if b is not None:
            lin += b.double()
        absg = a.abs() @ wat
        if r0 == 0:
            _pin_product(xq, wq, b, lin, absg)
        yield slice(r0, r1), lin, absg


def _pin_product(xq, wq, b, lin, absg):
    """The GPU fp64 product of the first four rows against the oracle's CPU product."""
    ops = (
        xq.codes[:4].view(torch.uint8).cpu().numpy(), xq.scales[:4].cpu().numpy(),
        wq.codes.view(torch.uint8).cpu().numpy(), wq.scales.cpu().numpy(),
    )
    ref = og.mx_gemm(*ops, bias=None if b is None else b.cpu().numpy())
    assert bool(((lin[:4].cpu() - ref).abs() <= 2.0**-20 * absg[:4].cpu()).all())


def _assert_within(err, bound, ref, stats):
    excess = (err - bound).max().item()
    assert excess <= 0.0, f"max excess over the bound {excess}"
    stats[0] = max(stats[0], err.max().item())
    stats[1] = max(stats[1], ref.abs().max().item())


def test_gemm_qkv_full_shape_every_element(pkg, dev):
    """QKV [32760, 5120] x [5120, 15360] + bias, with and without the Σy² partials of the first
    5120 columns: identical bf16 outputs, every element within the bound, the partials equal to
    the fp64 sums of the kernel's own squared bf16 outputs to fp32 summation error."""
    N = 3 * DIM
    _, xq, wq, b = _operands(pkg, dev, DIM, N, seed=21)
    y = pkg.mxfp8_linear(xq, wq)
    y_again = pkg.mxfp8_linear(xq, wq)
    assert torch.equal(y, y_again)
    del y_again
    ss = torch.full((M, N // 128), float("nan"), device=dev)
    y_ss = pkg.mxfp8_linear(xq, wq, row_sumsq=ss, sumsq_cols=DIM)
    assert torch.equal(y, y_ss)
    del y_ss
    ref_ss = y[:, :DIM].double().pow(2).view(M, DIM // 128, 128).sum(-1)
    got_ss = ss[:, : DIM // 128].double()
    assert bool(((got_ss - ref_ss).abs() <= 2e-5 * ref_ss).all())
    assert bool(torch.isnan(ss[:, DIM // 128 :]).all())
    stats = [0.0, 0.0]
    for rows, ref, absg in _chunks(xq, wq, b):
        err = (y[rows].double() - ref).abs()
        _assert_within(err, 2.0**-8 * ref.abs() + 2.0**-14 * absg, ref, stats)
    assert stats[0] / stats[1] <= 2e-2, stats


def test_gemm_up_full_shape_every_element(pkg, dev):
    """FFN up [32760, 5120] x [5120, 13824] with the GELU-tanh epilogue: bf16 output on every
    element within the bound of GELU(fp64 product), repeat bit-identical, and the MX output of the
    same GEMM within e4m3 rounding of the bf16 output on every element."""
    _, xq, wq, b = _operands(pkg, dev, DIM, FFN, seed=22)
    y = pkg.mxfp8_linear(xq, wq, epilogue="gelu_bf16")
    assert torch.equal(y, pkg.mxfp8_linear(xq, wq, epilogue="gelu_bf16"))
    y_mx = pkg.mxfp8_linear(xq, wq, epilogue="gelu_mx")
    y_mx2 = pkg.mxfp8_linear(xq, wq, epilogue="gelu_mx")
    assert torch.equal(y_mx.codes.view(torch.uint8), y_mx2.codes.view(torch.uint8))
    assert torch.equal(y_mx.scales, y_mx2.scales)
    del y_mx2
    stats = [0.0, 0.0]
    for rows, lin, absg in _chunks(xq, wq, b):
        ref = torch.nn.functional.gelu(lin, approximate="tanh")
        yr = y[rows].double()
        _assert_within((yr - ref).abs(), 2.0**-8 * ref.abs() + 2.0**-14 * (absg + 1e-3), ref, stats)
        dq = _dq(y_mx.codes[rows], y_mx.scales[rows])
        step = torch.exp2(y_mx.scales[rows].double() - 127.0 - 10.0).repeat_interleave(32, dim=1)
        assert bool(((dq - yr).abs() <= 2.0**-4 * yr.abs() + step).all())
    assert stats[0] / stats[1] <= 2e-2, stats


def test_gemm_down_full_shape_every_element(pkg, dev):
    """FFN down [32760, 13824] x [13824, 5120] with the gated-residual epilogue
    ``bf16(res + bf16(y)·gate)``: every element within the row-subset test's bound, repeat
    bit-identical."""
    g, xq, wq, b = _operands(pkg, dev, FFN, DIM, seed=23)
    res = torch.randn(M, DIM, generator=g, device=dev).to(torch.bfloat16)
    gate = torch.randn(DIM, generator=g, device=dev)
    y = pkg.mxfp8_linear(xq, wq, epilogue="gated_residual", residual=res, gate=gate)
    assert torch.equal(y, pkg.mxfp8_linear(xq, wq, epilogue="gated_residual", residual=res, gate=gate))
    gd = gate.double()
    stats = [0.0, 0.0]
    for rows, lin, absg in _chunks(xq, wq, b):
        ref = res[rows].double() + lin.to(torch.bfloat16).double() * gd
        err = (y[rows].double() - ref).abs()
        bound = 2.0**-8 * ref.abs() + (2.0**-7 * lin.abs() + 2.0**-14 * absg) * gd.abs() + 1e-30
        _assert_within(err, bound, ref, stats)
    assert stats[0] / stats[1] <= 2e-2, stats
