"""GPU parity of the fused adaLN + quantization kernel against the canonical oracle (bit-exact).

Inputs follow the adaLN workload: x ~ N(0,1) bf16, shift/scale ~ N(0, 0.5), mul = 1 + scale,
LayerNorm without affine, eps 1e-6. Codes, e8m0 scales, bf16 outputs, packed ROW bytes and the
fused residual must all match bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import adaln as oracle_adaln
from oracle import fp8

pytestmark = pytest.mark.gpu


def _inputs(T, H, seed, residual=False, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, generator=g) * scale).to(torch.bfloat16)
    sc = torch.randn(H, generator=g) * 0.5
    sh = torch.randn(H, generator=g) * 0.5
    res = torch.randn(T, H, generator=g).to(torch.bfloat16) if residual else None
    gate = torch.randn(H, generator=g) if residual else None
    return x, 1 + sc, sh, res, gate


def _np(t):
    return None if t is None else t.float().numpy()


@pytest.mark.parametrize(
    "T,H",
    [(1, 32), (7, 96), (33, 544), (128, 5120), (257, 5120), (64, 13824), (5, 16384), (1560, 5120)],
)
def test_adaln_mx_bit_exact(pkg, dev, T, H):
    x, mul, add, _, _ = _inputs(T, H, seed=T * 7 + H)
    out = pkg.adaln_modulate(x.to(dev), mul.to(dev), add.to(dev), eps=1e-6, quant="mx")
    ref = oracle_adaln.adaln_quant(_np(x), mul.numpy(), add.numpy(), eps=1e-6, quant="mx")
    np.testing.assert_array_equal(out.scales.cpu().numpy(), ref["scales"])
    np.testing.assert_array_equal(out.codes.view(torch.uint8).cpu().numpy(), ref["codes"])


@pytest.mark.parametrize("norm_type", ["layer_norm", "rms_norm", "none"])
@pytest.mark.parametrize("quant", ["none", "mx", "row"])
def test_adaln_modes_bit_exact(pkg, dev, norm_type, quant):
    T, H = 200, 5120
    x, mul, add, _, _ = _inputs(T, H, seed=11, scale=3.0)
    out = pkg.adaln_modulate(x.to(dev), mul.to(dev), add.to(dev), eps=1e-6, norm_type=norm_type, quant=quant)
    ref = oracle_adaln.adaln_quant(_np(x), mul.numpy(), add.numpy(), eps=1e-6, norm_type=norm_type, quant=quant)
    if quant == "none":
        np.testing.assert_array_equal(out.float().cpu().numpy(), ref["y"])
    elif quant == "mx":
        np.testing.assert_array_equal(out.scales.cpu().numpy(), ref["scales"])
        np.testing.assert_array_equal(out.codes.view(torch.uint8).cpu().numpy(), ref["codes"])
    else:
        np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), ref["packed"])


@pytest.mark.parametrize("quant,norm", [("mx", "layer_norm"), ("row", "layer_norm"), ("none", "rms_norm"),
                                        ("row", "none")])
@pytest.mark.parametrize("with_gate", [True, False])
def test_adaln_fused_residual_bit_exact(pkg, dev, with_gate, quant, norm):
    """The reference's residual sites: x = bf16(h * gate + res) (gate optional), written out, then
    normalized, modulated and quantized; 300 rows (a partial workgroup of eight at the end)."""
    T, H = 300, 5120
    x, mul, add, res, gate = _inputs(T, H, seed=5, residual=True)
    gate = gate if with_gate else None
    res_out, out = pkg.adaln_modulate(
        x.to(dev), mul.to(dev), add.to(dev), eps=1e-6, norm_type=norm, quant=quant, residual=res.to(dev),
        gate=None if gate is None else gate.to(dev),
    )
    ref = oracle_adaln.adaln_quant(
        _np(x), mul.numpy(), add.numpy(), eps=1e-6, norm_type=norm, quant=quant, residual=_np(res),
        gate=None if gate is None else gate.numpy(),
    )
    np.testing.assert_array_equal(res_out.float().cpu().numpy(), ref["residual_out"])
    if quant == "mx":
        np.testing.assert_array_equal(out.scales.cpu().numpy(), ref["scales"])
        np.testing.assert_array_equal(out.codes.view(torch.uint8).cpu().numpy(), ref["codes"])
    elif quant == "row":
        np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), ref["packed"])
    else:
        np.testing.assert_array_equal(out.float().cpu().numpy(), ref["y"])


def test_adaln_batched_modulation(pkg, dev):
    # [B, S, H] with per-batch [B, 1, H] mul/add, as WanTransformerBlock passes them
    B, S, H = 2, 40, 5120
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    mul = 1 + torch.randn(B, 1, H, generator=g) * 0.5
    add = torch.randn(B, 1, H, generator=g) * 0.5
    out = pkg.adaln_modulate(x.to(dev), mul.to(dev), add.to(dev), eps=1e-6, quant="mx")
    assert out.codes.shape == (B, S, H) and out.scales.shape == (B, S, H // 32)
    for b in range(B):
        ref = oracle_adaln.adaln_quant(_np(x[b]), mul[b, 0].numpy(), add[b, 0].numpy(), eps=1e-6, quant="mx")
        np.testing.assert_array_equal(out.codes[b].view(torch.uint8).cpu().numpy(), ref["codes"])
        np.testing.assert_array_equal(out.scales[b].cpu().numpy(), ref["scales"])


def test_adaln_extreme_rows(pkg, dev):
    # constant rows, huge and tiny magnitudes, a wide dynamic range inside one row
    T, H = 8, 5120
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g)
    x[0] = 1.5
    x[1] *= 1e30
    x[2] *= 1e-30
    x[3, :64] *= 1e4
    x[4] = 0.0
    x = x.to(torch.bfloat16)
    mul = torch.ones(H)
    for quant in ("mx", "row", "none"):
        out = pkg.adaln_modulate(x.to(dev), mul.to(dev), None, eps=1e-6, quant=quant)
        ref = oracle_adaln.adaln_quant(_np(x), mul.numpy(), None, eps=1e-6, quant=quant)
        if quant == "mx":
            np.testing.assert_array_equal(out.codes.view(torch.uint8).cpu().numpy(), ref["codes"])
            np.testing.assert_array_equal(out.scales.cpu().numpy(), ref["scales"])
        elif quant == "row":
            np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), ref["packed"])
        else:
            np.testing.assert_array_equal(out.float().cpu().numpy(), ref["y"])


def test_empty_input(pkg, dev):
    x = torch.empty(0, 5120, dtype=torch.bfloat16, device=dev)
    out = pkg.adaln_modulate(x, eps=1e-6, quant="mx")
    assert out.codes.shape == (0, 5120)


def test_e4m3_conversion_kat_every_bf16(pkg, dev):
    """Hardware e4m3fn conversion (the one every kernel uses) vs the oracle on all bf16 inputs."""
    u = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    v = u[np.isfinite(u) & (np.abs(u) < 464.0)].copy()
    lib = pkg._lib.load()
    src = torch.from_numpy(v).to(dev)
    dst = torch.empty(v.size, dtype=torch.uint8, device=dev)
    pkg._lib.check(lib.wanmi_e4m3_encode(pkg._lib.ptr(src), pkg._lib.ptr(dst), v.size, pkg._lib.stream_of(src)), "e4m3")
    np.testing.assert_array_equal(dst.cpu().numpy(), fp8.e4m3_encode(v))


@pytest.mark.parametrize("case", ["layer_row", "rms_none_3d", "none_row_residual", "layer_none_residual_nogate"])
def test_adaln_quant_kernel_dropin(pkg, dev, case):
    """The kernel-level drop-in as the bridge launches it (adaln_kernels.py:150-201): bf16 ``[1, H]``
    mul / add, fp32 gate, OCP ROW output, a rank-3 hidden; bit-exact against the oracle."""
    A, NT, QT, DM = pkg.AdaLNQuantKernelArgs, pkg.NormType, pkg.QuantizationType, pkg.DtypeMode
    norm, quant, resid, shape = {
        "layer_row": (NT.LAYER_NORM, QT.ROW, False, (300, 5120)),
        "rms_none_3d": (NT.RMS_NORM, QT.NONE, False, (2, 37, 512)),
        "none_row_residual": (NT.NO_NORM, QT.ROW, True, (64, 1024)),
        "layer_none_residual_nogate": (NT.LAYER_NORM, QT.NONE, "nogate", (33, 544)),
    }[case]
    H = shape[-1]
    g = torch.Generator().manual_seed(H + len(shape))
    x = torch.randn(*shape, generator=g).to(torch.bfloat16)
    mul = (1 + 0.5 * torch.randn(1, H, generator=g)).to(torch.bfloat16)
    add = (0.5 * torch.randn(1, H, generator=g)).to(torch.bfloat16)
    res = torch.randn(*shape, generator=g).to(torch.bfloat16) if resid else None
    gate = torch.randn(1, H, generator=g) if resid is True else None
    args = A(norm_type=norm, quantization_type=quant, eps=1e-6)
    out = pkg.adaln_quant_kernel(x.to(dev), args, mul.to(dev), add.to(dev), DM.OCP,
                                 None if res is None else res.to(dev), None if gate is None else gate.to(dev))
    ref = oracle_adaln.adaln_quant(_np(x).reshape(-1, H), mul.float().numpy().reshape(H), add.float().numpy().reshape(H),
                                   eps=1e-6, norm_type=norm.value, quant=quant.value,
                                   residual=None if res is None else _np(res).reshape(-1, H),
                                   gate=None if gate is None else gate.numpy().reshape(H))
    if res is not None:
        res_out, out = out
        assert res_out.shape == shape
        np.testing.assert_array_equal(res_out.float().cpu().numpy().reshape(-1, H), ref["residual_out"])
    if quant == QT.ROW:
        assert out.shape == (*shape[:-1], H + 4) and out.dtype == torch.float8_e4m3fn
        np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy().reshape(-1, H + 4), ref["packed"])
    else:
        assert out.shape == shape and out.dtype == torch.bfloat16
        np.testing.assert_array_equal(out.float().cpu().numpy().reshape(-1, H), ref["y"])
