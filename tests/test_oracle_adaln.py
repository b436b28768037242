"""Pin the canonical adaLN oracle (CPU only).

- The fixed-grid fp64 statistics are checked against ``math.fsum`` (the exactly rounded sum) of
  the same grid terms, and the mean/variance against fsum of the raw values.
- The whole output is compared with the reference's eager path restated in torch
  (``_eager_adaln``, adaln_kernels.py:51-84, which uses ``F.layer_norm``): bf16 outputs may differ
  only by one ulp and only rarely (the eager fp32 reduction order is unspecified).
- LayerNorm invariants and the identity special cases.
"""

import math

import numpy as np
import pytest
import torch

from oracle import adaln, fp8


def _bf16(rng, shape, scale=1.0):
    return fp8.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def test_ordered_sums_within_fp32_error_bound():
    """The canonical fixed-order fp32 sum stays within the classical bound of the exactly rounded
    sum (math.fsum): |S - S_exact| <= (n_lane + 6) * 2^-24 * sum|x| for 80 terms per lane plus 6
    butterfly levels; an index slip (a dropped or doubled chunk) breaks it by orders of magnitude."""
    rng = np.random.default_rng(0)
    x = _bf16(rng, (6, 5120), scale=3.0)
    x[1] *= 1e-20
    x[2, :100] *= 1e6
    x[3] = 0.0
    x[4] += np.float32(50.0)
    x = fp8.bf16_round(x)
    for H in (5120, 4096 + 96):
        xs = x[:, :H]
        got = adaln._ordered_sum(adaln._lane_major(xs))[:, 0].astype(np.float64)
        n_lane = -(-H // 512) * 8
        for i, row in enumerate(xs.astype(np.float64)):
            exact = math.fsum(row)
            bound = (n_lane + 6) * 2.0**-24 * np.abs(row).sum()
            assert abs(got[i] - exact) <= bound + 1e-300, (H, i)


def test_lane_major_order_is_the_documented_one():
    # column c*512 + 8l + j is lane l's term number c*8 + j
    x = np.arange(1024, dtype=np.float32)[None]
    lm = adaln._lane_major(x)
    assert lm.shape == (1, 64, 16)
    assert lm[0, 3].tolist() == [24, 25, 26, 27, 28, 29, 30, 31, 536, 537, 538, 539, 540, 541, 542, 543]


def test_layer_norm_stats_match_exact_moments():
    rng = np.random.default_rng(1)
    x = _bf16(rng, (8, 5120), scale=2.0) + np.float32(0.5)
    mu, rstd = adaln.layer_norm_stats(x, 1e-6)
    for i, row in enumerate(x.astype(np.float64)):
        m = math.fsum(row) / row.size
        v = math.fsum((row - m) ** 2) / row.size
        assert abs(mu[i, 0] - m) <= 1e-6 * max(1.0, abs(m))
        assert abs(rstd[i, 0] - 1.0 / math.sqrt(v + 1e-6)) <= 2e-7 * rstd[i, 0]


@pytest.mark.parametrize("norm_type", ["layer_norm", "rms_norm"])
@pytest.mark.parametrize("with_residual", [False, True])
def test_matches_eager_reference_within_one_ulp(norm_type, with_residual):
    rng = np.random.default_rng(2)
    T, H = 64, 5120
    h = _bf16(rng, (T, H))
    mul = (1 + rng.standard_normal(H) * 0.5).astype(np.float32)
    add = (rng.standard_normal(H) * 0.5).astype(np.float32)
    res = _bf16(rng, (T, H)) if with_residual else None
    gate = rng.standard_normal(H).astype(np.float32) if with_residual else None
    y, res_out = adaln.adaln_y(h, mul, add, eps=1e-6, norm_type=norm_type, residual=res, gate=gate)
    y_eager = adaln.eager_adaln_y(h, mul, add, eps=1e-6, norm_type=norm_type, residual=res, gate=gate)
    # Allowed gap: one bf16 ulp of y plus the fp32 rounding scale of the terms summed into it
    # (y = xh*mul + add can cancel, amplifying a 1-ulp difference in mu/rstd relative to y).
    x = res_out if with_residual else h
    xh_mag = np.abs(x - x.mean(axis=-1, keepdims=True)) / (x.std(axis=-1, keepdims=True) + 1e-12)
    if norm_type == "rms_norm":
        xh_mag = np.abs(x) / np.sqrt((x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True))
    ulp_y = np.ldexp(1.0, fp8.exp_field(y) - 127 - 7)
    tol = ulp_y + 2.0**-20 * (xh_mag * np.abs(mul) + np.abs(add))
    diff = np.abs(y.astype(np.float64) - y_eager)
    assert np.all(diff <= tol), f"max excess {(diff - tol).max()}"
    assert (diff > 0).mean() < 0.02


def test_layer_norm_invariants_and_identities():
    rng = np.random.default_rng(3)
    x = fp8.bf16_round(_bf16(rng, (16, 1024), scale=4.0) + np.float32(3.0))
    y, _ = adaln.adaln_y(x, eps=1e-6)
    assert np.abs(y.mean(axis=-1)).max() < 2e-2
    assert np.abs(y.std(axis=-1) - 1).max() < 2e-2
    # norm "none" with no modulation is the identity on bf16 values
    y0, _ = adaln.adaln_y(x, norm_type="none")
    np.testing.assert_array_equal(y0, x)
    # a constant row normalizes to exactly zero
    c = np.full((1, 256), 7.25, np.float32)
    yc, _ = adaln.adaln_y(c, eps=1e-6)
    assert not yc.any()
    # mul = 1, add = 0 changes nothing
    y1, _ = adaln.adaln_y(x, np.ones(1024, np.float32), np.zeros(1024, np.float32), eps=1e-6)
    np.testing.assert_array_equal(y1, y)


def test_residual_output_is_bf16_of_fp32_gated_sum():
    rng = np.random.default_rng(4)
    h, r = _bf16(rng, (4, 256)), _bf16(rng, (4, 256))
    g = rng.standard_normal(256).astype(np.float32)
    _, res_out = adaln.adaln_y(h, residual=r, gate=g, norm_type="none")
    ref = (torch.from_numpy(h).float() * torch.from_numpy(g) + torch.from_numpy(r)).to(torch.bfloat16).float()
    np.testing.assert_array_equal(res_out, ref.numpy())
