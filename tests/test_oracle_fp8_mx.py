"""Pin the oracle's fp8 / bf16 / MX / ROW rules (CPU only).

- e4m3fn and bf16 rounding are checked against torch's own casts (the library routines the
  reference's torch refs use, adaln_quant_torch.py:35-38) on every bf16 bit pattern and on random
  fp32 values, including exact ties.
- The MX rule (shared exponent = block max - 7, adaln_quant_torch.py:151-175) is pinned by
  hand-derived known answers: a plausible slip (OCP's emax 8, dropping the clamp at 0, a per-row
  instead of per-32 block) changes at least one of them.
"""

import numpy as np
import pytest
import torch

from oracle import fp8, mx


def _all_finite_bf16(limit=464.0):
    u = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    return u[np.isfinite(u) & (np.abs(u) < limit)]


def test_e4m3_encode_matches_torch_on_every_bf16():
    v = _all_finite_bf16()
    ref = torch.from_numpy(v.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(fp8.e4m3_encode(v), ref)


def test_e4m3_encode_matches_torch_on_random_fp32_and_ties():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal(200_000) * np.exp2(rng.integers(-14, 8, 200_000))).astype(np.float32)
    v = np.clip(v, -448, 448)
    # exact midpoints between neighbouring e4m3 values (ties -> even), normal and subnormal
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    lo, hi = fp8.e4m3_decode(codes[:-1]), fp8.e4m3_decode(codes[1:])
    ties = ((lo.astype(np.float64) + hi) / 2).astype(np.float32)
    v = np.concatenate([v, ties, -ties]).astype(np.float32)
    ref = torch.from_numpy(v.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(fp8.e4m3_encode(v), ref)


def test_e4m3_decode_all_codes():
    c = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(c.copy()).view(torch.float8_e4m3fn).float().numpy()
    got = fp8.e4m3_decode(c)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok], ref[ok])
    assert fp8.e4m3_decode(np.array([0x7E], np.uint8))[0] == 448.0
    assert fp8.e4m3_decode(np.array([0x01], np.uint8))[0] == 2.0**-9


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(100_000) * np.exp2(rng.integers(-30, 30, 100_000))).astype(np.float32)
    ref = torch.from_numpy(v.copy()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(fp8.bf16_round(v), ref)


def _block(vals, fill=0.0):
    b = np.full(32, fill, np.float32)
    b[: len(vals)] = vals
    return b


def test_mx_known_answers():
    # max 1.0 (biased exp 127) -> s = 120 -> multiplier 2^7: 1.0 -> 128.0 (code 0x70), 0.5 -> 64
    codes, s = mx.mx_quantize(_block([1.0, 0.5, -1.0])[None])
    assert s.tolist() == [[120]]
    assert codes[0, :3].tolist() == [0x70, 0x68, 0xF0]
    # max 3.0 (exp 128) -> s = 121 -> 3 * 2^6 = 192 (code 0x74); 0.01 * 64 = 0.64 -> 0.625 (0x32)
    codes, s = mx.mx_quantize(_block([3.0, 0.01])[None])
    assert s.tolist() == [[121]]
    assert codes[0, :2].tolist() == [0x74, 0x32]
    # max 255.9 (exp 134) -> s = 127 -> multiplier 1 -> 255.9 rounds up to 256 (0x78)
    codes, s = mx.mx_quantize(_block([255.9])[None])
    assert s.tolist() == [[127]] and codes[0, 0] == 0x78
    # all-zero block: s = 0 (clamped), codes 0
    codes, s = mx.mx_quantize(np.zeros((1, 32), np.float32))
    assert s.tolist() == [[0]] and not codes.any()
    # tiny block: max exponent 3 < 7 -> s clamps to 0 -> multiplier 2^127
    tiny = np.float32(2.0**-124)  # biased exponent 3
    codes, s = mx.mx_quantize(_block([tiny])[None])
    assert s.tolist() == [[0]] and fp8.e4m3_decode(codes[0, :1])[0] == 8.0
    # two blocks get independent exponents
    y = np.concatenate([_block([1.0]), _block([16.0])])[None]
    codes, s = mx.mx_quantize(y)
    assert s.tolist() == [[120, 124]]
    assert codes[0, 0] == codes[0, 32] == 0x70


def test_mx_never_saturates_and_error_bound():
    rng = np.random.default_rng(2)
    y = fp8.bf16_round((rng.standard_normal((64, 512)) * np.exp2(rng.integers(-20, 20, (64, 1)))).astype(np.float32))
    codes, s = mx.mx_quantize(y)
    vals = fp8.e4m3_decode(codes)
    assert np.abs(vals).max() <= 256.0  # |y * 2^(127-s)| < 2^8 under the max-7 convention
    deq = mx.mx_dequantize(codes, s)
    # RNE error <= half an e4m3 ulp of the element's binade (relative 2^-4), or the subnormal grain
    blk_scale = np.repeat(np.ldexp(1.0, s.astype(np.int64) - 127), 32, axis=-1)
    bound = np.maximum(np.abs(y) * 2.0**-4, blk_scale * 2.0**-10)
    assert np.all(np.abs(deq - y) <= bound + 1e-30)


def test_row_quantize_known_answers():
    y = np.array([[448.0, -224.0, 1.0, 0.0]], np.float32)
    codes, dq = mx.row_quantize(y)
    assert dq[0, 0] == np.float32(1.0)
    assert codes[0].tolist() == [0x7E, 0xF6, 0x38, 0x00]
    packed = mx.row_pack(codes, dq)
    assert packed.shape == (1, 8)
    assert packed[0, 4:].tobytes() == np.float32(1.0).tobytes()
    c2, d2 = mx.row_unpack(packed)
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_array_equal(d2, dq)
    # all-zero row: dq floors at 1e-6
    codes, dq = mx.row_quantize(np.zeros((1, 8), np.float32))
    assert dq[0, 0] == np.float32(1e-6) and not codes.any()


@pytest.mark.parametrize("bad", [464.0, np.inf])
def test_e4m3_encode_rejects_out_of_range(bad):
    with pytest.raises(ValueError):
        fp8.e4m3_encode(np.array([bad], np.float32))
