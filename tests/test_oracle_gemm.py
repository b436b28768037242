"""Pin the MXFP8 projection oracle (CPU only).

- ``mx_gemm`` against brute-force scalar loops on tiny, non-square shapes, with different block
  scales in every 32-block, per-row and per-column scales and a bias: a transposed operand, a
  misplaced block scale, or the bias applied before the scales fails it. The loops decode the e4m3
  codes with torch's own float8_e4m3fn cast, independently of the oracle's integer decoder.
- ``gelu_tanh`` at published values of the tanh approximation of GELU (which differ from the
  exact erf form by up to ~4e-4 near x = -3, and from the sigmoid form x * sigmoid(1.702 x) by
  ~2e-2), plus its odd-part identity gelu(x) - gelu(-x) = x.
- ``quantize_weight``: the GEMM layout is the transpose of the reference's ``x @ W`` weight.
"""

import math

import numpy as np
import torch

from oracle import fp8
from oracle import gemm as og
from oracle import mx as omx


def _random_mx(rng, rows, K):
    codes = rng.integers(0, 256, size=(rows, K), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x10  # no NaN codes
    scales = rng.integers(118, 136, size=(rows, K // 32), dtype=np.uint8)
    return codes, scales


def _decode(code: int, scale: int) -> float:
    v = float(torch.tensor([code], dtype=torch.uint8).view(torch.float8_e4m3fn).float()[0])
    return v * 2.0 ** (int(scale) - 127)


def test_mx_gemm_matches_brute_force_loops():
    rng = np.random.default_rng(0)
    M, N, K = 3, 5, 96
    a_c, a_s = _random_mx(rng, M, K)
    w_c, w_s = _random_mx(rng, N, K)
    r = rng.uniform(0.5, 2.0, M).astype(np.float32)
    c = rng.uniform(0.5, 2.0, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    got = og.mx_gemm(a_c, a_s, w_c, w_s, bias=b, row_scale=r, col_scale=c).numpy()
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += _decode(a_c[m, k], a_s[m, k // 32]) * _decode(w_c[n, k], w_s[n, k // 32])
            want = acc * float(r[m]) * float(c[n]) + float(b[n])
            assert abs(got[m, n] - want) <= 1e-12 * (abs(want) + 1.0), (m, n, got[m, n], want)


def test_abs_gemm_is_the_magnitude_product():
    rng = np.random.default_rng(1)
    a_c, a_s = _random_mx(rng, 4, 64)
    w_c, w_s = _random_mx(rng, 6, 64)
    got = og.abs_gemm(a_c, a_s, w_c, w_s).numpy()
    for m in range(4):
        for n in range(6):
            want = sum(abs(_decode(a_c[m, k], a_s[m, k // 32]) * _decode(w_c[n, k], w_s[n, k // 32])) for k in range(64))
            assert abs(got[m, n] - want) <= 1e-12 * want


def test_gelu_tanh_published_values():
    # 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) at x = 1, -1, 2, -3, 0
    x = torch.tensor([1.0, -1.0, 2.0, -3.0, 0.0], dtype=torch.float64)
    want = [0.8411919906082768, -0.15880800939172324, 1.9545976940877752, -0.0036373920817729943, 0.0]
    got = og.gelu_tanh(x)
    for g_, w_ in zip(got.tolist(), want):
        assert abs(g_ - w_) <= 1e-12, (g_, w_)
    # distinguishable from the exact erf GELU at x = -3 (-0.0040496)
    erf_gelu = -3.0 * 0.5 * (1.0 + math.erf(-3.0 / math.sqrt(2.0)))
    assert abs(float(got[3]) - erf_gelu) > 3e-4
    # odd-part identity of any GELU of the form x * F(x) with F(x) + F(-x) = 1
    t = torch.linspace(-6, 6, 121, dtype=torch.float64)
    assert torch.allclose(og.gelu_tanh(t) - og.gelu_tanh(-t), t, atol=1e-12)


def test_quantize_weight_is_the_transposed_mx_layout():
    rng = np.random.default_rng(2)
    K, N = 96, 40
    w = fp8.bf16_round(rng.standard_normal((K, N)).astype(np.float32) * 0.02)
    codes, scales = og.quantize_weight(w)
    assert codes.shape == (N, K) and scales.shape == (N, K // 32)
    deq = omx.mx_dequantize(codes, scales)
    # each dequantized element is within half an e4m3 step (2^-4 relative) of W[k, n]
    err = np.abs(deq - w.T.astype(np.float64))
    assert bool((err <= 2.0**-4 * np.abs(w.T) + 2.0**-9 * np.repeat(np.abs(w.T).reshape(N, -1, 32).max(-1), 32, -1)).all())
    assert not np.allclose(deq[:, :N], w[:N, :N].astype(np.float64), atol=1e-3)
