"""Bit-level fp8 e4m3fn, bf16 and e8m0 helpers (numpy) -- oracle, test infrastructure only.

Reference semantics: ``_fp8_e4m3fn_round`` (vllm_omni_neuron/kernels/nkilib/experimental/norm/
adaln_quant_torch.py:35-38) rounds through torch's float8_e4m3fn cast: round to nearest even,
subnormals with a 2^-9 grain, max finite 448 (adaln_quant_torch.py:28). This module restates that
conversion with integer arithmetic so the oracle does not depend on the cast it is checked against.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (nearest even) and return them as fp32. Finite inputs only."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of fp32 values, rounding to nearest even."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32/fp64 values -> e4m3fn codes (uint8), round to nearest even.

    Values with |x| >= 464 would round past the largest finite code; callers clip to +-448 first
    (the MX and ROW rules both do), so such inputs are rejected here. Values exactly representable
    in fp32 take an integer path on the fp32 bits; other fp64 values are rounded from their fp64
    magnitude directly (no double rounding through fp32).
    """
    x = np.asarray(x)
    x32 = x.astype(np.float32)
    if x.dtype != np.float32 and not np.array_equal(x32.astype(x.dtype), x):
        return _e4m3_encode_f64(x)
    u = x32.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    mag = u & np.uint32(0x7FFFFFFF)
    if np.any(mag >= np.float32(464.0).view(np.uint32)):  # also catches inf / nan
        raise ValueError("e4m3_encode: input outside the finite e4m3fn rounding range")
    # normal range (|x| >= 2^-6, biased fp32 exponent >= 121): round the 23-bit mantissa to 3 bits,
    # nearest even; a carry moves into the exponent, and rebiasing 127 -> 7 subtracts 120 << 3
    rne = (mag + np.uint32(0x7FFFF) + ((mag >> 20) & 1)) >> 20
    normal = (rne.astype(np.int64) - (120 << 3))
    # subnormal range (and zero): magnitude in units of 2^-9, nearest even (exact in fp32); 8 is the
    # smallest normal, which the same integer encodes
    sub = np.rint(mag.view(np.float32) * np.float32(512.0)).astype(np.int64)
    code = np.where(mag >= np.uint32(121 << 23), normal, sub)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def _e4m3_encode_f64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    if np.any(~np.isfinite(a)) or np.any(a >= 464.0):
        raise ValueError("e4m3_encode: input outside the finite e4m3fn rounding range")
    code = np.zeros(a.shape, dtype=np.int64)
    # Subnormal range (and zero): magnitude in units of 2^-9, nearest even. A result of 8 is the
    # smallest normal (exponent field 1, mantissa 0), which the same integer encodes.
    sub = a < 2.0**-6
    code[sub] = np.rint(a[sub] * 2.0**9).astype(np.int64)
    # Normal range: e = floor(log2 a) taken from the fp64 exponent; mantissa rounded to 3 bits.
    nrm = ~sub
    if np.any(nrm):
        an = a[nrm]
        e = np.frexp(an)[1] - 1  # an = m * 2^e, m in [1, 2)
        q = np.rint(np.ldexp(an, 3 - e)).astype(np.int64)  # in [8, 16]
        carry = q == 16
        e = e + carry
        q = np.where(carry, 8, q)
        code[nrm] = ((e + 7) << 3) | (q - 8)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    """e4m3fn codes -> fp32 values (0x7F / 0xFF, the NaN codes, decode to NaN)."""
    c = np.asarray(c, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    v = np.where(e == 0, np.ldexp(m.astype(np.float64), -9), np.ldexp(1.0 + m / 8.0, e - 7))
    v = np.where((c & 0x7F) == 0x7F, np.nan, v)
    return (s * v).astype(np.float32)


def e8m0_value(s: np.ndarray) -> np.ndarray:
    """e8m0 shared-exponent bytes -> 2^(s - 127) as fp64."""
    return np.ldexp(1.0, np.asarray(s, dtype=np.int64) - 127)


def exp_field(x: np.ndarray) -> np.ndarray:
    """Biased fp32 exponent field of each value (0 for zeros and subnormals)."""
    return ((np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 23) & 0xFF).astype(np.int64)
