"""The allocation-free exact attention (``wanmi_attention_exact_noalloc``, static device scratch)
against ``wanmi_attention_exact`` (caller-provided row-sum workspace), through the C ABI.

Inputs are the loose-bound case of the exact drop-in test (half the query rows underflow under the
constant-max bound, so the rescue kernel runs and reads the scratch row sums). Two calls in a row,
the second with a smaller input (fewer queries, fewer keys, fewer heads), each bit-identical to the
allocating entry point on the same inputs; a size beyond the scratch is refused before any launch.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

HD = 128


def _case(Sq, Sk, N, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Sq, N, HD, generator=g) * 9.0
    q[0::2, :, 0] = 0.0
    q[1::2] = 0.05 * q[1::2]
    q[1::2, :, 0] = 50.0
    k = torch.randn(Sk, N, HD, generator=g)
    k[0] = 0.0
    k[0, :, 0] = 400.0
    v = torch.randn(Sk, N, HD, generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def _run(pkg, dev, q, k, v, noalloc):
    lib = pkg._lib.load()
    ops = pkg.attention_ops
    Sq, N, _ = q.shape
    Sk = k.shape[0]
    qd, kd = q.to(dev), k.to(dev)
    vt, s_pad = ops.transpose_heads(v.to(dev))
    kmax = ops.head_max_norm(kd)
    out = torch.full((N, HD, Sq), float("nan"), dtype=torch.bfloat16, device=dev)  # d-major
    args = [ctypes.c_void_p(qd.data_ptr()), qd.stride(1), qd.stride(0), ctypes.c_void_p(kd.data_ptr()), kd.stride(1),
            kd.stride(0), ctypes.c_void_p(vt.data_ptr()), s_pad, ctypes.c_void_p(kmax.data_ptr()), Sq, Sk, N, HD,
            HD**-0.5, ops.OUT_DMAJOR, ctypes.c_void_p(out.data_ptr()), out.stride(0), 1, out.stride(1)]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if noalloc:
        st = lib.wanmi_attention_exact_noalloc(*args, stream)
    else:
        row_sum = torch.empty((N, Sq), dtype=torch.float32, device=dev)
        st = lib.wanmi_attention_exact(*args, ctypes.c_void_p(row_sum.data_ptr()), stream)
    pkg._lib.check(st, "exact attention")
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_the_allocating_entry_point(pkg, dev):
    for Sq, Sk, N, seed in ((700, 1900, 8, 1), (150, 500, 4, 2)):  # the second call smaller
        q, k, v = _case(Sq, Sk, N, seed)
        ref = _run(pkg, dev, q, k, v, noalloc=False)
        got = _run(pkg, dev, q, k, v, noalloc=True)
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got, ref), (Sq, Sk, N)
        assert float(got[:, :, 0::2].float().abs().max()) > 0.1  # the rescued rows are not zero


def test_noalloc_refuses_more_rows_than_its_scratch(pkg, dev):
    lib = pkg._lib.load()
    heads, Sq = 64, (1 << 22) // 64 + 1  # one row sum past the 4M the library holds
    st = lib.wanmi_attention_exact_noalloc(None, 0, 0, None, 0, 0, None, 64, None, Sq, 64, heads, HD, 0.1,
                                           pkg.attention_ops.OUT_DMAJOR, None, 0, 0, 0, None)
    assert st == pkg._lib.WANMI_ERR_ARG
    assert b"exceed" in lib.wanmi_last_error()
