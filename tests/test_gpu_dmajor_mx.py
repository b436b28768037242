"""The o-projection's d-major -> token-major MX pass (``wanmi_dmajor_to_mx``) against the two-pass
form it replaces (a transposing copy, then the adaLN kernel's NO_NORM / MX mode, itself bit-exact
against the oracle's MX rule): codes and scales bit-identical on every tested shape, stride and
value range, and the o-projection drop-in unchanged by it."""

import pytest
import torch

from oracle import mx as oracle_mx

pytestmark = pytest.mark.gpu


def _two_pass(pkg, att):
    B, N, D, S = att.shape
    x = att.permute(0, 3, 1, 2).reshape(B * S, N * D).contiguous()
    return pkg.adaln_kernels.adaln_quant_2d(x, None, None, eps=0.0, norm_type="none", quant="mx")


def _att(dev, B, N, S, seed, S_alloc=None):
    g = torch.Generator(device=dev).manual_seed(seed)
    full = torch.randn(B, N, 128, S_alloc or S, device=dev, generator=g)
    # magnitudes from 2^-20 to 2^12 across heads and tokens, a zero block and a one-hot block
    full = full * torch.exp2(torch.randint(-20, 13, (1, N, 1, S_alloc or S), device=dev, generator=g).float())
    full[:, 0, :32, 0] = 0.0
    if (S_alloc or S) > 1:
        full[:, 0, 32:64, 1] = 0.0
        full[:, 0, 40, 1] = -3.0
    return full.to(torch.bfloat16)[..., :S]


@pytest.mark.parametrize("B,N,S", [(1, 40, 1560), (2, 3, 64), (1, 2, 8), (3, 1, 200), (1, 40, 32760)])
def test_dmajor_to_mx_matches_the_two_pass_form(pkg, dev, B, N, S):
    att = _att(dev, B, N, S, seed=S + N)
    got = pkg.attention_ops.dmajor_to_mx(att)
    ref = _two_pass(pkg, att)
    torch.cuda.synchronize()
    assert torch.equal(got.codes.view(torch.uint8), ref.codes.view(torch.uint8))
    assert torch.equal(got.scales, ref.scales)


def test_dmajor_to_mx_strided_and_unaligned(pkg, dev):
    # a view whose channel rows are longer than S (d_stride > S): the fused pass
    att = _att(dev, 2, 4, 96, seed=5, S_alloc=136)
    assert att.stride(2) == 136
    got = pkg.attention_ops.dmajor_to_mx(att)
    ref = _two_pass(pkg, att)
    assert torch.equal(got.codes.view(torch.uint8), ref.codes.view(torch.uint8))
    assert torch.equal(got.scales, ref.scales)
    # S not a multiple of 8 takes the two-pass form (same bits by construction)
    att = _att(dev, 1, 3, 77, seed=6)
    got = pkg.attention_ops.dmajor_to_mx(att)
    ref = _two_pass(pkg, att)
    assert torch.equal(got.codes.view(torch.uint8), ref.codes.view(torch.uint8))


def test_dmajor_to_mx_against_the_oracle(pkg, dev):
    att = _att(dev, 1, 2, 40, seed=9)
    got = pkg.attention_ops.dmajor_to_mx(att)
    x = att.permute(0, 3, 1, 2).reshape(40, 256).float().cpu().numpy()
    codes, scales = oracle_mx.mx_quantize(x)
    assert (got.codes.view(torch.uint8).cpu().numpy() == codes).all()
    assert (got.scales.cpu().numpy() == scales).all()


def test_dmajor_to_mx_refuses_bad_strides_in_the_abi(pkg, dev):
    lib = pkg._lib.load()
    x = torch.zeros(1, 1, 128, 12, dtype=torch.bfloat16, device=dev)
    codes = torch.empty(12, 128, dtype=torch.uint8, device=dev)
    scales = torch.empty(12, 4, dtype=torch.uint8, device=dev)
    st = lib.wanmi_dmajor_to_mx(x.data_ptr(), 1, 1, 12, x.stride(0), x.stride(1), x.stride(2), codes.data_ptr(),
                                scales.data_ptr(), None)
    assert st != 0 and b"multiple of 8" in lib.wanmi_last_error()
