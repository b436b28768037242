"""Every tensor whose pointer reaches the C ABI is checked on the host first (CPU only).

A wrong dtype, shape or layout raises ValueError before anything is launched; a tensor that is
not on a GPU raises RuntimeError ("no CPU fallback"). These run on CPU tensors, so a check that
were missing would surface as the device error instead of the ValueError asserted here.
"""

import pytest
import torch

N, K, M = 256, 128, 8


@pytest.fixture(scope="module")
def w(pkg):
    codes = torch.zeros(N, K, dtype=torch.uint8).view(torch.float8_e4m3fn)
    scales = torch.full((N, K // 32), 127, dtype=torch.uint8)
    return pkg.MXWeight(codes, scales, None, torch.zeros(N))


@pytest.fixture(scope="module")
def x(pkg):
    return pkg.MXTensor(torch.zeros(M, K, dtype=torch.uint8).view(torch.float8_e4m3fn),
                        torch.full((M, K // 32), 127, dtype=torch.uint8))


def test_linear_weight_vectors(pkg, w, x):
    bad = [
        w._replace(bias=torch.zeros(N, dtype=torch.bfloat16)),  # bias dtype
        w._replace(bias=torch.zeros(N + 1)),  # bias shape
        w._replace(col_scale=torch.zeros(2, N)),  # col_scale shape
        w._replace(scales=torch.zeros(N, K // 16, dtype=torch.uint8)),  # scales shape
        w._replace(scales=torch.zeros(N, K // 32, dtype=torch.float32)),  # scales dtype
    ]
    for wb in bad:
        with pytest.raises(ValueError):
            pkg.mxfp8_linear(x, wb)


def test_linear_activation_and_epilogue_operands(pkg, w, x):
    with pytest.raises(ValueError, match="activation scales"):
        pkg.mxfp8_linear(x._replace(scales=torch.zeros(M, 3, dtype=torch.uint8)), w)
    with pytest.raises(ValueError, match="residual"):
        pkg.mxfp8_linear(x, w, epilogue="gated_residual", residual=torch.zeros(M, N), gate=torch.ones(N))
    with pytest.raises(ValueError, match="gate"):
        pkg.mxfp8_linear(x, w, epilogue="gated_residual", residual=torch.zeros(M, N, dtype=torch.bfloat16),
                         gate=torch.ones(N, dtype=torch.float16))
    with pytest.raises(ValueError, match="out"):
        pkg.mxfp8_linear(x, w, out=torch.zeros(M, N))
    with pytest.raises(ValueError, match="row_sumsq"):
        pkg.mxfp8_linear(x, w, row_sumsq=torch.zeros(M, 3), sumsq_cols=128)
    with pytest.raises(ValueError, match="ROW-packed"):
        pkg.mxfp8_linear(torch.zeros(M, K + 4, dtype=torch.bfloat16), w)
    # well-formed but on the host: the device check fires
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.mxfp8_linear(x, w)


def test_qk_norm_rope_tables(pkg):
    ops = pkg.attention_ops
    S, W = 16, 512
    xq = torch.zeros(S, W, dtype=torch.bfloat16)
    g = torch.ones(W)
    ok = torch.zeros(S, 64)
    for cos, sin in [
        (ok.to(torch.bfloat16), ok),  # half-width dtype would read past the table
        (torch.zeros(1, S, 1, 128), torch.zeros(1, S, 1, 128)),  # the reference's interleaved [1,S,1,128]
        (torch.zeros(S + 1, 64), torch.zeros(S + 1, 64)),  # wrong S
        (ok.t().contiguous().t(), ok),  # not contiguous
        (ok, None),
    ]:
        with pytest.raises(ValueError):
            ops.qk_rmsnorm_rope_(xq, g, cos=cos, sin=sin)
    with pytest.raises(ValueError):
        ops.qk_rmsnorm_rope_(xq, torch.ones(W - 1))
    with pytest.raises(ValueError):
        ops.qk_rmsnorm_rope_(xq, g, rope_pairs="bogus")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.qk_rmsnorm_rope_(xq, g, cos=ok, sin=ok)


def test_attention_operands(pkg):
    ops = pkg.attention_ops
    Sq, Sk, Nh = 32, 64, 4
    q = torch.zeros(Sq, Nh, 128, dtype=torch.bfloat16)
    k = torch.zeros(Sk, Nh, 128, dtype=torch.bfloat16)
    vt = torch.zeros(Nh, 128, 64, dtype=torch.bfloat16)
    km = torch.ones(Nh)
    with pytest.raises(ValueError, match="vt"):
        ops.attention_core(q, k, vt[:, :, :32], km, 0.1)
    with pytest.raises(ValueError, match="kmax"):
        ops.attention_core(q, k, vt, km.double(), 0.1)
    qp = ops.QPrep(torch.zeros(Sq, Nh), torch.ones(Nh * 128), torch.zeros(Sq, 64, dtype=torch.bfloat16),
                   torch.zeros(Sq, 64))
    with pytest.raises(ValueError, match="cos"):
        ops.attention_core(q, k, vt, km, 0.1, q_prep=qp)
    with pytest.raises(ValueError, match="sumsq"):
        ops.attention_core(q, k, vt, km, 0.1, q_prep=ops.QPrep(torch.zeros(Sq, Nh - 1), torch.ones(Nh * 128)))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.attention_core(q, k, vt, km, 0.1)


def test_drop_in_argument_checks(pkg, w):
    ops, ct = pkg.attention_ops, pkg.common_types
    packed = torch.zeros(1, M, K + 4, dtype=torch.uint8).view(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="output channels"):
        ops.row_mx_qkv_proj(packed, w, num_heads=4, head_dim=128, num_kv_heads=4)
    with pytest.raises(NotImplementedError):
        ops.row_mx_qkv_proj(packed, w, num_heads=2, head_dim=64, num_kv_heads=0)
    with pytest.raises(NotImplementedError, match="across-heads"):  # RoPE needs the K norm too
        cfg = ct.QKNormConfig(q_norm=ct.NormType.RMS_NORM_ACROSS_HEADS, k_norm=None)
        wk = pkg.MXWeight(torch.zeros(3 * 512, K, dtype=torch.uint8).view(torch.float8_e4m3fn),
                          torch.full((3 * 512, K // 32), 127, dtype=torch.uint8))
        ops.row_mx_qkv_proj(packed, wk, num_heads=4, head_dim=128, num_kv_heads=4, fused_rope=True,
                            qk_norm_pre_rope=cfg, qk_norm_pre_rope_q_gamma=torch.ones(512))
    with pytest.raises(NotImplementedError):
        ops.row_mx_qkv_proj(packed, w, num_heads=2, head_dim=128, replica_groups=[[0, 1]])
    with pytest.raises(ValueError, match="weight scale"):
        pkg.row_mx_mlp(packed, w, w, up_w_scale=torch.ones(N + 1))
    with pytest.raises(ValueError, match="K/4, N, 4"):
        pkg.packed_weight_to_mx(torch.zeros(K, N, dtype=torch.uint8).view(torch.float8_e4m3fn))
    with pytest.raises(ValueError, match="bf16"):
        pkg.row_quantize_packed(torch.zeros(M, K))
    with pytest.raises(ValueError, match=r"\[T, H\]"):
        pkg.row_quantize_packed(torch.zeros(K, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):  # no CPU fallback
        pkg.row_quantize_packed(torch.zeros(M, K, dtype=torch.bfloat16))


def test_packed_reference_weight_layout(pkg):
    """[K/4, N, 4] with four consecutive contraction values innermost -> codes [N, K]."""
    K4, Nn = 16, 256
    phys = torch.arange(K4 * Nn * 4, dtype=torch.int64).remainder(251).to(torch.uint8).view(K4, Nn, 4)
    mw = pkg.packed_weight_to_mx(phys.view(torch.float8_e4m3fn), torch.full((1, Nn), 0.5))
    codes = mw.codes.view(torch.uint8)
    for n, k in [(0, 0), (3, 5), (255, 63), (17, 30)]:
        assert int(codes[n, k]) == int(phys[k // 4, n, k % 4])
    assert mw.rope_pairs == "halves" and bool((mw.scales == 127).all())
    assert mw.col_scale.shape == (Nn,) and float(mw.col_scale[7]) == 0.5


def test_registered_attention_op(pkg):
    """``wan_transformer::attention_cte`` is registered as a functional torch op (the reference's
    ``nki_op`` registration), propagates shapes without running ([BN, S_q, D] -> [BN, D, S_q]) and
    refuses CPU tensors (no CPU fallback)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    op = torch.ops.wan_transformer.attention_cte
    with FakeTensorMode():
        q = torch.empty(6, 300, 128, dtype=torch.bfloat16)
        k = torch.empty(6, 77, 128, dtype=torch.bfloat16)
        o = op(q, k, k)
        assert o.shape == (6, 128, 300) and o.dtype == torch.bfloat16
    with pytest.raises(RuntimeError):
        op(torch.zeros(2, 8, 128, dtype=torch.bfloat16), torch.zeros(2, 8, 128, dtype=torch.bfloat16),
           torch.zeros(2, 8, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="BN, S, 128"):
        pkg.attention_ops.attention_cte(torch.zeros(2, 8, 128), torch.zeros(3, 8, 128), torch.zeros(3, 8, 128))
    assert pkg.attention_ops.register_torch_ops() is False  # registered once per process


def test_adaln_quant_kernel_argument_checks(pkg):
    """The kernel-level adaLN drop-in keeps the reference's checks (adaln_quant.py:70-114, 242-290)
    and refuses what gfx950 does not produce, all before any launch."""
    A, NT, QT, DM = pkg.AdaLNQuantKernelArgs, pkg.NormType, pkg.QuantizationType, pkg.DtypeMode
    with pytest.raises(ValueError, match="normalization"):
        A(norm_type=NT.RMS_NORM_ACROSS_HEADS)
    with pytest.raises(ValueError, match="quantization"):
        A(quantization_type=QT.ROW_MX)
    with pytest.raises(ValueError, match="Lower bound"):
        A(lower_bound=-1.0)
    with pytest.raises(ValueError, match="Epsilon"):
        A(eps=-1e-6)
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    k = pkg.adaln_quant_kernel
    with pytest.raises(NotImplementedError, match="MX"):
        k(x, A(quantization_type=QT.MX), dtype_mode=DM.OCP)
    with pytest.raises(NotImplementedError, match="NON_OCP"):
        k(x, A(quantization_type=QT.ROW))  # the reference's default dtype mode
    with pytest.raises(NotImplementedError, match="clip bound"):
        k(x, A(quantization_type=QT.ROW, lower_bound=8.0), dtype_mode=DM.OCP)
    with pytest.raises(ValueError, match="Rank of hidden"):
        k(torch.zeros(64, dtype=torch.bfloat16), A())
    with pytest.raises(ValueError, match="gate requires residual"):
        k(x, A(), gate=torch.ones(64))
    with pytest.raises(ValueError, match="vector length"):
        k(x, A(), mul=torch.ones(32))
    with pytest.raises(ValueError, match="first dimension"):
        k(x, A(), add=torch.ones(2, 64))
    with pytest.raises(ValueError, match="residual"):
        k(x, A(), residual=torch.zeros(4, 32, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):  # no CPU fallback
        k(x, A(quantization_type=QT.ROW), dtype_mode=DM.OCP)


def _wan_mlp_kwargs(pkg, **over):
    """The argument set the Wan FFN passes to the nkilib mlp kernel (row_mx_kernels.py:172-198)."""
    ct = pkg.common_types
    kw = dict(skip_gate_proj=True, activation_fn=ct.ActFnType.GELU_Tanh_Approx, normalization_type=ct.NormType.NO_NORM,
              quantization_type=ct.QuantizationType.ROW_MX, quant_clipping_bound=None, output_dtype="bfloat16",
              force_cte_mode=True, dtype_mode=ct.DtypeMode.AUTO,
              gate_up_w_layout=ct.MLPGateUpWeightLayout.H_X4_INNERMOST)
    kw.update(over)
    return kw


def test_kernel_mlp_rejects_other_configurations(pkg, w):
    """The nkilib mlp signature runs only Wan's configuration; everything else is refused before
    any tensor is touched (NotImplementedError), and a malformed weight is a ValueError."""
    ct = pkg.common_types
    x = torch.zeros(M, K + 4, dtype=torch.uint8).view(torch.float8_e4m3fn)
    bad = [
        dict(skip_gate_proj=False),
        dict(activation_fn=ct.ActFnType.SiLU),
        dict(normalization_type=ct.NormType.RMS_NORM),
        dict(quantization_type=ct.QuantizationType.MX),
        dict(fused_add_tensor=torch.zeros(M, K, dtype=torch.bfloat16)),
        dict(store_fused_add_result=True),
        dict(quant_clipping_bound=240.0),
        dict(up_clamp_upper_limit=7.0),
        dict(store_output_in_sbuf=True),
        dict(transposed_in=True),
        dict(mode=ct.ComputationMode.DECODE),
        dict(dtype_mode=ct.DtypeMode.NON_OCP),
        dict(output_dtype=torch.float32),
        dict(down_in_scale=torch.ones(1)),
    ]
    for over in bad:
        with pytest.raises(NotImplementedError):
            pkg.kernels.mlp(x, w, w, w, **_wan_mlp_kwargs(pkg, **over))
    with pytest.raises(ValueError, match="MXWeight or a packed"):
        pkg.kernels.mlp(x, torch.zeros(K, N), torch.zeros(K, N), w, **_wan_mlp_kwargs(pkg))
    # the supported configuration with host tensors reaches the device check
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.kernels.mlp(x, w, w, w, **_wan_mlp_kwargs(pkg))


def test_kernel_qkv_shim_rejections(pkg):
    ct = pkg.common_types
    x = torch.zeros(1, M, K + 4, dtype=torch.uint8).view(torch.float8_e4m3fn)
    wt = torch.zeros(K // 4, 3 * 128, 4, dtype=torch.uint8).view(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="d_head"):
        pkg.kernels.torch_compatible_row_mx_qkv(x, wt, torch.ones(1, 384))
    with pytest.raises(NotImplementedError, match="replica"):
        pkg.kernels.torch_compatible_row_mx_qkv(x, wt, torch.ones(1, 384), None, 128, 1, 1, replica_groups=((0, 1),))
    with pytest.raises(NotImplementedError):
        pkg.kernels.torch_compatible_row_mx_qkv(x, wt, torch.ones(1, 384), None, 128, 1, 1,
                                                qk_norm_pre_rope_q_norm=ct.NormType.RMS_NORM)


@pytest.mark.parametrize("head_dim", [64, 112, 256])
def test_rope_refuses_head_dims_whose_split_disagrees(pkg, head_dim):
    """rope.py builds axis tables 2*(hd//6) wide and slices them at hd//3 (rope.py:54-55, 91-95);
    where those differ the reference's tables are not per-pair rotations, so these are refused."""
    with pytest.raises(NotImplementedError, match="split"):
        pkg.rope_tables((1, 2, 3), head_dim=head_dim, device="cpu")
    with pytest.raises(NotImplementedError, match="split"):
        pkg.WanRotaryPosEmbed(head_dim, (1, 2, 2), 1024)
    pkg.WanRotaryPosEmbed(128, (1, 2, 2), 1024)  # the Wan head_dim is accepted


def test_dmajor_to_mx_and_stream_helpers(pkg):
    ops = pkg.attention_ops
    with pytest.raises(ValueError, match="bf16"):
        ops.dmajor_to_mx(torch.zeros(1, 2, 128, 8))  # fp32
    with pytest.raises(ValueError, match="bf16"):
        ops.dmajor_to_mx(torch.zeros(2, 128, 8, dtype=torch.bfloat16))  # rank 3
    with pytest.raises(NotImplementedError, match="head_dim"):
        ops.dmajor_to_mx(torch.zeros(1, 2, 64, 8, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.dmajor_to_mx(torch.zeros(1, 2, 128, 8, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg._lib.hbm_stream_fold(torch.zeros(16384, dtype=torch.uint8), torch.zeros(32768, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg._lib.hbm_stream_copy(torch.zeros(16, dtype=torch.uint8), torch.zeros(16, dtype=torch.uint8))
