"""The reference-form drop-ins, called as the reference's modules call them, against the oracle.

- ``row_mx_qkv_proj`` as ``WanSelfAttentionFP8.forward`` calls it (row_mx_modules.py:340-404):
  the ROW-packed activation of ``adaln_modulate(quant="row")``, the reference's packed
  ``[H/4, I, 4]`` FP8 weight with Q/K channels de-interleaved per head, per-channel
  ``weight_scales [1, I]`` (three checkpoint scalars expanded), a de-interleaved ``[1, I]`` bias and
  ``[1, dim]`` gammas, rotate-half caches ``[B, S, 128]`` built from Wan's interleaved tables
  (row_mx_modules.py:51-76), ``QKNormConfig(RMS_NORM_ACROSS_HEADS, RMS_NORM_ACROSS_HEADS)``, batch 2,
  BSD and NBSd layouts; and as ``WanCrossAttentionFP8._project_query`` calls it (Q only, no RoPE,
  NBSd). The oracle computes the ROW_MX projection (``psum * r_s * c_n + b``, qkv_cte.py:3996-4021)
  in fp64 on the natural channel order, the across-heads RMSNorm and Wan's interleaved RoPE, and
  the result is compared after de-interleaving its Q/K channels the same way.
- ``row_mx_mlp`` with a ROW-packed input and per-channel ``*_w_scale`` against the oracle's
  ROW_MX MLP (up -> GELU-tanh -> bf16 -> MX -> down, mlp_torch.py:471-597).
- ``row_mx_o_proj`` on d-major ``[B, N, D, S]`` attention with the reference's partition-expanded
  ``[128, H]`` weight scale against MX quantization of the token-major activation and the fp64
  product.

Bars: the GEMM bars of the projection tests (max |err| / max |ref| <= 2e-2, cosine >= 0.999) per
output section; the NBSd result must be exactly the BSD result re-laid out.
"""

import numpy as np
import pytest
import torch

from oracle import gemm as og
from oracle import mx as omx
from oracle import rope as orope

pytestmark = pytest.mark.gpu

HD = 128


def _close(got, ref, what, bar=2e-2, cos_bar=0.999):
    got, ref = got.double().flatten(), ref.double().flatten()
    rel = float((got - ref).abs().max() / ref.abs().max())
    cos = float(torch.nn.functional.cosine_similarity(got, ref, dim=0))
    assert rel <= bar and cos >= cos_bar, (what, rel, cos)


def _per_tensor_fp8(w: torch.Tensor):
    """[K, N] fp32 -> (fp8 codes [K, N], scalar scale): absmax per-tensor quantization, as the
    ComfyUI FP8-scaled checkpoint stores a linear."""
    s = float(w.abs().max()) / 448.0
    return (w / s).to(torch.float8_e4m3fn), s


def _deinterleave_cols(n_heads: int) -> torch.Tensor:
    perm = torch.cat([torch.arange(0, HD, 2), torch.arange(1, HD, 2)])
    return (torch.arange(n_heads)[:, None] * HD + perm[None]).reshape(-1)


def _pack(codes_kn: torch.Tensor) -> torch.Tensor:
    """[K, N] fp8 -> the reference's [K/4, N, 4] (four consecutive contraction values innermost)."""
    K, N = codes_kn.shape
    return codes_kn.view(torch.uint8).reshape(K // 4, 4, N).permute(0, 2, 1).contiguous().view(torch.float8_e4m3fn)


def _row_mx_oracle(packed: torch.Tensor, w_codes_kn: torch.Tensor, col_scale, bias) -> torch.Tensor:
    """fp64 ROW_MX projection of a ROW-packed [T, K + 4] activation: (codes . dq_row) @ W * c + b."""
    p = packed.reshape(-1, packed.shape[-1]).view(torch.uint8).cpu().numpy()
    codes, dq = omx.row_unpack(p)
    K = codes.shape[-1]
    neutral_a = np.full((codes.shape[0], K // 32), 127, np.uint8)
    wc = w_codes_kn.view(torch.uint8).t().contiguous().cpu().numpy()
    neutral_w = np.full((wc.shape[0], K // 32), 127, np.uint8)
    return og.mx_gemm(codes, neutral_a, wc, neutral_w, bias=bias, row_scale=dq.reshape(-1), col_scale=col_scale)


@pytest.fixture(scope="module")
def qkv_case(pkg, dev):
    B, grid, nh = 2, (1, 15, 20), 8
    S, dim = grid[0] * grid[1] * grid[2], nh * HD
    g = torch.Generator().manual_seed(11)
    h = torch.randn(B, S, dim, generator=g).to(torch.bfloat16)
    mul, add = 1 + 0.5 * torch.randn(dim, generator=g), 0.5 * torch.randn(dim, generator=g)
    wq, sq = _per_tensor_fp8(torch.randn(dim, dim, generator=g) * 0.02)
    wk, sk = _per_tensor_fp8(torch.randn(dim, dim, generator=g) * 0.03)
    wv, sv = _per_tensor_fp8(torch.randn(dim, dim, generator=g) * 0.01)
    w_nat = torch.cat([wq, wk, wv], dim=1)  # [K, 3 dim], natural channel order
    scales = torch.cat([torch.full((dim,), s) for s in (sq, sk, sv)])
    bias = 0.1 * torch.randn(3 * dim, generator=g)
    gq, gk = 1 + 0.1 * torch.randn(dim, generator=g), 1 + 0.1 * torch.randn(dim, generator=g)
    # the reference loader's layout: Q/K columns de-interleaved per head, V untouched
    qk_perm = _deinterleave_cols(nh)
    order = torch.cat([qk_perm, dim + qk_perm, torch.arange(2 * dim, 3 * dim)])
    w_ref = w_nat.view(torch.uint8)[:, order].contiguous().view(torch.float8_e4m3fn)
    packed = pkg.adaln_modulate(h.to(dev), mul.to(dev), add.to(dev), eps=1e-6, quant="row")
    cos, sin = orope.wan_rope(grid)
    base_c, base_s = cos[:, 0::2], sin[:, 1::2]
    cos_cache = torch.cat([base_c, base_c], -1)[None].expand(B, S, HD).contiguous()
    sin_cache = torch.cat([base_s, base_s], -1)[None].expand(B, S, HD).contiguous()
    # oracle, natural order: ROW_MX projection -> bf16 -> across-heads RMS -> interleaved RoPE
    lin = _row_mx_oracle(packed, w_nat, scales.numpy(), bias.numpy()).float().to(torch.bfloat16).view(B, S, 3 * dim)
    q = orope.rms_norm_across_heads(lin[..., :dim], gq).view(B, S, nh, HD)
    k = orope.rms_norm_across_heads(lin[..., dim : 2 * dim], gk).view(B, S, nh, HD)
    q = orope.apply_rotary_emb_wan(q, cos[None, :, None], sin[None, :, None]).view(B, S, dim)
    k = orope.apply_rotary_emb_wan(k, cos[None, :, None], sin[None, :, None]).view(B, S, dim)
    ref_nat = torch.cat([q, k, lin[..., 2 * dim :]], dim=-1)
    return dict(B=B, S=S, nh=nh, dim=dim, packed=packed, w_ref=w_ref, w_nat=w_nat, order=order, scales=scales,
                bias=bias, gq=gq, gk=gk, cos_cache=cos_cache, sin_cache=sin_cache, ref_nat=ref_nat, lin=lin)


def _call_self(pkg, c, dev, weight, layout, scales, bias, gq, gk):
    ct = pkg.common_types
    return pkg.row_mx_qkv_proj(
        c["packed"], weight, scales.to(dev)[None], bias.to(dev)[None], num_heads=c["nh"], head_dim=HD,
        num_kv_heads=c["nh"], fused_rope=True, cos_cache=c["cos_cache"].to(dev), sin_cache=c["sin_cache"].to(dev),
        qk_norm_pre_rope=ct.QKNormConfig(ct.NormType.RMS_NORM_ACROSS_HEADS, ct.NormType.RMS_NORM_ACROSS_HEADS, 1e-6),
        qk_norm_pre_rope_q_gamma=gq.to(dev)[None], qk_norm_pre_rope_k_gamma=gk.to(dev)[None], norm_eps=1e-6,
        output_layout=layout,
    )


def test_qkv_proj_reference_packed_weight(pkg, dev, qkv_case):
    c = qkv_case
    dim, order = c["dim"], c["order"]
    ct = pkg.common_types
    w = _pack(c["w_ref"]).to(dev)
    out = _call_self(pkg, c, dev, w, None, c["scales"][order], c["bias"][order], c["gq"][order[:dim]],
                     c["gk"][order[dim : 2 * dim] - dim])
    assert out.shape == (c["B"], c["S"], 3 * dim) and out.dtype == torch.bfloat16
    ref = c["ref_nat"][..., order]  # the reference's channel order
    got = out.cpu()
    for name, sl in (("Q", slice(0, dim)), ("K", slice(dim, 2 * dim)), ("V", slice(2 * dim, 3 * dim))):
        for b in range(c["B"]):
            _close(got[b, :, sl], ref[b, :, sl], f"{name} batch {b}")
    # NBSd is the same result laid out [N, B, S, d]
    nbsd = _call_self(pkg, c, dev, w, ct.QKVOutputLayout.NBSd, c["scales"][order], c["bias"][order],
                      c["gq"][order[:dim]], c["gk"][order[dim : 2 * dim] - dim])
    assert nbsd.shape == (3 * c["nh"], c["B"], c["S"], HD) and nbsd.is_contiguous()
    assert torch.equal(nbsd.cpu(), got.view(c["B"], c["S"], 3 * c["nh"], HD).permute(2, 0, 1, 3))


def test_qkv_proj_natural_order_mxweight(pkg, dev, qkv_case):
    """The same projection from an MXWeight in Wan's natural order (interleaved RoPE pairs)."""
    c = qkv_case
    dim = c["dim"]
    codes = c["w_nat"].view(torch.uint8).t().contiguous().view(torch.float8_e4m3fn).to(dev)
    mw = pkg.MXWeight(codes, torch.full((3 * dim, dim // 32), 127, dtype=torch.uint8, device=dev))
    out = _call_self(pkg, c, dev, mw, None, c["scales"], c["bias"], c["gq"], c["gk"]).cpu()
    for name, sl in (("Q", slice(0, dim)), ("K", slice(dim, 2 * dim)), ("V", slice(2 * dim, 3 * dim))):
        _close(out[:, :, sl], c["ref_nat"][:, :, sl], name)


def test_cross_query_projection_nbsd(pkg, dev, qkv_case):
    """``WanCrossAttentionFP8._project_query``: Q only (num_kv_heads 0), across-heads norm, no RoPE."""
    c = qkv_case
    dim, nh = c["dim"], c["nh"]
    ct = pkg.common_types
    wq = c["w_nat"][:, :dim]
    out = pkg.row_mx_qkv_proj(
        c["packed"], _pack(wq).to(dev), c["scales"][:dim].to(dev)[None], c["bias"][:dim].to(dev)[None], num_heads=nh,
        head_dim=HD, qk_norm_pre_rope=ct.QKNormConfig(ct.NormType.RMS_NORM_ACROSS_HEADS, None, 1e-6),
        qk_norm_pre_rope_q_gamma=c["gq"].to(dev)[None], norm_eps=1e-6, output_layout=ct.QKVOutputLayout.NBSd,
    )
    assert out.shape == (nh, c["B"], c["S"], HD)
    ref = orope.rms_norm_across_heads(c["lin"][..., :dim], c["gq"]).view(c["B"], c["S"], nh, HD).permute(2, 0, 1, 3)
    _close(out.cpu(), ref, "cross Q")


@pytest.mark.parametrize("shape", [(512, 5120), (2, 37, 96), (0, 64)])
def test_row_quantize_packed(pkg, dev, shape):
    """The context row-pack (row_mx_kernels.py:12-45) bit for bit against the oracle's ROW rule,
    2-D and batched, with a zero row (dequant scale floored at 1e-6) and rows of very different
    magnitudes."""
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=g)
    if x.numel():
        flat = x.view(-1, shape[-1])
        flat[0] = 0.0
        flat[-1] *= 3.0e4
        if flat.shape[0] > 2:
            flat[1] *= 1.0e-5
    x = x.to(torch.bfloat16)
    out = pkg.row_quantize_packed(x.to(dev))
    assert out.dtype == torch.float8_e4m3fn and out.shape == (*shape[:-1], shape[-1] + 4)
    codes, dq = omx.row_quantize(x.float().numpy())
    np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), omx.row_pack(codes, dq))


def test_row_packed_context_cross_kv(pkg, dev, qkv_case):
    """``WanCrossAttentionFP8.project_kv`` on the row-packed context (row_mx_modules.py:509-542,
    wan2_2_transformer.py:1686-1696): K with the across-heads norm and V, both NBSd, from one packed
    input, against the fp64 ROW_MX projections of the oracle's packing."""
    c = qkv_case
    dim, nh = c["dim"], c["nh"]
    ct = pkg.common_types
    g = torch.Generator().manual_seed(5)
    ctx = torch.randn(1, 96, dim, generator=g).to(torch.bfloat16)
    packed = pkg.row_quantize_packed(ctx.to(dev))
    codes, dq = omx.row_quantize(ctx.float().numpy())
    np.testing.assert_array_equal(packed.view(torch.uint8).cpu().numpy(), omx.row_pack(codes, dq))
    wk, wv = c["w_nat"][:, dim : 2 * dim], c["w_nat"][:, 2 * dim :]
    sk, sv = c["scales"][dim : 2 * dim], c["scales"][2 * dim :]
    bk, bv = c["bias"][dim : 2 * dim], c["bias"][2 * dim :]
    key = pkg.row_mx_qkv_proj(
        packed, _pack(wk).to(dev), sk.to(dev)[None], bk.to(dev)[None], num_heads=nh, head_dim=HD,
        qk_norm_pre_rope=ct.QKNormConfig(ct.NormType.RMS_NORM_ACROSS_HEADS, None, 1e-6),
        qk_norm_pre_rope_q_gamma=c["gk"].to(dev)[None], norm_eps=1e-6, output_layout=ct.QKVOutputLayout.NBSd,
    )
    value = pkg.row_mx_qkv_proj(packed, _pack(wv).to(dev), sv.to(dev)[None], bv.to(dev)[None], num_heads=nh,
                                head_dim=HD, output_layout=ct.QKVOutputLayout.NBSd)
    assert key.shape == value.shape == (nh, 1, 96, HD)
    lin_k = _row_mx_oracle(packed, wk, sk.numpy(), bk.numpy()).float().to(torch.bfloat16).view(1, 96, dim)
    lin_v = _row_mx_oracle(packed, wv, sv.numpy(), bv.numpy()).float().to(torch.bfloat16).view(1, 96, dim)
    ref_k = orope.rms_norm_across_heads(lin_k, c["gk"]).view(1, 96, nh, HD).permute(2, 0, 1, 3)
    _close(key.cpu(), ref_k, "cross K")
    _close(value.cpu(), lin_v.view(1, 96, nh, HD).permute(2, 0, 1, 3), "cross V")


def test_row_mx_mlp(pkg, dev):
    B, S, dim, ffn = 2, 200, 1024, 2816
    g = torch.Generator().manual_seed(12)
    h = torch.randn(B, S, dim, generator=g).to(torch.bfloat16)
    wu, su = _per_tensor_fp8(torch.randn(dim, ffn, generator=g) * 0.02)
    wd, sd = _per_tensor_fp8(torch.randn(ffn, dim, generator=g) * 0.02)
    bu, bd = 0.1 * torch.randn(ffn, generator=g), 0.1 * torch.randn(dim, generator=g)
    packed = pkg.adaln_modulate(h.to(dev), eps=1e-6, quant="row")

    def mxw(codes_kn):
        n, k = codes_kn.shape[1], codes_kn.shape[0]
        return pkg.MXWeight(codes_kn.view(torch.uint8).t().contiguous().view(torch.float8_e4m3fn).to(dev),
                            torch.full((n, k // 32), 127, dtype=torch.uint8, device=dev))

    up_scale = torch.full((1, ffn), su)
    down_scale = torch.full((128, dim), sd)  # partition-expanded, as the reference loads it
    out = pkg.row_mx_mlp(packed, mxw(wu), mxw(wd), up_scale.to(dev), down_scale.to(dev), bu.to(dev)[None],
                         bd.to(dev)[None])
    assert out.shape == (B, S, dim) and out.dtype == torch.bfloat16
    up = _row_mx_oracle(packed, wu, np.full(ffn, su, np.float32), bu.numpy())
    gel = og.gelu_tanh(up).float().to(torch.bfloat16).float().numpy()
    ic, isc = omx.mx_quantize(gel)
    wdc = wd.view(torch.uint8).t().contiguous().numpy()
    ref = og.mx_gemm(ic, isc, wdc, np.full((dim, ffn // 32), 127, np.uint8), bias=bd.numpy(),
                     col_scale=np.full(dim, sd, np.float32))
    _close(out.cpu().view(B * S, dim), ref, "row_mx_mlp")


def test_row_mx_o_proj(pkg, dev):
    B, nh, S, dim = 2, 8, 300, 1024
    g = torch.Generator().manual_seed(13)
    att = torch.randn(B, nh, HD, S, generator=g).to(torch.bfloat16)  # d-major [B, N, D, S]
    wo, so = _per_tensor_fp8(torch.randn(nh * HD, dim, generator=g) * 0.02)
    bo = 0.1 * torch.randn(dim, generator=g)
    codes = wo.view(torch.uint8).t().contiguous()
    mw = pkg.MXWeight(codes.view(torch.float8_e4m3fn).to(dev),
                      torch.full((dim, nh * HD // 32), 127, dtype=torch.uint8, device=dev))
    out = pkg.row_mx_o_proj(att.to(dev), mw, torch.full((128, dim), so, device=dev), bo.to(dev)[None])
    assert out.shape == (B, S, dim)
    x = att.permute(0, 3, 1, 2).reshape(B * S, nh * HD).float().numpy()
    xc, xs = omx.mx_quantize(x)
    ref = og.mx_gemm(xc, xs, codes.numpy(), np.full((dim, nh * HD // 32), 127, np.uint8), bias=bo.numpy(),
                     col_scale=np.full(dim, so, np.float32))
    _close(out.cpu().view(B * S, dim), ref, "row_mx_o_proj")


def test_torch_compatible_row_mx_qkv(pkg, dev, qkv_case):
    """The kernel-level QKV shim (qkv_shim.py:26-77) with the QK norm as flat scalars, as
    ``row_mx_qkv_proj`` calls it (row_mx_kernels.py:91-111): the reference's packed de-interleaved
    weight, rotate-half caches, both norms across heads; the result must be the oracle's, and
    bit-identical to the same projection through ``row_mx_qkv_proj``."""
    c = qkv_case
    dim, order = c["dim"], c["order"]
    ct = pkg.common_types
    w = _pack(c["w_ref"]).to(dev)
    scales, bias = c["scales"][order].to(dev)[None], c["bias"][order].to(dev)[None]
    gq, gk = c["gq"][order[:dim]].to(dev)[None], c["gk"][order[dim : 2 * dim] - dim].to(dev)[None]
    out = pkg.kernels.torch_compatible_row_mx_qkv(
        hidden=c["packed"], qkv_weights=w, qkv_w_scale=scales, bias=bias, d_head=HD, num_q_heads=c["nh"],
        num_kv_heads=c["nh"], output_layout=ct.QKVOutputLayout.BSD, fused_rope=True,
        cos_cache=c["cos_cache"].to(dev), sin_cache=c["sin_cache"].to(dev),
        qk_norm_pre_rope_q_norm=ct.NormType.RMS_NORM_ACROSS_HEADS,
        qk_norm_pre_rope_k_norm=ct.NormType.RMS_NORM_ACROSS_HEADS, qk_norm_pre_rope_eps=1e-6,
        qk_norm_pre_rope_q_gamma=gq, qk_norm_pre_rope_k_gamma=gk, replica_groups=None,
    )
    assert out.shape == (c["B"], c["S"], 3 * dim)
    ref = c["ref_nat"][..., order]
    got = out.cpu()
    for name, sl in (("Q", slice(0, dim)), ("K", slice(dim, 2 * dim)), ("V", slice(2 * dim, 3 * dim))):
        for b in range(c["B"]):
            _close(got[b, :, sl], ref[b, :, sl], f"shim {name} batch {b}")
    via = _call_self(pkg, c, dev, w, None, c["scales"][order], c["bias"][order], c["gq"][order[:dim]],
                     c["gk"][order[dim : 2 * dim] - dim])
    assert torch.equal(out, via)
    # no norm given: the plain ROW_MX projection in NBSd
    plain = pkg.kernels.torch_compatible_row_mx_qkv(
        c["packed"], w, scales, bias, HD, c["nh"], c["nh"], ct.QKVOutputLayout.NBSd)
    lin = c["lin"][..., order]
    for b in range(c["B"]):
        _close(plain[:, b].permute(1, 0, 2).reshape(c["S"], 3 * dim).cpu(), lin[b], f"shim plain batch {b}")


@pytest.mark.parametrize("batched", [False, True])
def test_kernel_mlp_wan_configuration(pkg, dev, batched):
    """The nkilib ``mlp`` kernel signature (mlp.py:53) in exactly the configuration the Wan FFN
    launches (row_mx_kernels.py:172-198: gate-less, GELU-tanh, ROW_MX, gate tensors aliasing the up
    tensors, the up bias in the reference's tiled [128, tiles, 4] form, the down bias [1, H], the
    down scale partition-expanded), against the oracle's ROW_MX MLP; the packed [K/4, N, 4] weights
    are taken as the reference passes them. Returns a one-element list, [B, S, H]."""
    ct = pkg.common_types
    S, dim, ffn = 260, 1024, 2816
    g = torch.Generator().manual_seed(21)
    h = torch.randn(S, dim, generator=g).to(torch.bfloat16)
    wu, su = _per_tensor_fp8(torch.randn(dim, ffn, generator=g) * 0.02)
    wd, sd = _per_tensor_fp8(torch.randn(ffn, dim, generator=g) * 0.02)
    bu, bd = 0.1 * torch.randn(ffn, generator=g), 0.1 * torch.randn(dim, generator=g)
    packed = pkg.adaln_modulate(h.to(dev), eps=1e-6, quant="row")
    if batched:
        packed = packed.view(2, S // 2, dim + 4)
    tiles = (ffn + 511) // 512
    bu_tiled = torch.nn.functional.pad(bu, (0, tiles * 512 - ffn)).reshape(tiles, 128, 4).permute(1, 0, 2).contiguous()
    up_w, down_w = _pack(wu).to(dev), _pack(wd).to(dev)
    up_s, down_s = torch.full((1, ffn), su, device=dev), torch.full((128, dim), sd, device=dev)
    res = pkg.kernels.mlp(
        hidden_tensor=packed, gate_proj_weights_tensor=up_w, up_proj_weights_tensor=up_w,
        down_proj_weights_tensor=down_w, normalization_weights_tensor=None, gate_proj_bias_tensor=bu_tiled.to(dev),
        up_proj_bias_tensor=bu_tiled.to(dev), down_proj_bias_tensor=bd.to(dev)[None], normalization_bias_tensor=None,
        fused_add_tensor=None, store_fused_add_result=False, activation_fn=ct.ActFnType.GELU_Tanh_Approx,
        normalization_type=ct.NormType.NO_NORM, quantization_type=ct.QuantizationType.ROW_MX, gate_w_scale=up_s,
        up_w_scale=up_s, down_w_scale=down_s, gate_up_in_scale=None, down_in_scale=None, quant_clipping_bound=None,
        output_dtype="bfloat16", store_output_in_sbuf=False, eps=1e-6, skip_gate_proj=True,
        use_tkg_gate_up_proj_column_tiling=False, use_tkg_down_proj_column_tiling=False,
        use_tkg_down_proj_optimized_layout=False, gate_clamp_upper_limit=None, gate_clamp_lower_limit=None,
        up_clamp_upper_limit=None, up_clamp_lower_limit=None, force_cte_mode=True, dtype_mode=ct.DtypeMode.AUTO,
        gate_up_w_layout=ct.MLPGateUpWeightLayout.H_X4_INNERMOST,
    )
    assert isinstance(res, list) and len(res) == 1
    out = res[0]
    assert out.shape == ((2, S // 2, dim) if batched else (1, S, dim)) and out.dtype == torch.bfloat16
    up = _row_mx_oracle(packed, wu, np.full(ffn, su, np.float32), bu.numpy())
    gel = og.gelu_tanh(up).float().to(torch.bfloat16).float().numpy()
    ic, isc = omx.mx_quantize(gel)
    wdc = wd.view(torch.uint8).t().contiguous().numpy()
    ref = og.mx_gemm(ic, isc, wdc, np.full((dim, ffn // 32), 127, np.uint8), bias=bd.numpy(),
                     col_scale=np.full(dim, sd, np.float32))
    _close(out.cpu().view(S, dim), ref, "kernels.mlp")
