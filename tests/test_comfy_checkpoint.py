"""ComfyUI FP8 checkpoint bookkeeping and host-side conversion (CPU).

Follows the reference's contract for the format (vllm_omni_neuron/diffusion/quantization/
comfy_fp8_checkpoint.py): the name mappings consume every checkpoint tensor the block needs
exactly once, with the norm3 -> norm2 and modulation -> scale_shift_table renames; validation
rejects a wrong dtype, rank or a non-scalar / missing scale; the native split hands weights and
scales to separate parameters. The conversion to the GEMM layout is checked bit for bit: the
codes are the checkpoint's bytes, concatenated [Q | K | V] for the fused projection, block scales
neutral, and codes * col_scale reproduces the checkpoint's dequantized weight exactly.
"""

import copy
import json
import struct

import pytest
import torch

from comfy_ckpt import BLOCK_LINEARS, TOP_LINEARS, write_checkpoint


@pytest.fixture(scope="module")
def ck(pkg):
    return pkg.comfy_fp8_checkpoint


@pytest.fixture(scope="module")
def ckpt2(tmp_path_factory):
    path = tmp_path_factory.mktemp("ckpt") / "wan_fp8_scaled.safetensors"
    tensors = write_checkpoint(path, num_layers=2, dim=256, ffn=512, seed=3)
    return path, tensors


def _header(tensors):
    dt = {torch.float8_e4m3fn: "F8_E4M3", torch.float32: "F32", torch.float16: "F16"}
    return {k: {"dtype": dt[v.dtype], "shape": list(v.shape)} for k, v in tensors.items()}


def test_key_counts_match_the_documented_format(ckpt2):
    _, t = ckpt2
    per_block = [k for k in t if k.startswith("blocks.0.")]
    top = [k for k in t if not k.startswith("blocks.")]
    assert len(per_block) == 47 and len(top) == 28
    assert sum(v.dtype == torch.float8_e4m3fn for v in t.values()) == 2 * 10 + 6 + 1


def test_header_reader(ck, ckpt2):
    path, t = ckpt2
    h = ck.read_safetensors_header(str(path))
    assert "__metadata__" not in h
    assert {k: (v["dtype"], v["shape"]) for k, v in h.items()} == {k: (v["dtype"], v["shape"])
                                                                    for k, v in _header(t).items()}
    # the raw format: 8-byte little-endian length, then the JSON header
    raw = path.read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    assert json.loads(raw[8 : 8 + n])["__metadata__"] == {"format": "pt"}


def test_mappings_consume_each_tensor_once(ck, ckpt2):
    _, t = ckpt2
    m = ck.build_fp8_dequant_mappings(num_layers=2)
    sources = []
    for v in m.values():
        sources += v if isinstance(v, list) else [v]
    assert len(sources) == len(set(sources)), "a checkpoint tensor feeds two parameters"
    unused = {k for k in t if k.endswith(".scale_input")} | {"scaled_fp8"}
    assert set(sources) == set(t) - unused
    # the three renames
    assert m["blocks.1.norm2.weight"] == "blocks.1.norm3.weight"
    assert m["blocks.1.norm2.bias"] == "blocks.1.norm3.bias"
    assert m["blocks.0.scale_shift_table"] == "blocks.0.modulation"
    assert m["scale_shift_table"] == "head.modulation"
    assert m["blocks.0.attn1.qkv_proj_weight"] == [f"blocks.0.self_attn.{p}.{leaf}" for p in "qkv"
                                                   for leaf in ("weight", "scale_weight")]
    assert m["proj_out.weight"] == ["head.head.weight", "head.head.scale_weight"]


def test_native_split_and_parameter_names(ck):
    m = ck.build_fp8_mappings(num_layers=1, native_fp8_modules={"attn1", "attn2", "ffn"})
    assert m["blocks.0.attn1.qkv_proj_weight"] == [f"blocks.0.self_attn.{p}.weight" for p in "qkv"]
    assert m["blocks.0.attn1.qkv_proj_w_scale"] == [f"blocks.0.self_attn.{p}.scale_weight" for p in "qkv"]
    assert m["blocks.0.attn2.k_proj_weight"] == "blocks.0.cross_attn.k.weight"
    assert m["blocks.0.attn2.k_proj_w_scale"] == "blocks.0.cross_attn.k.scale_weight"
    assert m["blocks.0.ffn.down_proj_w_scale"] == "blocks.0.ffn.2.scale_weight"
    # modules loaded by dequantization keep the [weight, scale] pair
    m1 = ck.build_fp8_mappings(num_layers=1, native_fp8_modules={"ffn"})
    assert m1["blocks.0.attn1.o_proj_weight"] == ["blocks.0.self_attn.o.weight", "blocks.0.self_attn.o.scale_weight"]
    names = ck.fp8_transformed_parameter_names(num_layers=3, native_fp8_modules={"attn1", "attn2", "ffn"})
    assert len(names) == len(set(names)) == 3 * (8 + 2 + 4 + 2) + len(TOP_LINEARS)
    assert set(names) <= set(ck.build_fp8_mappings(num_layers=3, native_fp8_modules={"attn1", "attn2", "ffn"}))
    with pytest.raises(ValueError):
        ck.build_fp8_mappings(num_layers=1, native_fp8_modules={"norm"})
    with pytest.raises(ValueError):
        ck.fp8_transformed_parameter_names(1, native_fp8_modules={"attn3"})


def test_validate(ck, ckpt2):
    _, t = ckpt2
    h = _header(t)
    ck.validate_fp8_checkpoint(h, num_layers=2)
    cases = [
        ("blocks.1.ffn.0.weight", {"dtype": "BF16"}, "blocks.1.ffn.0.weight: stored as BF16, the format requires F8_E4M3"),
        ("blocks.0.cross_attn.o.weight", {"shape": [256, 256, 1]}, "cross_attn.o.weight: shape .* is not a 2-D"),
        ("blocks.0.self_attn.k.scale_weight", {"shape": [256]}, "self_attn.k.scale_weight: shape .* not a single scalar"),
        ("text_embedding.2.scale_weight", {"dtype": "F16"}, "stored as F16, the format requires F32"),
    ]
    for key, patch, msg in cases:
        bad = copy.deepcopy(h)
        bad[key].update(patch)
        with pytest.raises(ck.Fp8CheckpointError, match=msg):
            ck.validate_fp8_checkpoint(bad, num_layers=2)
    for key in ("blocks.1.self_attn.v.weight", "head.head.scale_weight"):
        bad = copy.deepcopy(h)
        del bad[key]
        with pytest.raises(ck.Fp8CheckpointError, match="missing"):
            ck.validate_fp8_checkpoint(bad, num_layers=2)
    # a reduced-layer file validates against its own layer count only; every problem is listed
    with pytest.raises(ck.Fp8CheckpointError, match="blocks.2.self_attn.q.weight: missing") as exc:
        ck.validate_fp8_checkpoint(h, num_layers=3)
    assert "20 problems" in str(exc.value)  # 10 checkpoint linears x 2 leaves of block 2, 8 shown


def test_host_block_layout_is_exact(ck, ckpt2):
    path, t = ckpt2
    f = ck.ComfyFp8Checkpoint(str(path), num_layers=2)
    blk = f.host_block(1)
    b = "blocks.1"
    projections = {
        "qkv": [f"{b}.self_attn.{p}" for p in "qkv"], "o": [f"{b}.self_attn.o"], "q2": [f"{b}.cross_attn.q"],
        "k2": [f"{b}.cross_attn.k"], "v2": [f"{b}.cross_attn.v"], "o2": [f"{b}.cross_attn.o"],
        "up": [f"{b}.ffn.0"], "down": [f"{b}.ffn.2"],
    }
    assert {p.split(".", 2)[2] for ps in projections.values() for p in ps} == set(BLOCK_LINEARS)
    for name, prefixes in projections.items():
        p = blk[name]
        ref_codes = torch.cat([t[f"{x}.weight"].view(torch.uint8) for x in prefixes])
        assert p.codes.dtype == torch.uint8 and torch.equal(p.codes, ref_codes), name
        widths = [t[f"{x}.weight"].shape[0] for x in prefixes]
        ref_cs = torch.cat([torch.full((w,), float(t[f"{x}.scale_weight"])) for x, w in zip(prefixes, widths)])
        assert torch.equal(p.col_scale, ref_cs), name
        assert torch.equal(p.bias, torch.cat([t[f"{x}.bias"].float() for x in prefixes])), name
        # GEMM-layout dequant (codes * 2^0 block scale * col_scale) == checkpoint dequant, bit for bit
        deq = p.codes.view(torch.float8_e4m3fn).float() * p.col_scale[:, None]
        ref = torch.cat([t[f"{x}.weight"].float() * t[f"{x}.scale_weight"] for x in prefixes])
        assert torch.equal(deq, ref), name
    assert torch.equal(blk["norm2_weight"], t[f"{b}.norm3.weight"].float())
    assert torch.equal(blk["norm2_bias"], t[f"{b}.norm3.bias"].float())
    assert torch.equal(blk["norm_q2"], t[f"{b}.cross_attn.norm_q.weight"].float())
    assert torch.equal(blk["norm_k"], t[f"{b}.self_attn.norm_k.weight"].float())
    assert blk["scale_shift_table"].shape == (6, 256)
    assert torch.equal(blk["scale_shift_table"], t[f"{b}.modulation"].float().reshape(6, 256))
    with pytest.raises(IndexError):
        f.host_block(2)


def test_block_weights_go_to_a_gpu_only(ck, ckpt2):
    path, _ = ckpt2
    f = ck.ComfyFp8Checkpoint(str(path), num_layers=2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ck.block_weights_from_host(f.host_block(0), "cpu")


def test_rejects_bad_tensors(ck):
    def get(key):
        return {"x.weight": torch.zeros(8, 40, dtype=torch.float8_e4m3fn), "x.scale_weight": torch.tensor([1.0]),
                "x.bias": torch.zeros(8, dtype=torch.float16), "y.weight": torch.zeros(8, 64, dtype=torch.float16),
                "y.scale_weight": torch.tensor(1.0), "y.bias": torch.zeros(8)}[key]

    with pytest.raises(ck.Fp8CheckpointError, match="multiple of 32"):
        ck.host_projection(get, ["x"])
    with pytest.raises(ck.Fp8CheckpointError, match="float8_e4m3fn"):
        ck.host_projection(get, ["y"])
