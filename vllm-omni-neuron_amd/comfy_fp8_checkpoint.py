"""ComfyUI FP8-scaled Wan2.2 checkpoints -> the MXFP8 GEMM layout of this package.

Counterpart of the reference's checkpoint bookkeeping
(vllm_omni_neuron/diffusion/quantization/comfy_fp8_checkpoint.py) and of its ROW_MX weight loaders
(row_mx_loaders.py). The public names below keep the reference's: header reader (:68-78), model
parameter -> checkpoint key mappings (:115-284) and validation (:287-321).

The file format (``Comfy-Org/Wan_2.2_ComfyUI_Repackaged``, ``split_files/diffusion_models/
wan2.2_t2v_{high,low}_noise_14B_fp8_scaled.safetensors``) stores every quantized linear as

    <prefix>.weight        F8_E4M3 [out, in]   per-tensor absmax quantized codes
    <prefix>.scale_weight  F32     [] or [1]   the tensor's dequant scale
    <prefix>.scale_input   F32                 activation calibration (unused)
    <prefix>.bias          F16     [out]

with native Wan names (``self_attn.{q,k,v,o}``, ``cross_attn.*``, ``ffn.{0,2}``), the
cross-attention LayerNorm under ``norm3`` and the block modulation under ``modulation``.

How a checkpoint becomes GEMM operands here. The reference's native path keeps the checkpoint's fp8
codes, expands each tensor's scalar scale to one fp32 scale per output channel, and runs its
projections with neutral MX block scales (row_mx_loaders.py:115-140, 194-260; the ROW_MX recipe,
qkv_cte.py:3996-4021). The MXFP8 GEMM here has exactly that operand set: ``MXWeight`` codes
``[N, K]`` (the checkpoint's ``[out, in]`` storage, so no transpose), e8m0 block scales fixed at
127 (2^0), a per-output-channel fp32 ``col_scale`` applied in the epilogue, and an fp32 bias. The
codes are therefore not re-quantized and the dequantized weight is reproduced bit for bit.
Two reference steps have no counterpart: the Q/K column de-interleave
(row_mx_loaders.py:26-71; this package's RoPE rotates Wan's interleaved pairs directly) and
the Neuron SBUF byte packing (``qkv_weight_pack_3d``, ``mx_shuffle_o_proj``).

Reading is host work (safetensors, no pickle); the tensors are then copied to the GPU once.
"""

from __future__ import annotations

import json
import struct
from collections.abc import Collection, Mapping
from typing import NamedTuple

import torch

from .block import BlockWeights
from .row_mx_kernels import MXWeight

#: Files under :data:`FP8_CHECKPOINT_SUBDIR` and the expert each one feeds (high noise first).
FP8_CHECKPOINT_FILES: dict[str, str] = {
    "transformer": "wan2.2_t2v_high_noise_14B_fp8_scaled.safetensors",
    "transformer_2": "wan2.2_t2v_low_noise_14B_fp8_scaled.safetensors",
}
FP8_CHECKPOINT_SUBDIR = "split_files/diffusion_models"
#: safetensors dtype string of the quantized weights
FP8_DTYPE_STR = "F8_E4M3"
NUM_BLOCKS = 40
SUPPORTED_NATIVE_FP8_MODULES = frozenset({"attn1", "attn2", "ffn"})

_NEUTRAL_MX_SCALE = 127  # e8m0 code of 2^0
_MX_BLOCK = 32


class Fp8CheckpointError(RuntimeError):
    """The file is not a Wan2.2 ComfyUI FP8-scaled checkpoint of the expected shape."""


def read_safetensors_header(path: str) -> dict[str, dict]:
    """The JSON header of a ``.safetensors`` file, ``{name: {dtype, shape, data_offsets}}``,
    without ``__metadata__``. The format is an 8-byte little-endian header length followed by the
    UTF-8 JSON header; nothing else of the file is read."""
    with open(path, "rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise Fp8CheckpointError(f"{path}: too short for a safetensors header")
        (n,) = struct.unpack("<Q", raw)
        header = json.loads(fh.read(n).decode("utf-8"))
    header.pop("__metadata__", None)
    return header


# ------------------------------------------------------------------------------------------------
# Name mapping (model parameter -> checkpoint key or keys)
# ------------------------------------------------------------------------------------------------

#: Top-level quantized linears: ComfyUI leaf -> Diffusers-style model prefix.
FP8_TOP_LINEAR_MAP: dict[str, str] = {
    "time_embedding.0": "condition_embedder.time_embedder.linear_1",
    "time_embedding.2": "condition_embedder.time_embedder.linear_2",
    "time_projection.1": "condition_embedder.time_proj",
    "text_embedding.0": "condition_embedder.text_embedder.linear_1",
    "text_embedding.2": "condition_embedder.text_embedder.linear_2",
    "head.head": "proj_out",
}

# The quantized projections of one block: model module, model projection, and the checkpoint
# linears whose output channels it concatenates (the fused self-attention QKV takes three).
_PROJECTIONS: tuple[tuple[str, str, tuple[str, ...]], ...] = (
    ("attn1", "qkv", ("self_attn.q", "self_attn.k", "self_attn.v")),
    ("attn1", "o", ("self_attn.o",)),
    ("attn2", "q", ("cross_attn.q",)),
    ("attn2", "k", ("cross_attn.k",)),
    ("attn2", "v", ("cross_attn.v",)),
    ("attn2", "o", ("cross_attn.o",)),
    ("ffn", "up", ("ffn.0",)),
    ("ffn", "down", ("ffn.2",)),
)
_SELF_QKV = ("q", "k", "v")
# Per-block plain tensors: model leaf -> checkpoint leaf (the three renames are the norm2/norm3 pair
# and modulation -> scale_shift_table).
_BLOCK_PLAIN = {
    "attn1.norm_q.weight": "self_attn.norm_q.weight",
    "attn1.norm_k.weight": "self_attn.norm_k.weight",
    "attn2.norm_q.weight": "cross_attn.norm_q.weight",
    "attn2.norm_k.weight": "cross_attn.norm_k.weight",
    "norm2.weight": "norm3.weight",
    "norm2.bias": "norm3.bias",
    "scale_shift_table": "modulation",
}
# What every quantized linear must hold: leaf -> (safetensors dtype, accepted shapes or a rank).
_QUANTIZED_LEAVES = {
    "weight": (FP8_DTYPE_STR, 2),
    "scale_weight": ("F32", ([], [1])),
}


def _check_native(native_fp8_modules: Collection[str]) -> frozenset:
    native = frozenset(native_fp8_modules)
    bad = native - SUPPORTED_NATIVE_FP8_MODULES
    if bad:
        raise ValueError(f"unsupported native FP8 modules: {sorted(bad)}")
    return native


def _block_projections(num_layers: int):
    """(model parameter prefix ``blocks.i.<module>.<proj>_proj``, module, checkpoint prefixes)."""
    for i in range(num_layers):
        for module, proj, sources in _PROJECTIONS:
            yield f"blocks.{i}.{module}.{proj}_proj", module, tuple(f"blocks.{i}.{src}" for src in sources)


def quantized_linear_prefixes(num_layers: int = NUM_BLOCKS) -> list[str]:
    """Checkpoint prefixes of every FP8 linear the model consumes (per block, then the top level)."""
    out = [src for _, _, sources in _block_projections(num_layers) for src in sources]
    return out + list(FP8_TOP_LINEAR_MAP)


def fp8_transformed_parameter_names(num_layers: int = NUM_BLOCKS,
                                    native_fp8_modules: Collection[str] = ()) -> list[str]:
    """Model parameters filled from quantized checkpoint tensors: the weight of every projection,
    and for the modules loaded natively (codes kept) also their per-channel ``*_w_scale``."""
    native = _check_native(native_fp8_modules)
    names = [f"{prefix}_weight" for prefix, _, _ in _block_projections(num_layers)]
    names += [f"{prefix}_w_scale" for prefix, module, _ in _block_projections(num_layers) if module in native]
    return names + [f"{model}.weight" for model in FP8_TOP_LINEAR_MAP.values()]


def build_fp8_dequant_mappings(num_layers: int = NUM_BLOCKS) -> dict[str, str | list[str]]:
    """Model parameter -> checkpoint key(s) when every projection is dequantized at load.

    A quantized weight maps to ``[weight, scale_weight]`` (the fused self-attention QKV to the six
    keys ``[qW, qS, kW, kS, vW, vS]``); biases, norms and modulation map to one key each.
    """
    m: dict[str, str | list[str]] = {}
    for prefix, _, sources in _block_projections(num_layers):
        m[f"{prefix}_weight"] = [f"{src}.{leaf}" for src in sources for leaf in ("weight", "scale_weight")]
        biases = [f"{src}.bias" for src in sources]
        m[f"{prefix}_bias"] = biases if len(biases) > 1 else biases[0]
    for i in range(num_layers):
        for model_leaf, ckpt_leaf in _BLOCK_PLAIN.items():
            m[f"blocks.{i}.{model_leaf}"] = f"blocks.{i}.{ckpt_leaf}"
    m["patch_embedding.weight"] = "patch_embedding.weight"
    m["patch_embedding.bias"] = "patch_embedding.bias"
    m["scale_shift_table"] = "head.modulation"
    for leaf, prefix in FP8_TOP_LINEAR_MAP.items():
        m[f"{prefix}.weight"] = [f"{leaf}.weight", f"{leaf}.scale_weight"]
        m[f"{prefix}.bias"] = f"{leaf}.bias"
    return m


def build_fp8_mappings(num_layers: int = NUM_BLOCKS,
                       native_fp8_modules: Collection[str] = ()) -> dict[str, str | list[str]]:
    """As :func:`build_fp8_dequant_mappings`, but for the natively loaded modules the weight maps
    to its code tensor(s) only and a separate ``*_w_scale`` parameter to its scale key(s)."""
    native = _check_native(native_fp8_modules)
    m = build_fp8_dequant_mappings(num_layers)
    for prefix, module, sources in _block_projections(num_layers):
        if module not in native:
            continue
        codes = [f"{src}.weight" for src in sources]
        scales = [f"{src}.scale_weight" for src in sources]
        m[f"{prefix}_weight"] = codes if len(codes) > 1 else codes[0]
        m[f"{prefix}_w_scale"] = scales if len(scales) > 1 else scales[0]
    return m


def _leaf_problems(header: Mapping[str, dict], key: str, dtype: str, shape_rule) -> list[str]:
    entry = header.get(key)
    if entry is None:
        return [f"{key}: missing tensor"]
    problems = []
    if entry.get("dtype") != dtype:
        problems.append(f"{key}: stored as {entry.get('dtype')}, the format requires {dtype}")
    shape = entry.get("shape")
    if isinstance(shape_rule, int):
        if not isinstance(shape, list) or len(shape) != shape_rule:
            problems.append(f"{key}: shape {shape} is not a 2-D [out, in] matrix")
    elif shape not in shape_rule:
        problems.append(f"{key}: shape {shape} is not a single scalar")
    return problems


def validate_fp8_checkpoint(header: Mapping[str, dict], num_layers: int = NUM_BLOCKS) -> None:
    """Check the header against the format: every quantized linear the model consumes has a 2-D
    ``F8_E4M3`` ``weight`` and a scalar ``F32`` ``scale_weight``. Raises :class:`Fp8CheckpointError`
    listing every problem found (a reduced-layer file is checked against its own layer count)."""
    problems = []
    for prefix in quantized_linear_prefixes(num_layers):
        for leaf, (dtype, shape_rule) in _QUANTIZED_LEAVES.items():
            problems += _leaf_problems(header, f"{prefix}.{leaf}", dtype, shape_rule)
    if problems:
        shown = "; ".join(problems[:8]) + (f"; ... ({len(problems)} problems)" if len(problems) > 8 else "")
        raise Fp8CheckpointError(f"not a Wan2.2 FP8-scaled checkpoint with {num_layers} blocks: {shown}")


# ------------------------------------------------------------------------------------------------
# Loading a block into the GEMM layout
# ------------------------------------------------------------------------------------------------


class HostProjection(NamedTuple):
    """One projection in GEMM layout, still on the host: e4m3fn codes ``[N, K]`` (as uint8),
    fp32 ``col_scale [N]`` (the checkpoint scalars expanded per output channel), fp32 ``bias [N]``."""

    codes: torch.Tensor
    col_scale: torch.Tensor
    bias: torch.Tensor


def _scalar(t: torch.Tensor, key: str) -> float:
    if t.numel() != 1:
        raise Fp8CheckpointError(f"{key} must be scalar, got {t.numel()} elements")
    return float(t.reshape(()).to(torch.float32))


def _codes(t: torch.Tensor, key: str) -> torch.Tensor:
    if t.dtype != torch.float8_e4m3fn or t.dim() != 2:
        raise Fp8CheckpointError(f"{key} must be 2-D float8_e4m3fn, got {t.dtype} {tuple(t.shape)}")
    if t.shape[1] % _MX_BLOCK:
        raise Fp8CheckpointError(f"{key}: in_features {t.shape[1]} is not a multiple of {_MX_BLOCK}")
    return t.contiguous().view(torch.uint8)


def host_projection(get, prefixes: list[str]) -> HostProjection:
    """The projection whose output channels are the concatenation of the checkpoint linears
    ``prefixes`` (one for a plain projection, three for the fused ``[Q | K | V]``)."""
    codes, scales, biases = [], [], []
    for p in prefixes:
        c = _codes(get(f"{p}.weight"), f"{p}.weight")
        s = _scalar(get(f"{p}.scale_weight"), f"{p}.scale_weight")
        b = get(f"{p}.bias").reshape(-1).to(torch.float32)
        if b.numel() != c.shape[0]:
            raise Fp8CheckpointError(f"{p}.bias has {b.numel()} elements for {c.shape[0]} outputs")
        codes.append(c)
        scales.append(torch.full((c.shape[0],), s, dtype=torch.float32))
        biases.append(b)
    if len({c.shape[1] for c in codes}) != 1:
        raise Fp8CheckpointError(f"{prefixes}: fused projections disagree on in_features")
    return HostProjection(torch.cat(codes).contiguous(), torch.cat(scales), torch.cat(biases))


def host_block_tensors(get, index: int) -> dict[str, object]:
    """Block ``index`` read through ``get(key) -> tensor`` (host tensors): the eight projections as
    :class:`HostProjection` and the norms and modulation as fp32."""
    b = f"blocks.{index}"
    out: dict[str, object] = {
        "qkv": host_projection(get, [f"{b}.self_attn.{p}" for p in _SELF_QKV]),
        "o": host_projection(get, [f"{b}.self_attn.o"]),
        "q2": host_projection(get, [f"{b}.cross_attn.q"]),
        "k2": host_projection(get, [f"{b}.cross_attn.k"]),
        "v2": host_projection(get, [f"{b}.cross_attn.v"]),
        "o2": host_projection(get, [f"{b}.cross_attn.o"]),
        "up": host_projection(get, [f"{b}.ffn.0"]),
        "down": host_projection(get, [f"{b}.ffn.2"]),
    }
    f32 = lambda key: get(f"{b}.{key}").to(torch.float32).contiguous()  # noqa: E731
    out["norm_q"] = f32("self_attn.norm_q.weight").reshape(-1)
    out["norm_k"] = f32("self_attn.norm_k.weight").reshape(-1)
    out["norm_q2"] = f32("cross_attn.norm_q.weight").reshape(-1)
    out["norm_k2"] = f32("cross_attn.norm_k.weight").reshape(-1)
    out["norm2_weight"] = f32("norm3.weight").reshape(-1)
    out["norm2_bias"] = f32("norm3.bias").reshape(-1)
    mod = f32("modulation")
    if mod.numel() % 6:
        raise Fp8CheckpointError(f"{b}.modulation has {mod.numel()} elements, not 6 x dim")
    out["scale_shift_table"] = mod.reshape(6, -1)
    return out


def _to_device(p: HostProjection, device) -> MXWeight:
    n, k = p.codes.shape
    codes = p.codes.to(device)
    scales = torch.full((n, k // _MX_BLOCK), _NEUTRAL_MX_SCALE, dtype=torch.uint8, device=device)
    return MXWeight(codes, scales, p.col_scale.to(device), p.bias.to(device))


def block_weights_from_host(t: Mapping[str, object], device) -> BlockWeights:
    """Copy one block's host tensors to ``device`` as the :class:`BlockWeights` the block runs on."""
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(f"block weights go to a ROCm GPU, not {dev}; the kernels never run on the host")
    proj = {k: _to_device(t[k], dev) for k in ("qkv", "o", "q2", "k2", "v2", "o2", "up", "down")}
    vec = {k: t[k].to(dev) for k in ("scale_shift_table", "norm_q", "norm_k", "norm2_weight", "norm2_bias",
                                     "norm_q2", "norm_k2")}
    return BlockWeights(vec["scale_shift_table"], proj["qkv"], vec["norm_q"], vec["norm_k"], proj["o"],
                        vec["norm2_weight"], vec["norm2_bias"], proj["q2"], proj["k2"], proj["v2"], vec["norm_q2"],
                        vec["norm_k2"], proj["o2"], proj["up"], proj["down"])


class ComfyFp8Checkpoint:
    """An open ComfyUI FP8 checkpoint file: validated header, per-tensor reads (memory-mapped by
    safetensors; nothing is unpickled), and per-block conversion to :class:`BlockWeights`."""

    def __init__(self, path: str, num_layers: int = NUM_BLOCKS):
        from safetensors import safe_open

        self.path = path
        self.num_layers = num_layers
        self.header = read_safetensors_header(path)
        validate_fp8_checkpoint(self.header, num_layers)
        self._file = safe_open(path, framework="pt", device="cpu")

    def get(self, key: str) -> torch.Tensor:
        if key not in self.header:
            raise Fp8CheckpointError(f"{self.path}: missing tensor {key}")
        return self._file.get_tensor(key)

    def host_block(self, index: int) -> dict[str, object]:
        if not 0 <= index < self.num_layers:
            raise IndexError(f"block {index} out of range [0, {self.num_layers})")
        return host_block_tensors(self.get, index)

    def block_weights(self, index: int, device) -> BlockWeights:
        return block_weights_from_host(self.host_block(index), device)

    def all_block_weights(self, device) -> list[BlockWeights]:
        """All blocks on ``device`` (≈14.4 GB of codes for the 14B expert), one block's host copy at
        a time."""
        return [self.block_weights(i, device) for i in range(self.num_layers)]
