"""Synthetic Wan2.2 ComfyUI FP8-scaled checkpoints for the loader tests.

The tensor set follows the format the reference documents for
``wan2.2_t2v_{high,low}_noise_14B_fp8_scaled.safetensors``
(vllm_omni_neuron/diffusion/quantization/comfy_fp8_checkpoint.py:8-27): per block 47 keys
(10 quantized linears x {weight F8_E4M3 [out, in], scale_weight F32 [], scale_input F32 [],
bias F16 [out]}, q/k RMSNorm gammas of both attentions, ``norm3`` weight/bias, ``modulation``
[1, 6, dim]) and 28 top-level keys (patch embedding, the six condition-embedder / head linears,
``head.modulation`` and the ``scaled_fp8`` marker). Weights are drawn N(0, std) and quantized the
way ComfyUI's scaled-fp8 files are: one absmax scale per tensor, ``codes = e4m3(W / scale)`` with
``scale = max|W| / 448``. Dimensions are parameters so the files stay small.
"""

from __future__ import annotations

import torch
from safetensors.torch import save_file

BLOCK_LINEARS = ("self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o", "cross_attn.q", "cross_attn.k",
                 "cross_attn.v", "cross_attn.o", "ffn.0", "ffn.2")
TOP_LINEARS = ("time_embedding.0", "time_embedding.2", "time_projection.1", "text_embedding.0", "text_embedding.2",
               "head.head")


def quantize_per_tensor(w: torch.Tensor):
    """bf16/fp32 [out, in] -> (e4m3fn codes, fp32 scalar scale) with the tensor's absmax at 448."""
    scale = w.float().abs().max() / 448.0
    return (w.float() / scale).to(torch.float8_e4m3fn), scale.reshape(()).to(torch.float32)


def make_tensors(num_layers: int, dim: int, ffn: int, seed: int = 0, std: float = 0.02, gamma_mean: float = 1.0):
    g = torch.Generator().manual_seed(seed)
    t: dict[str, torch.Tensor] = {}

    def linear(prefix, out_f, in_f):
        codes, scale = quantize_per_tensor(torch.randn(out_f, in_f, generator=g) * std)
        t[f"{prefix}.weight"] = codes
        t[f"{prefix}.scale_weight"] = scale
        t[f"{prefix}.scale_input"] = torch.tensor(1.0)
        t[f"{prefix}.bias"] = (torch.randn(out_f, generator=g) * std).half()

    def vec(n, mean=0.0):
        return (mean + torch.randn(n, generator=g) * std).half()

    shapes = {"ffn.0": (ffn, dim), "ffn.2": (dim, ffn)}
    for i in range(num_layers):
        b = f"blocks.{i}"
        for lin in BLOCK_LINEARS:
            linear(f"{b}.{lin}", *shapes.get(lin, (dim, dim)))
        for attn in ("self_attn", "cross_attn"):
            t[f"{b}.{attn}.norm_q.weight"] = vec(dim, gamma_mean)
            t[f"{b}.{attn}.norm_k.weight"] = vec(dim, gamma_mean)
        t[f"{b}.norm3.weight"] = vec(dim, 1.0)
        t[f"{b}.norm3.bias"] = vec(dim)
        t[f"{b}.modulation"] = (torch.randn(1, 6, dim, generator=g) * std).half()
    t["patch_embedding.weight"] = vec(dim * 16).reshape(dim, 16)
    t["patch_embedding.bias"] = vec(dim)
    for lin in TOP_LINEARS:
        linear(lin, dim, 64)
    t["head.modulation"] = (torch.randn(1, 2, dim, generator=g) * std).half()
    t["scaled_fp8"] = torch.empty(0, dtype=torch.float8_e4m3fn)
    return t


def write_checkpoint(path, num_layers: int = 1, dim: int = 256, ffn: int = 512, seed: int = 0, **kw):
    tensors = make_tensors(num_layers, dim, ffn, seed, **kw)
    save_file(tensors, str(path), metadata={"format": "pt"})
    return tensors
