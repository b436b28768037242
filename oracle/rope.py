"""Wan 3D rotary embeddings and the across-heads QK RMSNorm -- oracle, test infrastructure only.

Restates (torch on the CPU):

- ``WanRotaryPosEmbed`` (vllm_omni_neuron/diffusion/layers/rope.py:37-114): per-axis angles
  ``t * theta^(-2i/dim)`` in fp64 for dims t/h/w = 44/42/42 (head_dim 128), cos/sin cast to fp32
  and repeat-interleaved, concatenated per latent (f, h, w) position in raster order.
- ``apply_rotary_emb_wan`` (rope.py:8-34): interleaved pairs ``(x1, x2) -> (x1 cos - x2 sin,
  x1 sin + x2 cos)`` in fp32, cast back to the input dtype.
- ``DistributedRMSNorm.forward`` at tp=1 (diffusion/models/wan2_2/wan2_2_transformer.py:879-893):
  ``bf16((x / sqrt(sum(x^2)/n + eps)) * w)`` over the whole projected row (all heads).
- the rotate-half equivalence used by the reference's fused QKV kernel
  (row_mx_loaders.py:26-39 ``deinterleave_perm``; row_mx_modules.py:51-76 rotate-half caches).
"""

from __future__ import annotations

import numpy as np
import torch


def rope_axis_freqs(dim: int, max_seq_len: int, theta: float = 10000.0):
    """(cos, sin) fp32 [max_seq_len, dim], each angle repeated on two adjacent lanes (rope.py:70-83)."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    t = torch.arange(max_seq_len, dtype=torch.float64)
    freqs = torch.outer(t, freqs)
    return freqs.cos().float().repeat_interleave(2, dim=-1), freqs.sin().float().repeat_interleave(2, dim=-1)


def wan_rope(grid, head_dim: int = 128, max_seq_len: int = 1024, theta: float = 10000.0):
    """Interleaved (cos, sin) fp32 [S, head_dim] for a latent patch grid (F, H, W), S = F*H*W."""
    F_, H_, W_ = grid
    h_dim = w_dim = 2 * (head_dim // 6)
    t_dim = head_dim - h_dim - w_dim
    cos_parts, sin_parts = [], []
    for dim, n, shape in ((t_dim, F_, (F_, 1, 1)), (h_dim, H_, (1, H_, 1)), (w_dim, W_, (1, 1, W_))):
        c, s = rope_axis_freqs(dim, max_seq_len, theta)
        cos_parts.append(c[:n].view(*shape, -1).expand(F_, H_, W_, -1))
        sin_parts.append(s[:n].view(*shape, -1).expand(F_, H_, W_, -1))
    cos = torch.cat(cos_parts, dim=-1).reshape(F_ * H_ * W_, head_dim)
    sin = torch.cat(sin_parts, dim=-1).reshape(F_ * H_ * W_, head_dim)
    return cos.contiguous(), sin.contiguous()


def base_angles(cos: torch.Tensor, sin: torch.Tensor):
    """Interleaved [.., 128] tables -> one (cos, sin) per pair [.., 64] (``cos[..., 0::2]``,
    ``sin[..., 1::2]``, exactly what ``apply_rotary_emb_wan`` reads)."""
    return cos[..., 0::2].contiguous(), sin[..., 1::2].contiguous()


def apply_rotary_emb_wan(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, S, N, D]; cos/sin broadcastable to [B, S, 1, D] (interleaved). Same dtype out."""
    x1, x2 = x.unflatten(-1, (-1, 2)).unbind(-1)
    c = cos[..., 0::2]
    s = sin[..., 1::2]
    out = torch.stack((x1 * c - x2 * s, x1 * s + x2 * c), dim=-1)
    return out.flatten(-2, -1).to(x.dtype)


def rms_norm_across_heads(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """DistributedRMSNorm at tp=1 over the last dim (all heads): bf16 out."""
    xf = x.float()
    rms = torch.sqrt((xf**2).sum(dim=-1, keepdim=True) / x.shape[-1] + eps)
    return ((xf / rms) * weight.float()).to(x.dtype)


def deinterleave_perm(head_dim: int) -> torch.Tensor:
    """Channel order that turns interleaved pairs into the two rotate-half halves."""
    return torch.cat([torch.arange(0, head_dim, 2), torch.arange(1, head_dim, 2)])


def apply_rotate_half(x: torch.Tensor, cos_half: torch.Tensor, sin_half: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE with ``cat([base, base])`` caches (the reference kernel's convention)."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    rot = torch.cat([-x2, x1], dim=-1)
    return (x.float() * cos_half + rot.float() * sin_half).to(x.dtype)
