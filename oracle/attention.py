"""Softmax attention, exact and constant-max -- oracle, test infrastructure only.

- ``torch_attend`` restates ``_torch_attend`` (vllm_omni_neuron/diffusion/models/wan2_2/
  wan2_2_transformer.py:640-650): ``softmax(scale Q K^T) V`` with fp32 softmax, [B, N, S, D].
- ``const_max_attention`` restates the constant-max form of the reference's ring kernel
  (kernels/nkilib/experimental/attention/attention_const_max.py:69-490 and
  ring_attention_const_max_fwd.py:559-804): per-row bound ``c_i = s ||q_i|| max_j ||k_j||``,
  ``P = exp(s q k^T - c)``, ``o = P V / max(sum P, 1e-37)``.
"""

from __future__ import annotations

import torch

SUM_FLOOR = 1e-37  # ring_attention_const_max_fwd.py:657-663


def torch_attend(q, k, v, scale, dtype=torch.float32):
    """Exact attention over [..., S, D] tensors, computed in ``dtype`` (fp32 or fp64)."""
    scores = torch.matmul(q.to(dtype) * scale, k.to(dtype).transpose(-2, -1))
    attn = torch.softmax(scores, dim=-1)
    return torch.matmul(attn, v.to(dtype))


def const_max_bound(q, k, scale):
    """c [..., Sq, 1] = scale * ||q_i|| * max_j ||k_j|| over the last two dims of [..., S, D]."""
    qn = q.double().norm(dim=-1, keepdim=True)
    kmax = k.double().norm(dim=-1).amax(dim=-1, keepdim=True).unsqueeze(-1)
    return scale * qn * kmax


def const_max_attention(q, k, v, scale, c=None, dtype=torch.float64):
    """Constant-max attention; ``c`` overrides the bound (any constant per row gives the same o)."""
    if c is None:
        c = const_max_bound(q, k, scale)
    s = torch.matmul(q.to(dtype), k.to(dtype).transpose(-2, -1)) * scale
    p = torch.exp(s - c.to(dtype))
    den = p.sum(dim=-1, keepdim=True).clamp_min(SUM_FLOOR)
    return torch.matmul(p, v.to(dtype)) / den
