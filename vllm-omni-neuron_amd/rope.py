"""Wan 3D rotary-embedding tables, built on the GPU.

Drop-in for ``WanRotaryPosEmbed`` (vllm_omni_neuron/diffusion/layers/rope.py:37-114), which the
transformer calls once per forward (diffusion/models/wan2_2/wan2_2_transformer.py:1757): the same
constructor arguments, and ``forward(hidden_states [B, C, F, H, W])`` returns the interleaved
``(freqs_cos, freqs_sin)``, fp32 ``[1, S, 1, head_dim]`` with S = (F/p_t)(H/p_h)(W/p_w), on the
hidden states' device. The tables come from the ``wanmi_rope_tables`` kernel: pair j of an axis of
dim d (time 44, height 42, width 42 channels at head_dim 128) at position p has the angle
``p / theta^(2j/d)`` in fp64, cast to fp32 after cos / sin, exactly as the reference computes it.

:meth:`WanRotaryPosEmbed.pair_tables` gives the ``[S, head_dim/2]`` one-angle-per-pair tables the
attention kernels read, and :meth:`rotate_half_caches` the ``cat([base, base])`` caches of the
reference's fused QKV path (row_mx_modules.py:51-76).
"""

from __future__ import annotations

import torch

from . import _lib

_LAYOUT = {"pairs": 0, "interleaved": 1, "rotate_half": 2}


def _check_axis_split(head_dim: int) -> None:
    """The reference builds its axis tables with widths ``[hd - 4 (hd // 6), 2 (hd // 6), 2 (hd // 6)]``
    (rope.py:54-55) but slices them in ``forward`` at ``[hd - 2 (hd // 3), hd // 3, hd // 3]``
    (rope.py:91-95). The two agree only when ``hd // 3 == 2 (hd // 6)`` (every even head_dim except
    those of the form 6k + 4, such as 64, 112 and 256); otherwise the reference's slices cut pairs
    apart and mix axes, which no per-pair table reproduces, so such head_dims are refused."""
    if head_dim // 3 != 2 * (head_dim // 6):
        raise NotImplementedError(
            f"head_dim={head_dim}: the reference's axis widths 2*(head_dim//6)={2 * (head_dim // 6)} and its forward's "
            f"split head_dim//3={head_dim // 3} disagree; only head_dims where they agree (e.g. 128) are built")


def rope_tables(grid, *, head_dim: int = 128, max_seq_len: int = 1024, theta: float = 10000.0,
                layout: str = "pairs", device="cuda"):
    """``(cos, sin)`` fp32 for the latent patch grid ``(F, H, W)`` in raster order: ``[S, head_dim/2]``
    (``layout="pairs"``) or ``[S, head_dim]`` (``"interleaved"``: each angle twice, the reference's
    freqs layout; ``"rotate_half"``: ``cat([base, base])``)."""
    if layout not in _LAYOUT:
        raise ValueError(f"unknown layout {layout!r}")
    _check_axis_split(head_dim)
    F_, H_, W_ = (int(v) for v in grid)
    if min(F_, H_, W_) < 0:
        raise ValueError(f"grid sizes must be non-negative, got {grid}")
    if max(F_, H_, W_) > max_seq_len:
        raise ValueError(f"grid {tuple(grid)} exceeds max_seq_len={max_seq_len}")
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(f"rope tables are built on a ROCm GPU, not {dev}; no CPU fallback")
    lib = _lib.load()
    S = F_ * H_ * W_
    width = head_dim // 2 if layout == "pairs" else head_dim
    cos = torch.empty((S, width), dtype=torch.float32, device=dev)
    sin = torch.empty((S, width), dtype=torch.float32, device=dev)
    st = lib.wanmi_rope_tables(F_, H_, W_, int(head_dim), int(max_seq_len), float(theta), _LAYOUT[layout],
                               _lib.ptr(cos), _lib.ptr(sin), _lib.stream_of(cos))
    _lib.check(st, "wanmi_rope_tables")
    return cos, sin


class WanRotaryPosEmbed(torch.nn.Module):
    """Rotary position tables for video latents (time + height + width axes)."""

    def __init__(self, attention_head_dim: int, patch_size: tuple[int, int, int], max_seq_len: int,
                 theta: float = 10000.0):
        super().__init__()
        _check_axis_split(attention_head_dim)
        self.attention_head_dim = attention_head_dim
        self.patch_size = tuple(patch_size)
        self.max_seq_len = max_seq_len
        self.theta = theta

    def grid(self, hidden_states: torch.Tensor) -> tuple[int, int, int]:
        """Latent patch grid of ``hidden_states [B, C, F, H, W]`` (rope.py:86-88)."""
        _, _, f, h, w = hidden_states.shape
        p_t, p_h, p_w = self.patch_size
        return f // p_t, h // p_h, w // p_w

    def _tables(self, grid, layout, device):
        return rope_tables(grid, head_dim=self.attention_head_dim, max_seq_len=self.max_seq_len, theta=self.theta,
                           layout=layout, device=device)

    def forward(self, hidden_states: torch.Tensor):
        """``(freqs_cos, freqs_sin)`` fp32 ``[1, S, 1, head_dim]`` (interleaved), on the input's device."""
        grid = self.grid(hidden_states)
        cos, sin = self._tables(grid, "interleaved", hidden_states.device)
        return cos.view(1, -1, 1, self.attention_head_dim), sin.view(1, -1, 1, self.attention_head_dim)

    def pair_tables(self, grid, device="cuda"):
        """``(cos, sin)`` fp32 ``[S, head_dim/2]``: angle i of pair i, the attention kernels' tables."""
        return self._tables(grid, "pairs", device)

    def rotate_half_caches(self, grid, device="cuda"):
        """``(cos_cache, sin_cache)`` fp32 ``[S, head_dim]`` = ``cat([base, base])``."""
        return self._tables(grid, "rotate_half", device)
