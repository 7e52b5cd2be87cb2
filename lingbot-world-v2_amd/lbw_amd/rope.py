"""Wan 3-D RoPE tables for the fused q/k kernel.

The reference builds full ``[f*h*w, D/2]`` cos/sin grids on the CPU every forward and copies
them to the device (wan/modules/model_fast.py:858-931). The grid is a column concatenation
of per-axis angle rows (frame rows start at ``start_frame``), so the fused kernel only needs
the three per-axis tables: ``f*s0 + h*s1 + w*s1`` cos/sin pairs (22 KB at 720p instead of
1.8 MB), which it keeps in LDS and indexes by the token's (frame, row, column). The values
are computed exactly as the reference computes its grid: fp32 angles from
``rope_params`` (wan/modules/model.py:47-53) and torch's fp32 cos/sin on the CPU.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

MAX_LATENT_FRAMES = 2880  # wan/modules/model.py:44


def rope_params(max_seq_len: int, dim: int, theta: float = 10000.0) -> torch.Tensor:
    """wan/modules/model.py:47-53."""
    assert dim % 2 == 0
    return torch.outer(torch.arange(max_seq_len).float(),
                       1.0 / torch.pow(theta, torch.arange(0, dim, 2).float().div(dim)))


def wan_rope_freqs(head_dim: int = 128, max_frames: int = MAX_LATENT_FRAMES) -> torch.Tensor:
    """wan/modules/model.py:480-487: ``[max_frames, head_dim/2]`` fp32."""
    d = head_dim
    return torch.cat([rope_params(max_frames, d - 4 * (d // 6)),
                      rope_params(max_frames, 2 * (d // 6)),
                      rope_params(max_frames, 2 * (d // 6))], dim=1)


def axis_split(c: int):
    """model_fast.py:889-891: pairs per axis (frame, height, width)."""
    return c - 2 * (c // 3), c // 3, c // 3


@dataclass(frozen=True)
class RopeTables:
    """Packed per-axis tables on a device: cos_t, sin_t [f, s0]; cos_h, sin_h [h, s1];
    cos_w, sin_w [w, s1] (fp32, in that order)."""
    packed: torch.Tensor
    f: int
    h: int
    w: int
    s0: int
    s1: int
    start_frame: int

    @property
    def tokens(self) -> int:
        return self.f * self.h * self.w


_CACHE: dict = {}


def causal_rope_tables(freqs: torch.Tensor, grid, start_frame: int = 0,
                       device=None) -> RopeTables:
    """Per-axis tables for one chunk grid ``(f, h, w)`` at ``start_frame``, memoised on
    (freqs, grid, start_frame, device) as causal_rope_grids is (model_fast.py:858-876)."""
    f, h, w = (int(x) for x in grid)
    device = torch.device(device) if device is not None else torch.device("cpu")
    key = (id(freqs), tuple(freqs.shape), f, h, w, int(start_frame), str(device))
    hit = _CACHE.get(key)
    if hit is not None and hit[0] is freqs:
        return hit[1]
    c = freqs.size(1)
    s0, s1, _ = axis_split(c)
    if start_frame + f > freqs.shape[0]:
        raise ValueError(f"frames {start_frame}..{start_frame + f} exceed the RoPE table "
                         f"({freqs.shape[0]} rows)")
    fs = freqs.detach().cpu().float().split([s0, s1, s1], dim=1)
    at = fs[0][start_frame:start_frame + f]
    ah, aw = fs[1][:h], fs[2][:w]
    packed = torch.cat([torch.cos(at).flatten(), torch.sin(at).flatten(),
                        torch.cos(ah).flatten(), torch.sin(ah).flatten(),
                        torch.cos(aw).flatten(), torch.sin(aw).flatten()]).contiguous()
    t = RopeTables(packed.to(device), f, h, w, s0, s1, int(start_frame))
    _CACHE[key] = (freqs, t)
    return t
