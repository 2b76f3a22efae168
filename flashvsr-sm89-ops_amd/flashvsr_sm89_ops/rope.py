"""Wan 2.1 3-D rotary frequencies for a (frames, height, width) token grid.

The DiT's head_dim is split over (f, h, w) as head_dim-4*(head_dim//6),
2*(head_dim//6), 2*(head_dim//6) dims (44/42/42 for 128); each axis uses the
angles pos * theta^(-2i/dim).  Returned as the complex64 ``freqs_cis``
[f*h*w, 1, head_dim/2] that fused_rms_rope consumes without conversion.
"""
from __future__ import annotations

import torch


def _angles(n: int, dim: int, theta: float, offset: int = 0) -> torch.Tensor:
    inv = 1.0 / torch.pow(theta, torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    return torch.outer(torch.arange(offset, offset + n, dtype=torch.float64), inv)


def wan_freqs_cis(f: int, h: int, w: int, head_dim: int = 128, theta: float = 10000.0,
                  f_offset: int = 0, device=None) -> torch.Tensor:
    d6 = head_dim // 6
    af = _angles(f, head_dim - 4 * d6, theta, f_offset)
    ah = _angles(h, 2 * d6, theta)
    aw = _angles(w, 2 * d6, theta)
    ang = torch.cat([af[:, None, None, :].expand(f, h, w, -1),
                     ah[None, :, None, :].expand(f, h, w, -1),
                     aw[None, None, :, :].expand(f, h, w, -1)], dim=-1).reshape(f * h * w, 1, -1)
    fc = torch.polar(torch.ones_like(ang), ang).to(torch.complex64)
    return fc.to(device) if device is not None else fc
