"""Block masks for LCSA workloads, built on the host.

``local_block_mask`` is the 2-D sliding-window rule of the reference
(lcsa/reference.py:24-34).  ``window_plus_random_mask`` is the BASELINE C4
recipe: the local rule inside each latent time row, plus ``extra`` blocks per
(head, query block) drawn without replacement from the blocks not yet kept
(numpy PCG64 seeded generator, so every machine draws the same mask).
"""
from __future__ import annotations

import numpy as np
import torch


def local_block_mask(bh: int, bw: int, rng: int) -> np.ndarray:
    r, c = np.meshgrid(np.arange(bh), np.arange(bw), indexing="ij")
    r, c = r.reshape(-1), c.reshape(-1)
    lo_r, lo_c = r - rng // 2, c - rng // 2
    in_r = (r[None, :] >= lo_r[:, None]) & (r[None, :] < lo_r[:, None] + rng)
    in_c = (c[None, :] >= lo_c[:, None]) & (c[None, :] < lo_c[:, None] + rng)
    return in_r & in_c


def window_plus_random_mask(heads: int = 12, time_rows: int = 2, bh: int = 6, bw: int = 11,
                            local_range: int = 7, extra: int = 10, seed: int = 7,
                            device=None) -> torch.Tensor:
    nb = bh * bw
    n = time_rows * nb
    loc = local_block_mask(bh, bw, local_range)
    base = np.zeros((n, n), bool)
    for t in range(time_rows):
        base[t * nb:(t + 1) * nb, t * nb:(t + 1) * nb] = loc
    keep = np.broadcast_to(base, (heads, n, n)).copy()
    gen = np.random.Generator(np.random.PCG64(seed))
    for h in range(heads):
        for i in range(n):
            free = np.flatnonzero(~keep[h, i])
            if len(free):
                keep[h, i, gen.choice(free, size=min(extra, len(free)), replace=False)] = True
    t = torch.from_numpy(keep)
    return t.to(device) if device is not None else t


def density_mask(heads: int, nq: int, nk: int, density: float, seed: int,
                 device=None) -> torch.Tensor:
    """Seeded Bernoulli(density) block mask with the diagonal kept (sweeps)."""
    gen = np.random.Generator(np.random.PCG64(seed))
    keep = gen.random((heads, nq, nk)) < density
    idx = np.arange(min(nq, nk))
    keep[:, idx, idx] = True
    t = torch.from_numpy(keep)
    return t.to(device) if device is not None else t
