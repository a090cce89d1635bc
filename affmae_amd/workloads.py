"""Seeded synthetic inputs for the benchmark configurations of the hot path.

Generators run on the CPU with explicit ``torch.Generator`` seeds (so every
machine produces the same inputs) and return CPU tensors; callers move them
to the device.  Seeds: coordinates 0, features 1, weights 2, selection 3.
"""
from __future__ import annotations

import math

import torch


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def cfg1_coords(B: int = 2, N: int = 1024, seed: int = 0) -> torch.Tensor:
    """Config 1: N points uniform in [0, 1)^2, fp32 [B, N, 2]."""
    return torch.rand((B, N, 2), generator=_gen(seed), dtype=torch.float32)


def jittered_grid(B: int, side: int, keep: int, seed: int = 0) -> torch.Tensor:
    """Config 2 coordinates: keep `keep` of side*side cells per image (chosen
    without replacement), each at (col, row) + U(-0.5, 0.5).

    Tokens are listed in raster order of their cells, the spatially coherent
    order in which the encoder presents tokens after its scanline clustering.
    Returns fp32 [B, keep, 2] in grid units.
    """
    g = _gen(seed)
    out = torch.empty((B, keep, 2), dtype=torch.float32)
    for b in range(B):
        cells = torch.randperm(side * side, generator=g)[:keep].sort().values
        row = (cells // side).to(torch.float32)
        col = (cells % side).to(torch.float32)
        jit = torch.rand((keep, 2), generator=g, dtype=torch.float32) - 0.5
        out[b, :, 0] = col + jit[:, 0]
        out[b, :, 1] = row + jit[:, 1]
    return out


def cfg2(B: int = 32, N: int = 6272, H: int = 4, D: int = 32, dtype=torch.bfloat16):
    """Config 2: neighbourhood attention at the stage-1 shape of a 448^2 image,
    patch 4, 50% mask (112 x 112 grid, 6272 visible tokens).

    Returns a dict of CPU tensors: pos [B,N,2] fp32, q/k/v [B,H,N,D] ~ N(0,1)
    in `dtype`, blank_k/blank_v [H,D] ~ N(0, 0.2^2), pos_w [H,5] and pos_b [H]
    (a seeded Linear(5, H) initialisation).
    """
    side = 112
    pos = jittered_grid(B, side, N, seed=0)
    g = _gen(1)
    q = torch.randn((B, H, N, D), generator=g).to(dtype)
    k = torch.randn((B, H, N, D), generator=g).to(dtype)
    v = torch.randn((B, H, N, D), generator=g).to(dtype)
    g2 = _gen(2)
    bound = 1.0 / math.sqrt(5)
    pos_w = (torch.rand((H, 5), generator=g2) * 2 - 1) * bound
    pos_b = (torch.rand((H,), generator=g2) * 2 - 1) * bound
    blank_k = (torch.randn((H, D), generator=g2) * 0.2).to(dtype)
    blank_v = (torch.randn((H, D), generator=g2) * 0.2).to(dtype)
    return dict(pos=pos, q=q, k=k, v=v, pos_w=pos_w, pos_b=pos_b, blank_k=blank_k, blank_v=blank_v)
