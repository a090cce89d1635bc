"""Relative-position feature table used by the attention bias.

The table must match src/utils/pos_embed.py:9-24 of the reference row for
row, because ClusterAttention's ``pos_embed`` weights are trained against it:
row (ry * T + rx) holds the offset (x, y) = (rx - 127, ry - 127) as the
features (x, y, r, y / r, x / r) with r = sqrt(x^2 + y^2) and the undefined
entries of the zero offset set to 0.
"""
from __future__ import annotations

import torch

REL_POS_WIDTH = 1024 // 8 - 1
TABLE_WIDTH = 2 * REL_POS_WIDTH + 1


def build_pre_table(dtype=torch.float32) -> torch.Tensor:
    """[TABLE_WIDTH**2, 5] relative-position features."""
    ax = torch.arange(TABLE_WIDTH, dtype=torch.float32) - REL_POS_WIDTH
    ys, xs = torch.meshgrid(ax, ax, indexing="ij")
    r = torch.sqrt(xs * xs + ys * ys)
    safe = torch.where(r > 0, r, torch.ones_like(r))
    sin = torch.where(r > 0, ys / safe, torch.zeros_like(r))
    cos = torch.where(r > 0, xs / safe, torch.zeros_like(r))
    tab = torch.stack([xs, ys, r, sin, cos], dim=2).reshape(-1, 5)
    return tab.to(dtype)


pre_table_fp32 = build_pre_table(torch.float32)
pre_table_fp16 = pre_table_fp32.to(torch.float16)


def pe_index(pos: torch.Tensor, member_idx: torch.Tensor) -> torch.Tensor:
    """pe_idx[b,n,j] of BasicLayer (reference src/layers/aff.py:458-465).

    Offsets of the neighbour positions, shifted by +127, clamped to
    [0, 254] and truncated: (rel_y * 255 + rel_x) as int64.
    """
    B, N, d = pos.shape
    M = member_idx.shape[-1]
    pos_m = pos.gather(1, member_idx.reshape(B, -1, 1).expand(-1, -1, d)).reshape(B, N, M, d)
    rel = (pos_m - (pos.unsqueeze(2) - REL_POS_WIDTH)).clamp(0, TABLE_WIDTH - 1)
    return (rel[..., 1] * TABLE_WIDTH + rel[..., 0]).long()
