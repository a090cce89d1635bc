"""Neighbourhood index construction of the encoder's BasicLayer on gfx950.

``cluster_members`` replaces the torch gathers of BasicLayer.forward
(src/layers/aff.py:452-465): the members of every token's nnc nearest
clusters, the padding mask of those members and the relative-position table
index pe_idx, written by one kernel (aff_cluster_members).
"""
from __future__ import annotations

import torch

from .. import _lib
from ..utils.pos_embed import REL_POS_WIDTH


def _index(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def cluster_members(nearest: torch.Tensor, members: torch.Tensor, cluster_mask: torch.Tensor | None = None,
                    pos: torch.Tensor | None = None, rel_width: int = REL_POS_WIDTH, out_dtype=torch.int64,
                    with_mask: bool = True, with_pe: bool = True):
    """Gather the neighbourhoods of every token.

    nearest [B,N,nnc]: ids of each token's nearest clusters; members [B,K,m]:
    token ids of each cluster; cluster_mask [B,K,m] (nonzero = real member) or
    None; pos [B,N,2] token coordinates (needed for pe_idx).
    Returns (member_idx [B,N,nnc*m] out_dtype, mask [B,N,nnc*m] int64 or None,
    pe_idx [B,N,nnc*m] out_dtype or None), equal to the reference's
    ``member_idx.gather(...)``, ``cluster_mask.gather(...)`` and its pe_idx
    expression (aff.py:453-465).  The mask is returned only when a
    cluster_mask is given (as in the reference) and with_mask is set.
    """
    lib = _lib.load()
    dev = _lib.require_cuda(nearest, members, cluster_mask, pos)
    assert nearest.dim() == 3 and members.dim() == 3, "nearest must be [B,N,nnc] and members [B,K,m]"
    B, N, nnc = nearest.shape
    K, m = members.shape[1], members.shape[2]
    assert members.shape[0] == B, "batch sizes must match"
    nr = _index(nearest)
    mb = _index(members)
    cm = None
    if cluster_mask is not None:
        assert tuple(cluster_mask.shape) == (B, K, m), "cluster_mask must be [B,K,m]"
        cm = (cluster_mask != 0).to(torch.uint8)
        if cm.stride(-1) != 1:
            cm = cm.contiguous()
    p = None
    if with_pe:
        assert pos is not None and tuple(pos.shape) == (B, N, 2), "pe_idx needs pos [B,N,2]"
        p = pos.to(torch.float32)
        if p.stride(-1) != 1:
            p = p.contiguous()
    S = nnc * m
    out = torch.empty((B, N, S), dtype=out_dtype, device=dev)
    mask_u8 = torch.empty((B, N, S), dtype=torch.uint8, device=dev) if (cm is not None and with_mask) else None
    pe = torch.empty((B, N, S), dtype=out_dtype, device=dev) if with_pe else None
    st = lib.aff_cluster_members(
        nr.data_ptr(), 1 if nr.dtype == torch.int64 else 0, nr.stride(0), nr.stride(1),
        mb.data_ptr(), 1 if mb.dtype == torch.int64 else 0, mb.stride(0), mb.stride(1),
        cm.data_ptr() if cm is not None else None, cm.stride(0) if cm is not None else 0,
        cm.stride(1) if cm is not None else 0,
        p.data_ptr() if p is not None else None, p.stride(0) if p is not None else 0, p.stride(1) if p is not None else 0,
        B, N, K, nnc, m, int(rel_width),
        out.data_ptr(), 1 if out_dtype == torch.int64 else 0,
        mask_u8.data_ptr() if mask_u8 is not None else None,
        pe.data_ptr() if pe is not None else None, 1 if out_dtype == torch.int64 else 0,
        _lib.stream_ptr(dev))
    _lib.check(st, "aff_cluster_members")
    mask = mask_u8.to(torch.int64) if mask_u8 is not None else None
    return out, mask, pe
