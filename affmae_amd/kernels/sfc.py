"""Space-filling-curve keys and per-row argsort (HIP, gfx950).

Host side of aff_sfc_curve_keys / aff_sfc_anchor_keys / aff_sfc_argsort:
the curve parameters are derived exactly as the reference derives them
(src/utils/geometry.py:203-216 for the anchor grid, :335-372 / :405-446 for
the Peano / Hilbert digit levels), the per-token work runs on the GPU.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from .. import _lib

CURVES = {"": _lib.SFC_SCANLINE, "peano": _lib.SFC_PEANO, "hilbert": _lib.SFC_HILBERT}


def curve_levels(curve: int, h, w):
    """(levels, first_w, cur_h fp32, inv_h fp32, level_scale fp32) of the Peano /
    Hilbert order on an h x w canvas (geometry.py:335-372, 405-446)."""
    base = 3 if curve == _lib.SFC_PEANO else 2
    levels = math.ceil(math.log(h, base))
    assert levels >= 1, "h too short"
    if levels > _lib.SFC_MAX_LEVELS:
        raise NotImplementedError(f"space-filling curve with {levels} levels (at most {_lib.SFC_MAX_LEVELS})")
    first_w = 0
    if h != w:
        first_w = round(base * (w / h))
        if first_w == base:
            first_w = 0
    cur, last = [], h
    for _ in range(levels):
        last = last / base
        cur.append(last)
    cur_f = np.asarray(cur, dtype=np.float32)
    inv_f = np.float32(1.0) / cur_f
    scale = np.asarray([base ** (2 * (levels - i - 1)) for i in range(levels)], dtype=np.float32)
    return levels, first_w, cur_f, inv_f, scale


def curve_keys(pos, curve: int, h, w):
    """fp32 [B,N] curve keys of pos [B,N,2] (fp32) on an h x w canvas."""
    lib = _lib.load()
    dev = _lib.require_cuda(pos)
    p = pos if pos.dtype == torch.float32 and pos.stride(-1) == 1 else pos.to(torch.float32).contiguous()
    B, N, _ = p.shape
    keys = torch.empty((B, N), dtype=torch.float32, device=dev)
    a = _lib.SfcCurveArgs()
    a.pos, a.p_sb, a.p_sn = p.data_ptr(), p.stride(0), p.stride(1)
    a.B, a.N, a.curve, a.w = B, N, curve, int(w)
    if curve != _lib.SFC_SCANLINE:
        levels, first_w, cur_f, inv_f, scale = curve_levels(curve, h, w)
        a.levels, a.first_w = levels, first_w
        for i in range(levels):
            a.cur_h[i], a.inv_h[i], a.level_scale[i] = float(cur_f[i]), float(inv_f[i]), float(scale[i])
    elif int(h) * int(w) > (1 << 24):
        raise NotImplementedError("scanline keys beyond 2^24 cells")
    a.keys = keys.data_ptr()
    _lib.check(lib.aff_sfc_curve_keys(ctypes.byref(a), _lib.stream_ptr(dev)), "aff_sfc_curve_keys")
    return keys


def anchor_keys(pos, plw, plh, npw, cell_rank, prev_c, next_c):
    """fp32 [B,N] anchor keys (geometry.py:254-268); cell_rank int32 [ncell],
    prev_c / next_c fp32 [ncell, 2] on the device."""
    lib = _lib.load()
    dev = _lib.require_cuda(pos, cell_rank, prev_c, next_c)
    p = pos if pos.dtype == torch.float32 and pos.stride(-1) == 1 else pos.to(torch.float32).contiguous()
    B, N, _ = p.shape
    cr = cell_rank.to(torch.int32).contiguous()
    pc = prev_c.to(torch.float32).contiguous()
    nc = next_c.to(torch.float32).contiguous()
    keys = torch.empty((B, N), dtype=torch.float32, device=dev)
    a = _lib.SfcAnchorArgs()
    a.pos, a.p_sb, a.p_sn = p.data_ptr(), p.stride(0), p.stride(1)
    a.B, a.N, a.plw, a.plh, a.npw, a.ncell = B, N, float(plw), float(plh), int(npw), cr.numel()
    a.cell_rank, a.prev_c, a.next_c, a.keys = cr.data_ptr(), pc.data_ptr(), nc.data_ptr(), keys.data_ptr()
    ws_bytes = int(lib.aff_sfc_anchor_workspace_bytes(B, N))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _lib.check(lib.aff_sfc_anchor_keys(ctypes.byref(a), ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev)),
               "aff_sfc_anchor_keys")
    return keys


def argsort(keys):
    """int64 [B,N]: stable ascending argsort of each row of fp32 keys [B,N]."""
    lib = _lib.load()
    dev = _lib.require_cuda(keys)
    k = keys.to(torch.float32).contiguous()
    B, N = k.shape
    out = torch.empty((B, N), dtype=torch.int64, device=dev)
    ws_bytes = int(lib.aff_sfc_argsort_workspace_bytes(B, N))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _lib.check(lib.aff_sfc_argsort(k.data_ptr(), B, N, out.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev)),
               "aff_sfc_argsort")
    return out
