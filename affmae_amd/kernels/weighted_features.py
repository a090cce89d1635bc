"""Weighted neighbour features, the AFF merge op (HIP, gfx950).

Drop-in for src/layers/kernels/weighted_features.py of the reference
(``weighted_features`` :433, ``WeightedFeaturesFunction`` :401-430):

    out[b, i, ic, c] = sum_m weights[b, i, m, ic] * feat[b, nbhd_idx[b, i, m], c]

fp32 accumulation, output in ``feat.dtype``; inputs are not cast to fp16.
"""
from __future__ import annotations

import torch
from torch.amp import custom_fwd, custom_bwd

from .. import _lib


def _idx(t):
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    return t if t.stride(-1) == 1 else t.contiguous()


def _float(t):
    return t if t.dtype in _lib.DTYPE_CODE else t.to(torch.float32)


def weighted_features_launch(weights, feat, nbhd_idx, out=None):
    """weights [B,Nout,M,IC], feat [B,N,C], nbhd_idx [B,Nout,M] -> [B,Nout,IC,C]."""
    lib = _lib.load()
    dev = _lib.require_cuda(weights, feat, nbhd_idx)
    B, Nout, M, IC = weights.shape
    _, N, C = feat.shape
    assert feat.shape[0] == B and tuple(nbhd_idx.shape) == (B, Nout, M), "shape mismatch"
    w = _float(weights)
    f = _float(feat)
    if f.stride(-1) != 1:
        f = f.contiguous()
    idx = _idx(nbhd_idx)
    if out is None:
        out = torch.empty((B, Nout, IC, C), dtype=f.dtype, device=dev)
    st = lib.aff_weighted_features_fwd(
        w.data_ptr(), _lib.DTYPE_CODE[w.dtype], *w.stride(),
        f.data_ptr(), _lib.DTYPE_CODE[f.dtype], f.stride(0), f.stride(1),
        idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, idx.stride(0), idx.stride(1),
        B, Nout, N, M, C, IC, out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        _lib.stream_ptr(dev))
    _lib.check(st, "aff_weighted_features_fwd")
    return out


def weighted_features_backward(dout, weights, feat, nbhd_idx, need_weights=True, need_feat=True):
    """(d_weights [B,Nout,M,IC] or None, d_feat [B,N,C] or None) through aff_weighted_features_bwd
    (reference weighted_features.py:164-398, 421-430).  d_feat is a fixed-order sum: bitwise
    reproducible, no atomics."""
    lib = _lib.load()
    dev = _lib.require_cuda(dout, weights, feat, nbhd_idx)
    B, Nout, M, IC = weights.shape
    _, N, C = feat.shape
    w = _float(weights)
    f = _float(feat)
    if f.stride(-1) != 1:
        f = f.contiguous()
    idx = _idx(nbhd_idx)
    do = dout.to(f.dtype)
    if do.stride(-1) != 1:
        do = do.contiguous()
    dw = torch.empty((B, Nout, M, IC), dtype=w.dtype, device=dev) if need_weights else None
    df = torch.empty((B, N, C), dtype=f.dtype, device=dev) if need_feat else None
    ws_bytes = int(lib.aff_weighted_features_bwd_workspace_bytes(B, Nout, N, M)) if need_feat else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    st = lib.aff_weighted_features_bwd(
        do.data_ptr(), do.stride(0), do.stride(1), do.stride(2),
        w.data_ptr(), _lib.DTYPE_CODE[w.dtype], *w.stride(),
        f.data_ptr(), _lib.DTYPE_CODE[f.dtype], f.stride(0), f.stride(1),
        idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, idx.stride(0), idx.stride(1),
        B, Nout, N, M, C, IC,
        dw.data_ptr() if dw is not None else None, _lib.DTYPE_CODE[w.dtype],
        df.data_ptr() if df is not None else None, ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(st, "aff_weighted_features_bwd")
    return dw, df


class WeightedFeaturesFunction(torch.autograd.Function):
    """Autograd entry (reference weighted_features.py:401-430): backward returns
    (d_weights, d_feat, None)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, weights, feat, nbhd_idx):
        assert weights.is_cuda and feat.is_cuda and nbhd_idx.is_cuda
        ctx.save_for_backward(weights, feat, nbhd_idx)
        return weighted_features_launch(weights, feat, nbhd_idx)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        weights, feat, nbhd_idx = ctx.saved_tensors
        dw, df = weighted_features_backward(dout, weights, feat, nbhd_idx, need_weights=ctx.needs_input_grad[0],
                                            need_feat=ctx.needs_input_grad[1])
        return (dw.to(weights.dtype) if dw is not None else None, df.to(feat.dtype) if df is not None else None, None)


def weighted_features(weights: torch.Tensor, feat: torch.Tensor, nbhd_idx: torch.Tensor) -> torch.Tensor:
    return WeightedFeaturesFunction.apply(weights, feat, nbhd_idx)
