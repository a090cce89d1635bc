"""Weighted gather and the fused softmax-distance merge (HIP, gfx950).

``weighted_gather`` / ``WeightedGatherFunction`` /
``launch_weighted_gather_fwd_kernel`` are drop-ins for
src/layers/kernels/weighted_gather.py of the reference (:104-124, :329-364):

    out[b, i, c] = sum_m weights[b, i, m] * feat[b, nbhd_idx[b, i, m], c]

``softmax_merge`` fuses knn -> softmax(-distance / tau) -> weighted_gather of
features and coordinates (the config-3 downsampling merge) into one kernel
after the KNN.
"""
from __future__ import annotations

import torch
from torch.amp import custom_fwd, custom_bwd

from .. import _lib
from .knn import knn_launch
from .weighted_features import weighted_features_backward


def _idx(t):
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    return t if t.stride(-1) == 1 else t.contiguous()


def _float(t):
    return t if t.dtype in _lib.DTYPE_CODE else t.to(torch.float32)


def launch_weighted_gather_fwd_kernel(nbhd_idx, weights, feat, out=None):
    """nbhd_idx [B,N,M], weights [B,N,M], feat [B,N_old,C] -> [B,N,C] in feat.dtype."""
    lib = _lib.load()
    dev = _lib.require_cuda(nbhd_idx, weights, feat)
    B, N, M = weights.shape
    _, N_old, C = feat.shape
    assert tuple(nbhd_idx.shape) == (B, N, M) and feat.shape[0] == B, "shape mismatch"
    w = _float(weights)
    f = _float(feat)
    if f.stride(-1) != 1:
        f = f.contiguous()
    idx = _idx(nbhd_idx)
    if out is None:
        out = torch.empty((B, N, C), dtype=f.dtype, device=dev)
    st = lib.aff_weighted_gather_fwd(
        idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, idx.stride(0), idx.stride(1),
        w.data_ptr(), _lib.DTYPE_CODE[w.dtype], w.stride(0), w.stride(1),
        f.data_ptr(), _lib.DTYPE_CODE[f.dtype], f.stride(0), f.stride(1),
        B, N, N_old, M, C, out.data_ptr(), out.stride(0), out.stride(1), _lib.stream_ptr(dev))
    _lib.check(st, "aff_weighted_gather_fwd")
    return out


class WeightedGatherFunction(torch.autograd.Function):
    """Autograd entry (reference weighted_gather.py:329-361): backward returns
    (None, d_weights, d_feat), the IC = 1 case of aff_weighted_features_bwd."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, nbhd_idx, weights, feat):
        assert nbhd_idx.is_cuda and weights.is_cuda and feat.is_cuda, "All inputs must be CUDA tensors."
        ctx.save_for_backward(nbhd_idx, weights, feat)
        return launch_weighted_gather_fwd_kernel(nbhd_idx, weights, feat)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        nbhd_idx, weights, feat = ctx.saved_tensors
        dw, df = weighted_features_backward(dout.unsqueeze(2), weights.unsqueeze(-1), feat, nbhd_idx,
                                            need_weights=ctx.needs_input_grad[1], need_feat=ctx.needs_input_grad[2])
        return (None, dw.squeeze(-1).to(weights.dtype) if dw is not None else None,
                df.to(feat.dtype) if df is not None else None)


def weighted_gather(nbhd_idx: torch.Tensor, weights: torch.Tensor, feat: torch.Tensor) -> torch.Tensor:
    return WeightedGatherFunction.apply(nbhd_idx, weights, feat)


def softmax_merge_launch(query_pos, src_pos, feat, nbhd_idx, tau, out=None, out_pos=None,
                         return_weights=False):
    """Fused softmax(-d/tau) weighted gather of features and coordinates.

    query_pos [B,Nout,2], src_pos [B,N,2] fp32; feat [B,N,C]; nbhd_idx [B,Nout,K].
    Returns (feat_out [B,Nout,C] in feat.dtype, pos_out [B,Nout,2] fp32, weights or None).
    """
    lib = _lib.load()
    dev = _lib.require_cuda(query_pos, src_pos, feat, nbhd_idx)
    B, Nout, K = nbhd_idx.shape
    _, N, C = feat.shape
    q = query_pos.to(torch.float32)
    q = q if q.stride(-1) == 1 else q.contiguous()
    sp = src_pos.to(torch.float32)
    sp = sp if sp.stride(-1) == 1 else sp.contiguous()
    f = _float(feat)
    if f.stride(-1) != 1:
        f = f.contiguous()
    idx = _idx(nbhd_idx)
    if out is None:
        out = torch.empty((B, Nout, C), dtype=f.dtype, device=dev)
    if out_pos is None:
        out_pos = torch.empty((B, Nout, 2), dtype=torch.float32, device=dev)
    w = torch.empty((B, Nout, K), dtype=torch.float32, device=dev) if return_weights else None
    st = lib.aff_softmax_merge_fwd(
        q.data_ptr(), q.stride(0), q.stride(1), sp.data_ptr(), sp.stride(0), sp.stride(1),
        f.data_ptr(), _lib.DTYPE_CODE[f.dtype], f.stride(0), f.stride(1),
        idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, idx.stride(0), idx.stride(1),
        B, Nout, N, K, C, float(tau), out.data_ptr(), out.stride(0), out.stride(1),
        out_pos.data_ptr(), out_pos.stride(0), out_pos.stride(1),
        w.data_ptr() if w is not None else None, _lib.stream_ptr(dev))
    _lib.check(st, "aff_softmax_merge_fwd")
    return out, out_pos, w


def softmax_merge(query_pos, src_pos, feat, k=48, tau=0.1, nbhd_idx=None, return_weights=False):
    """Merge source tokens into query points: each query takes its k nearest
    sources (exact KNN, ties to the lower index) with weights softmax(-d/tau).

    Returns (feat_out, pos_out) or (feat_out, pos_out, nbhd_idx, weights).
    """
    if nbhd_idx is None:
        nbhd_idx = knn_launch(query_pos, src_pos, k, out_dtype=torch.int32)
    fo, po, w = softmax_merge_launch(query_pos, src_pos, feat, nbhd_idx, tau, return_weights=return_weights)
    if return_weights:
        return fo, po, nbhd_idx, w
    return fo, po
