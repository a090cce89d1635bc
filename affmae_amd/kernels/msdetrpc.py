"""Multi-slot deformable gather (HIP, gfx950).

Drop-in for src/layers/kernels/msdetrpc.py of the reference
(``MSDETRPCFunction`` :372-390, ``launch_msdetrpc_forward`` :305-325):

    out[b, n, c] = sum_m sum_k attn[b, n, m] * nn_weight[b, n, m, k] * val[b, nn_idx[b, n, m, k], c]
"""
from __future__ import annotations

import torch
from torch.autograd import Function
from torch.amp import custom_fwd, custom_bwd

from .. import _lib


def launch_msdetrpc_forward(nn_idx, nn_weight, attn, val):
    lib = _lib.load()
    dev = _lib.require_cuda(nn_idx, nn_weight, attn, val)
    B, N, M, K = nn_idx.shape
    _, Nval, C = val.shape
    idx = nn_idx if nn_idx.dtype in (torch.int32, torch.int64) else nn_idx.to(torch.int64)
    idx = idx if idx.stride(-1) == 1 else idx.contiguous()
    w = nn_weight if nn_weight.dtype in _lib.DTYPE_CODE else nn_weight.to(torch.float32)
    w = w if w.stride(-1) == 1 else w.contiguous()
    a = attn if attn.dtype in _lib.DTYPE_CODE else attn.to(torch.float32)
    a = a if a.stride(-1) == 1 else a.contiguous()
    v = val if val.dtype in _lib.DTYPE_CODE else val.to(torch.float32)
    if v.stride(-1) != 1 or v.data_ptr() % 16:
        v = v.contiguous()
    out = torch.empty((B, N, C), dtype=v.dtype, device=dev)
    st = lib.aff_msdetrpc_fwd(idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, idx.stride(0), idx.stride(1),
                              idx.stride(2), w.data_ptr(), _lib.DTYPE_CODE[w.dtype], w.stride(0), w.stride(1),
                              w.stride(2), a.data_ptr(), _lib.DTYPE_CODE[a.dtype], a.stride(0), a.stride(1),
                              v.data_ptr(), _lib.DTYPE_CODE[v.dtype], v.stride(0), v.stride(1),
                              B, N, M, K, Nval, C, out.data_ptr(), out.stride(0), out.stride(1),
                              _lib.stream_ptr(dev))
    _lib.check(st, "aff_msdetrpc_fwd")
    return out


class MSDETRPCFunction(Function):
    """Autograd entry (reference msdetrpc.py:372-390): backward returns
    (None, d_nn_weight, d_attn, d_val) through aff_deform_bwd (GIVEN weights;
    d_val is a fixed-order sum, no float atomics)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, nn_idx, nn_weight, attn, val):
        ctx.save_for_backward(nn_idx, nn_weight, attn, val)
        return launch_msdetrpc_forward(nn_idx, nn_weight, attn, val)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, d_out):
        nn_idx, nn_weight, attn, val = ctx.saved_tensors
        n = ctx.needs_input_grad
        d_nw, d_att, d_val = launch_msdetrpc_backward(d_out, nn_idx, nn_weight, attn, val,
                                                      want=(n[1], n[2], n[3]))
        return None, d_nw, d_att, d_val


def launch_msdetrpc_backward(d_out, nn_idx, nn_weight, attn, val, want=(True, True, True)):
    """(d_nn_weight [B,N,M,K], d_attn [B,N,M], d_val [B,Nval,C]) (reference msdetrpc.py:328-369)."""
    from .fused_deform_attn import deform_backward_launch
    B, N, M, K = nn_idx.shape
    g = deform_backward_launch(_lib.DEFORM_BWD_GIVEN, d_out.unsqueeze(2), idx=nn_idx.unsqueeze(2),
                               weights=nn_weight.unsqueeze(2), attn=attn.unsqueeze(2), values=val.unsqueeze(2),
                               want_weights=want[0], want_attn=want[1], want_values=want[2])
    d_nw = g["d_weights"].reshape(nn_weight.shape).to(nn_weight.dtype) if want[0] else None
    d_att = g["d_attn"].reshape(attn.shape).to(attn.dtype) if want[1] else None
    d_val = g["d_values"].reshape(val.shape).to(val.dtype) if want[2] else None
    return d_nw, d_att, d_val
