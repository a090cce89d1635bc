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
    """Autograd entry (forward only: the backward kernels are not built yet)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, nn_idx, nn_weight, attn, val):
        return launch_msdetrpc_forward(nn_idx, nn_weight, attn, val)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, d_out):
        raise NotImplementedError("MSDETRPC backward is not implemented in affmae_amd yet")
