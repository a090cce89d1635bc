"""LayerNorm for the encoder's glue (HIP, gfx950): token rows and [B, C, H, W]
maps, the latter with the masked patch embedding's mask and GELU fused.

The reference normalises with torch's ``nn.LayerNorm`` (src/layers/aff.py:96,
108, 296, 494, 726) and ``LayerNorm2dImages`` (aff.py:514-526) between the
masked convolutions of the patch embedding (aff.py:610-632).  These kernels
compute the same function (fp32 statistics, biased variance) and may write
the dtype an autocast consumer would cast to, so a Linear under autocast
reads the normalised rows once, in bf16, with no separate cast pass.

``norm(module, x)`` is what the encoder modules call: inference (no autograd
graph to record) on a GPU runs the HIP kernel; a forward that records
gradients calls the module itself, whose backward torch owns.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import _lib


def _needs_graph(x, module) -> bool:
    if not torch.is_grad_enabled():
        return False
    return x.requires_grad or any(p.requires_grad for p in module.parameters())


def _affine(module):
    w = module.weight
    b = module.bias
    if w is not None and w.dtype != torch.float32:
        w = w.float()
    if b is not None and b.dtype != torch.float32:
        b = b.float()
    return w, b


def _out_dtype(x, to_autocast: bool):
    if torch.is_autocast_enabled("cuda"):
        # F.layer_norm runs in fp32 under autocast; its Linear consumer casts to the autocast dtype
        return torch.get_autocast_dtype("cuda") if to_autocast else torch.float32
    return x.dtype


def layer_norm_rows(x, weight, bias, eps, out_dtype=None):
    """LayerNorm over the last dimension of x [..., C] through aff_layer_norm_fwd."""
    lib = _lib.load()
    dev = _lib.require_cuda(x, weight, bias)
    C = x.shape[-1]
    x2 = x.reshape(-1, C)
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 or (x2.stride(0) * x2.element_size()) % 16:
        x2 = x2.contiguous()
    out_dtype = out_dtype or x.dtype
    weight, bias = (t.float().contiguous() if t is not None else None for t in (weight, bias))
    y = torch.empty(x.shape, dtype=out_dtype, device=dev)
    st = lib.aff_layer_norm_fwd(x2.data_ptr(), _lib.DTYPE_CODE[x2.dtype], x2.stride(0),
                                y.data_ptr(), _lib.DTYPE_CODE[out_dtype], C,
                                weight.data_ptr() if weight is not None else None,
                                bias.data_ptr() if bias is not None else None,
                                x2.shape[0], C, float(eps), _lib.stream_ptr(dev))
    _lib.check(st, "aff_layer_norm_fwd")
    return y


def layer_norm_map(x, weight, bias, eps, keep=None, cell=1, gelu=False, token_major=False, out_dtype=None):
    """LayerNorm over the channels of x [B, C, H, W] through aff_layer_norm_map_fwd:
    x * keep (token mask [B, (H/cell)*(W/cell)], broadcast over each cell x cell
    block), LayerNorm, optional exact GELU.  Returns [B, C, H, W] or, with
    token_major, [B, H*W, C]."""
    lib = _lib.load()
    dev = _lib.require_cuda(x, weight, bias, keep)
    B, C, H, W = x.shape
    x = x.contiguous()
    if keep is not None:
        keep = keep.to(torch.float32).reshape(B, -1).contiguous()
        assert keep.shape[1] == (H // cell) * (W // cell), "keep mask does not match the map"
    out_dtype = out_dtype or x.dtype
    weight, bias = (t.float().contiguous() if t is not None else None for t in (weight, bias))
    shape = (B, H * W, C) if token_major else (B, C, H, W)
    y = torch.empty(shape, dtype=out_dtype, device=dev)
    st = lib.aff_layer_norm_map_fwd(x.data_ptr(), _lib.DTYPE_CODE[x.dtype], y.data_ptr(), _lib.DTYPE_CODE[out_dtype],
                                    weight.data_ptr() if weight is not None else None,
                                    bias.data_ptr() if bias is not None else None,
                                    keep.data_ptr() if keep is not None else None, int(cell),
                                    B, C, H, W, 1 if token_major else 0, 1 if gelu else 0, float(eps),
                                    _lib.stream_ptr(dev))
    _lib.check(st, "aff_layer_norm_map_fwd")
    return y


def fast_path(module, x) -> bool:
    """True when ``norm(module, x)`` runs the HIP kernel."""
    return (isinstance(module, nn.LayerNorm) and len(module.normalized_shape) == 1 and x.is_cuda
            and x.dtype in _lib.DTYPE_CODE and x.shape[-1] % 8 == 0 and x.shape[-1] <= 4096
            and not _needs_graph(x, module))


def norm(module, x, to_autocast: bool = False):
    """module(x) for an nn.LayerNorm over the last dimension.  to_autocast: the
    only consumer is a Linear, so under autocast the output may be written in
    the autocast dtype (the value that Linear would compute with)."""
    if not fast_path(module, x):
        return module(x)
    w, b = _affine(module)
    return layer_norm_rows(x, w, b, module.eps, _out_dtype(x, to_autocast))
