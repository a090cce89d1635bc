"""Exact K-nearest neighbours over point coordinates (HIP, gfx950).

Drop-in for src/layers/kernels/knn.py of the reference: same function names,
argument meaning, return dtypes and assertion messages.  One kernel family
serves every k (the reference switches to cdist+topk / KeOps above k=8,
knn.py:1391-1393); results are ordered by (squared distance, index), i.e.
ties keep the lower reference index as the reference's streaming kernels do
(knn.py:313-330).
"""
from __future__ import annotations

import ctypes

import torch
from torch.autograd import Function
from torch.amp import custom_fwd

from .. import _lib


def _as_f32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _require_2d(D: int) -> None:
    """The reference accepts D in {2, 3, 4}: D = 2 runs the grid-bucketed search,
    D = 3 / 4 the brute-force exact search (k <= 64)."""
    if D not in (1, 2, 3, 4):
        raise NotImplementedError(f"affmae_amd KNN supports 1 <= D <= 4 (got D={D})")


def knn_launch(query: torch.Tensor, ref: torch.Tensor, k: int, out_dtype=torch.int32,
               return_dist: bool = False):
    """Call aff_knn on [B,M,D] / [B,N,D] fp32 views; returns idx (and d2)."""
    lib = _lib.load()
    dev = _lib.require_cuda(query, ref)
    _require_2d(query.shape[-1])
    q = _as_f32(query)
    r = _as_f32(ref)
    B, M, D = q.shape
    N = r.shape[1]
    idx = torch.empty((B, M, k), dtype=out_dtype, device=dev)
    d2 = torch.empty((B, M, k), dtype=torch.float32, device=dev) if return_dist else None
    ws_bytes = lib.aff_knn_workspace_bytes(B, M, N, D, k)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=dev)
    st = lib.aff_knn(q.data_ptr(), q.stride(0), q.stride(1), r.data_ptr(), r.stride(0), r.stride(1),
                     B, M, N, D, k, idx.data_ptr(), 1 if out_dtype == torch.int64 else 0,
                     d2.data_ptr() if d2 is not None else None, ws.data_ptr(), ws_bytes,
                     _lib.stream_ptr(dev))
    _lib.check(st, "aff_knn")
    return (idx, d2) if return_dist else idx


def knn_forward(query, ref, k, D=2, use_v2=True, use_heuristic=True):
    """K nearest neighbours of each query among ref (reference: knn.py:1368-1540).

    query [B,M,D], ref [B,N,D] -> int32 indices [B,M,k], ascending by
    (distance, index).  ``use_heuristic`` is accepted for signature
    compatibility (there is no autotuning here); ``use_v2=False`` raises as
    in the reference.
    """
    assert query.is_cuda and ref.is_cuda, "Inputs must be on CUDA"
    assert query.dim() == 3 and ref.dim() == 3, "Expected 3D tensors [B, N, D]"
    assert query.shape[0] == ref.shape[0], "Batch sizes must match"
    assert query.shape[2] == ref.shape[2] == D, f"Expected D={D}, got query D={query.shape[2]}, ref D={ref.shape[2]}"
    assert D in [2, 3, 4], f"D must be 2, 3, or 4, got {D}"
    assert k <= ref.shape[1], f"k={k} exceeds number of reference points N={ref.shape[1]}"
    _require_2d(D)
    if not use_v2:
        raise ValueError(
            f"use_v2=False is deprecated. Only optimized K=4/K=8 kernels are supported. "
            f"Got K={k}, use_v2={use_v2}")
    return knn_launch(query, ref, k, out_dtype=torch.int32)


class KNNFunction(Function):
    """Autograd wrapper (forward only; indices carry no gradient). knn.py:1543-1582."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, query, ref, k, D=2):
        with torch.no_grad():
            q = query.detach()
            r = ref.detach()
            assert q.is_cuda and r.is_cuda, "Inputs must be on CUDA"
            assert q.dim() == 3 and r.dim() == 3, "Expected 3D tensors [B, N, D]"
            assert q.shape[0] == r.shape[0], "Batch sizes must match"
            assert q.shape[2] == r.shape[2] == D, f"Expected D={D}, got query D={q.shape[2]}, ref D={r.shape[2]}"
            assert D in [2, 3, 4], f"D must be 2, 3, or 4, got {D}"
            assert k <= r.shape[1], f"k={k} exceeds number of reference points N={r.shape[1]}"
            _require_2d(D)
            # int64 written directly by the kernel (no cast pass)
            return knn_launch(q, r, k, out_dtype=torch.int64)

    @staticmethod
    def backward(ctx, grad_output):
        return None, None, None, None


def knn_hip(query, ref, k, D=2):
    """int64 [B,M,k] neighbour indices (the reference's knn_triton, knn.py:1585-1611)."""
    return KNNFunction.apply(query, ref, k, D)


def knn_pytorch_large(query, ref, k):
    """int64 [B,M,k] (knn.py:1312-1332).  The reference materialises cdist + topk;
    here the exact HIP KNN serves it (ties: lower index first, where topk leaves
    the order unspecified)."""
    return knn_hip(query, ref, k, D=query.shape[-1])


def knn_large_k_fallback(query, ref, k):
    """int64 [B,M,k] (knn.py:1335-1365): the reference's k > 8 dispatch to KeOps or
    cdist; the exact HIP KNN covers every k here."""
    return knn_hip(query, ref, k, D=query.shape[-1])


def knn(query, database, k, return_dist=False, D=None):
    """Public KNN (knn.py:1615-1648): int64 indices and optional squared distances.

    The distances are the kernel's own d2 = (qx-rx)^2 + (qy-ry)^2 in fp32,
    bit-identical to the reference's gather-and-recompute (knn.py:1636-1646)
    for fp32 inputs.
    """
    if D is None:
        D = query.shape[-1]
    if not return_dist:
        return knn_hip(query, database, k, D=D)
    assert query.is_cuda and database.is_cuda, "Inputs must be on CUDA"
    assert query.dim() == 3 and database.dim() == 3, "Expected 3D tensors [B, N, D]"
    assert query.shape[0] == database.shape[0], "Batch sizes must match"
    assert query.shape[2] == database.shape[2] == D, f"Expected D={D}, got query D={query.shape[2]}, ref D={database.shape[2]}"
    assert k <= database.shape[1], f"k={k} exceeds number of reference points N={database.shape[1]}"
    _require_2d(D)
    with torch.no_grad():
        idx, d2 = knn_launch(query.detach(), database.detach(), k, out_dtype=torch.int64, return_dist=True)
    return idx, d2.to(query.dtype) if query.dtype != torch.float32 else d2
