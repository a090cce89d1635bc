"""aff_knn_noalloc: aff_knn with its workspace in the library's static device array.

Called through the C ABI and checked bit-for-bit (indices and squared
distances) against aff_knn with a caller-allocated workspace, on two calls in
a row, the second with a smaller input, and then once more on the first
input.  A request larger than the static array fails before any launch.
"""
import ctypes

import pytest
import torch

from affmae_amd import _lib, workloads
from affmae_amd.kernels.knn import knn_launch

pytestmark = pytest.mark.gpu


def _noalloc(q, r, k):
    """aff_knn_noalloc on fp32 [B,M,2] / [B,N,2] -> (int32 idx, fp32 d2)."""
    lib = _lib.load()
    B, M, _ = q.shape
    N = r.shape[1]
    idx = torch.full((B, M, k), -7, dtype=torch.int32, device=q.device)
    d2 = torch.full((B, M, k), -1.0, dtype=torch.float32, device=q.device)
    st = lib.aff_knn_noalloc(q.data_ptr(), q.stride(0), q.stride(1), r.data_ptr(), r.stride(0), r.stride(1),
                             B, M, N, 2, k, idx.data_ptr(), 0, d2.data_ptr(), _lib.stream_ptr(q.device))
    _lib.check(st, "aff_knn_noalloc")
    return idx, d2


def _case(B, M, N, seed, dev):
    g = torch.Generator().manual_seed(seed)
    r = workloads.cfg1_coords(B, N, seed=seed) * 80.0
    q = r[:, :M].clone() if M <= N else torch.rand((B, M, 2), generator=g) * 80.0
    q[:, ::3] += torch.rand((B, (M + 2) // 3, 2), generator=g) * 0.5
    return q.to(dev), r.to(dev)


def test_noalloc_matches_aff_knn_twice(dev):
    lib = _lib.load()
    # 1) the cfg2 shape: B=32 images of 6272 points, k=48 (6.5 MiB of scratch)
    print("[noalloc] call 1: B=32 N=6272 self k=48", flush=True)
    w = workloads.cfg2(B=32, N=6272, H=1, D=32)
    pos = w["pos"].to(dev)
    assert lib.aff_knn_workspace_bytes(32, 6272, 6272, 2, 48) <= _lib.KNN_NOALLOC_SCRATCH_BYTES
    i1, d1 = _noalloc(pos, pos, 48)
    ri1, rd1 = knn_launch(pos, pos, 48, out_dtype=torch.int32, return_dist=True)
    torch.cuda.synchronize()
    assert torch.equal(i1, ri1) and torch.equal(d1, rd1)

    # 2) a smaller cross query right after: 3 images, 700 queries among 1000 points, k=16
    print("[noalloc] call 2: B=3 M=700 N=1000 k=16", flush=True)
    q, r = _case(3, 700, 1000, seed=5, dev=dev)
    i2, d2 = _noalloc(q, r, 16)
    ri2, rd2 = knn_launch(q, r, 16, out_dtype=torch.int32, return_dist=True)
    torch.cuda.synchronize()
    assert torch.equal(i2, ri2) and torch.equal(d2, rd2)

    # 3) the first input again: the scratch left by call 2 does not leak into the result
    print("[noalloc] call 3: B=32 N=6272 self k=48 again", flush=True)
    i3, d3 = _noalloc(pos, pos, 48)
    torch.cuda.synchronize()
    assert torch.equal(i3, ri1) and torch.equal(d3, rd1)


def test_noalloc_rejects_oversize(dev):
    """A workspace need above the static array is refused on the host, before any launch."""
    lib = _lib.load()
    B, N, k = 128, 6272, 48
    assert lib.aff_knn_workspace_bytes(B, N, N, 2, k) > _lib.KNN_NOALLOC_SCRATCH_BYTES
    dummy = 0x10000  # never dereferenced: the size check fails first
    st = lib.aff_knn_noalloc(dummy, N * 2, 2, dummy, N * 2, 2, B, N, N, 2, k, dummy, 0, None,
                             _lib.stream_ptr(dev))
    assert st == _lib.AFF_ERR_WORKSPACE
    assert b"static scratch" in lib.aff_last_error()
