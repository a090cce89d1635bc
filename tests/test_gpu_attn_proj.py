"""Attention with ClusterAttention's output projection fused (aff_nbhd_attn_proj_fwd).

Reference: the fp64 oracle attention (oracle.nbhd_attn, pinned in
tests/test_oracle.py) times the projection weight rounded to the kernel's
dtype, plus the bias rounded to that dtype too, as the Linear the kernel
replaces computes under autocast (reference attention.py:204-205 after the
local attention).  Tolerance: 2e-2 of max|y| (bf16 / fp16: the attention output is
rounded to 16 bits before the projection, as the two-step composition does).
The fused result is also compared with the two-step GPU composition
(nbhd_attn_fwd, then an fp32 GEMM of its 16-bit output) at 1e-2 of max|y|.
Cases: 1-4 heads, N not a multiple of 32, blank tokens, a mask, and a raster
token order whose 32-query unions overflow (the per-row fallback inside the
fused kernel).
"""
import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels.knn import knn
from affmae_amd.kernels.local_attn import nbhd_attn_fwd, nbhd_attn_proj_fwd, record_paths

pytestmark = pytest.mark.gpu


def _case(B, N, H, M, dtype, seed, order="sfc"):
    g = torch.Generator().manual_seed(seed)
    side = int(np.ceil(np.sqrt(N * 2)))
    pos = workloads.jittered_grid(B, side, N, seed=seed, order=order)
    q = torch.randn(B, H, N, 32, generator=g).to(dtype)
    k = torch.randn(B, H, N, 32, generator=g).to(dtype)
    v = torch.randn(B, H, N, 32, generator=g).to(dtype)
    C = H * 32
    w = (torch.randn(C, C, generator=g) / np.sqrt(C)).float()
    b = (0.1 * torch.randn(C, generator=g)).float()
    table = (0.3 * torch.randn(255 * 255, H, generator=g)).float()
    return pos, q, k, v, w, b, table


def _oracle_y(oracle_mod, q, k, v, idx, scale, dense, mask, bk, bv, w, b, dtype):
    out, _ = oracle_mod.nbhd_attn(q.double().cpu().numpy(), k.double().cpu().numpy(), v.double().cpu().numpy(),
                                  idx.cpu().numpy(), scale, bias=dense, mask=mask,
                                  blank_k=None if bk is None else bk.double().cpu().numpy(),
                                  blank_v=None if bv is None else bv.double().cpu().numpy())
    B, H, N, D = q.shape
    o = torch.from_numpy(out).permute(0, 2, 1, 3).reshape(B, N, H * D)
    return o @ w.to(dtype).double().T + b.to(dtype).double()


@pytest.mark.parametrize("H", [1, 2, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("blank,masked", [(False, False), (True, True)])
def test_fused_projection(oracle_mod, dev, H, dtype, blank, masked):
    from affmae_amd.utils.pos_embed import pe_index
    B, N, M = 2, 1000, 48
    pos, q, k, v, w, b, table = _case(B, N, H, M, dtype, seed=H * 10 + int(blank))
    idx = knn(pos.to(dev), pos.to(dev), M)
    pe = pe_index(pos, idx.cpu()).to(dev)
    g = torch.Generator().manual_seed(5)
    mask = (torch.rand(B, 1, N, M, generator=g) > 0.2) if masked else None
    bk = (0.2 * torch.randn(H, 32, generator=g)).to(dtype) if blank else None
    bv = (0.2 * torch.randn(H, 32, generator=g)).to(dtype) if blank else None
    scale = 32 ** -0.5
    args = dict(pe_idx=pe, pe_table=table.to(dev), mask=mask.to(dev) if masked else None,
                blank_k=bk.to(dev) if blank else None, blank_v=bv.to(dev) if blank else None)
    print(f"[attn proj] H={H} {dtype} blank={blank} mask={masked}", flush=True)
    with record_paths() as paths:
        y = nbhd_attn_proj_fwd(q.to(dev), k.to(dev), v.to(dev), idx, scale, w.to(dev), b.to(dev), **args)
    assert y is not None and list(paths) == ["wave+proj"]
    o2, _ = nbhd_attn_fwd(q.to(dev), k.to(dev), v.to(dev), idx, scale, return_lse=False, **args)
    y2 = o2.permute(0, 2, 1, 3).reshape(B, N, H * 32).float() @ w.to(dtype).float().to(dev).T + b.to(dtype).float().to(dev)
    torch.cuda.synchronize()
    dense = oracle_mod.table_bias(pe.cpu().numpy(), table.double().numpy())
    ref = _oracle_y(oracle_mod, q, k, v, idx, scale, dense, None if mask is None else mask.numpy(), bk, bv, w, b,
                    dtype)
    scale_y = float(ref.abs().max())
    assert float((y.double().cpu() - ref).abs().max()) <= 2e-2 * scale_y
    assert float((y.double().cpu() - y2.double().cpu()).abs().max()) <= 1e-2 * scale_y


def test_fused_projection_fallback_tiles(oracle_mod, dev):
    """Raster-ordered tokens: many 32-query unions exceed 224 rows and take the per-row
    routine inside the fused kernel; the result is the same."""
    from affmae_amd.utils.pos_embed import pe_index
    B, N, H, M = 2, 3000, 4, 48
    pos, q, k, v, w, b, table = _case(B, N, H, M, torch.bfloat16, seed=77, order="raster")
    idx = knn(pos.to(dev), pos.to(dev), M)
    pe = pe_index(pos, idx.cpu()).to(dev)
    y = nbhd_attn_proj_fwd(q.to(dev), k.to(dev), v.to(dev), idx, 32 ** -0.5, w.to(dev), b.to(dev), pe_idx=pe,
                           pe_table=table.to(dev))
    torch.cuda.synchronize()
    dense = oracle_mod.table_bias(pe.cpu().numpy(), table.double().numpy())
    ref = _oracle_y(oracle_mod, q, k, v, idx, 32 ** -0.5, dense, None, None, None, w, b, torch.bfloat16)
    assert float((y.double().cpu() - ref).abs().max()) <= 2e-2 * float(ref.abs().max())


def test_fused_projection_declines_other_shapes(dev):
    q = torch.randn(1, 8, 64, 32, device=dev, dtype=torch.bfloat16)
    idx = torch.zeros(1, 64, 8, dtype=torch.int64, device=dev)
    w = torch.randn(256, 256, device=dev)
    assert nbhd_attn_proj_fwd(q, q, q, idx, 0.1, w) is None                       # 8 heads
    q4 = torch.randn(1, 4, 64, 32, device=dev)
    assert nbhd_attn_proj_fwd(q4, q4, q4, idx, 0.1, torch.randn(128, 128, device=dev)) is None   # fp32
