"""Weighted features / weighted gather / softmax merge / ClusterMerging on the GPU vs the oracle.

Tolerances: fp32 -> max|out - ref| <= 1e-5 * max|ref|; bf16 / fp16 -> 2e-2
max-abs against the oracle on the same rounded inputs.
"""
import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels import knn, weighted_features, weighted_gather, softmax_merge
from affmae_amd.kernels.weighted_gather import launch_weighted_gather_fwd_kernel, softmax_merge_launch
from affmae_amd.layers import ClusterMerging
from affmae_amd.utils.geometry import upsample_feature_shepard, inverse_distance_weighting

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _close(out, ref, dtype):
    out = _np(out).astype(np.float64)
    if dtype == torch.float32:
        scale = max(np.abs(ref).max(), 1e-30)
        assert np.abs(out - ref).max() <= 1e-5 * scale, f"rel err {np.abs(out - ref).max() / scale:.3e}"
        # elementwise: 1e-5 of each element plus a floor of 1e-6 of the output scale (the floor covers
        # outputs that cancel to ~0, where fp32 summation order alone moves the last bits)
        bad = np.abs(out - ref) > 1e-5 * np.abs(ref) + 1e-6 * scale
        assert not bad.any(), f"elementwise rel err at {np.argwhere(bad)[:3].tolist()}"
    else:
        assert np.abs(out - ref).max() <= 2e-2, f"abs err {np.abs(out - ref).max():.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("C,IC", [(64, 4), (128, 4), (96, 3), (512, 4), (1024, 2), (12, 4), (8, 1)])
def test_weighted_features(oracle_mod, dev, dtype, C, IC):
    g = torch.Generator().manual_seed(C * 10 + IC)
    B, N, Nout, M = 2, 500, 200, 48
    # convex weights per (row, ic): unit-scale outputs, where a 2e-2 bound is
    # meaningful for bf16 (its half-ulp alone is 0.031 above 8)
    w = torch.softmax(torch.randn((B, Nout, M, IC), generator=g), dim=2).to(dtype)
    f = torch.randn((B, N, C), generator=g).to(dtype)
    idx = torch.randint(0, N, (B, Nout, M), generator=g)
    out = weighted_features(w.to(dev), f.to(dev), idx.to(dev))
    assert out.shape == (B, Nout, IC, C) and out.dtype == dtype
    _close(out, oracle_mod.weighted_features(_np(w), _np(f), idx.numpy()), dtype)


@pytest.mark.parametrize("C", [128, 2, 13, 64])
def test_weighted_gather(oracle_mod, dev, C):
    g = torch.Generator().manual_seed(C)
    B, N, Nout, M = 3, 400, 150, 20
    w = torch.rand((B, Nout, M), generator=g)
    f = torch.randn((B, N, C), generator=g)
    idx = torch.randint(0, N, (B, Nout, M), generator=g, dtype=torch.int32)
    out = weighted_gather(idx.to(dev), w.to(dev), f.to(dev))
    _close(out, oracle_mod.weighted_gather(idx.numpy(), w.numpy(), f.numpy()), torch.float32)


def test_weighted_gather_out_of_range_and_strided(oracle_mod, dev):
    g = torch.Generator().manual_seed(5)
    B, N, Nout, M, C = 2, 100, 30, 8, 32
    w = torch.rand((B, Nout, M), generator=g)
    fbig = torch.randn((B, N, 2 * C), generator=g)
    f = fbig[..., :C]                                   # row stride 2C
    idx = torch.randint(0, N, (B, Nout, M), generator=g)
    idx[..., 3] = N + 7
    idx[..., 5] = -1
    out = launch_weighted_gather_fwd_kernel(idx.to(dev), w.to(dev), fbig.to(dev)[..., :C])
    _close(out, oracle_mod.weighted_gather(idx.numpy(), w.numpy(), f.contiguous().numpy()), torch.float32)


@pytest.mark.parametrize("B", [2, 32])
def test_cfg3_softmax_merge(oracle_mod, dev, B):
    """Config 3: 6272 -> 2509 merged points, k=48, C=128 bf16, tau=0.1 (B=32 is the full config)."""
    w = workloads.cfg3(B=B)
    sp, mp, f = w["src_pos"].to(dev), w["merged_pos"].to(dev), w["feat"].to(dev)
    print(f"[merge cfg3] B={B}", flush=True)
    fo, po, idx, wt = softmax_merge(mp, sp, f, k=48, tau=0.1, return_weights=True)
    assert fo.dtype == torch.bfloat16 and po.dtype == torch.float32
    oi, _ = oracle_mod.knn(w["merged_pos"].numpy(), w["src_pos"].numpy(), 48)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    ro, rp, rw = oracle_mod.softmax_merge(w["merged_pos"].numpy(), w["src_pos"].numpy(), _np(w["feat"]), oi, 0.1)
    _close(fo, ro, torch.bfloat16)
    _close(po, rp, torch.float32)
    _close(wt, rw, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_softmax_merge_general(oracle_mod, dev, dtype):
    g = torch.Generator().manual_seed(7)
    B, N, Nout, K, C = 2, 700, 90, 24, 40
    sp = torch.rand((B, N, 2), generator=g)
    qp = torch.rand((B, Nout, 2), generator=g)
    f = torch.randn((B, N, C), generator=g).to(dtype)
    idx = knn(qp.to(dev), sp.to(dev), K)
    fo, po, wt = softmax_merge_launch(qp.to(dev), sp.to(dev), f.to(dev), idx, 0.05, return_weights=True)
    ro, rp, rw = oracle_mod.softmax_merge(qp.numpy(), sp.numpy(), _np(f), idx.cpu().numpy(), 0.05)
    _close(fo, ro, dtype)
    _close(po, rp, torch.float32)


def test_shepard_upsampling(oracle_mod, dev):
    """upsample_feature_shepard (geometry.py:97-167): knn + IDW weights + weighted_gather."""
    g = torch.Generator().manual_seed(8)
    B, N, Nq, C = 2, 300, 120, 16
    db = torch.rand((B, N, 2), generator=g)
    q = torch.rand((B, Nq, 2), generator=g)
    f = torch.randn((B, N, C), generator=g)
    up = upsample_feature_shepard(q.to(dev), db.to(dev), f.to(dev), k=4, power=3)
    oi, od = oracle_mod.knn(q.numpy(), db.numpy(), 4)
    ipd = 1.0 / (od.astype(np.float64) ** 3 + 1e-10)
    ww = ipd / (ipd.sum(-1, keepdims=True) + 1e-12)
    _close(up, oracle_mod.weighted_gather(oi, ww, f.numpy()), torch.float32)


def test_cluster_merging_module(oracle_mod, dev):
    """ClusterMerging forward vs the same steps with the oracle's weighted_features."""
    torch.manual_seed(0)
    b, n, c, nbhd = 2, 512, 32, 48
    m = ClusterMerging(dim=c, out_dim=64, ds_rate=0.25, reserve_on=False).to(dev).eval()
    pos = workloads.jittered_grid(b, 32, n, seed=1).to(dev)
    feat = torch.randn((b, n, c), device=dev)
    member_idx = knn(pos, pos, nbhd)
    from affmae_amd.utils.pos_embed import pe_index
    pe_idx = pe_index(pos, member_idx)
    lp = torch.rand((b, n, 1), device=dev)
    with torch.no_grad():
        pos_down, feat_down = m(pos, feat, member_idx, None, lp, 2, pe_idx, 0)
        keep = int(n * 0.25)
        assert pos_down.shape == (b, keep, 2) and feat_down.shape == (b, keep, 64)
        # recompute with the oracle for the merge step
        idx = lp.view(b, n).topk(keep, dim=1, sorted=False)[1].unsqueeze(2)
        assert torch.equal(pos_down, pos.gather(1, idx.expand(-1, -1, 2)))
        mi = member_idx.gather(1, idx.expand(-1, -1, nbhd))
        pe = pe_idx.gather(1, idx.expand(-1, -1, nbhd))
        lpm = lp.gather(1, mi.view(b, -1, 1)).reshape(b, keep, nbhd, 1)
        from affmae_amd.utils.pos_embed import pre_table_fp32
        tab = m.weight_net(pre_table_fp32.to(dev))
        wts = tab.gather(0, pe.reshape(-1, 1).expand(-1, 4)).reshape(b, keep, nbhd, 4) * lpm
        merged = oracle_mod.weighted_features(_np(wts), _np(feat), mi.cpu().numpy()).reshape(b, keep, 4 * c)
        ref = m.linear(m.norm(torch.from_numpy(merged).float().to(dev)))
    _close(feat_down, _np(ref).astype(np.float64), torch.float32)


def test_idw_weights(dev):
    d = torch.rand((2, 10, 3), device=dev) + 0.1
    w = inverse_distance_weighting(d, power=3)
    ipd = 1.0 / (d.double() ** 3 + 1e-10)
    ref = ipd / (ipd.sum(2, keepdim=True) + 1e-12)
    assert torch.allclose(w.double(), ref, rtol=1e-5)


@pytest.mark.parametrize("reserve_on,dtype", [(True, torch.float32), (False, torch.bfloat16), (True, torch.bfloat16)])
def test_cluster_merging_module_reserve_and_bf16(oracle_mod, dev, reserve_on, dtype):
    """ClusterMerging with the reference constructor's default reserve_on=True (grid tokens
    at multiples of 2 * stride are always kept, after the sampled ones) and under bf16
    autocast: the kept positions are checked against the rule, and the merged features
    against the oracle's weighted_features on the module's own (autocast) weight table,
    followed by the module's norm and linear."""
    torch.manual_seed(1)
    b, side_x, side_y, c, nbhd, stride = 2, 32, 16, 32, 48, 2
    n = side_x * side_y
    ys, xs = torch.meshgrid(torch.arange(side_y), torch.arange(side_x), indexing="ij")
    grid = torch.stack([xs, ys], -1).reshape(1, n, 2).float()
    perm = torch.stack([torch.randperm(n, generator=torch.Generator().manual_seed(10 + i)) for i in range(b)])
    pos = grid.expand(b, -1, -1).gather(1, perm.unsqueeze(-1).expand(-1, -1, 2)).contiguous().to(dev)
    reserve = ((pos.long() % (2 * stride)) == 0).all(-1)
    reserve_num = int(reserve[0].sum()) if reserve_on else 0
    assert (reserve.sum(1) == reserve[0].sum()).all()
    m = ClusterMerging(dim=c, out_dim=64, ds_rate=0.25, reserve_on=reserve_on).to(dev).eval()
    feat = torch.randn((b, n, c), device=dev)
    member_idx = knn(pos, pos, nbhd)
    from affmae_amd.utils.pos_embed import pe_index
    pe_idx = pe_index(pos, member_idx)
    lp = torch.rand((b, n, 1), device=dev)
    keep = int(n * 0.25)
    ac = torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype == torch.bfloat16)
    with torch.no_grad(), ac:
        pos_down, feat_down = m(pos, feat, member_idx, None, lp, stride, pe_idx, reserve_num)
        assert pos_down.shape == (b, keep, 2) and feat_down.shape == (b, keep, 64)
        # kept token of each output row, recovered from its (unique) position
        key = (pos[..., 1] * side_x + pos[..., 0]).long()
        inv = torch.empty_like(key)
        inv.scatter_(1, key, torch.arange(n, device=dev).expand(b, -1))
        idx = inv.gather(1, (pos_down[..., 1] * side_x + pos_down[..., 0]).long()).unsqueeze(2)
        if reserve_on:
            tail = reserve.gather(1, idx[:, keep - reserve_num:, 0])
            assert tail.all() and int(reserve.gather(1, idx[..., 0]).sum()) == b * reserve_num
        mi = member_idx.gather(1, idx.expand(-1, -1, nbhd))
        pe = pe_idx.gather(1, idx.expand(-1, -1, nbhd))
        lpm = lp.gather(1, mi.view(b, -1, 1)).reshape(b, keep, nbhd, 1)
        tab = m._weights_table(dev, feat.dtype)
        wts = tab.gather(0, pe.reshape(-1, 1).expand(-1, 4)).reshape(b, keep, nbhd, 4) * lpm
        merged = oracle_mod.weighted_features(_np(wts), _np(feat), mi.cpu().numpy()).reshape(b, keep, 4 * c)
        ref = m.linear(m.norm(torch.from_numpy(merged).float().to(dev)))
    _close(feat_down.float(), _np(ref).astype(np.float64), dtype)
