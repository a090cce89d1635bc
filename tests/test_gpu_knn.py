"""KNN on the GPU through the C ABI, bit-exact against the oracle.

Indices must match exactly (ties -> lower index); squared distances must be
bit-identical (both are fl(fl(dx*dx) + fl(dy*dy)) in fp32).
"""
import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels import knn, knn_forward
from affmae_amd.kernels.knn import knn_launch

pytestmark = pytest.mark.gpu


def _check(query, ref, k, oracle_mod, dev, out_dtype=torch.int64):
    print(f"[knn] B={query.shape[0]} M={query.shape[1]} N={ref.shape[1]} k={k}", flush=True)
    idx, d2 = knn_launch(query.to(dev), ref.to(dev), k, out_dtype=out_dtype, return_dist=True)
    torch.cuda.synchronize()
    oi, od = oracle_mod.knn(query.float().cpu().numpy(), ref.float().cpu().numpy(), k)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), oi)
    np.testing.assert_array_equal(d2.cpu().numpy(), od)


def test_golden_cfg1(golden_dir, dev):
    g = np.load(golden_dir / "knn_cfg1.npz")
    pos = torch.from_numpy(g["pos"]).to(dev)
    idx, d2 = knn(pos, pos, 48, return_dist=True)
    assert idx.dtype == torch.int64
    np.testing.assert_array_equal(idx.cpu().numpy(), g["idx"].astype(np.int64))
    np.testing.assert_array_equal(d2.cpu().numpy(), g["d2"])


def test_golden_ties(golden_dir, dev):
    g = np.load(golden_dir / "knn_ties.npz")
    idx = knn(torch.from_numpy(g["query"]).to(dev), torch.from_numpy(g["ref"]).to(dev), 24)
    np.testing.assert_array_equal(idx.cpu().numpy(), g["idx"].astype(np.int64))


def test_cfg2_full_batch(oracle_mod, dev):
    """The benchmark shape: B=32, N=6272 jittered grid, k=48, self-KNN."""
    pos = workloads.jittered_grid(32, 112, 6272, seed=0)
    _check(pos, pos, 48, oracle_mod, dev, out_dtype=torch.int32)


@pytest.mark.parametrize("k,out_dtype", [(5, torch.int64), (13, torch.int32), (20, torch.int64),
                                         (48, torch.int64), (64, torch.int32)])
def test_more_waves_than_resident(oracle_mod, dev, k, out_dtype):
    """40 images of 6272 points: more waves than the GPU holds at once, so the
    windowed kernel writes whole output rows through LDS (every column-chunk
    width: k below, at and above half the candidate cap)."""
    pos = workloads.jittered_grid(40, 112, 6272, seed=k)
    _check(pos, pos, k, oracle_mod, dev, out_dtype=out_dtype)


def test_cfg3_cross(oracle_mod, dev):
    """Merged points (a seeded weighted subset) against all source tokens."""
    src = workloads.jittered_grid(4, 112, 6272, seed=0) / 112.0
    g = torch.Generator().manual_seed(3)
    sel = torch.stack([torch.multinomial(torch.rand(6272, generator=g), 2509, replacement=False, generator=g)
                       for _ in range(4)])
    merged = src.gather(1, sel.unsqueeze(-1).expand(-1, -1, 2))
    _check(merged, src, 48, oracle_mod, dev)


@pytest.mark.parametrize("k", [1, 4, 6, 8, 13, 24, 25, 64])
def test_uniform_various_k(oracle_mod, dev, k):
    pos = workloads.cfg1_coords(B=2, N=1024, seed=7 + k)
    _check(pos, pos, k, oracle_mod, dev)


@pytest.mark.parametrize("k", [65, 100])
def test_large_k_exact_path(oracle_mod, dev, k):
    pos = workloads.cfg1_coords(B=1, N=300, seed=11)
    _check(pos, pos, k, oracle_mod, dev)


def test_k_equals_n(oracle_mod, dev):
    pos = workloads.cfg1_coords(B=2, N=40, seed=12)
    _check(pos, pos, 40, oracle_mod, dev)


def test_cluster_means_small_k(oracle_mod, dev):
    """The encoder's call: tokens against means of 8-token clusters, k = 6."""
    pos = workloads.jittered_grid(2, 112, 6272, seed=5)
    means = pos.view(2, 784, 8, 2).mean(2)
    _check(pos, means, 6, oracle_mod, dev)


def test_lattice_ties_and_duplicates(oracle_mod, dev):
    g = torch.stack(torch.meshgrid(torch.arange(40), torch.arange(30), indexing="xy"), -1).reshape(1, -1, 2).float()
    ref = torch.cat([g, g.flip(1)], 1)                     # every point twice
    q = torch.cat([g, g + 0.5], 1)
    _check(q, ref, 48, oracle_mod, dev)


def test_all_points_identical(oracle_mod, dev):
    ref = torch.full((1, 200, 2), 0.25)
    q = torch.tensor([[[0.25, 0.25], [0.3, 0.1]]])
    _check(q, ref, 10, oracle_mod, dev)


def test_collinear_points(oracle_mod, dev):
    x = torch.rand(1, 500, generator=torch.Generator().manual_seed(9))
    ref = torch.stack([x, torch.zeros_like(x)], -1)
    _check(ref, ref, 48, oracle_mod, dev)


def test_query_far_outside(oracle_mod, dev):
    ref = workloads.cfg1_coords(B=1, N=800, seed=13)
    q = torch.tensor([[[50.0, -30.0], [0.5, 0.5], [-2.0, 0.1]]])
    _check(q, ref, 48, oracle_mod, dev)


def test_tiny_sizes(oracle_mod, dev):
    _check(torch.zeros(1, 1, 2), torch.ones(1, 1, 2), 1, oracle_mod, dev)
    pos = workloads.cfg1_coords(B=3, N=65, seed=14)
    _check(pos[:, :7], pos, 3, oracle_mod, dev)


def test_strided_and_fp16_inputs(oracle_mod, dev):
    base = workloads.cfg1_coords(B=2, N=1024, seed=15)
    wide = torch.cat([base, torch.rand(2, 1024, 3)], -1).to(dev)   # [B,N,5]
    view = wide[..., :2]                                             # coordinate stride 1, point stride 5
    idx = knn_forward(view, view, 8)
    assert idx.dtype == torch.int32
    oi, _ = oracle_mod.knn(base.numpy(), base.numpy(), 8)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    h = base.half()
    idx = knn(h.to(dev), h.to(dev), 8)
    oi, _ = oracle_mod.knn(h.float().numpy(), h.float().numpy(), 8)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)


def test_repeated_calls_deterministic(dev):
    pos = workloads.jittered_grid(4, 112, 6272, seed=0).to(dev)
    a = knn(pos, pos, 48)
    b = knn(pos, pos, 48)
    assert torch.equal(a, b)


def test_k_too_large_raises(dev):
    pos = torch.rand(1, 10, 2, device=dev)
    with pytest.raises(AssertionError, match="exceeds number of reference points"):
        knn(pos, pos, 11)


def test_reference_fallback_names(oracle_mod, dev):
    """knn_large_k_fallback / knn_pytorch_large (knn.py:1312-1365) and knn_keops
    (geometry.py:56-95, Euclidean distances) give the exact neighbours."""
    from affmae_amd.kernels.knn import knn_large_k_fallback, knn_pytorch_large
    from affmae_amd.utils.geometry import knn_keops
    pos = workloads.cfg1_coords(B=2, N=700, seed=21)
    q = pos[:, :300]
    oi, od = oracle_mod.knn(q.numpy(), pos.numpy(), 20)
    for fn in (knn_large_k_fallback, knn_pytorch_large):
        idx = fn(q.to(dev), pos.to(dev), 20)
        assert idx.dtype == torch.int64
        np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    idx, dist = knn_keops(q.to(dev).half(), pos.to(dev).half(), 20, return_dist=True)
    oih, odh = oracle_mod.knn(q.half().float().numpy(), pos.half().float().numpy(), 20)
    np.testing.assert_array_equal(idx.cpu().numpy(), oih)
    np.testing.assert_allclose(dist.cpu().numpy(), np.sqrt(odh.astype(np.float64)), rtol=1e-6)
    np.testing.assert_array_equal(knn_keops(q.to(dev), pos.to(dev), 20).cpu().numpy(), oi)


@pytest.mark.parametrize("D", [1, 3, 4])
@pytest.mark.parametrize("k", [1, 4, 8, 13, 16, 32, 48, 64])
def test_other_dims_bruteforce(oracle_mod, dev, D, k):
    """D = 1 / 3 / 4 (the brute-force search): bit-exact indices and squared distances."""
    g = torch.Generator().manual_seed(D * 100 + k)
    ref = torch.rand(2, 1500, D, generator=g)
    q = torch.rand(2, 700, D, generator=g)
    _check(q, ref, k, oracle_mod, dev)


@pytest.mark.parametrize("D", [3, 4])
def test_other_dims_lattice_ties(oracle_mod, dev, D):
    """Integer lattice with duplicated points: many equal distances, ties to the lower index."""
    g = torch.Generator().manual_seed(D)
    ref = torch.randint(0, 4, (2, 900, D), generator=g).float()
    q = torch.randint(0, 4, (2, 300, D), generator=g).float() + 0.5 * (torch.rand(2, 300, D, generator=g) > 0.5)
    for k in (8, 24):
        _check(q, ref, k, oracle_mod, dev, out_dtype=torch.int32)


def test_other_dims_reference_names(oracle_mod, dev):
    """knn / knn_forward accept D = 3 and 4 like the reference's dispatch (knn.py:1368-1540)."""
    g = torch.Generator().manual_seed(9)
    ref = torch.rand(1, 400, 3, generator=g)
    q = torch.rand(1, 100, 3, generator=g)
    oi, _ = oracle_mod.knn(q.numpy(), ref.numpy(), 6)
    np.testing.assert_array_equal(knn(q.to(dev), ref.to(dev), 6).cpu().numpy(), oi)
    out = knn_forward(q.to(dev), ref.to(dev), 6, D=3)
    assert out.dtype == torch.int32
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), oi)
    with pytest.raises(NotImplementedError):
        knn(q.to(dev), ref.to(dev), 65)
