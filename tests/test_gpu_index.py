"""BasicLayer neighbourhood index construction on the GPU (aff_cluster_members
and the neighbourhood_index glue) against the CPU oracle: member ids, padding
mask and pe_idx must be bit-exact (integer outputs)."""
import math

import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels import cluster_members
from affmae_amd.layers import neighbourhood_index
from affmae_amd.utils.geometry import space_filling_cluster

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("itype", [torch.int32, torch.int64])
@pytest.mark.parametrize("with_mask", [False, True])
def test_cluster_members_random(oracle_mod, dev, itype, with_mask):
    g = torch.Generator().manual_seed(7)
    B, N, K, m, nnc = 3, 517, 66, 8, 6
    print(f"[index] {itype} mask={with_mask}", flush=True)
    members = torch.randint(0, N, (B, K, m), generator=g)
    members[0, 3, 2] = N + 5                                       # member out of range
    cmask = (torch.rand((B, K, m), generator=g) > 0.1).long() if with_mask else None
    nearest = torch.stack([torch.stack([torch.randperm(K, generator=g)[:nnc] for _ in range(N)]) for _ in range(B)])
    nearest[1, 4, 0] = K + 1                                      # cluster id out of range
    pos = torch.rand((B, N, 2), generator=g) * 60
    mi, mk, pe = cluster_members(nearest.to(itype).to(dev), members.to(itype).to(dev),
                                 None if cmask is None else cmask.to(dev), pos.to(dev), out_dtype=itype)
    torch.cuda.synchronize()
    mo, ko, po = oracle_mod.cluster_members(nearest.numpy(), members.numpy(),
                                            None if cmask is None else cmask.numpy(), pos.numpy())
    assert mi.dtype == itype and pe.dtype == itype
    assert np.array_equal(mi.cpu().numpy(), mo)
    assert np.array_equal(pe.cpu().numpy(), po)
    if with_mask:
        assert np.array_equal(mk.cpu().numpy(), ko)
    else:
        assert mk is None


@pytest.mark.parametrize("n,cluster,nbhd", [(2048, 8, 48), (1999, 8, 48), (300, 1, 16), (40, 8, 48)])
def test_neighbourhood_index_against_oracle(oracle_mod, dev, n, cluster, nbhd):
    """Jittered-grid tokens of a 64 x 64 canvas.  The space-filling clustering is torch
    code on either device (its float sort keys are not bit-identical across devices), so
    the exact checks take the GPU's own clustering as input: oracle KNN of the cluster
    centres and oracle gathers must equal the glue's member_idx, mask and pe_idx bit for
    bit.  The clustering itself must reorder pos and feat by one permutation and agree
    with the CPU ranking on nearly every token."""
    B, c, side = 2, 16, 64
    print(f"[index glue] n={n} cluster={cluster} nbhd={nbhd}", flush=True)
    pos = workloads.jittered_grid(B, side, n, seed=3, order="raster") + 0.5
    feat = torch.randn((B, n, c), generator=torch.Generator().manual_seed(4))
    pos_g, feat_g, mi, mk, pe, glob, nb = neighbourhood_index(pos.to(dev), feat.to(dev), side, side, cluster, nbhd)
    k = math.ceil(n / cluster)
    nnc = min(int(round(nbhd / cluster)), k)
    assert nb == cluster * nnc and glob == (nbhd >= n)
    if k == n:
        assert torch.equal(pos_g.cpu(), pos) and torch.equal(feat_g.cpu(), feat)
        pos_r, cmean = pos, pos
        members, cmask = np.broadcast_to(np.arange(n).reshape(1, n, 1), (B, n, 1)), None
    else:
        pr, cm_g, mem_g, msk_g, reorder = space_filling_cluster(pos.to(dev), cluster, side, side, no_reorder=False)
        reorder = reorder.cpu()
        perm = reorder[..., 0]
        assert torch.equal(perm.sort(dim=1).values, torch.arange(n).expand(B, -1))
        assert torch.equal(pos_g.cpu(), pos.gather(1, reorder.expand(-1, -1, 2)))
        assert torch.equal(feat_g.cpu(), feat.gather(1, reorder.expand(-1, -1, c)))
        cpu_perm = space_filling_cluster(pos, cluster, side, side, no_reorder=False)[4][..., 0]
        assert (cpu_perm == perm).float().mean() > 0.95
        pos_r, cmean = pr.cpu(), cm_g.cpu()
        members, cmask = mem_g.cpu().numpy(), None if msk_g is None else msk_g.cpu().numpy()
    nearest, _ = oracle_mod.knn(pos_r.numpy(), cmean.numpy(), nnc)
    mo, ko, po = oracle_mod.cluster_members(nearest, members, cmask, pos_r.numpy())
    assert np.array_equal(mi.cpu().numpy(), mo)
    assert (mk is None) == (ko is None)
    if ko is not None:
        assert np.array_equal(mk.cpu().numpy(), ko)
    if glob:
        assert tuple(pe.shape) == (B, n, n)
    else:
        assert np.array_equal(pe.cpu().numpy(), po)
