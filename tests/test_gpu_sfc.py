"""Space-filling-curve keys and argsort (aff_sfc_*) on the GPU.

Reference: oracle/sfc.py, the reference's orderings (geometry.py:170-460)
restated in torch and evaluated by torch on the same GPU, so the keys must be
bit-identical (the kernels reproduce the device arithmetic of those torch ops:
reciprocal-multiply division by a scalar, fmod, fp32 sums in order).  The
argsort is checked against torch's stable sort; the whole clustering against
the product's independent CPU ordering and against sorting the oracle's keys.
"""
import math

import pytest
import torch

from affmae_amd.kernels import sfc
from affmae_amd.utils.geometry import space_filling_cluster

pytestmark = pytest.mark.gpu


def _jitter(B, side, n, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    pos = []
    for _ in range(B):
        cells = torch.randperm(side * side, generator=g)[:n]
        p = torch.stack([cells % side, cells // side], -1).float()
        pos.append(p + torch.rand(p.shape, generator=g) * 0.98)
    return (torch.stack(pos) * scale).contiguous()


@pytest.mark.parametrize("curve,h,w,scale", [("peano", 27, 27, 1.0), ("peano", 20, 20, 1.0), ("peano", 30, 60, 1.0),
                                             ("peano", 81, 81, 1.0), ("hilbert", 32, 32, 1.0),
                                             ("hilbert", 20, 20, 1.0), ("scanline", 25, 40, 1.0)])
def test_curve_keys_bitwise(dev, curve, h, w, scale):
    from oracle import sfc as osfc
    side = min(h, w)
    pos = _jitter(2, side, side * side // 2, h + w, scale).to(dev)
    if curve == "scanline":
        pos = pos.floor()                 # the scanline branch indexes integer cells
        ref = osfc.scanline_keys(h, w, pos).float()
        got = sfc.curve_keys(pos, sfc.CURVES[""], h, w)
    else:
        ref = (osfc.peano_keys if curve == "peano" else osfc.hilbert_keys)(h, w, pos)
        got = sfc.curve_keys(pos, sfc.CURVES[curve], h, w)
    torch.cuda.synchronize()
    assert torch.equal(got, ref.to(torch.float32))


@pytest.mark.parametrize("sf_type", ["", "peano", "hilbert"])
def test_anchor_keys_and_ranking_bitwise(dev, sf_type):
    from oracle import sfc as osfc
    side = 64
    pos = _jitter(3, side, 2000, 7).to(dev)
    ranking = space_filling_cluster(pos, 8, side, side, sf_type=sf_type)[4][..., 0]
    key = osfc.anchor_keys(pos, 8, side, side, sf_type)
    torch.cuda.synchronize()
    assert torch.equal(ranking, key.sort(dim=1, stable=True)[1])


def test_scanline_ranking_matches_cpu_path(dev):
    side = 112
    pos = _jitter(4, side, 6272, 11)
    gpu = space_filling_cluster(pos.to(dev), 8, side, side)
    cpu = space_filling_cluster(pos, 8, side, side)
    torch.cuda.synchronize()
    for a, b in zip(gpu, cpu):
        if a is None:
            assert b is None
            continue
        assert torch.equal(a.cpu(), b)


def test_argsort_stable_with_ties(dev):
    g = torch.Generator().manual_seed(5)
    keys = torch.randint(0, 50, (4, 5000), generator=g).float()
    keys[1, ::7] = -3.5
    keys[2, :] = 0.0
    keys[3, ::3] = -0.0
    got = sfc.argsort(keys.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), keys.sort(dim=1, stable=True)[1])


def test_non_anchor_orders(dev):
    """use_anchor=False on integer grid tokens: the ranking is the sorted curve keys."""
    from oracle import sfc as osfc
    side = 27
    ys, xs = torch.meshgrid(torch.arange(side), torch.arange(side), indexing="ij")
    pos = torch.stack([xs, ys], -1).reshape(1, -1, 2).float()
    perm = torch.randperm(side * side, generator=torch.Generator().manual_seed(2))
    pos = pos[:, perm].to(dev)
    for sf in ("", "peano"):
        r = space_filling_cluster(pos, 9, side, side, sf_type=sf, use_anchor=False)[4][0, :, 0]
        key = osfc.peano_keys(side, side, pos)[0] if sf else osfc.scanline_keys(side, side, pos)[0].float()
        assert torch.equal(r, key.sort(stable=True)[1])


def test_hilbert_wide_canvas_rejected(dev):
    pos = torch.rand(1, 10, 2, device=dev) * 4
    with pytest.raises(NotImplementedError):
        sfc.curve_keys(pos, sfc.CURVES["hilbert"], 4, 16)
