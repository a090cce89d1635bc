"""Geometry helpers on the hot path (reference src/utils/geometry.py).

``inverse_distance_weighting`` (geometry.py:40-53) is elementwise torch
work; ``upsample_feature_shepard`` (geometry.py:97-167) runs the HIP KNN and
weighted-gather kernels; ``space_filling_cluster`` (geometry.py:170-319) is
the token ordering and balanced clustering the encoder runs before every
stage's attention blocks (aff.py:436-446): its curve keys and sort run on
the HIP kernels (aff_sfc_*), the gathers and cluster means are torch.
"""
from __future__ import annotations

import math

import torch

from ..kernels.knn import knn as hip_knn
from ..kernels.weighted_gather import weighted_gather


def knn_keops(query, database, k, return_dist=False):
    """geometry.py:56-95: int64 indices [b,n_,k] of the k nearest database points and,
    with return_dist, their Euclidean distances (the reference's KeOps Kmin of
    sqrt(sum (q - x)^2)), from the exact HIP KNN in fp32, no autograd."""
    with torch.no_grad():
        q = query.detach().float()
        d = database.detach().float()
        if not return_dist:
            return hip_knn(q, d, k)
        idx, d2 = hip_knn(q, d, k, return_dist=True)
        return idx, d2.sqrt()


def inverse_distance_weighting(dist, power=3):
    """w = (1 / (d^p + 1e-10)) / (sum + 1e-12) in fp32 (callers pass squared distances)."""
    with torch.autocast(device_type=dist.device.type, enabled=False):
        dist = dist.to(torch.float32)
        ipd = 1.0 / (dist.pow(power) + 1e-10)
        return ipd / (ipd.sum(dim=2, keepdim=True) + 1e-12)


def upsample_feature_shepard(query, database, feature, database_idx=None, k=4, power=3,
                             custom_kernel=True, nn_idx=None, return_weight_only=False):
    """Interpolate database features at query positions from their k nearest
    database points with inverse-distance weights (geometry.py:97-167)."""
    b, n_, d = database.shape
    n = query.shape[1]
    with torch.autocast(device_type=query.device.type, enabled=False):
        database = database.to(torch.float32)
        query = query.to(torch.float32)
        if nn_idx is not None:
            k = nn_idx.shape[-1]
        else:
            k = min(k, n_)
            nn_idx = hip_knn(query, database, k=k, return_dist=False)
        nn_pos = database.gather(index=nn_idx.view(b, -1, 1).expand(-1, -1, 2), dim=1).reshape(b, n, k, d)
        nn_dist = (query.unsqueeze(2) - nn_pos).pow(2).sum(-1)
        nn_weights = inverse_distance_weighting(nn_dist, power=power)
        if return_weight_only:
            return nn_weights
        c = feature.shape[-1]
        assert feature.shape[1] == n_
        if custom_kernel:
            up = weighted_gather(nn_idx, nn_weights, feature)
        else:
            nn_f = feature.gather(index=nn_idx.view(b, -1).unsqueeze(2).expand(-1, -1, c), dim=1).reshape(b, n, k, c)
            up = nn_f.mul(nn_weights.unsqueeze(3)).sum(dim=2).to(feature.dtype)
        if database_idx is not None:
            up.scatter_(dim=1, index=database_idx.long().expand(-1, -1, c), src=feature)
        return up


def _scanline_rank(nh: int, nw: int, width: int, device) -> torch.Tensor:
    """Rank of each cell of an nh x nw grid (row-major ids) along horizontal
    scanlines whose direction alternates per row (geometry.py:217-229: the
    sort key is x + y*width on even rows and (width-1) - x + y*width on odd rows)."""
    ys, xs = torch.meshgrid(torch.arange(nh, device=device), torch.arange(nw, device=device), indexing="ij")
    odd = (ys % 2) == 1
    key = torch.where(odd, (width - 1) - xs, xs) + ys * width
    order = key.reshape(-1).sort()[1]
    rank = torch.empty_like(order)
    rank[order] = torch.arange(order.numel(), device=device)
    return rank, order


def _anchor_grid(n, m, h, w, sf_type):
    """Patch grid of the anchor ordering (geometry.py:203-216): (rows, cols, row
    height, column width); Peano / Hilbert round the rows to a power of 3 / 2."""
    k = int(math.ceil(n / m))
    patch_len = (h * w / k) ** 0.5
    nph = int(round(h / patch_len))
    npw = int(round(w / patch_len))
    plh, plw = h / nph, w / npw
    if sf_type in ("peano", "hilbert"):
        base = 3 if sf_type == "peano" else 2
        nph = max(base, int(base ** round(math.log(nph, base))))
        plh = h / nph
        npw = int(round(w / h * base) * (nph / base))
        plw = w / npw
    return nph, npw, plh, plw


def _neighbour_centres(ordered_grid, plw, plh, dev):
    """Patch centres in curve order and those of the previous / next patch on the
    curve, extrapolated at both ends (geometry.py:238-248)."""
    # per-column scalars (no host-to-device copy, so the ordering can be graph-captured);
    # the same fp32 products and sums as with a [plw, plh] tensor
    centres = torch.stack([ordered_grid[:, 0] * plw + plw / 2 - 0.5, ordered_grid[:, 1] * plh + plh / 2 - 0.5], -1)
    plhw = (plw, plh)
    npch = centres.shape[0]
    prev_c = torch.zeros_like(centres)
    prev_c[1:] = centres[:npch - 1]
    prev_c[0] = prev_c[1] - (prev_c[2] - prev_c[1])
    next_c = torch.zeros_like(centres)
    next_c[:npch - 1] = centres[1:]
    next_c[-1] = next_c[-2] + (next_c[-2] - next_c[-3])
    return plhw, prev_c, next_c


def _ranking_hip(pos, m, h, w, sf_type, use_anchor):
    """pos_ranking [b,n,1] of GPU tokens: curve / anchor keys and the argsort on the HIP kernels."""
    from ..kernels import sfc
    b, n, _ = pos.shape
    dev = pos.device
    curve = sfc.CURVES[sf_type]
    if not use_anchor:
        return sfc.argsort(sfc.curve_keys(pos, curve, h, w)).unsqueeze(2)
    nph, npw, plh, plw = _anchor_grid(n, m, h, w, sf_type)
    ys, xs = torch.meshgrid(torch.arange(nph, device=dev), torch.arange(npw, device=dev), indexing="ij")
    grid = torch.stack([xs, ys], dim=2).reshape(-1, 2)
    if curve == sfc.CURVES[""]:
        rank, order = _scanline_rank(nph, npw, w, dev)
    else:
        order = sfc.argsort(sfc.curve_keys(grid.float().unsqueeze(0), curve, nph, npw))[0]
        rank = torch.empty_like(order)
        rank[order] = torch.arange(order.numel(), device=dev)
    _, prev_c, next_c = _neighbour_centres(grid[order], plw, plh, dev)
    keys = sfc.anchor_keys(pos, plw, plh, npw, rank, prev_c, next_c)
    return sfc.argsort(keys).unsqueeze(2)


def _ranking_torch(pos, m, h, w, use_anchor):
    """pos_ranking [b,n,1] of CPU tokens along the scanline curve (the host-side
    ordering of synthetic inputs; GPU tokens take the HIP kernels)."""
    b, n, d = pos.shape
    dev = pos.device
    if use_anchor:
        nph, npw, plh, plw = _anchor_grid(n, m, h, w, "")
        rank, order = _scanline_rank(nph, npw, w, dev)
        ys, xs = torch.meshgrid(torch.arange(nph, device=dev), torch.arange(npw, device=dev), indexing="ij")
        grid = torch.stack([xs, ys], dim=2).reshape(-1, 2)[order]          # cells in curve order
        plhw, prev_c, next_c = _neighbour_centres(grid, plw, plh, dev)
        cell = (pos / torch.tensor(plhw, dtype=torch.float32, device=dev)).floor()
        cell = (cell[..., 0] + cell[..., 1] * npw).long()                  # row-major patch id
        prank = rank.unsqueeze(0).expand(b, -1).gather(1, cell)             # b x n
        d_prev = (pos - prev_c[prank]).pow(2).sum(-1)
        d_next = (pos - next_c[prank]).pow(2).sum(-1)
        ratio = d_prev / (d_next + 1e-5)
        key = prank.unsqueeze(2) * (ratio.max() + 1) + ratio.unsqueeze(2)
        return key.sort(dim=1, stable=True)[1]
    rank, _ = _scanline_rank(h, w, w, dev)
    pid = (pos[..., 0] + pos[..., 1] * w).long().reshape(-1)
    return rank.gather(0, pid).reshape(b, n).sort(stable=True)[1].unsqueeze(2)


def space_filling_cluster(pos, m, h, w, no_reorder=False, sf_type="", use_anchor=True):
    """Balanced clustering along a space-filling curve (geometry.py:170-319).

    pos [b,n,2] token positions (x, y) on an h x w canvas, m the cluster size.
    With anchors (the default, used by the encoder) the canvas is cut into
    ~n/m patches visited along the curve (alternating horizontal scanlines
    for sf_type '', or the Peano / Hilbert curve); a token's rank is its
    patch's rank, ties inside a patch broken by the ratio of its squared
    distances to the previous and next patch centres (geometry.py:199-268).
    Without anchors the tokens themselves are ordered along the curve.  Keys
    and sort run on the HIP kernels for GPU tokens (equal keys keep the lower
    token index first); CPU tokens (synthetic input generation) are ordered
    by torch along the scanline curve.  Returns, like the reference,
      no_reorder=False: (pos reordered, cluster_mean_pos [b,k,2],
                         member_idx [b,k,m], cluster_mask [b,k,m] or None,
                         pos_ranking [b,n,1])
      no_reorder=True:  (cluster_mean_pos, member_idx, cluster_mask)
    """
    if sf_type not in ("", "peano", "hilbert"):
        sf_type = ""          # the reference treats every other value as the scanline curve
    with torch.no_grad():
        pos = pos.detach()
        if pos.dtype != torch.float:
            pos = pos.to(torch.float)
        b, n, d = pos.shape
        k = int(math.ceil(n / m))
        dev = pos.device
        if pos.is_cuda:
            pos_ranking = _ranking_hip(pos, m, h, w, sf_type, use_anchor)
        else:
            if sf_type:
                raise NotImplementedError("space_filling_cluster: Peano / Hilbert orders run on GPU tokens only")
            pos_ranking = _ranking_torch(pos, m, h, w, use_anchor)

        pos = pos.gather(1, pos_ranking.expand(-1, -1, d))
        if k * m == n:
            cluster_mask = None
            cluster_mean_pos = pos.reshape(b, k, m, d).mean(2)
        else:
            pos_pad = torch.zeros(b, k * m, d, dtype=pos.dtype, device=dev)
            pos_pad[:, :n] = pos
            cluster_mask = torch.zeros(b, k * m, device=dev).long()
            cluster_mask[:, :n] = 1
            cluster_mask = cluster_mask.reshape(b, k, m)
            cluster_mean_pos = pos_pad.reshape(b, k, m, d).sum(2) / cluster_mask.sum(2, keepdim=True)

        if no_reorder:
            if k * m == n:
                member_idx = pos_ranking.reshape(b, k, m)
            else:
                member_idx = torch.zeros(b, k * m, device=dev, dtype=torch.int64)
                member_idx[:, :n] = pos_ranking.squeeze(2)
                member_idx = member_idx.reshape(b, k, m)
            return cluster_mean_pos, member_idx, cluster_mask
        member_idx = torch.arange(k * m, device=dev)
        member_idx[n:] = 0
        member_idx = member_idx.unsqueeze(0).expand(b, -1).reshape(b, k, m)
        return pos, cluster_mean_pos, member_idx, cluster_mask, pos_ranking
