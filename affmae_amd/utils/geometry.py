"""Geometry helpers on the hot path (reference src/utils/geometry.py).

``inverse_distance_weighting`` (geometry.py:40-53) is elementwise torch
work; ``upsample_feature_shepard`` (geometry.py:97-167) runs the HIP KNN and
weighted-gather kernels.
"""
from __future__ import annotations

import torch

from ..kernels.knn import knn as hip_knn
from ..kernels.weighted_gather import weighted_gather


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
