"""AFF layer pieces with the reference's signatures (src/layers/aff.py).

``neighbourhood_index`` is the index construction of BasicLayer.forward
(aff.py:414-465): space-filling clustering, nearest-cluster KNN and the
fused member / mask / pe_idx gather.  ``ClusterMerging`` is the AFF
downsampling layer (aff.py:122-299).

``ClusterMerging`` keeps the constructor, forward signature and parameter
names (``weight_net``, ``norm``, ``linear``, ``global_norm``,
``global_linear``) of the reference so state_dicts load unchanged.  Token
selection, index gathers and the small ``weight_net`` table evaluation are
torch ops as in the reference; the merge itself, ``weighted_features``, runs
on the HIP kernel.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from ..kernels.knn import knn
from ..kernels.nbhd_index import cluster_members
from ..kernels.weighted_features import weighted_features
from ..utils.geometry import space_filling_cluster
from ..utils.pos_embed import REL_POS_WIDTH, TABLE_WIDTH, pre_table_fp32


def neighbourhood_index(pos, feat, h, w, cluster_size, nbhd_size, global_attention=False):
    """Neighbourhood construction of BasicLayer.forward (reference
    src/layers/aff.py:414-465), before its attention blocks run.

    pos [b,n,2], feat [b,n,c] on an h x w canvas.  Tokens are clustered along
    the space-filling curve into k = ceil(n / cluster_size) clusters (tokens
    and features reordered so that each cluster is contiguous), every token's
    nnc = min(round(nbhd_size / cluster_size), k) nearest cluster centres are
    found by the exact KNN kernel, and one fused kernel gathers their members,
    padding mask and relative-position table index.  Returns
    (pos, feat, member_idx [b,n,nnc*m] int64, cluster_mask [b,n,nnc*m] int64
    or None, pe_idx int64, global_attn, nbhd_size): the neighbourhood size is
    rounded to a multiple of the cluster size as in the reference, and when it
    covers every token (global attention) pe_idx is the dense [b,n,n] index.
    The reference's training-time cache of the first stage's clustering is a
    pure reuse of the same result and is not kept here.
    """
    b, n, d = pos.shape
    c = feat.shape[2]
    assert cluster_size > 0, "cluster_size must be positive"
    global_attn = bool(global_attention) or nbhd_size >= n
    k = int(math.ceil(n / float(cluster_size)))
    nnc = min(int(round(nbhd_size / float(cluster_size))), k)
    nbhd = cluster_size * nnc
    if k == n:
        cluster_mean_pos = pos
        members = torch.arange(n, device=pos.device).reshape(1, n, 1).expand(b, -1, -1)
        cmask = None
    else:
        pos, cluster_mean_pos, members, cmask, reorder = space_filling_cluster(pos, cluster_size, h, w,
                                                                               no_reorder=False)
        feat = feat.gather(1, reorder.expand(-1, -1, c))
    assert members.shape[1] == k and members.shape[2] == cluster_size, "member_idx shape incorrect!"
    nearest = knn(pos, cluster_mean_pos, nnc)
    member_idx, cluster_mask, pe_idx = cluster_members(nearest, members, cmask, pos, with_pe=not global_attn)
    if global_attn:
        rel = ((pos[:, None, :, :] + REL_POS_WIDTH) - pos[:, :, None, :]).clamp(0, TABLE_WIDTH - 1)
        pe_idx = (rel[..., 1] * TABLE_WIDTH + rel[..., 0]).long()
    return pos, feat, member_idx, cluster_mask, pe_idx, global_attn, nbhd


class ClusterMerging(nn.Module):
    """Adaptive downsampling: keep int(n * ds_rate) tokens and merge each one's
    neighbourhood with learned position-dependent weights."""

    def __init__(self, dim, out_dim, norm_layer=nn.LayerNorm, alpha=4.0, ds_rate=0.25, reserve_on=True):
        super().__init__()
        self.dim = dim
        self.pos_dim = 2
        self.alpha = alpha
        self.ds_rate = ds_rate
        self.reserve_on = reserve_on
        inner_ch = 4
        self.weight_net = nn.Sequential(
            nn.Linear(self.pos_dim + 3, inner_ch, bias=True),
            nn.LayerNorm(inner_ch),
            nn.GELU(),
        )
        self.norm = norm_layer(inner_ch * dim)
        self.linear = nn.Linear(dim * inner_ch, out_dim)
        self.global_norm = norm_layer(dim)
        self.global_linear = nn.Linear(dim, out_dim)
        self._weights_table_cache = {}

    def clear_weights_cache(self):
        self._weights_table_cache.clear()

    def _weights_table(self, device, dtype):
        key = (device, dtype)
        if not self.training and key in self._weights_table_cache:
            return self._weights_table_cache[key]
        tab = self.weight_net(pre_table_fp32.to(device=device, dtype=dtype))
        if not self.training:
            self._weights_table_cache[key] = tab
        return tab

    def forward(self, pos, feat, member_idx, cluster_mask, learned_prob, stride, pe_idx, reserve_num):
        """pos [b,n,2], feat [b,n,c], member_idx/cluster_mask/pe_idx [b,n,nbhd],
        learned_prob [b,n,1] -> (pos_down [b,n',2], feat_down [b,n',out_dim])."""
        b, n, c = feat.shape
        d = pos.shape[2]
        keep_num = int(n * self.ds_rate)
        pos_long = pos.long()
        if torch.is_autocast_enabled():
            cast_dtype = torch.get_autocast_dtype("cuda") or torch.float16
        else:
            cast_dtype = torch.float32

        final_prob = None
        if learned_prob is not None:
            final_prob = learned_prob.detach().view(b, n)
        if self.reserve_on:
            reserve_mask = ((pos_long % (stride * 2)) == 0).all(dim=-1).to(cast_dtype)
            final_prob = final_prob + (reserve_mask * (-100))
            sample_num = keep_num - reserve_num
        else:
            sample_num = keep_num

        sample_idx = final_prob.topk(sample_num, dim=1, sorted=False)[1]
        if self.reserve_on:
            reserve_idx = reserve_mask.nonzero(as_tuple=True)[1].reshape(b, reserve_num)
            idx = torch.cat([sample_idx, reserve_idx], dim=-1).unsqueeze(2)
        else:
            idx = sample_idx.unsqueeze(2)
        n_down = idx.shape[1]
        assert n_down == keep_num, "n not equal to keep num!"
        pos_down = pos.gather(index=idx.expand(-1, -1, d), dim=1)

        if member_idx is None:
            feat_down = feat.gather(index=idx.expand(-1, -1, c), dim=1)
            feat_down = self.global_linear(self.global_norm(feat_down))
            return pos_down, feat_down

        nbhd_size = member_idx.shape[-1]
        member_idx = member_idx.gather(index=idx.expand(-1, -1, nbhd_size), dim=1)
        pe_idx = pe_idx.gather(index=idx.expand(-1, -1, nbhd_size), dim=1)
        if cluster_mask is not None:
            cluster_mask = cluster_mask.gather(index=idx.expand(-1, -1, nbhd_size), dim=1)
        lp = None
        if learned_prob is not None:
            lp = learned_prob.gather(index=member_idx.view(b, -1, 1), dim=1).reshape(b, n_down, nbhd_size, 1)

        weights_table = self._weights_table(pe_idx.device, feat.dtype)
        inner_ch = weights_table.shape[-1]
        weights = weights_table.gather(index=pe_idx.reshape(-1, 1).expand(-1, inner_ch), dim=0)
        weights = weights.reshape(*pe_idx.shape, inner_ch)
        if lp is not None:
            if cluster_mask is not None:
                lp = lp * cluster_mask.unsqueeze(3)
            weights = weights * lp
        elif cluster_mask is not None:
            weights = weights * cluster_mask.unsqueeze(3)

        feat_down = weighted_features(weights, feat, member_idx.view(b, n_down, -1)).reshape(b, n_down, -1)
        feat_down = self.norm(feat_down)
        feat_down = self.linear(feat_down)
        return pos_down, feat_down
