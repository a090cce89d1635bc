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
import torch.nn.functional as F

from ..kernels.knn import knn
from ..kernels.layer_norm import layer_norm_map, norm
from ..kernels.nbhd_index import cluster_members
from ..kernels.weighted_features import weighted_features
from ..utils.geometry import space_filling_cluster
from ..utils.pos_embed import REL_POS_WIDTH, TABLE_WIDTH, pre_table_fp32
from .attention import ClusterAttention


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
        self.weight_net[0].inp = 'norm'     # initialisation tags read by AFFEncoder.init_weights
        self.norm = norm_layer(inner_ch * dim)
        self.linear = nn.Linear(dim * inner_ch, out_dim)
        self.linear.inp = 'norm'
        self.global_norm = norm_layer(dim)
        self.global_linear = nn.Linear(dim, out_dim)
        self.global_linear.inp = 'norm'
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
            feat_down = self.global_linear(norm(self.global_norm, feat_down, to_autocast=True))
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
        # element gather of table rows (an index_select of 4-wide rows launches one block per row)
        flat = pe_idx.unsqueeze(-1) * inner_ch + torch.arange(inner_ch, device=pe_idx.device)
        weights = torch.take(weights_table, flat)
        if lp is not None:
            if cluster_mask is not None:
                lp = lp * cluster_mask.unsqueeze(3)
            weights = weights * lp
        elif cluster_mask is not None:
            weights = weights * cluster_mask.unsqueeze(3)

        feat_down = weighted_features(weights, feat, member_idx.view(b, n_down, -1)).reshape(b, n_down, -1)
        feat_down = norm(self.norm, feat_down, to_autocast=True)
        feat_down = self.linear(feat_down)
        return pos_down, feat_down


# ------------------------------------------------------------------- encoder --
# The AFF encoder (reference src/layers/aff.py:21-120, 302-508, 511-736):
# transformer blocks over each token's neighbourhood, one BasicLayer per
# stage, the masked convolutional patch embedding and the 4-stage encoder.
# GEMMs, LayerNorm, GELU and the convolutions are torch; KNN, the
# neighbourhood gathers, the attention and the merge run on the HIP kernels.

class DropPath(nn.Module):
    """Stochastic depth per sample (timm's DropPath, which the reference's blocks use,
    aff.py:12, 68): in training each sample's branch is dropped with probability p
    and the kept ones are scaled by 1 / (1 - p); identity in eval mode."""

    def __init__(self, drop_prob: float = 0.):
        super().__init__()
        self.drop_prob = float(drop_prob)

    def forward(self, x):
        if self.drop_prob == 0. or not self.training:
            return x
        keep = 1.0 - self.drop_prob
        gate = x.new_empty((x.shape[0],) + (1,) * (x.dim() - 1)).bernoulli_(keep)
        return x * gate / keep


class Mlp(nn.Module):
    """fc1 -> act -> drop -> fc2 -> drop (aff.py:21-39)."""

    def __init__(self, in_features, hidden_features=None, out_features=None, act_layer=nn.GELU, drop=0.):
        super().__init__()
        out_features = out_features or in_features
        hidden_features = hidden_features or in_features
        self.fc1 = nn.Linear(in_features, hidden_features)
        self.fc1.inp = 'norm'
        self.act = act_layer()
        self.fc2 = nn.Linear(hidden_features, out_features)
        self.fc2.inp = 'act'
        self.drop = nn.Dropout(drop)

    def forward(self, x):
        return self.drop(self.fc2(self.drop(self.act(self.fc1(x)))))


class ClusterTransformerBlock(nn.Module):
    """Pre-norm block: x + attn(norm1(x)), then + mlp(norm2(x)), with optional layer
    scale and stochastic depth (aff.py:42-120)."""

    def __init__(self, dim, num_heads, mlp_ratio=2., drop=0., attn_drop=0., drop_path=0., layer_scale=0.0,
                 act_layer=nn.GELU, norm_layer=nn.LayerNorm):
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.mlp_ratio = mlp_ratio
        self.norm1 = norm_layer(dim)
        self.attn = ClusterAttention(dim, num_heads=num_heads, proj_drop=drop)
        self.drop_path = DropPath(drop_path) if drop_path > 0. else nn.Identity()
        self.norm2 = norm_layer(dim)
        self.mlp = Mlp(in_features=dim, hidden_features=int(dim * mlp_ratio), act_layer=act_layer, drop=drop)
        self.layer_scale = False
        if layer_scale is not None and type(layer_scale) in (int, float) and layer_scale > 0:
            self.layer_scale = True
            self.gamma1 = nn.Parameter(layer_scale * torch.ones(dim), requires_grad=True)
            self.gamma2 = nn.Parameter(layer_scale * torch.ones(dim), requires_grad=True)

    def forward(self, feat, member_idx, cluster_mask, pe_idx, global_attn):
        """feat [b,n,c]; member_idx / cluster_mask / pe_idx [b,n,nbhd] -> [b,n,c]."""
        b, n, c = feat.shape
        assert c == self.dim, "dim does not accord to input"
        a = self.attn(feat=norm(self.norm1, feat, to_autocast=True), member_idx=member_idx,
                      cluster_mask=cluster_mask, pe_idx=pe_idx, global_attn=global_attn)
        if self.layer_scale:
            feat = feat + self.drop_path(self.gamma1 * a)
            return feat + self.drop_path(self.gamma2 * self.mlp(norm(self.norm2, feat, to_autocast=True)))
        feat = feat + self.drop_path(a)
        return feat + self.drop_path(self.mlp(norm(self.norm2, feat, to_autocast=True)))

    def extra_repr(self) -> str:
        return f"dim={self.dim}, num_heads={self.num_heads}, mlp_ratio={self.mlp_ratio}"


class L2NormMerging(nn.Module):
    """Parameter-free downsampling (aff.py:302-334): the int(ds_rate * n) tokens of
    largest L2 norm are marked with a learned embedding before the stage's last
    block and kept after it."""

    def __init__(self, dim, ds_rate=0.4):
        super().__init__()
        self.ds_rate = ds_rate
        self.token_selection_embedding = nn.Parameter(torch.zeros(1, 1, dim))
        nn.init.normal_(self.token_selection_embedding, std=0.02)

    def forward(self, feat):
        b, n, c = feat.shape
        keep = int(self.ds_rate * n)
        scores = torch.norm(feat, p=2, dim=-1)
        _, indices = scores.topk(keep, dim=1)
        marked = torch.zeros_like(scores).scatter_(1, indices, 1.0)
        return feat + marked.unsqueeze(-1) * self.token_selection_embedding, indices


class BasicLayer(nn.Module):
    """One encoder stage (aff.py:337-508): neighbourhood construction, `depth`
    ClusterTransformerBlocks over it, then the downsampling to the next stage."""

    def __init__(self, dim, out_dim, cluster_size, nbhd_size, depth, num_heads, mlp_ratio,
                 alpha=4.0, ds_rate=0.25, reserve_on=False, global_attention=False, drop=0., attn_drop=0.,
                 drop_path=0., norm_layer=nn.LayerNorm, layer_scale=0.0, downsample=None):
        super().__init__()
        self.dim = dim
        self.nbhd_size = nbhd_size
        self.cluster_size = cluster_size
        self.depth = depth
        self.global_attention = global_attention
        self.blocks = nn.ModuleList([
            ClusterTransformerBlock(dim=dim, num_heads=num_heads, mlp_ratio=mlp_ratio, drop=drop,
                                    attn_drop=attn_drop,
                                    drop_path=drop_path[i] if isinstance(drop_path, list) else drop_path,
                                    layer_scale=layer_scale, norm_layer=norm_layer)
            for i in range(depth)])
        if downsample is None:
            self.downsample = None
        elif issubclass(downsample, ClusterMerging):
            self.downsample = downsample(dim=dim, out_dim=out_dim, norm_layer=norm_layer, alpha=alpha,
                                         ds_rate=ds_rate, reserve_on=reserve_on)
            self.prob_net = nn.Linear(dim, 1)
            self.prob_net.inp = 'norm'
        elif issubclass(downsample, L2NormMerging):
            self.downsample = downsample(dim=dim, ds_rate=ds_rate)
            self.downsample_norm = norm_layer(dim)
            self.downsample_proj = nn.Linear(dim, out_dim)
            self.downsample_proj.inp = "norm"
        else:
            raise ValueError(f"{downsample} method not supported!")
        self.ds_rate = ds_rate

    def forward(self, pos, feat, h, w, on_grid, stride):
        """pos [b,n,2], feat [b,n,c] on an h x w canvas; stride of the current token
        set.  Returns (pos, feat, pos_down, feat_down): the stage's tokens in
        cluster order and the downsampled set (the same tensors when the stage
        has no downsampling).  ``on_grid`` selects the reference's training-time
        reuse of the first stage's clustering, which is a cache of the same
        result: the clustering is simply recomputed here."""
        assert self.cluster_size > 0, 'self.cluster_size must be positive'
        pos, feat, member_idx, cluster_mask, pe_idx, global_attn, nbhd = neighbourhood_index(
            pos, feat, h, w, self.cluster_size, self.nbhd_size, self.global_attention)
        # the reference keeps the rounded neighbourhood size (aff.py:431)
        self.nbhd_size = nbhd

        selection = None
        for i, blk in enumerate(self.blocks):
            if i == len(self.blocks) - 1 and isinstance(self.downsample, L2NormMerging):
                feat, selection = self.downsample(feat)
            feat = blk(feat=feat, member_idx=member_idx, cluster_mask=cluster_mask, pe_idx=pe_idx,
                       global_attn=global_attn)

        if self.downsample is None:
            return pos, feat, pos, feat
        if isinstance(self.downsample, L2NormMerging):
            if selection is None:        # a stage without blocks selects nothing (as in the reference)
                return pos, feat, pos, feat
            feat_down = feat.gather(1, selection.unsqueeze(-1).expand(-1, -1, feat.shape[-1]))
            pos_down = pos.gather(1, selection.unsqueeze(-1).expand(-1, -1, pos.shape[-1]))
            return pos, feat, pos_down, self.downsample_proj(norm(self.downsample_norm, feat_down, to_autocast=True))
        learned_prob = self.prob_net(feat).sigmoid()
        reserve_num = math.ceil(h / (stride * 2)) * math.ceil(w / (stride * 2))
        pos_down, feat_down = self.downsample(pos=pos, feat=feat, member_idx=member_idx,
                                              cluster_mask=cluster_mask, learned_prob=learned_prob,
                                              stride=stride, pe_idx=pe_idx, reserve_num=reserve_num)
        return pos, feat, pos_down, feat_down

    def extra_repr(self) -> str:
        return f"dim={self.dim}, depth={self.depth}"


class LayerNorm2dImages(nn.Module):
    """LayerNorm over the channels of a [B,C,H,W] map (aff.py:511-526)."""

    def __init__(self, num_channels: int, eps: float = 1e-5):
        super().__init__()
        self.ln = nn.LayerNorm(num_channels, eps=eps)

    def forward(self, x):
        return self.ln(x.permute(0, 2, 3, 1)).permute(0, 3, 1, 2)


class AFFPatchEmbed(nn.Module):
    """Masked patch embedding (aff.py:529-640): log2(patch_size) stride-2 3x3
    convolutions, with LayerNorm + GELU between them; after every convolution the
    masked tokens' regions of the map are zeroed, so nothing of a masked patch
    leaks into a visible one.  Returns token positions (x, y) on the token grid,
    the [b, h*w, embed_dim] tokens, and the grid size h, w."""

    def __init__(self, img_size=None, patch_size=8, in_chans=3, embed_dim=768, norm_layer=None):
        super().__init__()
        if patch_size <= 0 or (patch_size & (patch_size - 1)) != 0:
            raise ValueError(f"patch_size must be a power of 2, but got {patch_size}")
        self.patch_size = patch_size
        self.num_patches = None
        if img_size is not None:
            hw = (img_size, img_size) if isinstance(img_size, int) else tuple(img_size)
            self.num_patches = (hw[0] // patch_size) * (hw[1] // patch_size)
        n_conv = int(math.log2(patch_size))
        self.projs = nn.ModuleList()
        self.lns = nn.ModuleList()
        self.acts = nn.ModuleList()
        self.norm = norm_layer(embed_dim) if norm_layer is not None else None
        ch = in_chans
        for i in range(n_conv):
            last = i == n_conv - 1
            out_ch = embed_dim if last else embed_dim // 2
            self.projs.append(nn.Conv2d(ch, out_ch, kernel_size=3, stride=2, padding=1))
            if not last:
                self.lns.append(LayerNorm2dImages(out_ch))
                self.acts.append(nn.GELU())
            ch = out_ch

    def _fused(self, x) -> bool:
        """Inference on a GPU with LayerNorm2dImages + exact GELU between the
        convolutions and a final LayerNorm: each mask / norm / GELU step runs as
        one HIP kernel."""
        if self.norm is None or not isinstance(self.norm, nn.LayerNorm) or not x.is_cuda:
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        if any(not isinstance(a, nn.GELU) or a.approximate != "none" for a in self.acts):
            return False
        chans = [ln.ln.normalized_shape[0] for ln in self.lns] + [self.norm.normalized_shape[0]]
        return all(c <= 64 for c in chans) and all(isinstance(ln, LayerNorm2dImages) for ln in self.lns)

    def forward(self, x, ids_masked):
        ps = self.patch_size
        H, W = x.shape[-2:]
        if W % ps:
            x = F.pad(x, (0, ps - W % ps))
        if H % ps:
            x = F.pad(x, (0, 0, 0, ps - H % ps))
        th, tw = x.shape[-2] // ps, x.shape[-1] // ps          # token grid
        keep = None
        if ids_masked is not None:
            B = x.shape[0]
            keep = torch.ones(B, th * tw, device=x.device, dtype=x.dtype)
            keep.scatter_(1, ids_masked, 0.0)
            keep = keep.view(B, 1, th, tw)
        fused = self._fused(x)
        for i, proj in enumerate(self.projs):
            x = proj(x)
            cell = max(ps >> (i + 1), 1)                       # map pixels per token side at this depth
            last = i == len(self.projs) - 1
            if fused:
                # mask, LayerNorm (+ GELU) in one pass; the last one writes the tokens [b, h*w, c]
                ln = self.norm if last else self.lns[i].ln
                to_ac = torch.is_autocast_enabled("cuda") and not last
                out_dtype = torch.get_autocast_dtype("cuda") if to_ac else (
                    torch.float32 if torch.is_autocast_enabled("cuda") else x.dtype)
                x = layer_norm_map(x, ln.weight, ln.bias, ln.eps, keep=keep, cell=cell, gelu=not last,
                                   token_major=last, out_dtype=out_dtype)
                continue
            if keep is not None:
                blocks = x.unflatten(3, (-1, cell)).unflatten(2, (-1, cell))   # b, c, th, cell, tw, cell
                x = (blocks * keep[:, :, :, None, :, None]).flatten(4, 5).flatten(2, 3)
            if i < len(self.lns):
                x = self.acts[i](self.lns[i](x))
        if fused:
            h, w = th, tw
            b = x.shape[0]
        else:
            b, c, h, w = x.shape
            x = x.flatten(2).transpose(1, 2)
            if self.norm is not None:
                x = self.norm(x)
        ys, xs = torch.meshgrid(torch.arange(h, device=x.device), torch.arange(w, device=x.device), indexing='ij')
        pos = torch.stack([xs, ys], dim=2).reshape(1, h * w, 2).expand(b, -1, -1).to(x.dtype)
        return pos, x, h, w


class AFFEncoder(nn.Module):
    """The 4-stage AFF encoder (aff.py:642-736).  forward(feat, pos, h, w) takes the
    visible tokens and their grid positions and returns, per stage i, the
    normalised stage output ``res{i+2}``, its positions ``res{i+2}_pos`` and the
    canvas size ``res{i+2}_spatial_shape``."""

    def __init__(self, img_size=384, patch_size=8, in_chans=1, embed_dims=(64, 128, 256, 448),
                 depths=(3, 3, 7, 4), num_heads=(2, 4, 8, 14), nbhd_sizes=(64, 64, 64, 64), cluster_size=8,
                 ds_rates=(0.4, 0.4, 0.4, 0.4), global_attention=False, drop_path_rate=0.1, alpha=10.0,
                 mlp_ratio=2, drop_rate=0, merging_method="l2norm"):
        super().__init__()
        embed_dims, depths, num_heads = list(embed_dims), list(depths), list(num_heads)
        nbhd_sizes, ds_rates = list(nbhd_sizes), list(ds_rates)
        self.num_layers = len(depths)
        self.patch_embed = AFFPatchEmbed(img_size=img_size, patch_size=patch_size, in_chans=in_chans,
                                         embed_dim=embed_dims[0], norm_layer=nn.LayerNorm)
        dpr = [x.item() for x in torch.linspace(0, drop_path_rate, sum(depths))]
        merging = {"l2norm": L2NormMerging, "cluster": ClusterMerging}.get(merging_method)
        if merging is None:
            raise ValueError(f"merging_method must be 'l2norm' or 'cluster', got {merging_method!r}")
        self.layers = nn.ModuleList()
        for i in range(self.num_layers):
            last = i == self.num_layers - 1
            self.layers.append(BasicLayer(
                dim=embed_dims[i], out_dim=None if last else embed_dims[i + 1], cluster_size=cluster_size,
                nbhd_size=nbhd_sizes[i], depth=depths[i], num_heads=num_heads[i], mlp_ratio=mlp_ratio,
                alpha=alpha, ds_rate=ds_rates[i], global_attention=global_attention, drop=drop_rate,
                downsample=None if last else merging,
                drop_path=dpr[sum(depths[:i]):sum(depths[:i + 1])]))
        self.norms = nn.ModuleList([nn.LayerNorm(d) for d in embed_dims])
        self.init_weights()

    def init_weights(self):
        """Tag-driven initialisation (aff.py:693-711): Linear layers tagged 'special',
        'norm', 'attn' or 'act' get their weight initialiser; untagged Linear biases
        are zeroed; norms start at weight 1, bias 0."""
        for m in self.modules():
            if isinstance(m, nn.Linear):
                tag = getattr(m, 'inp', None)
                if tag == 'special':
                    nn.init.normal_(m.weight, mean=0.0, std=0.3)
                    if m.bias is not None:
                        nn.init.constant_(m.bias, 0)
                elif tag == 'norm':
                    nn.init.xavier_uniform_(m.weight)
                elif tag == 'attn':
                    nn.init.trunc_normal_(m.weight, std=0.02)
                elif tag == 'act':
                    nn.init.kaiming_uniform_(m.weight, a=math.sqrt(5))
                elif tag is None and m.bias is not None:
                    nn.init.constant_(m.bias, 0)
            elif isinstance(m, (nn.LayerNorm, nn.GroupNorm, nn.BatchNorm2d)):
                if m.bias is not None:
                    nn.init.constant_(m.bias, 0)
                if m.weight is not None:
                    nn.init.constant_(m.weight, 1.0)

    def forward(self, feat, pos, h, w):
        out = {}
        for i, layer in enumerate(self.layers):
            pos_out, x_out, pos, feat = layer(pos, feat, h=h, w=w, on_grid=False, stride=2 ** (i + 1))
            name = f"res{i + 2}"
            out[name] = norm(self.norms[i], x_out)
            out[f"{name}_pos"] = pos_out
            out[f"{name}_spatial_shape"] = (h, w)
        return out

    def forward_with_pos(self, feat, pos, h, w):
        """Positions of every stage's tokens (aff.py:728-736, token visualisation)."""
        stages = []
        for i, layer in enumerate(self.layers):
            pos_out, _, pos, feat = layer(pos, feat, h=h, w=w, on_grid=False, stride=2 ** (i + 1))
            stages.append(pos_out)
        return stages
