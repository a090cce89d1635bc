"""Seeded synthetic inputs for the benchmark configurations of the hot path.

Generators run on the CPU with explicit ``torch.Generator`` seeds (so every
machine produces the same inputs) and return CPU tensors; callers move them
to the device.  Seeds: coordinates 0, features 1, weights 2, selection 3.
"""
from __future__ import annotations

import math

import torch


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def cfg1_coords(B: int = 2, N: int = 1024, seed: int = 0) -> torch.Tensor:
    """Config 1: N points uniform in [0, 1)^2, fp32 [B, N, 2]."""
    return torch.rand((B, N, 2), generator=_gen(seed), dtype=torch.float32)


def jittered_grid(B: int, side: int, keep: int, seed: int = 0, order: str = "sfc") -> torch.Tensor:
    """Config 2 coordinates: keep `keep` of side*side cells per image (chosen
    without replacement), each at (col, row) + U(-0.5, 0.5).

    order "sfc" (default) lists the tokens the way the encoder hands them to
    its attention blocks: ordered by space_filling_cluster on the cells' grid
    positions with cluster size 8 (reference aff.py:436-446 reorders feat and
    pos by that ranking before the blocks run).  order "raster" lists them in
    row-major cell order.  Returns fp32 [B, keep, 2] in grid units.
    """
    from .utils.geometry import space_filling_cluster

    g = _gen(seed)
    out = torch.empty((B, keep, 2), dtype=torch.float32)
    for b in range(B):
        cells = torch.randperm(side * side, generator=g)[:keep].sort().values
        row = (cells // side).to(torch.float32)
        col = (cells % side).to(torch.float32)
        if order == "sfc":
            cxy = torch.stack([col, row], -1).unsqueeze(0)
            rank = space_filling_cluster(cxy, 8, side, side)[4][0, :, 0]
            col, row = col[rank], row[rank]
        elif order != "raster":
            raise ValueError(f"unknown token order {order!r}")
        jit = torch.rand((keep, 2), generator=g, dtype=torch.float32) - 0.5
        out[b, :, 0] = col + jit[:, 0]
        out[b, :, 1] = row + jit[:, 1]
    return out


def cfg2(B: int = 32, N: int = 6272, H: int = 4, D: int = 32, dtype=torch.bfloat16, order: str = "sfc"):
    """Config 2: neighbourhood attention at the stage-1 shape of a 448^2 image,
    patch 4, 50% mask (112 x 112 grid, 6272 visible tokens).

    Returns a dict of CPU tensors: pos [B,N,2] fp32, q/k/v [B,H,N,D] ~ N(0,1)
    in `dtype`, blank_k/blank_v [H,D] ~ N(0, 0.2^2), pos_w [H,5] and pos_b [H]
    (a seeded Linear(5, H) initialisation).
    """
    side = 112
    pos = jittered_grid(B, side, N, seed=0, order=order)
    g = _gen(1)
    q = torch.randn((B, H, N, D), generator=g).to(dtype)
    k = torch.randn((B, H, N, D), generator=g).to(dtype)
    v = torch.randn((B, H, N, D), generator=g).to(dtype)
    g2 = _gen(2)
    bound = 1.0 / math.sqrt(5)
    pos_w = (torch.rand((H, 5), generator=g2) * 2 - 1) * bound
    pos_b = (torch.rand((H,), generator=g2) * 2 - 1) * bound
    blank_k = (torch.randn((H, D), generator=g2) * 0.2).to(dtype)
    blank_v = (torch.randn((H, D), generator=g2) * 0.2).to(dtype)
    return dict(pos=pos, q=q, k=k, v=v, pos_w=pos_w, pos_b=pos_b, blank_k=blank_k, blank_v=blank_v)


def cfg3(B: int = 32, N: int = 6272, M: int = 2509, C: int = 128, dtype=torch.bfloat16):
    """Config 3: weighted-gather downsampling merge at ratio 0.4.

    Source tokens: config-2 coordinates normalised by the grid side (112) and
    features ~ N(0, 1) [B, N, C].  Merged points: M tokens per image drawn
    without replacement with probability proportional to an importance score
    U(0, 1) (seed 3), listed in source order; their coordinates are the
    selected tokens' coordinates.  Returns CPU tensors src_pos, feat, sel
    [B, M] int64, merged_pos.
    """
    src_pos = jittered_grid(B, 112, N, seed=0) / 112.0
    feat = torch.randn((B, N, C), generator=_gen(1)).to(dtype)
    g = _gen(3)
    sel = torch.empty((B, M), dtype=torch.int64)
    for b in range(B):
        imp = torch.rand(N, generator=g)
        sel[b] = torch.multinomial(imp, M, replacement=False, generator=g).sort().values
    merged_pos = src_pos.gather(1, sel.unsqueeze(-1).expand(-1, -1, 2))
    return dict(src_pos=src_pos, feat=feat, sel=sel, merged_pos=merged_pos)


def cfg4(B: int = 32, H: int = 8, C: int = 32, P: int = 4, level_sizes=(6272, 2509, 1004, 402),
         dtype=torch.bfloat16, side: int = 112):
    """Config 4: multi-level deformable cross-attention of a dense pixel decoder.

    Queries: the side x side grid cell centres ((i + 0.5) / side), identical for
    every image.  Level 0: config-2 coordinates normalised by the side; level
    l + 1: a seeded subset of level l (probability proportional to U(0, 1)
    importance, without replacement).  Values [B, sum N_l, H, C] ~ N(0, 1);
    offsets [B, Nq, H, L, P, 2] ~ N(0, 0.02); attention logits ~ N(0, 1)
    softmaxed over L * P.  Returns CPU tensors and level_start.
    """
    L = len(level_sizes)
    lv0 = jittered_grid(B, side, level_sizes[0], seed=0) / float(side)
    levels = [lv0]
    g = _gen(3)
    for l in range(1, L):
        prev = levels[-1]
        sub = torch.empty((B, level_sizes[l], 2), dtype=torch.float32)
        for b in range(B):
            imp = torch.rand(prev.shape[1], generator=g)
            sel = torch.multinomial(imp, level_sizes[l], replacement=False, generator=g).sort().values
            sub[b] = prev[b, sel]
        levels.append(sub)
    kv_pos = torch.cat(levels, dim=1)
    level_start = [0]
    for n in level_sizes:
        level_start.append(level_start[-1] + n)
    ax = (torch.arange(side, dtype=torch.float32) + 0.5) / side
    ys, xs = torch.meshgrid(ax, ax, indexing="ij")
    qpos = torch.stack([xs, ys], -1).reshape(1, side * side, 2).expand(B, -1, -1).contiguous()
    Nq = side * side
    gv = _gen(1)
    values = torch.randn((B, level_start[-1], H, C), generator=gv).to(dtype)
    go = _gen(2)
    offsets = (torch.randn((B, Nq, H, L, P, 2), generator=go) * 0.02).to(dtype)
    logits = torch.randn((B, Nq, H, L * P), generator=go)
    attn = torch.softmax(logits, dim=-1).reshape(B, Nq, H, L, P).to(dtype)
    return dict(query_pos=qpos, kv_pos=kv_pos, level_start=level_start, values=values, offsets=offsets, attn=attn)


def cfg5(B: int = 8, img: int = 1024, patch: int = 4, mask_ratio: float = 0.5, seed: int = 0):
    """Config 5: B single-channel img x img images ~ N(0, 1) (seed `seed`) and a
    per-image random patch mask (seed `seed` + 3) with the reference's
    random_masking semantics (src/utils/masking.py:12-24): the patches are
    ranked by U(0, 1) noise, the first int(L * (1 - mask_ratio)) of that order
    are kept (ids_keep, in noise order) and the rest masked (ids_masked).
    Returns a dict of CPU tensors: images [B,1,img,img] fp32, ids_keep and
    ids_masked [B, *] int64 over the (img/patch)^2 patch grid."""
    L = (img // patch) ** 2
    images = torch.randn((B, 1, img, img), generator=_gen(seed), dtype=torch.float32)
    noise = torch.rand((B, L), generator=_gen(seed + 3))
    order = torch.argsort(noise, dim=1)
    keep = int(L * (1 - mask_ratio))
    return {"images": images, "ids_keep": order[:, :keep].contiguous(), "ids_masked": order[:, keep:].contiguous()}


def mae_encode(encoder, images, ids_keep, ids_masked, patch: int):
    """The MAE's encoder front end (reference src/models/aff_mae.py:109-134): zero the
    masked patches of the images, run the masked patch embedding, keep the visible
    tokens (in ids_keep order) with their grid positions, run the encoder.
    Returns the encoder's output dict."""
    B, C, Hh, Ww = images.shape
    th, tw = Hh // patch, Ww // patch
    keep = torch.ones((B, th * tw), device=images.device, dtype=images.dtype)
    keep.scatter_(1, ids_masked, 0.0)
    blocks = images.reshape(B, C, th, patch, tw, patch) * keep.view(B, 1, th, 1, tw, 1)
    pos, feat, h, w = encoder.patch_embed(blocks.reshape(B, C, Hh, Ww), ids_masked)
    vis_feat = feat.gather(1, ids_keep.unsqueeze(-1).expand(-1, -1, feat.shape[-1]))
    vis_pos = pos.gather(1, ids_keep.unsqueeze(-1).expand(-1, -1, 2))
    return encoder(vis_feat, vis_pos, h, w)


def cfg5_encoder(**overrides):
    """The AFF-small encoder of config 5: patch 4, dims 64/128/256/512, heads
    2/4/8/16 (head_dim 32), depths 2/2/6/2, cluster 8, neighbourhood 48 (6
    nearest clusters), 0.4 weighted-gather (ClusterMerging) downsampling,
    random init (seed 2), no stochastic depth (inference)."""
    from .layers.aff import AFFEncoder
    kw = dict(img_size=1024, patch_size=4, in_chans=1, embed_dims=(64, 128, 256, 512), depths=(2, 2, 6, 2),
              num_heads=(2, 4, 8, 16), nbhd_sizes=(48, 48, 48, 48), cluster_size=8, ds_rates=(0.4, 0.4, 0.4, 0.4),
              drop_path_rate=0.0, merging_method="cluster")
    kw.update(overrides)
    torch.manual_seed(2)
    return AFFEncoder(**kw)
