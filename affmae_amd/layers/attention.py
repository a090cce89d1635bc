"""Attention modules with the reference's signatures (src/layers/attention.py).

``DeformableCrossAttention`` / ``DeformableSelfAttention`` (attention.py:210-593)
keep the reference's constructors, forwards, parameter names and
initialisation; their fused branch runs the in-kernel K-NN deformable
kernel, the other branches the given-index and MSDETRPC kernels.

``ClusterAttention`` keeps the constructor, forward signature, parameter and
buffer names of the reference (attention.py:20-207) so state_dicts load
unchanged.  Its local branch runs the HIP neighbourhood-attention kernel
directly on strided views of the q / kv projections: no head permute copies,
the relative-position bias gathered in-kernel from the [T*T, H] table by
pe_idx (the [B,H,N,M] bias is never materialised), the cluster mask
broadcast over heads without expansion, and the output written in [B,N,H,D]
order so the projection reads it without a permute.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.fused_deform_attn import (
    fused_deformable_attention,
    fused_knn_deformable_cross_attention,
    fused_knn_deformable_self_attention,
)
from ..kernels.knn import knn as hip_knn
from ..kernels.local_attn import nbhd_attn_proj_fwd, ClusterAttnFunction
from ..kernels.msdetrpc import MSDETRPCFunction
from ..utils.pos_embed import pre_table_fp16, pre_table_fp32


class ClusterAttention(nn.Module):
    """Local attention over each token's neighbourhood plus a per-head blank token."""

    # pos_embed builds the bias table in fp32 even under autocast (pe_table)
    fp32_submodules = ("pos_embed",)

    def __init__(self, dim, num_heads, proj_drop=0.):
        super().__init__()
        self.dim = dim
        self.pos_dim = 2
        self.num_heads = num_heads
        head_dim = dim // num_heads
        assert head_dim * num_heads == dim, "dim must be divisible by num_heads"
        self.scale = head_dim ** -0.5

        self.register_buffer('pre_table_fp32', pre_table_fp32.clone())
        self.register_buffer('pre_table_fp16', pre_table_fp16.clone())

        self.q = nn.Linear(dim, dim)
        self.q.inp = 'attn'                 # initialisation tags read by AFFEncoder.init_weights
        self.kv = nn.Linear(dim, 2 * dim)
        self.kv.inp = 'attn'
        self.blank_k = nn.Parameter(torch.randn(dim) * 0.2)
        self.blank_v = nn.Parameter(torch.randn(dim) * 0.2)
        self.pos_embed = nn.Linear(self.pos_dim + 3, num_heads)
        self.pos_embed.inp = 'norm'
        self.proj = nn.Linear(dim, dim)
        self.proj.inp = 'norm'
        self.proj_drop = nn.Dropout(proj_drop)
        self._pe_table_cache = {}

    def clear_pe_table_cache(self):
        """Drop the eval-mode pe_table cache (needed after changing weights in eval mode)."""
        self._pe_table_cache.clear()

    def pe_table(self, dtype: torch.dtype) -> torch.Tensor:
        """pos_embed(pre_table): [T*T, H].

        fp16 runs use the fp16 table as the reference does (attention.py:85-90);
        fp32 and bf16 runs use the fp32 table and keep the result in fp32.
        Cached per (device, dtype) in eval mode, as in the reference.
        """
        if dtype == torch.float16:
            pre = self.pre_table_fp16
        else:
            pre = self.pre_table_fp32
            dtype = torch.float32
        key = (pre.device, dtype)
        if not self.training and key in self._pe_table_cache:
            return self._pe_table_cache[key]
        with torch.autocast(device_type=pre.device.type, enabled=False):
            w = self.pos_embed.weight.to(pre.dtype)
            b = self.pos_embed.bias.to(pre.dtype)
            tab = F.linear(pre, w, b)
        if not self.training:
            self._pe_table_cache[key] = tab
        return tab

    def _make_pos_bias(self, pe_idx: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """The dense bias [B,H,N,M] of pe_idx (attention.py:72-125), for callers that want
        it materialised.  forward() never builds it: the attention kernel reads the
        table row of each (query, neighbour) pair itself.  bf16 is accepted."""
        tab = self.pe_table(dtype)                                   # [T*T, H]
        return tab[pe_idx.long()].permute(0, 3, 1, 2).to(dtype)

    def forward(self, feat, member_idx, cluster_mask, pe_idx, global_attn: bool):
        """feat [B,N,C], member_idx / pe_idx [B,N,M], cluster_mask [B,N,M] or None -> [B,N,C]."""
        B, N, C = feat.shape
        H = self.num_heads
        Ch = C // H
        q = self.q(feat)
        kv = self.kv(feat)
        dtype = q.dtype

        if global_attn:
            return self._global(feat, q, kv, pe_idx)

        mask = None
        if cluster_mask is not None:
            mask = (cluster_mask > 0) if cluster_mask.dtype != torch.bool else cluster_mask
            mask = mask.unsqueeze(1)                                  # broadcast over heads
        if self._fuse_proj(q, kv):
            # inference: the projection runs in the attention kernel's epilogue
            qh = q.view(B, N, H, Ch).permute(0, 2, 1, 3)
            kvh = kv.view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
            y = nbhd_attn_proj_fwd(qh, kvh[..., :Ch], kvh[..., Ch:], member_idx, self.scale, self.proj.weight,
                                   self.proj.bias, pe_idx=pe_idx, pe_table=self.pe_table(dtype), mask=mask,
                                   blank_k=self.blank_k.view(H, Ch).to(dtype), blank_v=self.blank_v.view(H, Ch).to(dtype))
            if y is not None:
                return y
        out = ClusterAttnFunction.apply(q, kv, member_idx, pe_idx, self.pe_table(dtype), mask,
                                        self.blank_k.view(H, Ch), self.blank_v.view(H, Ch), self.scale, H)
        out = self.proj(out)
        return self.proj_drop(out)

    def _fuse_proj(self, q, kv):
        """The fused projection serves forwards that record no gradients, with the
        projection's dropout inactive."""
        if not q.is_cuda or (self.proj_drop.p > 0 and self.training):
            return False
        if torch.is_grad_enabled() and (q.requires_grad or kv.requires_grad
                                        or any(p.requires_grad for p in self.parameters())):
            return False
        return True

    def _global(self, feat, q, kv, pe_idx):
        """Dense attention with bias and blank token (attention.py:157-180), torch SDPA."""
        B, N, C = feat.shape
        H = self.num_heads
        Ch = C // H
        qh = q.view(B, N, H, Ch).permute(0, 2, 1, 3)
        kvh = kv.view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
        k, v = kvh[..., :Ch], kvh[..., Ch:]
        if pe_idx.shape[-1] != N:
            raise ValueError(f"Global attention requires M == N, but got M={pe_idx.shape[-1]} and N={N}")
        tab = self.pe_table(q.dtype)
        bias = tab.index_select(0, pe_idx.reshape(-1).long()).view(B, N, N, H).permute(0, 3, 1, 2)
        bias = F.pad(bias.to(q.dtype), (0, 1), "constant", 0.0)
        bk = self.blank_k.view(1, H, 1, Ch).expand(B, -1, -1, -1).to(q.dtype)
        bv = self.blank_v.view(1, H, 1, Ch).expand(B, -1, -1, -1).to(q.dtype)
        k_full = torch.cat([k, bk], dim=2)
        v_full = torch.cat([v, bv], dim=2)
        out = F.scaled_dot_product_attention(qh, k_full, v_full, attn_mask=bias)
        out = out.permute(0, 2, 1, 3).reshape(B, N, C)
        return self.proj_drop(self.proj(out))


# ------------------------------------------------------------------ deformable --
def _deform_reset(mod):
    """Parameter initialisation of the reference (attention.py:247-273)."""
    nn.init.constant_(mod.sampling_offsets.weight.data, 0.)
    thetas = torch.arange(mod.n_heads, dtype=torch.float32) * (2.0 * math.pi / mod.n_heads)
    grid_init = torch.stack([thetas.cos(), thetas.sin()], -1)
    grid_init = (grid_init / grid_init.abs().max(-1, keepdim=True)[0]).view(mod.n_heads, 1, 2).repeat(1, mod.n_points, 1)
    for i in range(mod.n_points):
        grid_init[:, i, :] *= i + 1
    with torch.no_grad():
        mod.sampling_offsets.bias = nn.Parameter(grid_init.view(-1))
    nn.init.constant_(mod.attention_weights.weight.data, 0.)
    nn.init.constant_(mod.attention_weights.bias.data, 0.)
    nn.init.xavier_uniform_(mod.value_proj.weight.data)
    nn.init.constant_(mod.value_proj.bias.data, 0.)
    nn.init.xavier_uniform_(mod.output_proj.weight.data)
    nn.init.constant_(mod.output_proj.bias.data, 0.)


def _deform_unfused(mod, query_pos, kv_pos, sampling_offsets, attention_weights, key_value_proj):
    """The reference's non-fused branches (attention.py:319-399): knn(k=4) of
    every sampling location, then the given-index fused kernel (use_fused) or
    explicit Shepard weights + MSDETRPC."""
    b, n_q, h, k, _ = sampling_offsets.shape
    n_kv = kv_pos.shape[1]
    c_ = mod.c_
    values = key_value_proj.reshape(b, n_kv, h, c_).permute(0, 2, 1, 3).reshape(b * h, n_kv, c_)
    loc = query_pos.unsqueeze(2).unsqueeze(3) + sampling_offsets
    loc = loc.permute(0, 2, 1, 3, 4).reshape(b * h, n_q * k, 2).contiguous()
    kv_loc = kv_pos.unsqueeze(1).expand(-1, h, -1, -1).reshape(b * h, n_kv, 2).contiguous()
    nb_idx = hip_knn(loc, kv_loc, k=4)
    if mod.use_fused:
        aw = attention_weights.permute(0, 2, 1, 3).reshape(b * h, n_q * k)
        out = fused_deformable_attention(loc, kv_loc, nb_idx, mod.shepard_power, aw, values, D=2)
        out = out.reshape(b * h, n_q, k, c_).sum(dim=2)
        return out.reshape(b, h, n_q, c_).permute(0, 2, 1, 3).reshape(b, n_q, h * c_)
    nb_pos = torch.gather(kv_loc.unsqueeze(1).expand(-1, n_q * k, -1, -1), 2,
                          nb_idx.unsqueeze(-1).expand(-1, -1, -1, 2))
    dist = torch.norm(nb_pos - loc.unsqueeze(2), dim=-1, p=2) + 1e-6
    power = F.relu(mod.shepard_power) + 1e-6
    nn_weights = F.softmax(-power * dist.unsqueeze(-1), dim=-2)
    out = MSDETRPCFunction.apply(nb_idx.reshape(b * h, n_q, k, 4), nn_weights.reshape(b * h, n_q, k, 4),
                                 attention_weights.permute(0, 2, 1, 3).reshape(b * h, n_q, k), values)
    return out.reshape(b, h, n_q, c_).permute(0, 2, 1, 3).reshape(b, n_q, h * c_)


class DeformableCrossAttention(nn.Module):
    """Single-level deformable cross attention (reference attention.py:210-404)."""

    def __init__(self, d_model, n_heads, n_points, shepard_power=3.0, shepard_power_learnable=True,
                 use_fused=False, use_fused_knn=True):
        super().__init__()
        self.d_model = d_model
        self.n_heads = n_heads
        self.n_points = n_points
        self.c_ = d_model // n_heads
        self.use_fused = use_fused
        self.use_fused_knn = use_fused_knn
        self.sampling_offsets = nn.Linear(d_model, n_heads * n_points * 2)
        self.attention_weights = nn.Linear(d_model, n_heads * n_points)
        self.value_proj = nn.Linear(d_model, d_model)
        self.output_proj = nn.Linear(d_model, d_model)
        self.shepard_power = nn.Parameter(torch.tensor(1.0))
        _deform_reset(self)

    def forward(self, query, query_pos, key_value, kv_pos):
        """query [b,n_q,c], query_pos [b,n_q,2], key_value [b,n_kv,c], kv_pos [b,n_kv,2] -> [b,n_q,c]."""
        b, n_q, c = query.shape
        n_kv = key_value.shape[1]
        h, k, c_ = self.n_heads, self.n_points, self.c_
        offs = self.sampling_offsets(query).view(b, n_q, h, k, 2)
        attn = F.softmax(self.attention_weights(query).view(b, n_q, h, k), dim=-1)
        vproj = self.value_proj(key_value)
        if self.use_fused_knn and k == 4:
            out = fused_knn_deformable_cross_attention(query_pos, kv_pos, offs, attn,
                                                       vproj.view(b, n_kv, h, c_), self.shepard_power, D=2)
            out = out.reshape(b, n_q, c)
        else:
            out = _deform_unfused(self, query_pos, kv_pos, offs, attn, vproj)
        return self.output_proj(out)


class DeformableSelfAttention(nn.Module):
    """Single-level deformable self attention (reference attention.py:407-593)."""

    def __init__(self, d_model, n_heads, n_points, shepard_power=3.0, shepard_power_learnable=True,
                 use_fused=False, use_fused_knn=True):
        super().__init__()
        self.d_model = d_model
        self.n_heads = n_heads
        self.n_points = n_points
        self.c_ = d_model // n_heads
        self.use_fused = use_fused
        self.use_fused_knn = use_fused_knn
        self.sampling_offsets = nn.Linear(d_model, n_heads * n_points * 2)
        self.attention_weights = nn.Linear(d_model, n_heads * n_points)
        self.value_proj = nn.Linear(d_model, d_model)
        self.output_proj = nn.Linear(d_model, d_model)
        self.shepard_power = nn.Parameter(torch.tensor(1.0))
        _deform_reset(self)

    def forward(self, x, pos):
        """x [b,n,c], pos [b,n,2] -> [b,n,c]."""
        b, n, c = x.shape
        h, k, c_ = self.n_heads, self.n_points, self.c_
        offs = self.sampling_offsets(x).view(b, n, h, k, 2)
        attn = F.softmax(self.attention_weights(x).view(b, n, h, k), dim=-1)
        vproj = self.value_proj(x)
        if self.use_fused_knn and k == 4:
            out = fused_knn_deformable_self_attention(pos, offs, attn, vproj.view(b, n, h, c_),
                                                      self.shepard_power, D=2)
            out = out.reshape(b, n, c)
        else:
            out = _deform_unfused(self, pos, pos, offs, attn, vproj)
        return self.output_proj(out)
