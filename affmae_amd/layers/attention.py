"""Attention modules with the reference's signatures (src/layers/attention.py).

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

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.local_attn import nbhd_attn_fwd
from ..utils.pos_embed import pre_table_fp16, pre_table_fp32


class ClusterAttention(nn.Module):
    """Local attention over each token's neighbourhood plus a per-head blank token."""

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
        self.kv = nn.Linear(dim, 2 * dim)
        self.blank_k = nn.Parameter(torch.randn(dim) * 0.2)
        self.blank_v = nn.Parameter(torch.randn(dim) * 0.2)
        self.pos_embed = nn.Linear(self.pos_dim + 3, num_heads)
        self.proj = nn.Linear(dim, dim)
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

        qh = q.view(B, N, H, Ch).permute(0, 2, 1, 3)                 # [B,H,N,Ch] view
        kvh = kv.view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)           # [B,H,N,2Ch] view
        k, v = kvh[..., :Ch], kvh[..., Ch:]
        mask = None
        if cluster_mask is not None:
            mask = (cluster_mask > 0) if cluster_mask.dtype != torch.bool else cluster_mask
            mask = mask.unsqueeze(1)                                  # broadcast over heads
        out = torch.empty((B, N, H, Ch), dtype=dtype, device=feat.device)
        nbhd_attn_fwd(qh, k, v, member_idx, self.scale,
                      pe_idx=pe_idx, pe_table=self.pe_table(dtype),
                      mask=mask,
                      blank_k=self.blank_k.view(H, Ch), blank_v=self.blank_v.view(H, Ch),
                      out=out.permute(0, 2, 1, 3), return_lse=False)
        out = self.proj(out.view(B, N, C))
        return self.proj_drop(out)

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
