"""Cross-attention pixel decoder over point tokens (reference src/layers/decoder.py).

``PositionEmbeddingSine`` (decoder.py:17-70), ``MSDecoderBlock`` (:73-165)
and ``CrossAttentionPixelDecoder`` (:168-371) keep the reference's
constructors, forward signatures and parameter names, so state_dicts load
unchanged.  The deformable self / cross attention of every block runs on the
HIP kernels (fused in-kernel K-NN + Shepard gather, forward and backward);
the LayerNorms run on the HIP LayerNorm at inference; the Linear layers and
the sine embedding are torch.
"""
from __future__ import annotations

import math
from collections import namedtuple
from typing import Callable, Dict, List, Optional, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.layer_norm import norm
from .attention import DeformableCrossAttention, DeformableSelfAttention

# What the decoder reads from each entry of ``input_shape`` (detectron2's ShapeSpec carries the same fields).
ShapeSpec = namedtuple("ShapeSpec", ["channels", "stride"])


class PositionEmbeddingSine(nn.Module):
    """Sine / cosine embedding of 2-D point positions (decoder.py:17-70).

    pos [b, n, 2] (x, y) -> [b, n, 2 * num_pos_feats]: the x features then the
    y features; each is sin of the even frequencies followed by cos of the odd
    ones, frequency i = temperature ** (2 * (i // 2) / num_pos_feats).  With
    ``normalize`` the coordinates are first divided by their maximum over the
    whole batch (+ 1e-6) and multiplied by ``scale`` (2 pi by default)."""

    def __init__(self, num_pos_feats=64, temperature=10000, normalize=False, scale=None):
        super().__init__()
        self.num_pos_feats = num_pos_feats
        self.temperature = temperature
        self.normalize = normalize
        if scale is not None and normalize is False:
            raise ValueError("normalize should be True if scale is passed")
        self.scale = 2 * math.pi if scale is None else scale

    def forward(self, pos):
        x = pos[:, :, 0]
        y = pos[:, :, 1]
        if self.normalize:
            x = x / (x.max() + 1e-6) * self.scale
            y = y / (y.max() + 1e-6) * self.scale
        i = torch.arange(self.num_pos_feats, dtype=torch.float32, device=pos.device)
        freq = self.temperature ** (2 * torch.div(i, 2, rounding_mode="floor") / self.num_pos_feats)

        def embed(v):
            t = v[:, :, None] / freq
            return torch.cat((t[:, :, 0::2].sin(), t[:, :, 1::2].cos()), dim=2)

        return torch.cat((embed(x), embed(y)), dim=2)

    def __repr__(self, _repr_indent=4):
        body = [f"num_pos_feats: {self.num_pos_feats}", f"temperature: {self.temperature}",
                f"normalize: {self.normalize}", f"scale: {self.scale}"]
        return "\n".join(["Positional encoding " + self.__class__.__name__] + [" " * _repr_indent + b for b in body])


class MSDecoderBlock(nn.Module):
    """Deformable self attention over the query tokens, deformable cross attention
    to the encoder tokens, then a feed-forward layer; post-norm residuals
    (decoder.py:73-165)."""

    def __init__(self, d_model=256, n_heads=8, n_points=4, d_ffn=1024, dropout=0.1, activation="relu",
                 shepard_power=3.0, shepard_power_learnable=True):
        super().__init__()
        self.self_attn = DeformableSelfAttention(d_model, n_heads, n_points, shepard_power, shepard_power_learnable)
        self.dropout1 = nn.Dropout(dropout)
        self.norm1 = nn.LayerNorm(d_model)
        self.cross_attn = DeformableCrossAttention(d_model, n_heads, n_points, shepard_power,
                                                   shepard_power_learnable)
        self.dropout2 = nn.Dropout(dropout)
        self.norm2 = nn.LayerNorm(d_model)
        self.linear1 = nn.Linear(d_model, d_ffn)
        self.activation = getattr(F, activation)
        self.dropout3 = nn.Dropout(dropout)
        self.linear2 = nn.Linear(d_ffn, d_model)
        self.dropout4 = nn.Dropout(dropout)
        self.norm3 = nn.LayerNorm(d_model)

    @staticmethod
    def with_pos_embed(tensor, pos_embed):
        return tensor if pos_embed is None else tensor + pos_embed

    def forward(self, query_tokens, query_pos, src, pos, pos_embed):
        """query_tokens [b,n_q,c], query_pos [b,n_q,2], src [b,n_src,c], pos [b,n_src,2],
        pos_embed [b,n_src,c] or None -> [b,n_q,c]."""
        q = query_tokens + self.dropout1(self.self_attn(query_tokens, query_pos))
        q = norm(self.norm1, q)
        q = q + self.dropout2(self.cross_attn(q, query_pos, self.with_pos_embed(src, pos_embed), pos))
        q = norm(self.norm2, q)
        q = q + self.dropout4(self.linear2(self.dropout3(self.activation(self.linear1(q)))))
        return norm(self.norm3, q)


class CrossAttentionPixelDecoder(nn.Module):
    """Masked-token decoder (decoder.py:168-371): the encoder stages are projected
    to ``conv_dim`` (Linear + LayerNorm) and embedded by their positions; the
    masked tokens (plus their own position embedding) pass through
    ``transformer_dec_layers`` MSDecoderBlocks per stage, coarsest stage first.
    ``forward_features`` returns the query tokens after every block.  The
    reference's ``forward`` body is empty (it returns None); here ``forward``
    returns ``forward_features``'s list."""

    def __init__(self, input_shape: Dict[str, "ShapeSpec"], *, transformer_dropout: float,
                 transformer_nheads: int, transformer_dim_feedforward: int, transformer_dec_layers: int,
                 conv_dim: int, mask_dim: int, norm: Optional[Union[str, Callable]] = None,
                 transformer_in_features: List[str], common_stride: int, shepard_power: float,
                 shepard_power_learnable: bool):
        super().__init__()
        t_shape = {k: v for k, v in input_shape.items() if k in transformer_in_features}
        shapes = sorted(input_shape.items(), key=lambda kv: kv[1].stride)
        self.in_features = [k for k, _ in shapes]
        self.feature_strides = [v.stride for _, v in shapes]
        self.feature_channels = [v.channels for _, v in shapes]
        t_shape = sorted(t_shape.items(), key=lambda kv: kv[1].stride)
        self.transformer_in_features = [k for k, _ in t_shape]
        t_channels = [v.channels for _, v in t_shape]
        self.transformer_feature_strides = [v.stride for _, v in t_shape]
        self.transformer_num_feature_levels = len(self.transformer_in_features)
        self.transformer_dec_layers = transformer_dec_layers
        self.conv_dim = conv_dim
        self.mask_dim = mask_dim
        self.common_stride = common_stride
        self.shepard_power = shepard_power
        self.shepard_power_learnable = shepard_power_learnable
        # coarsest (res5) first
        chans = t_channels[::-1] if self.transformer_num_feature_levels > 1 else t_channels[-1:]
        self.input_proj = nn.ModuleList([nn.Sequential(nn.Linear(c, conv_dim, bias=True), nn.LayerNorm(conv_dim))
                                         for c in chans])
        for proj in self.input_proj:
            nn.init.xavier_uniform_(proj[0].weight, gain=1)
            nn.init.constant_(proj[0].bias, 0)
        self.pe_layer = PositionEmbeddingSine(conv_dim // 2, normalize=True)
        self.decoder_blocks = nn.ModuleList([
            nn.ModuleList([MSDecoderBlock(d_model=conv_dim, n_heads=transformer_nheads, n_points=4,
                                          d_ffn=transformer_dim_feedforward, dropout=transformer_dropout,
                                          activation="relu", shepard_power=shepard_power,
                                          shepard_power_learnable=shepard_power_learnable)
                           for _ in range(transformer_dec_layers)])
            for _ in range(self.transformer_num_feature_levels)])

    @classmethod
    def from_config(cls, cfg, input_shape: Dict[str, "ShapeSpec"]):
        """Constructor arguments from a detectron2-style config (decoder.py:279-296)."""
        head = cfg.MODEL.SEM_SEG_HEAD
        return {
            "input_shape": {k: v for k, v in input_shape.items() if k in head.IN_FEATURES},
            "conv_dim": head.CONVS_DIM,
            "mask_dim": head.MASK_DIM,
            "norm": head.NORM,
            "transformer_dropout": cfg.MODEL.MASK_FORMER.DROPOUT,
            "transformer_nheads": cfg.MODEL.MASK_FORMER.NHEADS,
            "transformer_dim_feedforward": 1024,
            "transformer_dec_layers": head.TRANSFORMER_DEC_LAYERS,
            "transformer_in_features": head.DEFORMABLE_TRANSFORMER_ENCODER_IN_FEATURES,
            "common_stride": head.COMMON_STRIDE,
            "shepard_power": cfg.MODEL.AFF.SHEPARD_POWER / 2.0,
            "shepard_power_learnable": cfg.MODEL.AFF.SHEPARD_POWER_LEARNABLE,
        }

    def _proj(self, idx, x):
        lin, ln = self.input_proj[idx]
        return norm(ln, lin(x))

    def forward_features(self, features, masked_tokens, masked_pos):
        """features: {name: [b,n,c], name + '_pos': [b,n,2], name + '_spatial_shape': (h, w)};
        masked_tokens [b,n_q,conv_dim], masked_pos [b,n_q,2] -> list of [b,n_q,conv_dim],
        one per block, coarsest stage first."""
        srcs, poss, embeds = [], [], []
        for idx, f in enumerate(self.transformer_in_features[::-1]):
            pos = features[f + "_pos"]
            srcs.append(self._proj(idx, features[f]))
            poss.append(pos)
            embeds.append(self.pe_layer(pos))
        query = masked_tokens + self.pe_layer(masked_pos)
        intermediates = []
        for stage in range(self.transformer_num_feature_levels):
            for block in self.decoder_blocks[stage]:
                query = block(query_tokens=query, query_pos=masked_pos, src=srcs[stage], pos=poss[stage],
                              pos_embed=embeds[stage])
                intermediates.append(query)
        return intermediates

    def forward(self, features, masked_tokens, masked_pos):
        return self.forward_features(features, masked_tokens, masked_pos)


class GlobalSelfAttention(nn.Module):
    """Dense multi-head self attention (reference attention.py:596-628): qkv
    projection, softmax(q k^T / sqrt(d)) v per head, output projection.  The
    scores are formed in fp32 from contiguous operands."""

    def __init__(self, d_model, n_heads, dropout=0.0):
        super().__init__()
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.qkv = nn.Linear(d_model, 3 * d_model)
        self.out_proj = nn.Linear(d_model, d_model)
        self.dropout_p = dropout

    def forward(self, x, pos=None):
        b, n, c = x.shape
        qkv = self.qkv(x).reshape(b, n, 3, self.n_heads, self.head_dim).permute(2, 0, 3, 1, 4).float()
        q, k, v = qkv[0].contiguous(), qkv[1].contiguous(), qkv[2].contiguous()
        with torch.autocast(device_type=x.device.type, enabled=False):
            s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(self.head_dim))
            out = torch.matmul(torch.softmax(s, dim=-1), v)
        out = out.transpose(1, 2).reshape(b, n, c)
        if not torch.is_autocast_enabled(x.device.type):
            out = out.to(x.dtype)
        return self.out_proj(out)
