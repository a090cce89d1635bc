"""The reference's own PyTorch path for the hot path, restated in torch-CPU fp32.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: bench.py times these
functions as its reported CPU baseline (``cpu_baseline``, kind "port"), and
tests/test_oracle.py pins them against the C oracle.  The product package
``affmae_amd`` never imports this module.

* :func:`knn_cdist_topk` restates ``knn_pytorch_large``
  (src/layers/kernels/knn.py:1312-1332): cdist, squared, topk(largest=False).
  Its tie order is whatever topk returns (the reference leaves it unspecified).
* :func:`table_bias` restates ``ClusterAttention._make_pos_bias``'s gather
  (src/layers/attention.py:117-124): table rows by pe_idx, then [B,H,N,M].
* :func:`gathered_attention` restates the reference's PyTorch baseline of
  the neighbourhood attention (src/layers/kernels/local_attn.py:979-1006):
  expanded gathers of K and V, masked logits plus bias, softmax over the
  neighbours and the blank token, P V plus the blank value.
"""
from __future__ import annotations

import torch


def knn_cdist_topk(query: torch.Tensor, ref: torch.Tensor, k: int) -> torch.Tensor:
    """int64 [B,M,k] indices of the k smallest squared distances (knn.py:1326-1332)."""
    dist = torch.cdist(query.float(), ref.float(), p=2.0).pow(2)
    _, idx = torch.topk(dist, k, dim=-1, largest=False)
    return idx.to(torch.int64)


def table_bias(pe_idx: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """[B,H,N,M] bias = table[pe_idx, h] (attention.py:117-124)."""
    B, N, M = pe_idx.shape
    g = table.index_select(0, pe_idx.reshape(-1)).view(B, N, M, -1)
    return g.permute(0, 3, 1, 2)


def gathered_attention(q, k, v, member_index, sm_scale, bias=None, mask=None, blank_k=None, blank_v=None):
    """[B,H,N,D] output of the reference's gathered PyTorch attention (local_attn.py:979-1006)."""
    B, H, N, D = q.shape
    M = member_index.shape[-1]
    mi = member_index.unsqueeze(1).expand(-1, H, -1, -1)                              # [B,H,N,M]
    gi = mi.unsqueeze(4).expand(-1, -1, -1, -1, D)
    k_g = torch.gather(k.unsqueeze(2).expand(-1, -1, N, -1, -1), 3, gi)                # [B,H,N,M,D]
    v_g = torch.gather(v.unsqueeze(2).expand(-1, -1, N, -1, -1), 3, gi)
    scores = torch.matmul(q.unsqueeze(3), k_g.transpose(-2, -1)).squeeze(3) * sm_scale  # [B,H,N,M]
    if bias is not None:
        scores = scores + bias
    if mask is not None:
        scores = scores.masked_fill(mask.expand_as(scores) == 0, float("-inf"))
    if blank_k is not None:
        blank = (q * blank_k.view(1, H, 1, D)).sum(-1, keepdim=True) * sm_scale        # [B,H,N,1]
        probs = torch.softmax(torch.cat([scores, blank], dim=-1), dim=-1)
        p_nb, p_blank = probs[..., :M], probs[..., M:]
        return torch.matmul(p_nb.unsqueeze(3), v_g).squeeze(3) + p_blank * blank_v.view(1, H, 1, D)
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs.unsqueeze(3), v_g).squeeze(3)
