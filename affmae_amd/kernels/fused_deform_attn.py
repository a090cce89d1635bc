"""Deformable attention over point clouds with in-kernel exact K-NN (HIP, gfx950).

Drop-ins for src/layers/kernels/fused_deform_attn.py of the reference:
``fused_knn_deformable_cross_attention`` (:4095), ``fused_knn_deformable_self_attention``
(:4063), their autograd Functions, the ``*_forward`` / ``*_forward_save``
launchers (:2387-2654) and ``fused_deformable_attention`` (:694, given
neighbour indices).  ``ms_deformable_attention`` is the multi-level form:
L levels x P points, K-NN per level with inverse-distance or Shepard weights.

The sampling power is read on the device (no ``.item()`` host sync).
"""
from __future__ import annotations

import ctypes

import torch
from torch.autograd import Function
from torch.amp import custom_fwd, custom_bwd

from .. import _lib


def _f32pos(t):
    t = t.to(torch.float32)
    return t if t.stride(-1) == 1 else t.contiguous()


def _float(t):
    return t if t.dtype in _lib.DTYPE_CODE else t.to(torch.float32)


def _power_ptr(power, dev):
    if not torch.is_tensor(power):
        power = torch.tensor(float(power))
    p = power.detach().to(device=dev, dtype=torch.float32).reshape(1).contiguous()
    return p


def get_fused_knn_config(B: int, N: int, H: int, K: int, C_: int, L: int = 1, knn_k: int = 4) -> dict:
    """Launch shape of the fused KNN + deformable kernel for these sizes.

    Counterpart of ``get_fused_knn_config`` (fused_deform_attn.py:744-790), which
    picks Triton block sizes from a benchmark table.  The HIP kernel has no tuned
    parameters: its shape follows from the sizes exactly as ``aff_deform_fwd``
    derives it (K = sampling points per head and level, knn_k = neighbours per
    sample).  One wave takes ``rows_per_wave`` consecutive (batch, query, head)
    rows, one lane per (row, point) during the search; each row's gather uses
    C_ / 8 lanes of 8 channels with ``gather_rows_in_flight`` value rows in flight.
    """
    if min(B, N, H, K, C_, L, knn_k) < 1:
        raise ValueError("get_fused_knn_config: sizes must be >= 1")
    pl = max(0, (K - 1).bit_length())
    rows_per_wave = 64 >> pl
    pair_group = 8
    skp = (L * K * knn_k + pair_group - 1) // pair_group * pair_group
    per_wave = 8 * rows_per_wave * skp
    waves = 4 if per_wave * 4 <= 65536 else 1
    rows = B * N * H
    return {
        "rows_per_wave": rows_per_wave,
        "lanes_per_row_search": 1 << pl,
        "lanes_per_row_gather": max(1, C_ // 8),
        "waves_per_workgroup": waves,
        "workgroups": -(-rows // (rows_per_wave * waves)),
        "lds_bytes_per_workgroup": per_wave * waves,
        "gather_rows_in_flight": pair_group,
    }


def deform_launch(query_pos, kv_pos, level_start, offsets, attn, values, power, K, mode, return_knn=False):
    """aff_deform_fwd.

    query_pos [B,Nq,2]; kv_pos [B,Ntot,2] (levels concatenated, level l in
    rows [level_start[l], level_start[l+1])); offsets [B,Nq,H,L,P,2];
    attn [B,Nq,H,L,P]; values [B,Ntot,H,C]; power scalar tensor/float.
    Returns out [B,Nq,H,C] in values.dtype (and knn idx / d2 [B,Nq,H,L,P,K]).
    """
    lib = _lib.load()
    dev = _lib.require_cuda(query_pos, kv_pos, offsets, attn, values)
    B, Nq, H, L, P, two = offsets.shape
    assert two == 2, "offsets must be [B, Nq, H, L, P, 2]"
    assert tuple(attn.shape) == (B, Nq, H, L, P), "attn must be [B, Nq, H, L, P]"
    Ntot = kv_pos.shape[1]
    assert values.shape[:3] == (B, Ntot, H), "values must be [B, N_kv, H, C]"
    C = values.shape[3]
    assert len(level_start) == L + 1 and level_start[0] == 0 and level_start[-1] == Ntot
    qp = _f32pos(query_pos)
    kp = _f32pos(kv_pos)
    off = _float(offsets)
    if off.stride(-1) != 1 or off.stride(-2) != 2 or off.stride(-3) != 2 * P:
        off = off.contiguous()
    at = _float(attn)
    if at.stride(-1) != 1 or at.stride(-2) != P:
        at = at.contiguous()
    val = values if values.dtype in _lib.DTYPE_CODE else values.to(torch.float32)
    if val.stride(-1) != 1 or val.data_ptr() % 16:
        val = val.contiguous()
    pw = _power_ptr(power, dev)
    out = torch.empty((B, Nq, H, C), dtype=val.dtype, device=dev)
    kidx = kd2 = None
    if return_knn:
        kidx = torch.empty((B, Nq, H, L, P, K), dtype=torch.int32, device=dev)
        kd2 = torch.empty((B, Nq, H, L, P, K), dtype=torch.float32, device=dev)
    a = _lib.DeformArgs()
    a.mode = mode
    a.B, a.Nq, a.H, a.L, a.P, a.K, a.C = B, Nq, H, L, P, K, C
    a.query_pos, a.qp_sb, a.qp_sn = qp.data_ptr(), qp.stride(0), qp.stride(1)
    a.kv_pos, a.kp_sb, a.kp_sn = kp.data_ptr(), kp.stride(0), kp.stride(1)
    for i, v in enumerate(level_start):
        a.level_start[i] = int(v)
    a.offsets, a.off_dtype = off.data_ptr(), _lib.DTYPE_CODE[off.dtype]
    a.off_sb, a.off_sn, a.off_sh = off.stride(0), off.stride(1), off.stride(2)
    a.attn, a.attn_dtype = at.data_ptr(), _lib.DTYPE_CODE[at.dtype]
    a.at_sb, a.at_sn, a.at_sh = at.stride(0), at.stride(1), at.stride(2)
    a.dtype, a.values = _lib.DTYPE_CODE[val.dtype], val.data_ptr()
    a.v_sb, a.v_sn, a.v_sh = val.stride(0), val.stride(1), val.stride(2)
    a.power = pw.data_ptr()
    a.out, a.o_sb, a.o_sn, a.o_sh = out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)
    a.knn_idx = kidx.data_ptr() if kidx is not None else None
    a.knn_d2 = kd2.data_ptr() if kd2 is not None else None
    ws_bytes = lib.aff_deform_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=dev)
    st = lib.aff_deform_fwd(ctypes.byref(a), ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(st, "aff_deform_fwd")
    if return_knn:
        return out, kidx, kd2
    return out


def _single_level(offsets, attn):
    B, N, H, K, _ = offsets.shape
    return offsets.reshape(B, N, H, 1, K, 2), attn.reshape(B, N, H, 1, K)


def fused_knn_deform_cross_attn_forward(query_pos, kv_pos, offsets, attn_weights, values, power, D=2,
                                        use_heuristics=True):
    """[B,Nq,H,C_] (fused_deform_attn.py:2460-2523)."""
    assert D == 2, "Currently only D=2 is supported"
    assert offsets.shape[3] == 4, "Currently only K=4 sampling points supported"
    off, at = _single_level(offsets, attn_weights)
    return deform_launch(query_pos, kv_pos, [0, kv_pos.shape[1]], off, at, values, power, 4, _lib.DEFORM_SHEPARD)


def fused_knn_deform_self_attn_forward(pos, offsets, attn_weights, values, power, D=2, use_heuristics=True):
    """[B,N,H,C_] (fused_deform_attn.py:2387-2457)."""
    return fused_knn_deform_cross_attn_forward(pos, pos, offsets, attn_weights, values, power, D)


def fused_knn_deform_cross_attn_forward_save(query_pos, kv_pos, offsets, attn_weights, values, power, D=2):
    """(out, knn_idx [B,Nq,H,K,4] int32, knn_dist_sq [B,Nq,H,K,4]) (fused_deform_attn.py:2592-2654)."""
    assert D == 2, "Currently only D=2 is supported"
    B, Nq, H, K, _ = offsets.shape
    assert K == 4, "Currently only K=4 sampling points supported"
    off, at = _single_level(offsets, attn_weights)
    out, ki, kd = deform_launch(query_pos, kv_pos, [0, kv_pos.shape[1]], off, at, values, power, 4,
                                _lib.DEFORM_SHEPARD, return_knn=True)
    return out, ki.reshape(B, Nq, H, K, 4), kd.reshape(B, Nq, H, K, 4)


def fused_knn_deform_self_attn_forward_save(pos, offsets, attn_weights, values, power, D=2):
    """(out, knn_idx, knn_dist_sq) for self-attention (fused_deform_attn.py:2530-2589)."""
    return fused_knn_deform_cross_attn_forward_save(pos, pos, offsets, attn_weights, values, power, D)


class FusedKNNDeformSelfAttnFunction(Function):
    """Autograd entry (forward only: the backward kernels are not built yet)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, pos, offsets, attn_weights, values, power, D=2):
        return fused_knn_deform_self_attn_forward(pos, offsets, attn_weights, values, power, D)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        raise NotImplementedError("deformable attention backward is not implemented in affmae_amd yet")


class FusedKNNDeformCrossAttnFunction(Function):
    """Autograd entry (forward only: the backward kernels are not built yet)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, query_pos, kv_pos, offsets, attn_weights, values, power, D=2):
        return fused_knn_deform_cross_attn_forward(query_pos, kv_pos, offsets, attn_weights, values, power, D)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        raise NotImplementedError("deformable attention backward is not implemented in affmae_amd yet")


def fused_knn_deformable_self_attention(pos, offsets, attn_weights, values, power, D=2):
    """pos [B,N,2], offsets [B,N,H,4,2], attn [B,N,H,4], values [B,N,H,C_] -> [B,N,H,C_]."""
    return FusedKNNDeformSelfAttnFunction.apply(pos, offsets, attn_weights, values, power, D)


def fused_knn_deformable_cross_attention(query_pos, kv_pos, offsets, attn_weights, values, power, D=2):
    """query_pos [B,Nq,2], kv_pos [B,Nkv,2], offsets [B,Nq,H,4,2], attn [B,Nq,H,4],
    values [B,Nkv,H,C_] -> [B,Nq,H,C_]."""
    return FusedKNNDeformCrossAttnFunction.apply(query_pos, kv_pos, offsets, attn_weights, values, power, D)


def ms_deformable_attention(query_pos, kv_pos, level_start, offsets, attn, values, power=3.0, k=3,
                            weighting="idw", return_knn=False):
    """Multi-level deformable attention: each of the P points per level is
    interpolated from its k nearest points of that level by inverse-distance
    (``weighting='idw'``, weights 1/(d2^power + 1e-10) normalised) or Shepard
    softmax weights, scaled by attn (softmaxed over levels x points)."""
    mode = _lib.DEFORM_IDW if weighting == "idw" else _lib.DEFORM_SHEPARD
    return deform_launch(query_pos, kv_pos, list(level_start), offsets, attn, values, power, k, mode,
                         return_knn=return_knn)


# -------------------------------------------------------- given indices ----
def deform_sample_launch(eps_mode, sampling_locs, kv_pos, nb_idx, power, attn_weights=None, values=None,
                         want_weights=False, weights_dtype=torch.float32):
    lib = _lib.load()
    dev = _lib.require_cuda(sampling_locs, kv_pos, nb_idx, attn_weights, values)
    B, N, D = sampling_locs.shape
    Nkv = kv_pos.shape[1]
    K = nb_idx.shape[-1]
    sl = _f32pos(sampling_locs)
    kv = _f32pos(kv_pos)
    idx = nb_idx if nb_idx.dtype in (torch.int32, torch.int64) else nb_idx.to(torch.int64)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    pw = _power_ptr(power, dev)
    out = None
    C = 0
    dt = _lib.AFF_F32
    if values is not None:
        val = values if values.dtype in _lib.DTYPE_CODE else values.to(torch.float32)
        if val.stride(-1) != 1 or val.data_ptr() % 16:
            val = val.contiguous()
        C = val.shape[-1]
        dt = _lib.DTYPE_CODE[val.dtype]
        out = torch.empty((B, N, C), dtype=val.dtype, device=dev)
    else:
        val = None
    at = None
    if attn_weights is not None:
        at = _float(attn_weights)
    w = torch.empty((B, N, K), dtype=weights_dtype, device=dev) if want_weights else None
    st = lib.aff_deform_sample_fwd(
        eps_mode, sl.data_ptr(), sl.stride(0), sl.stride(1), kv.data_ptr(), kv.stride(0), kv.stride(1),
        idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, idx.stride(0), idx.stride(1),
        pw.data_ptr(), B, N, Nkv, K, D,
        at.data_ptr() if at is not None else None, _lib.DTYPE_CODE[at.dtype] if at is not None else 0,
        at.stride(0) if at is not None else 0, at.stride(1) if at is not None else 0,
        val.data_ptr() if val is not None else None, dt,
        val.stride(0) if val is not None else 0, val.stride(1) if val is not None else 0, C,
        out.data_ptr() if out is not None else None, out.stride(0) if out is not None else 0,
        out.stride(1) if out is not None else 0,
        w.data_ptr() if w is not None else None, _lib.DTYPE_CODE[weights_dtype] if w is not None else 0,
        w.stride(0) if w is not None else 0, w.stride(1) if w is not None else 0,
        _lib.stream_ptr(dev))
    _lib.check(st, "aff_deform_sample_fwd")
    return out, w


def fused_deform_attn_forward(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D=2, use_heuristics=False):
    """[B,N,C] = attn * sum_k softmax_k(-p (sqrt(d2) + 1e-6)) values[idx] (fused_deform_attn.py:503-571)."""
    assert sampling_locs.shape[-1] == D
    out, _ = deform_sample_launch(0, sampling_locs, kv_pos, nb_idx, power, attn_weights, values)
    return out


class FusedDeformAttnFunction(Function):
    """Autograd entry (forward only: the backward kernels are not built yet)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D=2, use_heuristics=None):
        return fused_deform_attn_forward(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        raise NotImplementedError("fused deformable attention backward is not implemented in affmae_amd yet")


def fused_deformable_attention(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D=2, use_heuristics=None):
    """Given-index deformable attention (fused_deform_attn.py:694-718)."""
    return FusedDeformAttnFunction.apply(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D, use_heuristics)
