"""Deformable attention over point clouds with in-kernel exact K-NN (HIP, gfx950).

Drop-ins for src/layers/kernels/fused_deform_attn.py of the reference:
``fused_knn_deformable_cross_attention`` (:4095), ``fused_knn_deformable_self_attention``
(:4063), their autograd Functions, the ``*_forward`` / ``*_forward_save``
launchers (:2387-2654) and ``fused_deformable_attention`` (:694, given
neighbour indices).  ``ms_deformable_attention`` is the multi-level form:
L levels x P points, K-NN per level with inverse-distance or Shepard weights.
Every autograd Function has a backward through aff_deform_bwd (fixed-order
sums, no float atomics).

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


def _inner_contig(t, dims):
    """t with its last `dims` dimensions contiguous (a copy only when they are not)."""
    exp = 1
    for i in range(1, dims + 1):
        if t.shape[-i] != 1 and t.stride(-i) != exp:
            return t.contiguous()
        exp *= t.shape[-i]
    return t


def deform_backward_launch(mode, dout, *, idx, loc=None, offsets=None, kv_pos=None, attn=None, weights=None,
                           values=None, d_w_in=None, power=None, level_start=None, P=None, Nkv=None,
                           want_loc=False, want_attn=False, want_weights=False, want_kv=False, want_values=False,
                           want_power=False):
    """aff_deform_bwd over rows (b, q, h) of S samples x K neighbours.

    idx [B,Q,H,S,K]; loc [B,Q,D] fp32; offsets [B,Q,H,S,D]; kv_pos [B,Nkv,D];
    attn [B,Q,H,S]; weights / d_w_in [B,Q,H,S,K]; values [B,Nkv,H,C] and
    dout [B,Q,H,C] (or dout None with d_w_in).  level_start: row offsets of
    the levels (level of sample s = s // P).  Returns a dict with the wanted
    gradients: d_loc [B,Q,H,S,D], d_attn [B,Q,H,S], d_weights [B,Q,H,S,K],
    d_kv_pos [B,Nkv,D] (fp32), d_values [B,Nkv,H,C] (values.dtype), d_power [1].
    """
    lib = _lib.load()
    dev = _lib.require_cuda(idx, dout, loc, kv_pos, values, d_w_in)
    B, Q, H, S, K = idx.shape
    a = _lib.DeformBwdArgs()
    a.mode, a.B, a.Q, a.H, a.S, a.K = mode, B, Q, H, S, K
    D = loc.shape[-1] if loc is not None else (kv_pos.shape[-1] if kv_pos is not None else 0)
    a.D = D
    a.P = P or S
    if Nkv is None:
        Nkv = values.shape[1] if values is not None else kv_pos.shape[1]
    a.Nkv = Nkv
    ls = list(level_start) if level_start is not None else [0, Nkv]
    for i, v in enumerate(ls):
        a.level_start[i] = int(v)
    keep = []
    ix = idx if idx.dtype in (torch.int32, torch.int64) else idx.to(torch.int64)
    ix = _inner_contig(ix, 2)
    keep.append(ix)
    a.idx, a.idx_is_i64 = ix.data_ptr(), 1 if ix.dtype == torch.int64 else 0
    a.i_sb, a.i_sn, a.i_sh = ix.stride(0), ix.stride(1), ix.stride(2)
    if loc is not None:
        lc = _f32pos(loc)
        keep.append(lc)
        a.loc, a.loc_sb, a.loc_sn = lc.data_ptr(), lc.stride(0), lc.stride(1)
    if offsets is not None:
        of = _inner_contig(_float(offsets), 2)
        keep.append(of)
        a.offsets, a.off_dtype = of.data_ptr(), _lib.DTYPE_CODE[of.dtype]
        a.off_sb, a.off_sn, a.off_sh = of.stride(0), of.stride(1), of.stride(2)
    if kv_pos is not None:
        kp = _f32pos(kv_pos)
        keep.append(kp)
        a.kv_pos, a.kp_sb, a.kp_sn = kp.data_ptr(), kp.stride(0), kp.stride(1)
    if attn is not None:
        at = _inner_contig(_float(attn), 1)
        keep.append(at)
        a.attn, a.attn_dtype = at.data_ptr(), _lib.DTYPE_CODE[at.dtype]
        a.at_sb, a.at_sn, a.at_sh = at.stride(0), at.stride(1), at.stride(2)
    if weights is not None:
        wt = _inner_contig(_float(weights), 2)
        keep.append(wt)
        a.weights, a.w_dtype = wt.data_ptr(), _lib.DTYPE_CODE[wt.dtype]
        a.w_sb, a.w_sn, a.w_sh = wt.stride(0), wt.stride(1), wt.stride(2)
    C = 0
    vdtype = torch.float32
    if values is not None:
        v = values if values.dtype in _lib.DTYPE_CODE else values.to(torch.float32)
        if v.stride(-1) != 1 or v.data_ptr() % 16 or any((st * v.element_size()) % 16 for st in v.stride()[:3]):
            v = v.contiguous()
        do = dout.to(v.dtype)
        if do.stride(-1) != 1 or do.data_ptr() % 16 or any((st * do.element_size()) % 16 for st in do.stride()[:3]):
            do = do.contiguous()
        keep += [v, do]
        C, vdtype = v.shape[-1], v.dtype
        a.dtype, a.values = _lib.DTYPE_CODE[v.dtype], v.data_ptr()
        a.v_sb, a.v_sn, a.v_sh = v.stride(0), v.stride(1), v.stride(2)
        a.dout, a.do_sb, a.do_sn, a.do_sh = do.data_ptr(), do.stride(0), do.stride(1), do.stride(2)
    a.C = C
    if d_w_in is not None:
        dw = _inner_contig(d_w_in.to(torch.float32), 2)
        keep.append(dw)
        a.d_w_in, a.dwi_sb, a.dwi_sn, a.dwi_sh = dw.data_ptr(), dw.stride(0), dw.stride(1), dw.stride(2)
    pw = None
    if power is not None:
        pw = _power_ptr(power, dev)
        keep.append(pw)
        a.power = pw.data_ptr()
    out = {}
    f32 = dict(dtype=torch.float32, device=dev)
    if want_loc:
        out["d_loc"] = torch.empty((B, Q, H, S, D), **f32)
        a.d_loc = out["d_loc"].data_ptr()
    if want_attn:
        out["d_attn"] = torch.empty((B, Q, H, S), **f32)
        a.d_attn = out["d_attn"].data_ptr()
    if want_weights:
        out["d_weights"] = torch.empty((B, Q, H, S, K), **f32)
        a.d_weights = out["d_weights"].data_ptr()
    if want_kv:
        out["d_kv_pos"] = torch.empty((B, Nkv, D), **f32)
        a.d_kv_pos = out["d_kv_pos"].data_ptr()
    if want_values:
        out["d_values"] = torch.empty((B, Nkv, H, C), dtype=vdtype, device=dev)
        a.d_values = out["d_values"].data_ptr()
    if want_power:
        out["d_power"] = torch.empty((1,), **f32)
        a.d_power = out["d_power"].data_ptr()
    ws_bytes = int(lib.aff_deform_bwd_workspace_bytes(ctypes.byref(a)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    st = lib.aff_deform_bwd(ctypes.byref(a), ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(st, "aff_deform_bwd")
    return out


def _power_grad(d_power, power):
    if not torch.is_tensor(power):
        return None
    return d_power.reshape(power.shape).to(power.dtype)


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


def _save_power(ctx, power):
    """Tensors go through save_for_backward; a Python number is kept as is."""
    if torch.is_tensor(power):
        ctx.power_num = None
        return power
    ctx.power_num = float(power)
    return None


def _knn_deform_backward(ctx, dout, query_pos, kv_pos, offsets, attn_weights, values, power, kidx, need):
    """Gradients of the single-level fused KNN deformable attention (reference
    fused_deform_attn.py:2661-2930): need = (qpos, kvpos, offsets, attn, values, power)."""
    B, Nq, H, K, _ = offsets.shape
    pw = power if power is not None else ctx.power_num
    g = deform_backward_launch(
        _lib.DEFORM_BWD_SHEPARD, dout, idx=kidx.reshape(B, Nq, H, K, kidx.shape[-1]), loc=query_pos,
        offsets=offsets, kv_pos=kv_pos, attn=attn_weights, values=values, power=pw,
        want_loc=need[0] or need[2], want_attn=need[3], want_kv=need[1], want_values=need[4],
        want_power=need[5] and power is not None)
    d_qpos = g["d_loc"].sum(dim=(2, 3)).to(query_pos.dtype) if need[0] else None
    d_kv = g["d_kv_pos"].to(kv_pos.dtype) if need[1] else None
    d_off = g["d_loc"].to(offsets.dtype) if need[2] else None
    d_attn = g["d_attn"].to(attn_weights.dtype) if need[3] else None
    d_val = g["d_values"].to(values.dtype) if need[4] else None
    d_pow = _power_grad(g["d_power"], power) if "d_power" in g else None
    return d_qpos, d_kv, d_off, d_attn, d_val, d_pow


class FusedKNNDeformSelfAttnFunction(Function):
    """Autograd entry (reference fused_deform_attn.py:3981-4017): the forward keeps
    the neighbour indices it found; backward returns (d_pos, d_offsets,
    d_attn_weights, d_values, d_power, None) through aff_deform_bwd, where d_pos
    sums the position's query and key roles."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, pos, offsets, attn_weights, values, power, D=2):
        assert D == 2, "Currently only D=2 is supported"
        assert offsets.shape[3] == 4, "Currently only K=4 sampling points supported"
        if not any(ctx.needs_input_grad[:5]):
            return fused_knn_deform_self_attn_forward(pos, offsets, attn_weights, values, power, D)
        out, kidx, _ = fused_knn_deform_self_attn_forward_save(pos, offsets, attn_weights, values, power, D)
        ctx.save_for_backward(pos, offsets, attn_weights, values, kidx, _save_power(ctx, power))
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        pos, offsets, attn_weights, values, kidx, power = ctx.saved_tensors
        n = ctx.needs_input_grad
        need = (n[0], n[0], n[1], n[2], n[3], n[4])
        d_q, d_kv, d_off, d_attn, d_val, d_pow = _knn_deform_backward(ctx, dout, pos, pos, offsets, attn_weights,
                                                                       values, power, kidx, need)
        d_pos = (d_q + d_kv).to(pos.dtype) if n[0] else None
        return d_pos, d_off, d_attn, d_val, d_pow, None


class FusedKNNDeformCrossAttnFunction(Function):
    """Autograd entry (reference fused_deform_attn.py:4020-4056): backward returns
    (d_query_pos, d_kv_pos, d_offsets, d_attn_weights, d_values, d_power, None)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, query_pos, kv_pos, offsets, attn_weights, values, power, D=2):
        assert D == 2, "Currently only D=2 is supported"
        assert offsets.shape[3] == 4, "Currently only K=4 sampling points supported"
        if not any(ctx.needs_input_grad[:6]):
            return fused_knn_deform_cross_attn_forward(query_pos, kv_pos, offsets, attn_weights, values, power, D)
        out, kidx, _ = fused_knn_deform_cross_attn_forward_save(query_pos, kv_pos, offsets, attn_weights, values,
                                                                power, D)
        ctx.save_for_backward(query_pos, kv_pos, offsets, attn_weights, values, kidx, _save_power(ctx, power))
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        query_pos, kv_pos, offsets, attn_weights, values, kidx, power = ctx.saved_tensors
        grads = _knn_deform_backward(ctx, dout, query_pos, kv_pos, offsets, attn_weights, values, power, kidx,
                                     ctx.needs_input_grad[:6])
        return (*grads, None)


def fused_knn_deformable_self_attention(pos, offsets, attn_weights, values, power, D=2):
    """pos [B,N,2], offsets [B,N,H,4,2], attn [B,N,H,4], values [B,N,H,C_] -> [B,N,H,C_]."""
    return FusedKNNDeformSelfAttnFunction.apply(pos, offsets, attn_weights, values, power, D)


def fused_knn_deformable_cross_attention(query_pos, kv_pos, offsets, attn_weights, values, power, D=2):
    """query_pos [B,Nq,2], kv_pos [B,Nkv,2], offsets [B,Nq,H,4,2], attn [B,Nq,H,4],
    values [B,Nkv,H,C_] -> [B,Nq,H,C_]."""
    return FusedKNNDeformCrossAttnFunction.apply(query_pos, kv_pos, offsets, attn_weights, values, power, D)


class MSDeformAttnFunction(Function):
    """Autograd entry of the multi-level form: backward returns the gradients of
    (query_pos, kv_pos, offsets, attn, values, power) through aff_deform_bwd."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, query_pos, kv_pos, offsets, attn, values, power, level_start, k, mode):
        ctx.level_start, ctx.mode = tuple(level_start), mode
        if not any(ctx.needs_input_grad[:6]):
            return deform_launch(query_pos, kv_pos, list(level_start), offsets, attn, values, power, k, mode)
        out, kidx, _ = deform_launch(query_pos, kv_pos, list(level_start), offsets, attn, values, power, k, mode,
                                     return_knn=True)
        ctx.save_for_backward(query_pos, kv_pos, offsets, attn, values, kidx, _save_power(ctx, power))
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        query_pos, kv_pos, offsets, attn, values, kidx, power = ctx.saved_tensors
        n = ctx.needs_input_grad
        B, Nq, H, L, P, _ = offsets.shape
        pw = power if power is not None else ctx.power_num
        mode = _lib.DEFORM_BWD_SHEPARD if ctx.mode == _lib.DEFORM_SHEPARD else _lib.DEFORM_BWD_IDW
        g = deform_backward_launch(
            mode, dout, idx=kidx.reshape(B, Nq, H, L * P, kidx.shape[-1]), loc=query_pos,
            offsets=offsets.reshape(B, Nq, H, L * P, 2), kv_pos=kv_pos, attn=attn.reshape(B, Nq, H, L * P),
            values=values, power=pw, level_start=ctx.level_start, P=P,
            want_loc=n[0] or n[2], want_attn=n[3], want_kv=n[1], want_values=n[4], want_power=n[5] and power is not None)
        d_q = g["d_loc"].sum(dim=(2, 3)).to(query_pos.dtype) if n[0] else None
        d_kv = g["d_kv_pos"].to(kv_pos.dtype) if n[1] else None
        d_off = g["d_loc"].reshape(offsets.shape).to(offsets.dtype) if n[2] else None
        d_at = g["d_attn"].reshape(attn.shape).to(attn.dtype) if n[3] else None
        d_val = g["d_values"].to(values.dtype) if n[4] else None
        d_pow = _power_grad(g["d_power"], power) if "d_power" in g else None
        return d_q, d_kv, d_off, d_at, d_val, d_pow, None, None, None


def ms_deformable_attention(query_pos, kv_pos, level_start, offsets, attn, values, power=3.0, k=3,
                            weighting="idw", return_knn=False):
    """Multi-level deformable attention: each of the P points per level is
    interpolated from its k nearest points of that level by inverse-distance
    (``weighting='idw'``, weights 1/(d2^power + 1e-10) normalised) or Shepard
    softmax weights, scaled by attn (softmaxed over levels x points).
    Differentiable in every float input (MSDeformAttnFunction)."""
    mode = _lib.DEFORM_IDW if weighting == "idw" else _lib.DEFORM_SHEPARD
    if return_knn:
        return deform_launch(query_pos, kv_pos, list(level_start), offsets, attn, values, power, k, mode,
                             return_knn=True)
    return MSDeformAttnFunction.apply(query_pos, kv_pos, offsets, attn, values, power, tuple(level_start), k, mode)


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
    """Autograd entry (reference fused_deform_attn.py:654-690): backward returns
    (d_sampling_locs, d_kv_pos, None, d_power, d_attn_weights, d_values, None, None)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D=2, use_heuristics=None):
        out = fused_deform_attn_forward(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D)
        ctx.save_for_backward(sampling_locs, kv_pos, nb_idx, attn_weights, values, _save_power(ctx, power))
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        sl, kv, nb_idx, attn, values, power = ctx.saved_tensors
        n = ctx.needs_input_grad
        B, N, K = nb_idx.shape
        pw = power if power is not None else ctx.power_num
        g = deform_backward_launch(
            _lib.DEFORM_BWD_SAMPLE, dout.unsqueeze(2), idx=nb_idx.reshape(B, N, 1, 1, K), loc=sl, kv_pos=kv,
            attn=attn.reshape(B, N, 1, 1), values=values.unsqueeze(2), power=pw,
            want_loc=n[0], want_kv=n[1], want_power=n[3] and power is not None, want_attn=n[4], want_values=n[5])
        d_sl = g["d_loc"].reshape(B, N, -1).to(sl.dtype) if n[0] else None
        d_kv = g["d_kv_pos"].to(kv.dtype) if n[1] else None
        d_pow = _power_grad(g["d_power"], power) if "d_power" in g else None
        d_attn = g["d_attn"].reshape(attn.shape).to(attn.dtype) if n[4] else None
        d_val = g["d_values"].reshape(values.shape).to(values.dtype) if n[5] else None
        return d_sl, d_kv, None, d_pow, d_attn, d_val, None, None


def fused_deformable_attention(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D=2, use_heuristics=None):
    """Given-index deformable attention (fused_deform_attn.py:694-718)."""
    return FusedDeformAttnFunction.apply(sampling_locs, kv_pos, nb_idx, power, attn_weights, values, D, use_heuristics)
