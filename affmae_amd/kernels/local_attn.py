"""Neighbourhood (cluster) flash attention on gfx950.

Drop-in for src/layers/kernels/local_attn.py of the reference:
``launch_flash_nbhood_attn_fwd`` (local_attn.py:609-708) and
``FlashLocalAttentionFunction`` (local_attn.py:843-936) keep their names,
arguments, assertion messages and output shapes.  Differences by design:
inputs are not cast to fp16 (fp32, fp16 and bf16 run natively) and the
output keeps the input dtype without an fp16 round trip (local_attn.py:340).

``nbhd_attn_fwd`` is the extended entry used by ClusterAttention: strided
q/k/v/out views (no permute copies) and the bias either dense, gathered from
a [T*T, H] table by pe_idx, or computed from coordinates in-kernel.
"""
from __future__ import annotations

import contextlib
import ctypes

import torch
from torch.autograd import Function
from torch.amp import custom_fwd, custom_bwd

from .. import _lib
from ..utils.pos_embed import REL_POS_WIDTH

_SUPPORTED_D = (8, 16, 32, 64, 128)
PATH_NAMES = {0: "row", 2: "wave"}
_path_log = None


@contextlib.contextmanager
def record_paths():
    """Collect, in a list, the kernel family ("wave" or "row") that each
    aff_nbhd_attn_fwd call inside the block runs (aff_nbhd_attn_path)."""
    global _path_log
    prev, _path_log = _path_log, []
    try:
        yield _path_log
    finally:
        _path_log = prev


def _row_ok(t: torch.Tensor) -> bool:
    """Unit stride on the last dim and 16-byte aligned rows."""
    if t.stride(-1) != 1:
        return False
    es = t.element_size()
    if t.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def _prep_qkv(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    if t.dtype != dtype:
        t = t.to(dtype)
    if not _row_ok(t):
        t = t.contiguous()
    return t


def _idx(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.int64):
        t = t.to(torch.int64)
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _attn_args(q, k, v, member_idx, scale, *, bias=None, pe_idx=None, pe_table=None, pos=None, pos_weight=None,
               pos_bias=None, rel_width=REL_POS_WIDTH, mask=None, blank_k=None, blank_v=None):
    """Validate the inputs and fill an aff_nbhd_attn_args (no out / lse / workspace yet).
    Returns (args, keep, device): keep holds every tensor the args point into."""
    dev = _lib.require_cuda(q, k, v, member_idx, bias, pe_idx, pe_table, pos, mask, blank_k, blank_v)
    dtype = q.dtype
    if dtype not in _lib.DTYPE_CODE:
        raise NotImplementedError(f"dtype {dtype} not supported")
    B, H, N, D = q.shape
    M = member_idx.shape[-1]
    assert k.shape == q.shape and v.shape == q.shape, "q, k, v must have the same shape"
    assert tuple(member_idx.shape) == (B, N, M), f"member_idx must be [B,N,M], got {tuple(member_idx.shape)}"
    if D not in _SUPPORTED_D:
        raise NotImplementedError(f"head_dim {D} not compiled (supported: {_SUPPORTED_D})")
    q = _prep_qkv(q, dtype)
    k = _prep_qkv(k, dtype)
    v = _prep_qkv(v, dtype)
    mi = _idx(member_idx)

    a = _lib.NbhdAttnArgs()
    a.dtype = _lib.DTYPE_CODE[dtype]
    a.B, a.H, a.N, a.M, a.D = B, H, N, M, D
    a.scale = float(scale)
    a.q, (a.q_sb, a.q_sh, a.q_sn) = q.data_ptr(), q.stride()[:3]
    a.k, (a.k_sb, a.k_sh, a.k_sn) = k.data_ptr(), k.stride()[:3]
    a.v, (a.v_sb, a.v_sh, a.v_sn) = v.data_ptr(), v.stride()[:3]
    a.member_idx = mi.data_ptr()
    a.idx_is_i64 = 1 if mi.dtype == torch.int64 else 0
    a.mi_sb, a.mi_sn = mi.stride(0), mi.stride(1)
    keep = [q, k, v, mi]
    if bias is not None and bias.numel() > 0:
        assert tuple(bias.shape) == (B, H, N, M), \
            "bias must have shape [batch_size, n_heads, seq_len, neighbor_size]"
        bt = bias if bias.dtype in _lib.DTYPE_CODE else bias.to(torch.float32)
        if bt.stride(-1) != 1:
            bt = bt.contiguous()
        a.bias_mode = 1
        a.bias, a.bias_dtype = bt.data_ptr(), _lib.DTYPE_CODE[bt.dtype]
        a.bias_sb, a.bias_sh, a.bias_sn = bt.stride()[:3]
        keep.append(bt)
    elif pe_idx is not None:
        assert pe_table is not None and pe_table.dim() == 2 and pe_table.shape[1] == H, \
            "pe_table must be [rows, H]"
        assert tuple(pe_idx.shape) == (B, N, M), "pe_idx must be [B,N,M]"
        tb = pe_table.detach().to(torch.float32).contiguous()   # [T*T, H], ~1 MB: the fast path reads fp32
        pe = _idx(pe_idx)
        a.bias_mode = 2
        a.pe_idx, a.pe_is_i64 = pe.data_ptr(), 1 if pe.dtype == torch.int64 else 0
        a.pe_sb, a.pe_sn = pe.stride(0), pe.stride(1)
        a.table, a.table_dtype, a.table_rows = tb.data_ptr(), _lib.DTYPE_CODE[tb.dtype], tb.shape[0]
        keep += [tb, pe]
    elif pos is not None and pe_table is not None:
        assert pe_table.dim() == 2 and pe_table.shape[1] == H, "pe_table must be [rows, H]"
        assert tuple(pos.shape) == (B, N, 2), "pos must be [B,N,2]"
        tb = pe_table.detach().to(torch.float32).contiguous()
        p = pos.to(torch.float32)
        if p.stride(-1) != 1:
            p = p.contiguous()
        a.bias_mode = 4
        a.pos, a.pos_sb, a.pos_sn = p.data_ptr(), p.stride(0), p.stride(1)
        a.rel_width = int(rel_width)
        a.table, a.table_dtype, a.table_rows = tb.data_ptr(), _lib.DTYPE_CODE[tb.dtype], tb.shape[0]
        keep += [p, tb]
    elif pos is not None:
        assert pos_weight is not None and pos_bias is not None
        assert tuple(pos.shape) == (B, N, 2), "pos must be [B,N,2]"
        assert tuple(pos_weight.shape) == (H, 5) and tuple(pos_bias.shape) == (H,)
        p = pos.to(torch.float32)
        if p.stride(-1) != 1:
            p = p.contiguous()
        w = pos_weight.detach().to(torch.float32).contiguous()
        bb = pos_bias.detach().to(torch.float32).contiguous()
        a.bias_mode = 3
        a.pos, a.pos_sb, a.pos_sn = p.data_ptr(), p.stride(0), p.stride(1)
        a.pos_w, a.pos_b = w.data_ptr(), bb.data_ptr()
        keep += [p, w, bb]
    else:
        a.bias_mode = 0

    if mask is not None and mask.numel() > 0:
        if mask.dim() == 3:
            mask = mask.unsqueeze(1)
        assert mask.shape[0] == B and mask.shape[1] in (1, H) and tuple(mask.shape[2:]) == (N, M), \
            f"mask must have shape [batch_size, n_heads, seq_len, neighbor_size] (mask shape: {tuple(mask.shape)})"
        # a bool mask is read as its bytes (0 / 1) without a copy
        mk = mask.view(torch.uint8) if mask.dtype == torch.bool else (mask > 0).view(torch.uint8)
        if mk.stride(-1) != 1:
            mk = mk.contiguous()
        a.mask = mk.data_ptr()
        a.mask_sb, a.mask_sh, a.mask_sn = mk.stride(0), (mk.stride(1) if mk.shape[1] == H and H > 1 else 0), mk.stride(2)
        keep.append(mk)

    if blank_k is not None and blank_v is not None and blank_k.numel() > 0 and blank_v.numel() > 0:
        assert tuple(blank_k.shape) == (H, D), "blank_k must have shape [n_heads, head_dim]"
        assert tuple(blank_v.shape) == (H, D), "blank_v must have shape [n_heads, head_dim]"
        bk = blank_k.detach().to(dtype).contiguous()
        bv = blank_v.detach().to(dtype).contiguous()
        a.blank_k, a.blank_v = bk.data_ptr(), bv.data_ptr()
        keep += [bk, bv]

    return a, keep, dev


def nbhd_attn_fwd(q, k, v, member_idx, scale, *, bias=None, pe_idx=None, pe_table=None,
                  pos=None, pos_weight=None, pos_bias=None, rel_width=REL_POS_WIDTH, mask=None,
                  blank_k=None, blank_v=None, out=None, return_lse=True):
    """Neighbourhood attention forward through aff_nbhd_attn_fwd.

    q, k, v   : [B,H,N,D] (any strides with a unit stride on D), one dtype
    member_idx: [B,N,M] int32/int64
    bias      : dense [B,H,N,M], or
    pe_idx + pe_table: bias[b,h,n,j] = pe_table[pe_idx[b,n,j], h], or
    pos + pe_table: as above with pe_idx computed in-kernel from the
                coordinates exactly as the encoder does (aff.py:458-465), or
    pos + pos_weight [H,5] + pos_bias [H]: continuous relative-position bias
    mask      : [B,1|H,N,M] (nonzero = valid) or None
    blank_k/v : [H,D] or None
    out       : optional [B,H,N,D] view to write into (e.g. a [B,N,H,D] buffer
                permuted), otherwise allocated contiguous [B,H,N,D]
    Returns (out, lse [B,H,N] fp32 or None).
    """
    lib = _lib.load()
    a, keep, dev = _attn_args(q, k, v, member_idx, scale, bias=bias, pe_idx=pe_idx, pe_table=pe_table, pos=pos,
                              pos_weight=pos_weight, pos_bias=pos_bias, rel_width=rel_width, mask=mask,
                              blank_k=blank_k, blank_v=blank_v)
    dtype = q.dtype
    B, H, N, D = q.shape
    if out is None:
        out = torch.empty((B, H, N, D), dtype=dtype, device=dev)
    else:
        assert tuple(out.shape) == (B, H, N, D) and out.dtype == dtype and _row_ok(out), "bad out view"
    lse = torch.empty((B, H, N), dtype=torch.float32, device=dev) if return_lse else None
    keep.append(out)
    a.out, (a.o_sb, a.o_sh, a.o_sn) = out.data_ptr(), out.stride()[:3]
    a.lse = lse.data_ptr() if lse is not None else None
    if _path_log is not None:
        _path_log.append(PATH_NAMES.get(int(lib.aff_nbhd_attn_path(ctypes.byref(a))), "?"))
    ws_bytes = int(lib.aff_nbhd_attn_workspace_bytes(ctypes.byref(a)))
    if ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        a.ws, a.ws_bytes = ws.data_ptr(), ws_bytes
        keep.append(ws)
    st = lib.aff_nbhd_attn_fwd(ctypes.byref(a), _lib.stream_ptr(dev))
    _lib.check(st, "aff_nbhd_attn_fwd")
    del keep
    return out, lse


def nbhd_attn_proj_fwd(q, k, v, member_idx, scale, proj_w, proj_b=None, *, pe_idx=None, pe_table=None, pos=None,
                       rel_width=REL_POS_WIDTH, mask=None, blank_k=None, blank_v=None, out=None):
    """Attention with the output projection fused (aff_nbhd_attn_proj_fwd):
    [B,N,H*D] = concat_h attention(q, k, v)[:, h] @ proj_w^T + proj_b.

    q, k, v as for nbhd_attn_fwd; proj_w [H*D, H*D] (cast to q's dtype),
    proj_b [H*D] or None.  Returns None when the shape is outside the fused
    kernel's case (16-bit, head_dim 32, H <= 4, H*M <= 192), so the caller
    runs the two steps instead."""
    lib = _lib.load()
    B, H, N, D = q.shape
    C = H * D
    if q.dtype not in (torch.bfloat16, torch.float16) or D != 32 or H > 4 or tuple(proj_w.shape) != (C, C):
        return None
    a, keep, dev = _attn_args(q, k, v, member_idx, scale, pe_idx=pe_idx, pe_table=pe_table, pos=pos,
                              rel_width=rel_width, mask=mask, blank_k=blank_k, blank_v=blank_v)
    if out is None:
        out = torch.empty((B, N, C), dtype=q.dtype, device=dev)
    assert tuple(out.shape) == (B, N, C) and out.dtype == q.dtype and out.stride(-1) == 1 and out.stride(1) == C
    w = proj_w.detach().to(q.dtype).contiguous()
    # the bias rounded to q's dtype first, as the Linear it replaces adds it with 16-bit operands
    bias = proj_b.detach().to(q.dtype).to(torch.float32).contiguous() if proj_b is not None else None
    keep += [out, w] + ([bias] if bias is not None else [])
    a.out, a.o_sb, a.o_sh, a.o_sn = out.data_ptr(), out.stride(0), D, C
    st = lib.aff_nbhd_attn_proj_fwd(ctypes.byref(a), w.data_ptr(), bias.data_ptr() if bias is not None else None,
                                    _lib.stream_ptr(dev))
    if st == _lib.AFF_ERR_UNSUPPORTED:
        return None
    _lib.check(st, "aff_nbhd_attn_proj_fwd")
    if _path_log is not None:
        _path_log.append("wave+proj")
    del keep
    return out


def nbhd_attn_bwd(dout, q, k, v, member_idx, scale, out, lse, *, bias=None, pe_idx=None, pe_table=None, pos=None,
                  rel_width=REL_POS_WIDTH, mask=None, blank_k=None, blank_v=None, dq=None, dk=None, dv=None,
                  want_dbias=False, want_dtable=False):
    """Gradients of nbhd_attn_fwd through aff_nbhd_attn_bwd (reference local_attn.py:711-840).

    The inputs are the forward's (same bias form), plus its output `out` and
    `lse` and the upstream gradient `dout` [B,H,N,D].  dq / dk / dv may be
    given as [B,H,N,D] views to write into (e.g. the per-head slices of a
    projection's gradient), otherwise they are allocated.  Returns
    (dq, dk, dv, dbias [B,H,N,M] fp32 or None, dtable [rows,H] fp32 or None,
    dblank_k [H,D] fp32 or None, dblank_v [H,D] fp32 or None).  Every sum is
    formed in a fixed order, so the result is bitwise reproducible.
    """
    lib = _lib.load()
    a, keep, dev = _attn_args(q, k, v, member_idx, scale, bias=bias, pe_idx=pe_idx, pe_table=pe_table, pos=pos,
                              rel_width=rel_width, mask=mask, blank_k=blank_k, blank_v=blank_v)
    dtype = q.dtype
    B, H, N, D = q.shape
    M = member_idx.shape[-1]
    o = _prep_qkv(out, dtype)
    ls = lse.to(torch.float32).contiguous()
    do = _prep_qkv(dout, dtype)
    a.out, (a.o_sb, a.o_sh, a.o_sn) = o.data_ptr(), o.stride()[:3]
    a.lse = ls.data_ptr()
    keep += [o, ls, do]

    def grad_buf(t):
        if t is None:
            return torch.empty((B, H, N, D), dtype=dtype, device=dev)
        assert tuple(t.shape) == (B, H, N, D) and t.dtype == dtype and _row_ok(t), "bad gradient view"
        return t

    dq, dk, dv = grad_buf(dq), grad_buf(dk), grad_buf(dv)
    g = _lib.NbhdAttnBwdArgs()
    g.fwd = a
    g.dout, (g.do_sb, g.do_sh, g.do_sn) = do.data_ptr(), do.stride()[:3]
    g.dq, (g.dq_sb, g.dq_sh, g.dq_sn) = dq.data_ptr(), dq.stride()[:3]
    g.dk, (g.dk_sb, g.dk_sh, g.dk_sn) = dk.data_ptr(), dk.stride()[:3]
    g.dv, (g.dv_sb, g.dv_sh, g.dv_sn) = dv.data_ptr(), dv.stride()[:3]
    dbias = torch.empty((B, H, N, M), dtype=torch.float32, device=dev) if want_dbias else None
    dtable = None
    if want_dtable:
        assert a.bias_mode in (2, 4), "dtable needs a table bias (pe_idx or pos with pe_table)"
        dtable = torch.empty((int(a.table_rows), H), dtype=torch.float32, device=dev)
    dbk = dbv = None
    if a.blank_k:
        dbk = torch.empty((H, D), dtype=torch.float32, device=dev)
        dbv = torch.empty((H, D), dtype=torch.float32, device=dev)
    g.dbias = dbias.data_ptr() if dbias is not None else None
    g.dtable = dtable.data_ptr() if dtable is not None else None
    g.dblank_k = dbk.data_ptr() if dbk is not None else None
    g.dblank_v = dbv.data_ptr() if dbv is not None else None
    ws_bytes = int(lib.aff_nbhd_attn_bwd_workspace_bytes(ctypes.byref(g)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    g.ws, g.ws_bytes = ws.data_ptr(), ws_bytes
    keep.append(ws)
    st = lib.aff_nbhd_attn_bwd(ctypes.byref(g), _lib.stream_ptr(dev))
    _lib.check(st, "aff_nbhd_attn_bwd")
    del keep
    return dq, dk, dv, dbias, dtable, dbk, dbv


def launch_flash_nbhood_attn_fwd(q, k, v, member_index, sm_scale, bias=None, mask=None,
                                 blank_k=None, blank_v=None, exp2=False):
    """(o [B,H,N,D] in q.dtype, lse [B,H,N] fp32) — reference local_attn.py:609-708.

    ``exp2`` is accepted for compatibility; the result is the same function.
    """
    assert q.shape == k.shape and k.shape == v.shape, "q, k, v must have the same shape"
    assert q.dim() == 4 and q.shape == k.shape and q.shape == v.shape, "q, k, v must have 4 dimensions"
    assert q.shape[-1] == k.shape[-1] and k.shape[-1] == v.shape[-1], "q, k, v must have the same head dimension"
    assert q.shape[-1] % 8 == 0, "head_dim must be a multiple of 8"
    batch_size, n_heads, seq_len, head_dim = q.shape
    neighbor_size = member_index.shape[-1]
    assert neighbor_size % 8 == 0, "neighbor_size must be a multiple of 8"
    if mask is not None and mask.numel() > 0 and mask.shape[1] == 1:
        mask = mask.expand(batch_size, 1, seq_len, neighbor_size)
    return nbhd_attn_fwd(q, k, v, member_index, sm_scale, bias=bias, mask=mask,
                         blank_k=blank_k, blank_v=blank_v, return_lse=True)


class FlashLocalAttentionFunction(Function):
    """Autograd entry point (reference local_attn.py:843-936).

    forward(Q, K, V, member_idx, bias, mask, blank_k, blank_v, softmax_scale)
    -> [B,H,N,D] in Q's dtype; backward returns (dQ, dK, dV, None, dbias,
    None, dblank_k, dblank_v, None) like the reference, from aff_nbhd_attn_bwd.
    """

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, Q, K, V, member_idx, bias, mask, blank_k, blank_v, softmax_scale):
        out, lse = launch_flash_nbhood_attn_fwd(Q, K, V, member_idx, softmax_scale, bias=bias, mask=mask,
                                                blank_k=blank_k, blank_v=blank_v)
        ctx.save_for_backward(Q, K, V, member_idx, bias, mask, blank_k, blank_v, out, lse)
        ctx.scale = softmax_scale
        return out

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, grad_output):
        Q, K, V, member_idx, bias, mask, blank_k, blank_v, out, lse = ctx.saved_tensors
        has_bias = bias is not None and bias.numel() > 0
        has_blank = blank_k is not None and blank_v is not None and blank_k.numel() > 0
        dq, dk, dv, dbias, _, dbk, dbv = nbhd_attn_bwd(
            grad_output, Q, K, V, member_idx, ctx.scale, out, lse, bias=bias if has_bias else None, mask=mask,
            blank_k=blank_k if has_blank else None, blank_v=blank_v if has_blank else None,
            want_dbias=has_bias and ctx.needs_input_grad[4])
        return (dq, dk, dv, None, dbias.to(bias.dtype) if dbias is not None else None, None,
                dbk.to(blank_k.dtype) if has_blank else None, dbv.to(blank_v.dtype) if has_blank else None, None)


class ClusterAttnFunction(Function):
    """Autograd entry of ClusterAttention's local branch.

    forward(q [B,N,H*D], kv [B,N,H*2D], member_idx [B,N,M], pe_idx [B,N,M],
            table [T*T,H], mask [B,1,N,M] bool or None, blank_k [H,D], blank_v [H,D],
            scale, H) -> out [B,N,H*D]
    q is viewed per head as [B,H,N,D]; kv holds each head's [k_h | v_h] pair
    (the reference's interleave, attention.py:150-152).  The bias of
    (query, neighbour) is table[pe_idx, h], gathered in-kernel.  backward
    returns dq, dkv (written straight into the projections' layouts), dtable
    and the blank tokens' gradients from aff_nbhd_attn_bwd.
    """

    @staticmethod
    def forward(ctx, q, kv, member_idx, pe_idx, table, mask, blank_k, blank_v, scale, H):
        B, N, C = q.shape
        Ch = C // H
        qh = q.view(B, N, H, Ch).permute(0, 2, 1, 3)
        kvh = kv.view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
        out = torch.empty((B, N, H, Ch), dtype=q.dtype, device=q.device)
        need = any(ctx.needs_input_grad)
        _, lse = nbhd_attn_fwd(qh, kvh[..., :Ch], kvh[..., Ch:], member_idx, scale, pe_idx=pe_idx, pe_table=table,
                               mask=mask, blank_k=blank_k, blank_v=blank_v, out=out.permute(0, 2, 1, 3),
                               return_lse=need)
        if need:
            ctx.save_for_backward(q, kv, member_idx, pe_idx, table, mask, blank_k, blank_v, out, lse)
            ctx.scale, ctx.H = scale, H
        return out.view(B, N, C)

    @staticmethod
    def backward(ctx, grad_out):
        q, kv, member_idx, pe_idx, table, mask, blank_k, blank_v, out, lse = ctx.saved_tensors
        B, N, C = q.shape
        H = ctx.H
        Ch = C // H
        heads = lambda t, w: t.view(B, N, H, w).permute(0, 2, 1, 3)
        dq = torch.empty_like(q)
        dkv = torch.empty_like(kv)
        kvh, dkvh = heads(kv, 2 * Ch), heads(dkv, 2 * Ch)
        _, _, _, _, dtable, dbk, dbv = nbhd_attn_bwd(
            grad_out.to(q.dtype).reshape(B, N, H, Ch).permute(0, 2, 1, 3), heads(q, Ch), kvh[..., :Ch], kvh[..., Ch:], member_idx, ctx.scale,
            out.permute(0, 2, 1, 3), lse, pe_idx=pe_idx, pe_table=table, mask=mask, blank_k=blank_k,
            blank_v=blank_v, dq=heads(dq, Ch), dk=dkvh[..., :Ch], dv=dkvh[..., Ch:],
            want_dtable=ctx.needs_input_grad[4])
        return (dq, dkv, None, None, dtable.to(table.dtype) if dtable is not None else None, None,
                dbk.to(blank_k.dtype) if dbk is not None else None, dbv.to(blank_v.dtype) if dbv is not None else None,
                None, None)
