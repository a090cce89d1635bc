"""CPU oracle for the AFFMAE point-token hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import this package, and only as the
checker (or, for bench.py, as the timed CPU baseline).  The product package
``affmae_amd`` never imports it and has no CPU fallback.

Contents
--------
* ``oracle.c`` (built into ``oracle/liboracle.so`` by :func:`build`):
  exact fp32 KNN (``oracle_knn``) and fp64 neighbourhood attention
  (``oracle_nbhd_attn``), each citing the reference lines it restates.
* numpy restatements of the relative-position bias inputs:
  :func:`pre_table` (src/utils/pos_embed.py:9-24), :func:`pe_index`
  (src/layers/aff.py:458-465), :func:`cluster_members` (aff.py:452-465), :func:`table_bias`
  (src/layers/attention.py:72-125) and :func:`continuous_bias`.

How each function is pinned (independent checks, not re-typed formulas) is
listed in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
SRC = HERE / "oracle.c"

_lib = None


def build(verbose: bool = False) -> Path:
    """Compile oracle.c with gcc (OpenMP, no fp contraction)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
           str(SRC), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[oracle build] wrote {LIB_PATH}", flush=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < SRC.stat().st_mtime:
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i32 = ctypes.c_int
        L.oracle_knn.argtypes = [P, P, i32, i32, i32, i32, i32, P, P]
        L.oracle_knn.restype = i32
        L.oracle_nbhd_attn.argtypes = [P, P, P, P, P, P, P, P, ctypes.c_double,
                                       i32, i32, i32, i32, i32, P, P]
        L.oracle_nbhd_attn.restype = i32
        L.oracle_weighted_features.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, P]
        L.oracle_weighted_features.restype = i32
        L.oracle_softmax_merge.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, ctypes.c_double, P, P, P]
        L.oracle_softmax_merge.restype = i32
        L.oracle_deform_gather.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, i32, P]
        L.oracle_deform_gather.restype = i32
        L.oracle_num_threads.restype = i32
        L.oracle_set_num_threads.argtypes = [i32]
        _lib = L
    return _lib


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ----------------------------------------------------------------- KNN ----
def knn(query, ref, k: int):
    """Exact KNN: k smallest (d2, index) keys per query, ascending.

    query [B,M,D], ref [B,N,D] (fp32).  Returns (idx int64 [B,M,k],
    d2 fp32 [B,M,k]).  Restates src/layers/kernels/knn.py:258-337 and
    knn.py:1615-1648 (see oracle.c).
    """
    q = _f32(query)
    r = _f32(ref)
    B, M, D = q.shape
    N = r.shape[1]
    assert r.shape[0] == B and r.shape[2] == D
    assert 1 <= k <= N, f"k={k} exceeds number of reference points N={N}"
    idx = np.empty((B, M, k), dtype=np.int64)
    d2 = np.empty((B, M, k), dtype=np.float32)
    rc = lib().oracle_knn(_ptr(q), _ptr(r), B, M, N, D, k, _ptr(idx), _ptr(d2))
    if rc != 0:
        raise ValueError("oracle_knn rejected its arguments")
    return idx, d2


# ------------------------------------------------ neighbourhood attention ----
def nbhd_attn(q, k, v, member_idx, scale: float, bias=None, mask=None, blank_k=None, blank_v=None):
    """fp64 neighbourhood attention (src/layers/kernels/local_attn.py:80-340).

    q,k,v [B,H,N,D]; member_idx [B,N,M]; bias [B,H,N,M] or None;
    mask [B,H,N,M] / [B,1,N,M] (nonzero = valid) or None; blank_k/blank_v
    [H,D] or None.  Returns (out fp64 [B,H,N,D], lse fp64 [B,H,N]).
    """
    q = _f32(q); k = _f32(k); v = _f32(v)
    B, H, N, D = q.shape
    idx = np.ascontiguousarray(np.asarray(member_idx, dtype=np.int64))
    M = idx.shape[-1]
    assert idx.shape == (B, N, M)
    b = None if bias is None else _f32(np.broadcast_to(np.asarray(bias, dtype=np.float32), (B, H, N, M)))
    mk = None
    if mask is not None:
        mk = np.ascontiguousarray(np.broadcast_to(np.asarray(mask) != 0, (B, H, N, M)).astype(np.uint8))
    bk = None if blank_k is None else _f32(blank_k).reshape(H, D)
    bv = None if blank_v is None else _f32(blank_v).reshape(H, D)
    out = np.empty((B, H, N, D), dtype=np.float64)
    lse = np.empty((B, H, N), dtype=np.float64)
    lib().oracle_nbhd_attn(_ptr(q), _ptr(k), _ptr(v), _ptr(idx), _ptr(b), _ptr(mk), _ptr(bk), _ptr(bv),
                           float(scale), B, H, N, M, D, _ptr(out), _ptr(lse))
    return out, lse


# ------------------------------------------------------ weighted gathers ----
def weighted_features(weights, feat, nbhd_idx):
    """fp64 out[b,i,ic,c] = sum_m w[b,i,m,ic] f[b,idx,c] (weighted_features.py:30-111)."""
    w = _f32(weights)
    f = _f32(feat)
    idx = np.ascontiguousarray(np.asarray(nbhd_idx, dtype=np.int64))
    B, Nout, M, IC = w.shape
    N, C = f.shape[1], f.shape[2]
    assert idx.shape == (B, Nout, M) and f.shape[0] == B
    out = np.empty((B, Nout, IC, C), dtype=np.float64)
    lib().oracle_weighted_features(_ptr(w), _ptr(f), _ptr(idx), B, Nout, N, M, C, IC, _ptr(out))
    return out


def weighted_gather(nbhd_idx, weights, feat):
    """fp64 out[b,i,c] = sum_m w[b,i,m] f[b,idx,c] (weighted_gather.py:21-102)."""
    return weighted_features(np.asarray(weights)[..., None], feat, nbhd_idx)[:, :, 0, :]


def softmax_merge(query_pos, src_pos, feat, nbhd_idx, tau):
    """fp64 softmax(-d/tau) merge of features and coordinates.

    Returns (feat_out [B,Nout,C], pos_out [B,Nout,2], weights [B,Nout,K]).
    """
    q = _f32(query_pos)
    s = _f32(src_pos)
    f = _f32(feat)
    idx = np.ascontiguousarray(np.asarray(nbhd_idx, dtype=np.int64))
    B, Nout, K = idx.shape
    N, C = f.shape[1], f.shape[2]
    out = np.empty((B, Nout, C), dtype=np.float64)
    pos = np.empty((B, Nout, 2), dtype=np.float64)
    w = np.empty((B, Nout, K), dtype=np.float64)
    lib().oracle_softmax_merge(_ptr(q), _ptr(s), _ptr(f), _ptr(idx), B, Nout, N, K, C, float(tau),
                               _ptr(out), _ptr(pos), _ptr(w))
    return out, pos, w


# ----------------------------------------------------------- KNN (tree) ----
def knn_tree(query, ref, k: int):
    """Same result as :func:`knn` (exact fp32 keys, ties to the lower index)
    for large query sets: a scipy cKDTree proposes k + 8 candidates in fp64,
    their fp32 d2 is recomputed and ranked by (d2, index), and a query is
    re-run with more candidates whenever a point outside its candidate set
    could still rank within its first k.  query [M,2], ref [N,2] fp32 (one
    segment).  Returns (idx int64 [M,k], d2 fp32 [M,k]).
    """
    from scipy.spatial import cKDTree
    q = _f32(query)
    r = _f32(ref)
    M, N = q.shape[0], r.shape[0]
    assert 1 <= k <= N
    tree = cKDTree(r.astype(np.float64))
    idx = np.empty((M, k), dtype=np.int64)
    d2 = np.empty((M, k), dtype=np.float32)
    todo = np.arange(M)
    extra = 8
    while todo.size:
        kk = min(N, k + extra)
        dd, ii = tree.query(q[todo].astype(np.float64), k=kk)
        dd = np.asarray(dd, dtype=np.float64).reshape(len(todo), kk)
        ii = np.asarray(ii, dtype=np.int64).reshape(len(todo), kk)
        diff = q[todo][:, None, :] - r[ii]                  # fp32, no contraction in numpy
        c2 = (diff[..., 0] * diff[..., 0] + diff[..., 1] * diff[..., 1]).astype(np.float32)
        order = np.lexsort((ii, c2), axis=-1)
        ci = np.take_along_axis(ii, order, -1)[:, :k]
        cd = np.take_along_axis(c2, order, -1)[:, :k]
        # points outside the candidate set have fp64 distance >= dd[:, -1]
        bound = (dd[:, -1] ** 2) * (1 - 1e-5) - 1e-30
        safe = (kk == N) | (cd[:, -1].astype(np.float64) < bound)
        idx[todo[safe]] = ci[safe]
        d2[todo[safe]] = cd[safe]
        todo = todo[~safe]
        extra *= 4
    return idx, d2


# ----------------------------------------------------- deformable attention --
def deform_weights(d2, mode: str, power: float):
    """Per-sample neighbour weights in fp64 from fp32 squared distances.

    shepard: softmax(-max(p, 1e-6) * (sqrt(d2) + 1e-6)), denominator + 1e-8
             (fused_deform_attn.py:1296-1314);
    idw:     (1 / (d2^p + 1e-10)) / (sum + 1e-12) (geometry.py:49-52).
    Missing neighbours (d2 = inf) get weight 0.
    """
    d2 = np.asarray(d2, dtype=np.float64)
    valid = np.isfinite(d2)
    if mode == "shepard":
        p = max(power, 1e-6)
        lg = np.where(valid, -p * (np.sqrt(np.where(valid, d2, 0)) + 1e-6), -np.inf)
        mx = lg.max(axis=-1, keepdims=True)
        e = np.where(valid, np.exp(lg - mx), 0.0)
        return e / (e.sum(-1, keepdims=True) + 1e-8)
    u = np.where(valid, 1.0 / (np.where(valid, d2, 1.0) ** power + 1e-10), 0.0)
    return u / (u.sum(-1, keepdims=True) + 1e-12)


def deform(query_pos, kv_pos, level_start, offsets, attn, values, power: float, K: int, mode: str):
    """fp64 deformable attention with exact per-level K-NN (the semantics of
    aff_deform_fwd): query_pos [B,Nq,2], kv_pos [B,Ntot,2], offsets
    [B,Nq,H,L,P,2], attn [B,Nq,H,L,P], values [B,Ntot,H,C].
    Returns (out [B,Nq,H,C] fp64, knn_idx [B,Nq,H,L,P,K] level-local, -1 if missing).
    """
    qp = _f32(query_pos)
    kp = _f32(kv_pos)
    off = _f32(offsets)
    at = np.asarray(attn, dtype=np.float64)
    val = _f32(values)
    B, Nq, H, L, P, _ = off.shape
    C = val.shape[-1]
    Ntot = kp.shape[1]
    loc = (qp[:, :, None, None, None, :] + off).astype(np.float32)      # fp32 add
    rows = np.full((B, Nq, H, L, P, K), -1, dtype=np.int64)
    local = np.full((B, Nq, H, L, P, K), -1, dtype=np.int64)
    d2 = np.full((B, Nq, H, L, P, K), np.inf, dtype=np.float64)
    for b in range(B):
        for l in range(L):
            s0, s1 = level_start[l], level_start[l + 1]
            n = s1 - s0
            if n == 0:
                continue
            ke = min(K, n)
            pts = loc[b, :, :, l].reshape(-1, 2)
            ii, dd = knn_tree(pts, kp[b, s0:s1], ke)
            local[b, :, :, l, :, :ke] = ii.reshape(Nq, H, P, ke)
            rows[b, :, :, l, :, :ke] = ii.reshape(Nq, H, P, ke) + s0
            d2[b, :, :, l, :, :ke] = dd.reshape(Nq, H, P, ke)
    w = deform_weights(d2, mode, power) * at[..., None]
    out = np.empty((B, Nq, H, C), dtype=np.float64)
    S = L * P
    rows_c = np.ascontiguousarray(rows.reshape(B, Nq, H, S, K))
    w_c = np.ascontiguousarray(w.reshape(B, Nq, H, S, K))
    lib().oracle_deform_gather(_ptr(rows_c), _ptr(w_c), _ptr(val), B, Nq, H, S, K, Ntot, C, _ptr(out))
    return out, local


def deform_sample(sampling_locs, kv_pos, nb_idx, power: float, eps_mode: int, attn=None, values=None):
    """fp64 distance-softmax weights from given indices (fused_deform_attn.py:79-231
    for eps_mode 0: sqrt(d2) + 1e-6; mssample.py:17-125 for eps_mode 1:
    sqrt(d2 + 1e-6)), optionally gathered: returns (weights [B,N,K], out [B,N,C] or None).
    """
    sl = np.asarray(sampling_locs, dtype=np.float64)
    kv = np.asarray(kv_pos, dtype=np.float64)
    idx = np.asarray(nb_idx, dtype=np.int64)
    B, N, K = idx.shape
    Nkv = kv.shape[1]
    ok = (idx >= 0) & (idx < Nkv)
    nb = np.take_along_axis(kv, np.where(ok, idx, 0).reshape(B, -1, 1).repeat(kv.shape[2], 2), 1).reshape(B, N, K, -1)
    d2 = ((sl[:, :, None, :] - nb) ** 2).sum(-1)
    dist = np.sqrt(d2) + 1e-6 if eps_mode == 0 else np.sqrt(d2 + 1e-6)
    lg = np.where(ok, -max(power, 1e-6) * dist, -np.inf)
    e = np.where(ok, np.exp(lg - lg.max(-1, keepdims=True)), 0.0)
    w = e / (e.sum(-1, keepdims=True) + 1e-8)
    out = None
    if values is not None:
        a = np.ones((B, N)) if attn is None else np.asarray(attn, dtype=np.float64)
        out = weighted_gather(np.where(ok, idx, -1), (w * a[..., None]).astype(np.float32), values)
    return w, out


def msdetrpc(nn_idx, nn_weight, attn, val):
    """fp64 out[b,n,c] = sum_m sum_k attn[b,n,m] w[b,n,m,k] val[b, idx[b,n,m,k], c]
    (msdetrpc.py:25-109; its commented torch form at :529-530)."""
    idx = np.asarray(nn_idx, dtype=np.int64)
    B, N, M, K = idx.shape
    w = (np.asarray(attn, dtype=np.float64)[..., None] * np.asarray(nn_weight, dtype=np.float64))
    return weighted_features(w.reshape(B, N, M * K, 1).astype(np.float32), val, idx.reshape(B, N, M * K))[:, :, 0, :]


# ------------------------------------------------ relative-position bias ----
REL_POS_WIDTH = 1024 // 8 - 1          # src/utils/pos_embed.py:9
TABLE_WIDTH = 2 * REL_POS_WIDTH + 1    # pos_embed.py:10


def pre_table() -> np.ndarray:
    """[T*T, 5] fp32 rows (x, y, r, y/r, x/r), non-finite -> 0 (pos_embed.py:12-22).

    Row (ry * T + rx) holds offset (x, y) = (rx - 127, ry - 127).
    """
    t = np.arange(TABLE_WIDTH, dtype=np.float32) - REL_POS_WIDTH
    ys, xs = np.meshgrid(t, t, indexing="ij")
    with np.errstate(divide="ignore", invalid="ignore"):
        dis = np.sqrt(ys * ys + xs * xs)
        tab = np.stack([xs, ys, dis, ys / dis, xs / dis], axis=2)
    tab[~np.isfinite(tab)] = 0
    return tab.reshape(-1, 5).astype(np.float32)


def pe_index(pos, member_idx) -> np.ndarray:
    """pe_idx of BasicLayer (aff.py:458-465): truncated, clamped offsets + 127."""
    pos = np.asarray(pos, dtype=np.float32)
    idx = np.asarray(member_idx, dtype=np.int64)
    B, N, _ = pos.shape
    pos_m = np.take_along_axis(pos, idx.reshape(B, -1, 1).repeat(2, axis=2), axis=1).reshape(*idx.shape, 2)
    rel = pos_m - (pos[:, :, None, :] - REL_POS_WIDTH)
    rel = np.clip(rel, 0, TABLE_WIDTH - 1)
    return (rel[..., 1] * TABLE_WIDTH + rel[..., 0]).astype(np.int64)


def cluster_members(nearest, members, cmask=None, pos=None):
    """Neighbourhood gathers of BasicLayer (aff.py:452-465) by explicit indexing.

    member[b, n, ci * m + i] = members[b, nearest[b, n, ci], i]; a cluster id
    outside [0, K) or a member outside [0, N) gives member 0 with mask 0.
    mask likewise from cmask (returned only when cmask is given), pe_idx from
    pe_index() on the gathered members (when pos is given).
    """
    nearest = np.asarray(nearest, dtype=np.int64)
    members = np.asarray(members, dtype=np.int64)
    B, N, nnc = nearest.shape
    K, m = members.shape[1], members.shape[2]
    cok = (nearest >= 0) & (nearest < K)
    nc = np.where(cok, nearest, 0)
    bi = np.arange(B)[:, None, None, None]
    ii = np.arange(m)[None, None, None, :]
    mem = members[bi, nc[..., None], ii]                                  # [B, N, nnc, m]
    keep = np.broadcast_to(cok[..., None], mem.shape).copy()
    if cmask is not None:
        keep &= np.asarray(cmask)[bi, nc[..., None], ii] != 0
    bad = (mem < 0) | (mem >= N) | ~cok[..., None]
    mem = np.where(bad, 0, mem).reshape(B, N, nnc * m)
    keep = (keep & ~bad).reshape(B, N, nnc * m)
    pe = pe_index(pos, mem) if pos is not None else None
    return mem, (keep.astype(np.int64) if cmask is not None else None), pe


def table_bias(pe_idx, table) -> np.ndarray:
    """Dense [B,H,N,M] bias = table[pe_idx, h] (attention.py:117-124)."""
    table = np.asarray(table, dtype=np.float32)
    g = table[np.asarray(pe_idx, dtype=np.int64)]          # [B,N,M,H]
    return np.ascontiguousarray(np.transpose(g, (0, 3, 1, 2)))


def continuous_bias(pos, member_idx, w, b) -> np.ndarray:
    """Dense [B,H,N,M] bias = w . (dx, dy, r, dy/r, dx/r) + b in fp64.

    The continuous counterpart of table_bias(pe_index(...), pre_table() @ w.T + b):
    equal to it whenever every offset is an integer in [-127, 127].
    """
    pos = np.asarray(pos, dtype=np.float64)
    idx = np.asarray(member_idx, dtype=np.int64)
    B, N, _ = pos.shape
    pos_m = np.take_along_axis(pos, idx.reshape(B, -1, 1).repeat(2, axis=2), axis=1).reshape(*idx.shape, 2)
    d = pos_m - pos[:, :, None, :]
    dx, dy = d[..., 0], d[..., 1]
    r = np.sqrt(dx * dx + dy * dy)
    safe = np.where(r > 0, r, 1.0)
    f = np.stack([dx, dy, r, np.where(r > 0, dy / safe, 0.0), np.where(r > 0, dx / safe, 0.0)], axis=-1)
    out = f @ np.asarray(w, dtype=np.float64).T + np.asarray(b, dtype=np.float64)   # [B,N,M,H]
    return np.ascontiguousarray(np.transpose(out, (0, 3, 1, 2)))
