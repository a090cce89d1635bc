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
  (src/layers/aff.py:458-465), :func:`table_bias`
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
