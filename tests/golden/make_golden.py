"""Regenerate the golden fixtures in tests/golden from the CPU oracle.

The reference ships no golden vectors for this path (its tests compare
against modules that are absent, and its inline kernel tests regenerate
random data), so these fixtures are produced by the oracle from seeded
inputs.  The oracle itself is pinned by independent checks in
tests/test_oracle.py; the fixtures freeze its outputs so GPU runs (where the
oracle is rebuilt from source) and later rounds compare against the same
numbers.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402


def cfg1_coords(seed=0, B=2, N=1024):
    rng = np.random.default_rng(seed)
    return rng.random((B, N, 2), dtype=np.float32)


def make_knn_cfg1():
    pos = cfg1_coords()
    idx, d2 = oracle.knn(pos, pos, 48)
    np.savez_compressed(HERE / "knn_cfg1.npz", pos=pos, idx=idx.astype(np.int16), d2=d2)


def make_knn_ties():
    # 16x16 integer lattice (many exactly equal distances) plus every point
    # duplicated once: ties in d2 must resolve to the lower index.
    g = np.stack(np.meshgrid(np.arange(16), np.arange(16), indexing="xy"), -1).reshape(-1, 2).astype(np.float32)
    ref = np.concatenate([g, g[::-1]], 0)[None]            # [1, 512, 2]
    q = np.concatenate([g, g + 0.5], 0)[None]               # lattice points and cell centres
    idx, d2 = oracle.knn(q, ref, 24)
    np.savez_compressed(HERE / "knn_ties.npz", query=q, ref=ref, idx=idx.astype(np.int16), d2=d2)


def make_attn_cfg1():
    """Config-1 shaped attention (B=1, N=512 to keep the file small): fp32,
    H=2, D=32, k=48 KNN neighbours, continuous relative-position bias from a
    seeded Linear(5, 2), blank tokens ~ N(0, 0.2^2)."""
    B, N, H, D, M = 1, 512, 2, 32, 48
    pos = cfg1_coords(seed=1, B=B, N=N)
    idx, _ = oracle.knn(pos, pos, M)
    rng = np.random.default_rng(2)
    q = rng.standard_normal((B, H, N, D), dtype=np.float32)
    k = rng.standard_normal((B, H, N, D), dtype=np.float32)
    v = rng.standard_normal((B, H, N, D), dtype=np.float32)
    w = (rng.standard_normal((H, 5)) * 0.4).astype(np.float32)
    bb = (rng.standard_normal(H) * 0.1).astype(np.float32)
    blank_k = (rng.standard_normal((H, D)) * 0.2).astype(np.float32)
    blank_v = (rng.standard_normal((H, D)) * 0.2).astype(np.float32)
    bias = oracle.continuous_bias(pos, idx, w, bb).astype(np.float32)
    out, lse = oracle.nbhd_attn(q, k, v, idx, D ** -0.5, bias=bias, blank_k=blank_k, blank_v=blank_v)
    np.savez_compressed(HERE / "attn_cfg1.npz", pos=pos, idx=idx.astype(np.int16), q=q, k=k, v=v,
                        pos_w=w, pos_b=bb, blank_k=blank_k, blank_v=blank_v,
                        out=out.astype(np.float32), lse=lse.astype(np.float32))


if __name__ == "__main__":
    make_knn_cfg1()
    make_knn_ties()
    make_attn_cfg1()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
