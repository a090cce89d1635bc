"""Pins the CPU oracle with checks that do not re-type its formulas.

KNN (oracle.knn):
  * scipy cKDTree (a different algorithm) on tie-free random inputs;
  * hand-derived known answers on integer lattices, where distances tie
    exactly and the lower index must win;
  * brute-force set properties: ascending keys, no unselected point with a
    smaller (d2, index) key, self at rank 0 for distinct points.
Attention (oracle.nbhd_attn):
  * a dense formulation: an N x N logit matrix with -inf outside each
    neighbour list, softmax by scipy, compared with the gathered oracle;
  * closed forms: one neighbour and no blank -> that value row; all masked
    and no blank -> 0 with lse = -1e11 + log(M); all masked with a blank ->
    the blank value; a uniform bias without blank changes nothing;
  * lse against scipy.special.logsumexp of the logits.
Bias inputs:
  * pre_table known rows (3-4-5 triangle, axes, zero offset);
  * pe_index on hand-built offsets (clamp at +-127, truncation);
  * table_bias(pe_index(p), pre_table() @ W.T + b) == continuous_bias(p)
    on integer offsets inside the table.
Golden fixtures: the oracle reproduces tests/golden/*.npz.
"""
import numpy as np
import pytest
from scipy.spatial import cKDTree
from scipy.special import logsumexp, softmax


# ------------------------------------------------------------------ KNN ----
@pytest.mark.parametrize("k", [1, 8, 48])
def test_knn_matches_kdtree(oracle_mod, k):
    rng = np.random.default_rng(10 + k)
    ref = rng.random((2, 700, 2), dtype=np.float32)
    q = rng.random((2, 300, 2), dtype=np.float32)
    idx, d2 = oracle_mod.knn(q, ref, k)
    for b in range(2):
        tree = cKDTree(ref[b].astype(np.float64))
        dd, ii = tree.query(q[b].astype(np.float64), k=k)
        ii = ii.reshape(300, k)
        np.testing.assert_array_equal(idx[b], ii)
        np.testing.assert_allclose(np.sqrt(d2[b]), dd.reshape(300, k), rtol=1e-5, atol=1e-7)


def test_knn_lattice_ties_known_answer(oracle_mod):
    # 5x5 lattice, indices row-major; query at the centre (2,2) = index 12.
    g = np.stack(np.meshgrid(np.arange(5), np.arange(5), indexing="xy"), -1).reshape(1, 25, 2).astype(np.float32)
    q = np.array([[[2.0, 2.0]]], dtype=np.float32)
    idx, d2 = oracle_mod.knn(q, g, 9)
    # d=0: 12; d=1: 7 (2,1), 11 (1,2), 13 (3,2), 17 (2,3); d=2: 6, 8, 16, 18
    assert idx[0, 0].tolist() == [12, 7, 11, 13, 17, 6, 8, 16, 18]
    assert d2[0, 0].tolist() == [0, 1, 1, 1, 1, 2, 2, 2, 2]


def test_knn_duplicates_lower_index_first(oracle_mod):
    # every point stored twice (index i and i+4); equal distances -> lower index
    p = np.array([[0, 0], [1, 0], [0, 1], [1, 1]], dtype=np.float32)
    ref = np.concatenate([p, p], 0)[None]
    q = np.array([[[0.1, 0.0]]], dtype=np.float32)
    idx, _ = oracle_mod.knn(q, ref, 8)
    assert idx[0, 0].tolist() == [0, 4, 1, 5, 2, 6, 3, 7]


def test_knn_bruteforce_properties(oracle_mod):
    rng = np.random.default_rng(3)
    # coarse grid coordinates -> many exact ties
    ref = (rng.integers(0, 12, (1, 400, 2))).astype(np.float32)
    q = (rng.integers(0, 12, (1, 100, 2)) + 0.5 * rng.integers(0, 2, (1, 100, 2))).astype(np.float32)
    k = 30
    idx, d2 = oracle_mod.knn(q, ref, k)
    diff = q[0][:, None, :] - ref[0][None, :, :]
    full = (diff[..., 0] * diff[..., 0] + diff[..., 1] * diff[..., 1]).astype(np.float32)
    for m in range(100):
        keys = list(zip(d2[0, m].tolist(), idx[0, m].tolist()))
        assert keys == sorted(keys)
        assert len(set(idx[0, m].tolist())) == k
        kd, ki = keys[-1]
        sel = set(idx[0, m].tolist())
        for n in range(400):
            if n not in sel:
                assert (full[m, n], n) > (kd, ki)
        np.testing.assert_array_equal(d2[0, m], full[m, idx[0, m]])


def test_knn_self_first(oracle_mod):
    rng = np.random.default_rng(4)
    p = rng.random((1, 256, 2), dtype=np.float32)
    idx, d2 = oracle_mod.knn(p, p, 5)
    assert (idx[0, :, 0] == np.arange(256)).all()
    assert (d2[0, :, 0] == 0).all()


def test_knn_k_equals_n(oracle_mod):
    rng = np.random.default_rng(5)
    p = rng.random((1, 33, 2), dtype=np.float32)
    idx, _ = oracle_mod.knn(p, p, 33)
    assert all(sorted(r) == list(range(33)) for r in idx[0].tolist())
    with pytest.raises(AssertionError, match="exceeds number of reference points"):
        oracle_mod.knn(p, p, 34)


# ------------------------------------------------------------ attention ----
def _dense_attention(q, k, v, idx, scale, bias, mask, blank_k, blank_v):
    """Dense N x N formulation: logits everywhere, -inf outside neighbour lists."""
    B, H, N, D = q.shape
    M = idx.shape[-1]
    out = np.zeros((B, H, N, D))
    lse = np.zeros((B, H, N))
    for b in range(B):
        for h in range(H):
            full = scale * (q[b, h].astype(np.float64) @ k[b, h].astype(np.float64).T)   # [N, N]
            logits = np.full((N, N), -np.inf)
            for n in range(N):
                for j in range(M):
                    if mask is None or mask[b, 0, n, j]:
                        logits[n, idx[b, n, j]] = full[n, idx[b, n, j]] + (0 if bias is None else bias[b, h, n, j])
            cols = [logits]
            vals = [v[b, h].astype(np.float64)]
            if blank_k is not None:
                cols.append(scale * (q[b, h].astype(np.float64) @ blank_k[h].astype(np.float64))[:, None])
                vals.append(blank_v[h].astype(np.float64)[None, :])
            L = np.concatenate(cols, axis=1)
            V = np.concatenate(vals, axis=0)
            out[b, h] = softmax(L, axis=1) @ V
            lse[b, h] = logsumexp(L, axis=1)
    return out, lse


@pytest.mark.parametrize("with_blank,with_mask", [(False, False), (True, False), (True, True)])
def test_attention_matches_dense(oracle_mod, with_blank, with_mask):
    rng = np.random.default_rng(20)
    B, H, N, D, M = 2, 2, 40, 8, 12
    q = rng.standard_normal((B, H, N, D), dtype=np.float32)
    k = rng.standard_normal((B, H, N, D), dtype=np.float32)
    v = rng.standard_normal((B, H, N, D), dtype=np.float32)
    # distinct neighbours per row (dense formulation needs no duplicates)
    idx = np.stack([np.stack([rng.permutation(N)[:M] for _ in range(N)]) for _ in range(B)])
    bias = rng.standard_normal((B, H, N, M)).astype(np.float32)
    mask = None
    if with_mask:
        mask = (rng.random((B, 1, N, M)) > 0.3)
        mask[..., 0] = True          # keep >= 1 valid neighbour (dense form has no -1e11 floor)
    bk = rng.standard_normal((H, D)).astype(np.float32) if with_blank else None
    bv = rng.standard_normal((H, D)).astype(np.float32) if with_blank else None
    out, lse = oracle_mod.nbhd_attn(q, k, v, idx, 0.35, bias=bias, mask=mask, blank_k=bk, blank_v=bv)
    ref_out, ref_lse = _dense_attention(q, k, v, idx, 0.35, bias, mask, bk, bv)
    np.testing.assert_allclose(out, ref_out, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-12, atol=1e-12)


def test_attention_closed_forms(oracle_mod):
    rng = np.random.default_rng(21)
    B, H, N, D = 1, 2, 10, 8
    q = rng.standard_normal((B, H, N, D), dtype=np.float32)
    k = rng.standard_normal((B, H, N, D), dtype=np.float32)
    v = rng.standard_normal((B, H, N, D), dtype=np.float32)
    # one neighbour, no blank -> the neighbour's value row
    idx1 = rng.integers(0, N, (B, N, 1))
    out, _ = oracle_mod.nbhd_attn(q, k, v, idx1, 0.5)
    np.testing.assert_allclose(out[0, :, np.arange(N)], np.transpose(v[0][:, idx1[0, :, 0]], (1, 0, 2)), rtol=1e-11)
    # all masked, no blank -> zeros, lse = -1e11 + log(M)
    M = 6
    idx = rng.integers(0, N, (B, N, M))
    mask = np.zeros((B, 1, N, M), dtype=bool)
    out, lse = oracle_mod.nbhd_attn(q, k, v, idx, 0.5, mask=mask)
    assert np.all(out == 0)
    np.testing.assert_allclose(lse, -1e11 + np.log(M), rtol=0, atol=1e-3)
    # all masked with a blank token -> the blank value
    bk = rng.standard_normal((H, D)).astype(np.float32)
    bv = rng.standard_normal((H, D)).astype(np.float32)
    out, _ = oracle_mod.nbhd_attn(q, k, v, idx, 0.5, mask=mask, blank_k=bk, blank_v=bv)
    np.testing.assert_allclose(out[0], np.broadcast_to(bv[:, None, :], (H, N, D)), rtol=1e-11)
    # a uniform bias shift without blank changes nothing but lse
    b0 = (rng.integers(-16, 16, (B, H, N, M)) / 8).astype(np.float32)   # dyadic: +3 is exact
    o1, l1 = oracle_mod.nbhd_attn(q, k, v, idx, 0.5, bias=b0)
    o2, l2 = oracle_mod.nbhd_attn(q, k, v, idx, 0.5, bias=b0 + np.float32(3.0))
    np.testing.assert_allclose(o1, o2, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(l2 - l1, 3.0, rtol=1e-9)


def test_attention_out_of_range_index_is_masked(oracle_mod):
    rng = np.random.default_rng(22)
    B, H, N, D, M = 1, 1, 8, 8, 4
    q, k, v = (rng.standard_normal((B, H, N, D), dtype=np.float32) for _ in range(3))
    idx = rng.integers(0, N, (B, N, M))
    bad = idx.copy()
    bad[..., 1] = N + 5
    bad[..., 2] = -1
    mask = np.ones((B, 1, N, M), dtype=bool)
    mask[..., 1:3] = False
    o1, l1 = oracle_mod.nbhd_attn(q, k, v, bad, 0.3)
    o2, l2 = oracle_mod.nbhd_attn(q, k, v, idx, 0.3, mask=mask)
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(l1, l2)


# ----------------------------------------------------------------- bias ----
def test_pre_table_known_rows(oracle_mod):
    tab = oracle_mod.pre_table()
    T, c = oracle_mod.TABLE_WIDTH, oracle_mod.REL_POS_WIDTH
    assert tab.shape == (255 * 255, 5)
    row = lambda x, y: tab[(y + c) * T + (x + c)]
    np.testing.assert_allclose(row(4, 3), [4, 3, 5, 0.6, 0.8], rtol=1e-6)
    np.testing.assert_allclose(row(-3, -4), [-3, -4, 5, -0.8, -0.6], rtol=1e-6)
    np.testing.assert_allclose(row(0, 7), [0, 7, 7, 1, 0], rtol=1e-6)
    np.testing.assert_array_equal(row(0, 0), [0, 0, 0, 0, 0])
    np.testing.assert_allclose(row(-127, 127), [-127, 127, 127 * 2 ** 0.5, 2 ** -0.5, -(2 ** -0.5)], rtol=1e-6)


def test_pe_index_known_answers(oracle_mod):
    pos = np.array([[[10.0, 20.0], [13.0, 16.0], [10.7, 20.2], [400.0, -300.0]]], dtype=np.float32)
    idx = np.array([[[1, 2, 3]] * 4])
    pe = oracle_mod.pe_index(pos, idx)
    T, c = 255, 127
    # token 0: offsets (3,-4) -> (130, 123); (0.7, 0.2) -> 127.2*255 + 127.7 = 32563.7, truncated
    # as one float (aff.py:465 truncates after combining); (390, -320) -> clamped (254, 0)
    assert pe[0, 0].tolist() == [123 * T + 130, 32563, 0 * T + 254]


def test_table_bias_equals_continuous_bias_on_integer_offsets(oracle_mod):
    rng = np.random.default_rng(30)
    B, N, M, H = 2, 200, 16, 3
    pos = rng.integers(0, 100, (B, N, 2)).astype(np.float32)
    idx, _ = oracle_mod.knn(pos, pos, M)
    w = rng.standard_normal((H, 5)).astype(np.float32)
    bb = rng.standard_normal(H).astype(np.float32)
    table = (oracle_mod.pre_table().astype(np.float64) @ w.T.astype(np.float64) + bb).astype(np.float64)
    tb = oracle_mod.table_bias(oracle_mod.pe_index(pos, idx), table)
    cb = oracle_mod.continuous_bias(pos, idx, w, bb)
    np.testing.assert_allclose(tb, cb, rtol=1e-6, atol=1e-5)   # pre_table is fp32


# --------------------------------------------------------------- golden ----
def test_golden_knn(oracle_mod, golden_dir):
    g = np.load(golden_dir / "knn_cfg1.npz")
    idx, d2 = oracle_mod.knn(g["pos"], g["pos"], 48)
    np.testing.assert_array_equal(idx, g["idx"].astype(np.int64))
    np.testing.assert_array_equal(d2, g["d2"])
    t = np.load(golden_dir / "knn_ties.npz")
    idx, d2 = oracle_mod.knn(t["query"], t["ref"], 24)
    np.testing.assert_array_equal(idx, t["idx"].astype(np.int64))


def test_golden_attention(oracle_mod, golden_dir):
    g = np.load(golden_dir / "attn_cfg1.npz")
    idx = g["idx"].astype(np.int64)
    bias = oracle_mod.continuous_bias(g["pos"], idx, g["pos_w"], g["pos_b"]).astype(np.float32)
    out, lse = oracle_mod.nbhd_attn(g["q"], g["k"], g["v"], idx, 32 ** -0.5, bias=bias,
                                    blank_k=g["blank_k"], blank_v=g["blank_v"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(lse, g["lse"], rtol=1e-6, atol=1e-6)
