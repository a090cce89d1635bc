"""The MFMA path of aff_nbhd_attn_fwd (bf16 / fp16, head_dim 32, M <= 64).

The wave kernel serves these calls, and aff_nbhd_attn_path() confirms it for
every test: one workgroup per (32 consecutive queries, group of up to
min(4, 192 // M) heads), one wave per head.  Its set-up deduplicates the
tile's neighbour indices into a union of at most 224 token rows; tiles it
cannot take (a wider union, an index window over 8192, an index repeated
within one query, a per-head mask) run the per-row routine for the group's
heads inside the same workgroup.  The cases with H * M > 192 (the encoder's
8- and 16-head stages) run several head groups per tile.

Each case below is built so that one of those branches runs, and every
result is checked against the fp64 oracle (oracle/oracle.c) at the
bf16/fp16 tolerance of 2e-2 max-abs on the output and the LSE.
"""
import numpy as np
import pytest
import torch

from affmae_amd.kernels import knn, nbhd_attn_fwd
from affmae_amd.kernels.local_attn import record_paths
from affmae_amd.utils.pos_embed import pre_table_fp32, pe_index

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _np(t):
    return t.detach().float().cpu().numpy()


def _grid_coords(B, N, seed):
    """N jittered points on a sqrt(2N)-wide integer grid, raster order (KNN neighbours are local)."""
    g = torch.Generator().manual_seed(seed)
    side = int(np.ceil(np.sqrt(2 * N)))
    out = torch.empty((B, N, 2))
    for b in range(B):
        cells = torch.randperm(side * side, generator=g)[:N].sort().values
        xy = torch.stack([cells % side, cells // side], -1).float()
        out[b] = xy + torch.rand((N, 2), generator=g) - 0.5
    return out


def _check(out, lse, ro, rl, what):
    err = np.abs(_np(out).astype(np.float64) - ro).max()
    assert err <= TOL, f"{what}: out abs err {err:.3e}"
    if lse is not None:
        # a fully masked row has lse = -1e11 + log(M): fp32 holds it to within one ulp (8192),
        # so the bound adds the fp32 representation error of the reference value
        lerr = np.abs(_np(lse).astype(np.float64) - rl) - 2.0 ** -23 * np.abs(rl)
        assert lerr.max() <= TOL, f"{what}: lse abs err {lerr.max():.3e}"


def _qkv(B, H, N, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn((B, H, N, 32), generator=g).to(dtype) for _ in range(3))
    bk = (torch.randn((H, 32), generator=g) * 0.5).to(dtype)
    bv = (torch.randn((H, 32), generator=g) * 0.5).to(dtype)
    return q, k, v, bk, bv


def _path(bias_mode, H, M):
    """The kernel family aff_nbhd_attn_fwd picks for 16-bit head_dim-32 inputs, M <= 64:
    the wave kernel, in workgroups of min(H, 192 // M) heads."""
    return "wave"


def _run(oracle_mod, dev, q, k, v, idx, scale, dense_bias=None, mask=None, bk=None, bv=None, expect=None, **kw):
    """Run the kernel and the oracle; `expect` ("wave" / "row") is the path the call must take."""
    print(f"[tile] B,H,N={tuple(q.shape[:3])} M={idx.shape[-1]} {q.dtype} {sorted(kw)} expect={expect}", flush=True)
    g = lambda t: None if t is None else t.to(dev)
    with record_paths() as paths:
        out, lse = nbhd_attn_fwd(g(q), g(k), g(v), g(idx), scale, mask=g(mask), blank_k=g(bk), blank_v=g(bv), **kw)
    torch.cuda.synchronize()
    if expect is not None:
        assert paths == [expect], f"expected the {expect} path, ran {paths}"
    ro, rl = oracle_mod.nbhd_attn(_np(q), _np(k), _np(v), idx.cpu().numpy(), scale,
                                  bias=dense_bias, mask=None if mask is None else mask.cpu().numpy(),
                                  blank_k=None if bk is None else _np(bk), blank_v=None if bv is None else _np(bv))
    return out, lse, ro, rl


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias_mode", ["none", "dense", "table", "coords", "continuous"])
def test_tile_bias_modes(oracle_mod, dev, dtype, bias_mode):
    """KNN neighbours (no repeats, local union) -> the MFMA branch; N = 997 leaves a ragged last tile."""
    B, H, N, M = 2, 4, 997, 48
    pos = _grid_coords(B, N, seed=11)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    q, k, v, bk, bv = _qkv(B, H, N, dtype, seed=12)
    lin = torch.nn.Linear(5, H)
    torch.nn.init.uniform_(lin.weight, -0.4, 0.4)
    w, bb = lin.weight.detach(), lin.bias.detach()
    table = (pre_table_fp32.double() @ w.double().T + bb.double()).float()
    kw, dense = {}, None
    if bias_mode in ("table", "coords", "dense"):
        pe = pe_index(pos, idx)
        dense = table[pe].permute(0, 3, 1, 2).contiguous()
        if bias_mode == "table":
            kw = dict(pe_idx=pe.to(dev), pe_table=table.to(dev))
        elif bias_mode == "coords":
            kw = dict(pos=pos.to(dev), pe_table=table.to(dev))
        else:
            dense = dense.to(dtype).float()
            kw = dict(bias=dense.to(dtype).to(dev))
        dense = dense.numpy()
    elif bias_mode == "continuous":
        dense = oracle_mod.continuous_bias(pos.numpy(), idx.numpy(), w.numpy(), bb.numpy()).astype(np.float32)
        kw = dict(pos=pos.to(dev), pos_weight=w.to(dev), pos_bias=bb.to(dev))
    out, lse, ro, rl = _run(oracle_mod, dev, q, k, v, idx, 32 ** -0.5, dense_bias=dense, bk=bk, bv=bv,
                            expect=_path(bias_mode, H, M), **kw)
    assert out.dtype == dtype
    _check(out, lse, ro, rl, bias_mode)


@pytest.mark.parametrize("M", [0, 8, 24, 40, 64])
def test_tile_neighbour_counts(oracle_mod, dev, M):
    B, H, N = 1, 2, 300
    pos = _grid_coords(B, N, seed=20 + M)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu() if M else torch.zeros((B, N, 0), dtype=torch.int64)
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=21)
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, bk=bk, bv=bv, expect=_path("none", H, M)), f"M={M}")


@pytest.mark.parametrize("blank", [False, True])
def test_tile_shared_mask_and_masked_rows(oracle_mod, dev, blank):
    """A [B,1,N,M] mask keeps the MFMA branch; every fifth query is fully masked."""
    B, H, N, M = 2, 4, 400, 48
    pos = _grid_coords(B, N, seed=30)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=31)
    mask = torch.rand((B, 1, N, M), generator=torch.Generator().manual_seed(32)) > 0.3
    mask[:, :, ::5] = False
    out, lse, ro, rl = _run(oracle_mod, dev, q, k, v, idx, 0.3, mask=mask,
                            bk=bk if blank else None, bv=bv if blank else None, expect="wave")
    _check(out, lse, ro, rl, "shared mask")
    if not blank:
        assert torch.all(out[:, :, ::5].float() == 0)


def test_tile_fallback_repeated_index(oracle_mod, dev):
    """Neighbour lists that repeat an index count it twice in the softmax (per-row branch)."""
    B, H, N, M = 1, 4, 256, 48
    pos = _grid_coords(B, N, seed=40)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    idx[:, 7::16, 5] = idx[:, 7::16, 9]          # one query in every tile repeats a neighbour
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=41)
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, bk=bk, bv=bv, expect="wave"), "repeat")


def test_tile_fallback_wide_union(oracle_mod, dev):
    """Distinct random neighbours over 4000 tokens: the 32-query union exceeds 224 rows."""
    B, H, N, M = 1, 2, 4000, 48
    g = torch.Generator().manual_seed(50)
    idx = torch.stack([torch.randperm(N, generator=g)[:M] for _ in range(N)]).unsqueeze(0)
    q, k, v, bk, bv = _qkv(B, H, N, torch.float16, seed=51)
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, bk=bk, bv=bv, expect="wave"), "wide union")


def test_tile_fallback_wide_window_mixed(oracle_mod, dev):
    """Local neighbours everywhere except a few queries that also reach a token 9000 rows away:
    their tiles exceed the 8192-index window and take the per-row branch, the rest stay on MFMA."""
    B, H, N, M = 1, 4, 10000, 32
    pos = _grid_coords(B, N, seed=60)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    far = torch.arange(0, 800, 37)
    idx[0, far, 3] = (far + 9000) % N
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=61)
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, bk=bk, bv=bv, expect="wave"), "wide window")


def test_tile_fallback_per_head_mask(oracle_mod, dev):
    B, H, N, M = 1, 4, 200, 24
    pos = _grid_coords(B, N, seed=70)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=71)
    mask = torch.rand((B, H, N, M), generator=torch.Generator().manual_seed(72)) > 0.5
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, mask=mask, bk=bk, bv=bv, expect="wave"), "per-head mask")


def test_tile_out_of_range_indices(oracle_mod, dev):
    B, H, N, M = 1, 2, 320, 16
    pos = _grid_coords(B, N, seed=80)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    idx[..., 2] = N
    idx[..., 11] = -1
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=81)
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, bk=bk, bv=bv, expect="wave"), "out of range")


def test_tile_strided_interleaved_kv(oracle_mod, dev):
    """ClusterAttention layout: q from [B,N,H*D], k/v the halves of each head's slice of [B,N,H*2D],
    output written through a permuted [B,N,H,D] view."""
    B, N, H, D, M = 2, 500, 4, 32, 48
    pos = _grid_coords(B, N, seed=90)
    idx = knn(pos.to(dev), pos.to(dev), M, ).to(torch.int32)
    g = torch.Generator().manual_seed(91)
    qf = torch.randn((B, N, H * D), generator=g).bfloat16()
    kvf = torch.randn((B, N, 2 * H * D), generator=g).bfloat16()
    qd, kvd = qf.to(dev), kvf.to(dev)
    qh = qd.view(B, N, H, D).permute(0, 2, 1, 3)
    kvh = kvd.view(B, N, H, 2 * D).permute(0, 2, 1, 3)
    out_buf = torch.empty((B, N, H, D), device=dev, dtype=torch.bfloat16)
    nbhd_attn_fwd(qh, kvh[..., :D], kvh[..., D:], idx, 0.25, out=out_buf.permute(0, 2, 1, 3), return_lse=False)
    torch.cuda.synchronize()
    kc = kvf.view(B, N, H, 2 * D).permute(0, 2, 1, 3)
    ro, _ = oracle_mod.nbhd_attn(_np(qf.view(B, N, H, D).permute(0, 2, 1, 3).contiguous()),
                                 _np(kc[..., :D].contiguous()), _np(kc[..., D:].contiguous()),
                                 idx.cpu().numpy(), 0.25)
    _check(out_buf.permute(0, 2, 1, 3), None, ro, None, "strided")


# ------------------------------------------------------------ head groups --
# H * M > 192: several workgroups of up to 4 heads per tile.

def _table(H, seed):
    """[T*T, H] bias table: a seeded Linear(5, H) over the offset features."""
    g = torch.Generator().manual_seed(seed)
    w = torch.rand((H, 5), generator=g) * 0.8 - 0.4
    bb = torch.rand((H,), generator=g) * 0.2 - 0.1
    return (pre_table_fp32.double() @ w.double().T + bb.double()).float()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,M", [(8, 48), (16, 32), (16, 48)])
@pytest.mark.parametrize("bias_mode", ["table", "coords"])
def test_tile_kernel_many_heads(oracle_mod, dev, dtype, H, M, bias_mode):
    """The encoder's 8- and 16-head stages (M = 48, nnc = 6) on integer grid coordinates, as
    the encoder's tokens are; N = 997 leaves a ragged last tile."""
    B, N = 2, 997
    pos = _grid_coords(B, N, seed=100 + H + M).round()
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    q, k, v, bk, bv = _qkv(B, H, N, dtype, seed=101)
    table = _table(H, seed=102)
    pe = pe_index(pos, idx)
    dense = table[pe].permute(0, 3, 1, 2).contiguous().numpy()
    kw = dict(pe_idx=pe.to(dev), pe_table=table.to(dev)) if bias_mode == "table" else \
        dict(pos=pos.to(dev), pe_table=table.to(dev))
    out, lse, ro, rl = _run(oracle_mod, dev, q, k, v, idx, 32 ** -0.5, dense_bias=dense, bk=bk, bv=bv,
                            expect=_path(bias_mode, H, M), **kw)
    assert out.dtype == dtype
    _check(out, lse, ro, rl, f"tile H={H} M={M} {bias_mode}")


@pytest.mark.parametrize("case", ["repeat", "wide_union", "per_head_mask", "shared_mask"])
def test_tile_kernel_flagged_tiles(oracle_mod, dev, case):
    """Tiles the set-up rejects (a repeated index, a union over 224 rows, a per-head mask) run
    the per-row routine for each head group; a shared mask stays on the matrix cores."""
    B, H, N, M = 1, 8, 640, 48
    pos = _grid_coords(B, N, seed=110).round()
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    mask = None
    if case == "repeat":
        idx[:, 7::32, 5] = idx[:, 7::32, 9]       # one query in every tile repeats a neighbour
    elif case == "wide_union":
        g = torch.Generator().manual_seed(111)
        far = torch.randint(0, N, (N // 2, M), generator=g)
        idx[0, 64:64 + N // 2] = far              # tiles 2..11: random neighbours, unions past 224 rows
    elif case == "per_head_mask":
        mask = torch.rand((B, H, N, M), generator=torch.Generator().manual_seed(112)) > 0.4
    else:
        mask = torch.rand((B, 1, N, M), generator=torch.Generator().manual_seed(113)) > 0.4
        mask[:, :, ::7] = False
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=114)
    table = _table(H, seed=115)
    pe = pe_index(pos, idx)
    dense = table[pe].permute(0, 3, 1, 2).contiguous().numpy()
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, dense_bias=dense, mask=mask, bk=bk, bv=bv,
                 expect="wave", pe_idx=pe.to(dev), pe_table=table.to(dev)), f"flagged {case}")


def test_tile_kernel_no_bias_no_blank(oracle_mod, dev):
    B, H, N, M = 2, 16, 300, 24
    pos = _grid_coords(B, N, seed=120)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    q, k, v, _, _ = _qkv(B, H, N, torch.float16, seed=121)
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, expect="wave"), "tile no bias")


@pytest.mark.parametrize("bias_mode", ["dense", "continuous"])
def test_tile_kernel_dense_and_continuous(oracle_mod, dev, bias_mode):
    """H * M > 192 with the dense and continuous bias forms: head groups of the wave kernel."""
    B, H, N, M = 2, 8, 500, 48
    pos = _grid_coords(B, N, seed=130)
    idx = knn(pos.to(dev), pos.to(dev), M).cpu()
    q, k, v, bk, bv = _qkv(B, H, N, torch.bfloat16, seed=131)
    g = torch.Generator().manual_seed(132)
    if bias_mode == "dense":
        dense = (torch.randn((B, H, N, M), generator=g) * 0.5).bfloat16().float()
        kw = dict(bias=dense.bfloat16().to(dev))
        dense = dense.numpy()
    else:
        w = torch.rand((H, 5), generator=g) * 0.8 - 0.4
        bb = torch.rand((H,), generator=g) * 0.2 - 0.1
        dense = oracle_mod.continuous_bias(pos.numpy(), idx.numpy(), w.numpy(), bb.numpy()).astype(np.float32)
        kw = dict(pos=pos.to(dev), pos_weight=w.to(dev), pos_bias=bb.to(dev))
    _check(*_run(oracle_mod, dev, q, k, v, idx, 0.3, dense_bias=dense, bk=bk, bv=bv, expect="wave", **kw),
           f"tile {bias_mode}")
