"""Neighbourhood attention on the GPU through the C ABI against the fp64 oracle.

Tolerances (from the north-star spec): fp32 inputs -> max|out - ref| <=
1e-5 * max|ref| (relative to the output scale) and the same for lse;
bf16 / fp16 inputs -> max-abs error <= 2e-2 against the oracle evaluated on
the same rounded inputs.  The reference's own inline test case
(local_attn.py:939-1022) is reproduced with its tolerance atol = 1e-2.
"""
import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels import launch_flash_nbhood_attn_fwd, nbhd_attn_fwd, knn
from affmae_amd.kernels.local_attn import FlashLocalAttentionFunction
from affmae_amd.utils.pos_embed import pre_table_fp32, pe_index

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5
LOWP_ABS = 2e-2


def _np(t):
    return t.detach().float().cpu().numpy()


def _assert_fp32(out, lse, ro, rl):
    scale = max(np.abs(ro).max(), 1e-30)
    o64 = _np(out).astype(np.float64)
    err = np.abs(o64 - ro).max()
    assert err <= FP32_REL * scale, f"out rel err {err / scale:.3e}"
    # elementwise: 1e-5 of each element plus a floor of 1e-6 of the output scale (outputs that
    # cancel to ~0 keep only the absolute error of fp32 summation order)
    bad = np.abs(o64 - ro) > FP32_REL * np.abs(ro) + 1e-6 * scale
    assert not bad.any(), f"out elementwise rel err at {np.argwhere(bad)[:3].tolist()}"
    if lse is not None:
        lscale = max(np.abs(rl).max(), 1.0)
        lerr = np.abs(_np(lse).astype(np.float64) - rl).max()
        assert lerr <= FP32_REL * lscale, f"lse rel err {lerr / lscale:.3e}"


def _assert_lowp(out, lse, ro, rl):
    err = np.abs(_np(out).astype(np.float64) - ro).max()
    assert err <= LOWP_ABS, f"out abs err {err:.3e}"
    if lse is not None:
        lerr = np.abs(_np(lse).astype(np.float64) - rl).max()
        assert lerr <= LOWP_ABS, f"lse abs err {lerr:.3e}"


def _rand_case(B, H, N, D, M, dtype, seed, dev, mask=False, blank=True, bias=True):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn((B, H, N, D), generator=g).to(dtype) for _ in range(3))
    idx = torch.randint(0, N, (B, N, M), generator=g)
    b = (torch.randn((B, H, N, M), generator=g) * 2).to(dtype) if bias else None
    mk = (torch.rand((B, 1, N, M), generator=g) > 0.25) if mask else None
    bk = (torch.randn((H, D), generator=g) * 0.5).to(dtype) if blank else None
    bv = (torch.randn((H, D), generator=g) * 0.5).to(dtype) if blank else None
    cpu = dict(q=q, k=k, v=v, idx=idx, bias=b, mask=mk, bk=bk, bv=bv)
    gpu = {n: (t.to(dev) if t is not None else None) for n, t in cpu.items()}
    return cpu, gpu


def _oracle(oracle_mod, c, scale):
    return oracle_mod.nbhd_attn(_np(c["q"]), _np(c["k"]), _np(c["v"]), c["idx"].numpy(), scale,
                                bias=None if c["bias"] is None else _np(c["bias"]),
                                mask=None if c["mask"] is None else c["mask"].numpy(),
                                blank_k=None if c["bk"] is None else _np(c["bk"]),
                                blank_v=None if c["bv"] is None else _np(c["bv"]))


# ---------------------------------------------------------------- golden --
def test_golden_cfg1_continuous_bias(golden_dir, dev):
    g = np.load(golden_dir / "attn_cfg1.npz")
    t = {n: torch.from_numpy(g[n]).to(dev) for n in ("q", "k", "v", "pos", "pos_w", "pos_b", "blank_k", "blank_v")}
    idx = torch.from_numpy(g["idx"].astype(np.int64)).to(dev)
    out, lse = nbhd_attn_fwd(t["q"], t["k"], t["v"], idx, 32 ** -0.5, pos=t["pos"], pos_weight=t["pos_w"],
                             pos_bias=t["pos_b"], blank_k=t["blank_k"], blank_v=t["blank_v"])
    _assert_fp32(out, lse, g["out"].astype(np.float64), g["lse"].astype(np.float64))


# ------------------------------------------------------- config 1 (fp32) --
@pytest.mark.parametrize("bias_mode", ["dense", "table", "continuous"])
def test_cfg1_fp32_knn_neighbours(oracle_mod, dev, bias_mode):
    """B=2, N=1024 uniform points, k=48 KNN neighbours, C=64 / 2 heads / D=32, fp32."""
    B, N, H, D, M = 2, 1024, 2, 32, 48
    pos = workloads.cfg1_coords(B, N, seed=0)
    if bias_mode == "table":
        pos = torch.floor(pos * 32)          # integer offsets -> table rows are exact
    pos_d = pos.to(dev)
    idx = knn(pos_d, pos_d, M)
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn((B, H, N, D), generator=g) for _ in range(3))
    lin = torch.nn.Linear(5, H)
    torch.nn.init.uniform_(lin.weight, -0.4, 0.4)
    w, bb = lin.weight.detach(), lin.bias.detach()
    bk, bv = torch.randn((H, D), generator=g) * 0.2, torch.randn((H, D), generator=g) * 0.2
    idx_np = idx.cpu().numpy()
    if bias_mode == "continuous":
        dense = oracle_mod.continuous_bias(pos.numpy(), idx_np, w.numpy(), bb.numpy())
        kw = dict(pos=pos_d, pos_weight=w.to(dev), pos_bias=bb.to(dev))
    else:
        table = (oracle_mod.pre_table().astype(np.float64) @ w.numpy().T.astype(np.float64) + bb.numpy()).astype(np.float32)
        pe = oracle_mod.pe_index(pos.numpy(), idx_np)
        dense = oracle_mod.table_bias(pe, table)
        if bias_mode == "dense":
            kw = dict(bias=torch.from_numpy(dense).to(dev))
        else:
            kw = dict(pe_idx=torch.from_numpy(pe).to(dev), pe_table=torch.from_numpy(table).to(dev))
    out, lse = nbhd_attn_fwd(q.to(dev), k.to(dev), v.to(dev), idx, D ** -0.5, blank_k=bk.to(dev),
                             blank_v=bv.to(dev), **kw)
    ro, rl = oracle_mod.nbhd_attn(q.numpy(), k.numpy(), v.numpy(), idx_np, D ** -0.5,
                                  bias=dense.astype(np.float32), blank_k=bk.numpy(), blank_v=bv.numpy())
    _assert_fp32(out, lse, ro, rl)


# --------------------------------------------------------- config 2 (bf16) --
@pytest.mark.parametrize("B", [2, 32])
def test_cfg2_bf16(oracle_mod, dev, B):
    """Benchmark shape (B=32 is the full config): N=6272, H=4, D=32, k=48, bf16,
    bias = Linear(5,4)(pre_table)[pe_idx] read in-kernel from the table."""
    w = workloads.cfg2(B=B)
    pos = w["pos"].to(dev)
    idx = knn(pos, pos, 48)
    pe = pe_index(pos, idx)
    table = (pre_table_fp32.double() @ w["pos_w"].double().T + w["pos_b"].double()).float()
    print(f"[attn cfg2] B={B}", flush=True)
    out, lse = nbhd_attn_fwd(w["q"].to(dev), w["k"].to(dev), w["v"].to(dev), idx, 32 ** -0.5,
                             pe_idx=pe, pe_table=table.to(dev), blank_k=w["blank_k"].to(dev),
                             blank_v=w["blank_v"].to(dev))
    assert out.dtype == torch.bfloat16
    # bias mode 4 (table row computed in-kernel from the coordinates) must pick
    # exactly the rows torch's pe_idx picks: identical output bits
    out4, lse4 = nbhd_attn_fwd(w["q"].to(dev), w["k"].to(dev), w["v"].to(dev), idx, 32 ** -0.5,
                               pos=pos, pe_table=table.to(dev), blank_k=w["blank_k"].to(dev),
                               blank_v=w["blank_v"].to(dev))
    assert torch.equal(out4, out) and torch.equal(lse4, lse)
    dense = table[pe.cpu()].permute(0, 3, 1, 2).contiguous().numpy()
    ro, rl = oracle_mod.nbhd_attn(_np(w["q"]), _np(w["k"]), _np(w["v"]), idx.cpu().numpy(), 32 ** -0.5,
                                  bias=dense, blank_k=_np(w["blank_k"]), blank_v=_np(w["blank_v"]))
    _assert_lowp(out, lse, ro, rl)


# ------------------------------------------------ the reference's own case --
def test_reference_inline_case(oracle_mod, dev):
    """local_attn.py:939-1022: B=5, H=2, N=128, D=64, M=64, fp16, scale 0.5,
    structured q/k/v columns, blank *5, bias *5 with its first 5 columns = 1,
    random member indices, all-ones mask; atol 1e-2 on O and LSE."""
    g = torch.Generator().manual_seed(0)
    B, H, N, D, M = 5, 2, 128, 64, 64
    q, k, v = (torch.randn((B, H, N, D), generator=g).half() for _ in range(3))
    q[:, :, :, :10] = 1.0
    k[:, :, :, :5] = 0.1
    v[:, :, :, :5] = 1.0
    bk = (torch.randn((H, D), generator=g) * 5.0).half()
    bv = (torch.randn((H, D), generator=g) * 5.0).half()
    bias = (torch.randn((B, H, N, M), generator=g) * 5.0).half()
    bias[:, :, :, :5] = 1.0
    idx = torch.randint(0, N, (B, N, M), generator=g, dtype=torch.int32)
    mask = torch.ones((B, 1, N, M), dtype=torch.int32)
    out, lse = launch_flash_nbhood_attn_fwd(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), 0.5, bias=bias.to(dev),
                                            mask=mask.to(dev), blank_k=bk.to(dev), blank_v=bv.to(dev))
    ro, rl = oracle_mod.nbhd_attn(_np(q), _np(k), _np(v), idx.numpy(), 0.5, bias=_np(bias), mask=mask.numpy(),
                                  blank_k=_np(bk), blank_v=_np(bv))
    assert np.abs(_np(out) - ro).max() <= 1e-2
    assert np.abs(_np(lse) - rl).max() <= 1e-2


# ----------------------------------------------------------- edge cases --
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [8, 16, 32, 64, 128])
def test_dtypes_and_head_dims(oracle_mod, dev, dtype, D):
    c, g = _rand_case(2, 3, 200, D, 24, dtype, seed=D, dev=dev, mask=True)
    out, lse = nbhd_attn_fwd(g["q"], g["k"], g["v"], g["idx"], D ** -0.5, bias=g["bias"], mask=g["mask"],
                             blank_k=g["bk"], blank_v=g["bv"])
    ro, rl = _oracle(oracle_mod, c, D ** -0.5)
    (_assert_fp32 if dtype == torch.float32 else _assert_lowp)(out, lse, ro, rl)


@pytest.mark.parametrize("M", [1, 5, 13, 48, 70])
def test_neighbour_counts(oracle_mod, dev, M):
    c, g = _rand_case(1, 2, 150, 32, M, torch.float32, seed=100 + M, dev=dev)
    out, lse = nbhd_attn_fwd(g["q"], g["k"], g["v"], g["idx"], 0.2, bias=g["bias"], blank_k=g["bk"], blank_v=g["bv"])
    _assert_fp32(out, lse, *_oracle(oracle_mod, c, 0.2))


def test_no_blank_no_bias(oracle_mod, dev):
    c, g = _rand_case(2, 2, 100, 32, 16, torch.float32, seed=5, dev=dev, blank=False, bias=False)
    out, lse = nbhd_attn_fwd(g["q"], g["k"], g["v"], g["idx"], 0.3)
    _assert_fp32(out, lse, *_oracle(oracle_mod, c, 0.3))


def test_all_masked_rows(oracle_mod, dev):
    for blank in (False, True):
        c, g = _rand_case(1, 2, 64, 32, 8, torch.float32, seed=6, dev=dev, blank=blank)
        mask = torch.ones((1, 1, 64, 8), dtype=torch.bool)
        mask[:, :, ::3] = False                   # every third row fully masked
        c["mask"], g["mask"] = mask, mask.to(dev)
        out, lse = nbhd_attn_fwd(g["q"], g["k"], g["v"], g["idx"], 0.3, bias=g["bias"], mask=g["mask"],
                                 blank_k=g["bk"], blank_v=g["bv"])
        ro, rl = _oracle(oracle_mod, c, 0.3)
        _assert_fp32(out, lse, ro, rl)
        if not blank:
            assert torch.all(out[:, :, ::3] == 0)


def test_per_head_mask(oracle_mod, dev):
    c, g = _rand_case(2, 4, 80, 16, 12, torch.float32, seed=7, dev=dev)
    mask = torch.rand((2, 4, 80, 12), generator=torch.Generator().manual_seed(1)) > 0.5
    c["mask"], g["mask"] = mask, mask.to(dev)
    out, lse = nbhd_attn_fwd(g["q"], g["k"], g["v"], g["idx"], 0.3, bias=g["bias"], mask=g["mask"],
                             blank_k=g["bk"], blank_v=g["bv"])
    ro, rl = oracle_mod.nbhd_attn(_np(c["q"]), _np(c["k"]), _np(c["v"]), c["idx"].numpy(), 0.3,
                                  bias=_np(c["bias"]), mask=mask.numpy(), blank_k=_np(c["bk"]), blank_v=_np(c["bv"]))
    _assert_fp32(out, lse, ro, rl)


def test_out_of_range_indices_are_masked(oracle_mod, dev):
    c, g = _rand_case(1, 2, 60, 32, 8, torch.float32, seed=8, dev=dev)
    bad = c["idx"].clone()
    bad[..., 2] = 60
    bad[..., 5] = -3
    out, lse = nbhd_attn_fwd(g["q"], g["k"], g["v"], bad.to(dev), 0.3, bias=g["bias"], blank_k=g["bk"], blank_v=g["bv"])
    c["idx"] = bad
    _assert_fp32(out, lse, *_oracle(oracle_mod, c, 0.3))


def test_strided_views_and_int32_index(oracle_mod, dev):
    """ClusterAttention-style views: q from [B,N,C], k/v interleaved per head in [B,N,2C]."""
    B, N, H, D, M = 2, 300, 4, 32, 16
    g = torch.Generator().manual_seed(9)
    qf = torch.randn((B, N, H * D), generator=g)
    kvf = torch.randn((B, N, 2 * H * D), generator=g)
    idx = torch.randint(0, N, (B, N, M), generator=g, dtype=torch.int32)
    qh = qf.view(B, N, H, D).permute(0, 2, 1, 3)
    kvh = kvf.view(B, N, H, 2 * D).permute(0, 2, 1, 3)
    k, v = kvh[..., :D], kvh[..., D:]
    out_buf = torch.empty((B, N, H, D), device=dev)
    qd, kvd = qf.to(dev), kvf.to(dev)
    qhd = qd.view(B, N, H, D).permute(0, 2, 1, 3)
    kvhd = kvd.view(B, N, H, 2 * D).permute(0, 2, 1, 3)
    nbhd_attn_fwd(qhd, kvhd[..., :D], kvhd[..., D:], idx.to(dev), 0.25, out=out_buf.permute(0, 2, 1, 3),
                  return_lse=False)
    ro, _ = oracle_mod.nbhd_attn(qh.contiguous().numpy(), k.contiguous().numpy(), v.contiguous().numpy(),
                                 idx.numpy(), 0.25)
    _assert_fp32(out_buf.permute(0, 2, 1, 3), None, ro, None)


def test_autograd_function_forward(oracle_mod, dev):
    c, g = _rand_case(1, 2, 64, 32, 16, torch.float32, seed=10, dev=dev)
    out = FlashLocalAttentionFunction.apply(g["q"], g["k"], g["v"], g["idx"], g["bias"], None, g["bk"], g["bv"], 0.3)
    ro, _ = _oracle(oracle_mod, c, 0.3)
    _assert_fp32(out, None, ro, None)


# ----------------------------------------------------- ClusterAttention module --
@pytest.mark.parametrize("with_mask", [False, True])
def test_cluster_attention_module(oracle_mod, dev, with_mask):
    """ClusterAttention.forward (attention.py:127-207) against the oracle: the module's own
    q / kv / proj weights, per-head interleaved [k_h | v_h], the table bias built
    from the oracle's pre_table and pe_index, the cluster mask and the blank token.
    Also pins _make_pos_bias to the oracle's dense table bias."""
    from affmae_amd.layers import ClusterAttention
    B, N, C, H, M = 2, 512, 64, 2, 48
    Ch = C // H
    pos = torch.floor(workloads.cfg1_coords(B, N, seed=3) * 32)
    pos_d = pos.to(dev)
    idx = knn(pos_d, pos_d, M)
    idx_np = idx.cpu().numpy()
    pe = oracle_mod.pe_index(pos.numpy(), idx_np)
    torch.manual_seed(5)
    m = ClusterAttention(C, H).to(dev).eval()
    with torch.no_grad():
        m.blank_k.normal_(0, 0.3)
        m.blank_v.normal_(0, 0.3)
    g = torch.Generator().manual_seed(6)
    feat = torch.randn((B, N, C), generator=g)
    cmask = (torch.rand((B, N, M), generator=g) > 0.2) if with_mask else None
    with torch.no_grad():
        out = m(feat.to(dev), idx, None if cmask is None else cmask.to(dev), torch.from_numpy(pe).to(dev), False)
        w, bb = m.pos_embed.weight.double().cpu().numpy(), m.pos_embed.bias.double().cpu().numpy()
        table = (oracle_mod.pre_table().astype(np.float64) @ w.T + bb).astype(np.float32)
        dense = oracle_mod.table_bias(pe, table).astype(np.float32)
        pb = m._make_pos_bias(torch.from_numpy(pe).to(dev), torch.float32)
        np.testing.assert_allclose(_np(pb), dense, rtol=1e-6, atol=1e-6)
        q = m.q(feat.to(dev)).view(B, N, H, Ch).permute(0, 2, 1, 3)
        kv = m.kv(feat.to(dev)).view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
        ro, _ = oracle_mod.nbhd_attn(_np(q), _np(kv[..., :Ch]), _np(kv[..., Ch:]), idx_np, m.scale, bias=dense,
                                     mask=None if cmask is None else cmask.unsqueeze(1).numpy(),
                                     blank_k=_np(m.blank_k.view(H, Ch)), blank_v=_np(m.blank_v.view(H, Ch)))
        ref = m.proj(torch.from_numpy(ro.astype(np.float32)).to(dev).permute(0, 2, 1, 3).reshape(B, N, C))
    scale = float(ref.abs().max())
    err = float((out - ref).abs().max())
    assert err <= 1e-5 * max(scale, 1.0), f"rel err {err / scale:.3e}"



def test_cluster_attention_module_bf16(oracle_mod, dev):
    """ClusterAttention under bf16 autocast (the encoder's mode; with <= 4 heads and no
    gradient the output projection runs fused in the attention kernel): against the fp64
    oracle attention on the module's own bf16 q / k / v and the same autocast projection."""
    from affmae_amd.layers import ClusterAttention
    B, N, C, H, M = 2, 512, 64, 2, 48
    Ch = C // H
    pos = torch.floor(workloads.cfg1_coords(B, N, seed=3) * 32)
    pos_d = pos.to(dev)
    idx = knn(pos_d, pos_d, M)
    idx_np = idx.cpu().numpy()
    pe = oracle_mod.pe_index(pos.numpy(), idx_np)
    torch.manual_seed(7)
    m = ClusterAttention(C, H).to(dev).eval()
    with torch.no_grad():
        m.blank_k.normal_(0, 0.3)
        m.blank_v.normal_(0, 0.3)
    feat = torch.randn((B, N, C), generator=torch.Generator().manual_seed(9)).to(dev)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = m(feat, idx, None, torch.from_numpy(pe).to(dev), False)
        q = m.q(feat).view(B, N, H, Ch).permute(0, 2, 1, 3)
        kv = m.kv(feat).view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
        assert q.dtype == torch.bfloat16
        table = m.pos_embed(pre_table_fp32.to(dev)).float()
        dense = oracle_mod.table_bias(pe, _np(table)).astype(np.float64)
        ro, _ = oracle_mod.nbhd_attn(_np(q), _np(kv[..., :Ch]), _np(kv[..., Ch:]), idx_np, m.scale, bias=dense,
                                     blank_k=_np(m.blank_k.view(H, Ch).bfloat16()),
                                     blank_v=_np(m.blank_v.view(H, Ch).bfloat16()))
        ref = m.proj(torch.from_numpy(ro.astype(np.float32)).to(dev).permute(0, 2, 1, 3).reshape(B, N, C))
    assert out.dtype == torch.bfloat16
    err = float((out.float() - ref.float()).abs().max())
    assert err <= LOWP_ABS, f"abs err {err:.3e}"


def test_cfg2_raster_order_bf16(oracle_mod, dev):
    """The benchmark shape on raster-ordered tokens: most 32-query tiles have a neighbour
    union wider than the kernel's 224 slots and run as two 16-query halves (or, if a half
    is still too wide, the per-row routine)."""
    w = workloads.cfg2(B=2, order="raster")
    pos = w["pos"].to(dev)
    idx = knn(pos, pos, 48)
    table = (pre_table_fp32.double() @ w["pos_w"].double().T + w["pos_b"].double()).float()
    out, lse = nbhd_attn_fwd(w["q"].to(dev), w["k"].to(dev), w["v"].to(dev), idx, 32 ** -0.5,
                             pos=pos, pe_table=table.to(dev), blank_k=w["blank_k"].to(dev),
                             blank_v=w["blank_v"].to(dev))
    pe = pe_index(pos, idx)
    dense = table[pe.cpu()].permute(0, 3, 1, 2).contiguous().numpy()
    ro, rl = oracle_mod.nbhd_attn(_np(w["q"]), _np(w["k"]), _np(w["v"]), idx.cpu().numpy(), 32 ** -0.5,
                                  bias=dense, blank_k=_np(w["blank_k"]), blank_v=_np(w["blank_v"]))
    _assert_lowp(out, lse, ro, rl)
