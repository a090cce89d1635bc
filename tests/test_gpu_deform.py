"""Deformable attention kernels on the GPU vs the oracle.

Neighbour indices returned by the kernel must equal the oracle's exactly;
outputs within 1e-5 relative (fp32) or 2e-2 max-abs (bf16 / fp16).
"""
import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels import (
    fused_deformable_attention,
    fused_knn_deformable_cross_attention,
    fused_knn_deformable_self_attention,
    ms_deformable_attention,
    mssample,
    knn,
)
from affmae_amd.kernels.fused_deform_attn import fused_knn_deform_cross_attn_forward_save
from affmae_amd.kernels.msdetrpc import MSDETRPCFunction
from affmae_amd.layers import DeformableCrossAttention, DeformableSelfAttention

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _close(out, ref, dtype):
    out = _np(out).astype(np.float64)
    if dtype == torch.float32:
        scale = max(np.abs(ref).max(), 1e-30)
        assert np.abs(out - ref).max() <= 1e-5 * scale, f"rel err {np.abs(out - ref).max() / scale:.3e}"
        # elementwise: 1e-5 of each element plus a floor of 1e-6 of the output scale (the floor covers
        # outputs that cancel to ~0, where fp32 summation order alone moves the last bits)
        bad = np.abs(out - ref) > 1e-5 * np.abs(ref) + 1e-6 * scale
        assert not bad.any(), f"elementwise rel err at {np.argwhere(bad)[:3].tolist()}"
    else:
        assert np.abs(out - ref).max() <= 2e-2, f"abs err {np.abs(out - ref).max():.3e}"


def _cross_case(B, Nq, Nkv, H, C, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    qp = torch.rand((B, Nq, 2), generator=g)
    kp = torch.rand((B, Nkv, 2), generator=g)
    off = (torch.randn((B, Nq, H, 4, 2), generator=g) * 0.03).to(dtype)
    att = torch.softmax(torch.randn((B, Nq, H, 4), generator=g), -1).to(dtype)
    val = torch.randn((B, Nkv, H, C), generator=g).to(dtype)
    return qp, kp, off, att, val


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fused_knn_cross_shepard(oracle_mod, dev, dtype):
    """The live decoder kernel (fused_deform_attn.py:1188-1335): 4 points, 4-NN, Shepard."""
    B, Nq, Nkv, H, C = 2, 500, 800, 8, 32
    qp, kp, off, att, val = _cross_case(B, Nq, Nkv, H, C, dtype, seed=1)
    power = torch.tensor(1.7, device=dev)
    out, ki, kd = fused_knn_deform_cross_attn_forward_save(qp.to(dev), kp.to(dev), off.to(dev), att.to(dev),
                                                            val.to(dev), power)
    assert out.dtype == dtype and out.shape == (B, Nq, H, C)
    ro, ri = oracle_mod.deform(qp.numpy(), kp.numpy(), [0, Nkv], _np(off).reshape(B, Nq, H, 1, 4, 2),
                               _np(att).reshape(B, Nq, H, 1, 4), _np(val), 1.7, 4, "shepard")
    np.testing.assert_array_equal(ki.cpu().numpy().reshape(ri.shape), ri)
    _close(out, ro, dtype)
    out2 = fused_knn_deformable_cross_attention(qp.to(dev), kp.to(dev), off.to(dev), att.to(dev), val.to(dev), power)
    assert torch.equal(out, out2)


def test_fused_knn_self_shepard(oracle_mod, dev):
    B, N, H, C = 2, 600, 4, 16
    g = torch.Generator().manual_seed(2)
    pos = torch.rand((B, N, 2), generator=g)
    off = torch.randn((B, N, H, 4, 2), generator=g) * 0.02
    att = torch.softmax(torch.randn((B, N, H, 4), generator=g), -1)
    val = torch.randn((B, N, H, C), generator=g)
    out = fused_knn_deformable_self_attention(pos.to(dev), off.to(dev), att.to(dev), val.to(dev),
                                              torch.tensor(1.0, device=dev))
    ro, _ = oracle_mod.deform(pos.numpy(), pos.numpy(), [0, N], off.numpy().reshape(B, N, H, 1, 4, 2),
                              att.numpy().reshape(B, N, H, 1, 4), val.numpy(), 1.0, 4, "shepard")
    _close(out, ro, torch.float32)


def test_fewer_points_than_neighbours(oracle_mod, dev):
    qp, kp, off, att, val = _cross_case(1, 50, 3, 2, 8, torch.float32, seed=3)
    out = fused_knn_deformable_cross_attention(qp.to(dev), kp.to(dev), off.to(dev), att.to(dev), val.to(dev),
                                               torch.tensor(0.5, device=dev))
    ro, _ = oracle_mod.deform(qp.numpy(), kp.numpy(), [0, 3], off.numpy().reshape(1, 50, 2, 1, 4, 2),
                              att.numpy().reshape(1, 50, 2, 1, 4), val.numpy(), 0.5, 4, "shepard")
    _close(out, ro, torch.float32)


@pytest.mark.parametrize("B", [2])
def test_cfg4_multilevel_idw(oracle_mod, dev, B):
    """Config 4: Nq=12544, C=256 (H=8 x 32), L=4 levels, P=4, 3-NN IDW (p=3), bf16."""
    w = workloads.cfg4(B=B)
    print(f"[deform cfg4] B={B}", flush=True)
    out, ki, _ = ms_deformable_attention(w["query_pos"].to(dev), w["kv_pos"].to(dev), w["level_start"],
                                         w["offsets"].to(dev), w["attn"].to(dev), w["values"].to(dev),
                                         power=3.0, k=3, weighting="idw", return_knn=True)
    assert out.dtype == torch.bfloat16 and out.shape == (B, 12544, 8, 32)
    ro, ri = oracle_mod.deform(w["query_pos"].numpy(), w["kv_pos"].numpy(), w["level_start"], _np(w["offsets"]),
                               _np(w["attn"]), _np(w["values"]), 3.0, 3, "idw")
    np.testing.assert_array_equal(ki.cpu().numpy(), ri)
    _close(out, ro, torch.bfloat16)


def test_cfg4_full_batch_oracle_sample(oracle_mod, dev):
    """Full config (B=32) against the oracle on three of its images (first, one inside,
    last) and every 7th query of them: images and queries are computed independently, so
    the oracle runs on those alone."""
    w = workloads.cfg4(B=32)
    out, ki, _ = ms_deformable_attention(w["query_pos"].to(dev), w["kv_pos"].to(dev), w["level_start"],
                                         w["offsets"].to(dev), w["attn"].to(dev), w["values"].to(dev),
                                         power=3.0, k=3, weighting="idw", return_knn=True)
    pick, qs = [0, 13, 31], slice(0, None, 7)
    sub = lambda t: t[pick][:, qs]
    ro, ri = oracle_mod.deform(sub(w["query_pos"]).numpy(), w["kv_pos"][pick].numpy(), w["level_start"],
                               _np(sub(w["offsets"])), _np(sub(w["attn"])), _np(w["values"][pick]), 3.0, 3, "idw")
    np.testing.assert_array_equal(ki[pick][:, qs].cpu().numpy(), ri)
    _close(out[pick][:, qs], ro, torch.bfloat16)


def test_cfg4_full_batch_consistency(dev):
    """Full config (B=32): images are independent, so images 0-1 of the full
    batch must equal the B=2 run bit for bit; every output finite."""
    w = workloads.cfg4(B=32)
    args = lambda t: (t["query_pos"].to(dev), t["kv_pos"].to(dev), t["level_start"], t["offsets"].to(dev),
                      t["attn"].to(dev), t["values"].to(dev))
    out = ms_deformable_attention(*args(w), power=3.0, k=3, weighting="idw")
    small = {n: (v[:2] if torch.is_tensor(v) else v) for n, v in w.items()}
    out2 = ms_deformable_attention(*args(small), power=3.0, k=3, weighting="idw")
    assert torch.equal(out[:2], out2)
    assert torch.isfinite(out.float()).all()


def test_cfg4_single_level_shepard(oracle_mod, dev):
    """The single-level K=4 Shepard drop-in at config-4 shapes (level 0 only)."""
    w = workloads.cfg4(B=2, level_sizes=(6272,))
    off = w["offsets"][:, :, :, 0]                       # [B,Nq,H,4,2]
    att = torch.softmax(w["attn"][:, :, :, 0].float(), -1).bfloat16()
    out = fused_knn_deformable_cross_attention(w["query_pos"].to(dev), w["kv_pos"].to(dev), off.to(dev),
                                               att.to(dev), w["values"].to(dev), torch.tensor(1.0, device=dev))
    ro, _ = oracle_mod.deform(w["query_pos"].numpy(), w["kv_pos"].numpy(), [0, 6272],
                              _np(off).reshape(2, 12544, 8, 1, 4, 2), _np(att).reshape(2, 12544, 8, 1, 4),
                              _np(w["values"]), 1.0, 4, "shepard")
    _close(out, ro, torch.bfloat16)


def _edge_points(name, B, N, g):
    if name == "lattice_ties":        # exact fp32 lattice with duplicates: many equal distances
        return torch.randint(0, 16, (B, N, 2), generator=g).float() / 16
    if name == "clustered":           # most points in a tiny box: very long candidate lists
        kv = torch.rand((B, N, 2), generator=g)
        m = N * 9 // 10
        kv[:, :m] = 0.4 + torch.rand((B, m, 2), generator=g) * 1e-3
        return kv
    if name == "identical":           # zero extent
        return torch.tensor([0.3, 0.7]).expand(B, N, 2).contiguous()
    if name == "elongated":           # 100:1 aspect ratio
        kv = torch.rand((B, N, 2), generator=g)
        kv[..., 1] *= 0.01
        return kv
    return torch.rand((B, N, 2), generator=g)


@pytest.mark.parametrize("name,K,off_sd", [("uniform", 3, 0.02), ("lattice_ties", 3, 0.0), ("lattice_ties", 8, 0.0),
                                           ("clustered", 3, 0.05), ("identical", 4, 0.05), ("elongated", 3, 0.03),
                                           ("uniform", 8, 0.6)])
def test_neighbour_search_edge_cases(oracle_mod, dev, name, K, off_sd):
    """Exact neighbour sets on inputs that stress the fine-cell candidate lists:
    ties and duplicates, dense clusters (lists beyond their cap), zero extent,
    elongated sets, and samples far outside the points (off_sd = 0.6)."""
    print(f"[deform edge] {name} K={K} off_sd={off_sd}", flush=True)
    g = torch.Generator().manual_seed(11)
    B, Nq, H, L, P, C = 2, 300, 2, 2, 2, 8
    sizes = (400, 90)
    kv = torch.cat([_edge_points(name, B, n, g) for n in sizes], dim=1)
    if name == "lattice_ties":
        qp = torch.randint(0, 32, (B, Nq, 2), generator=g).float() / 32
        off = torch.randint(-4, 5, (B, Nq, H, L, P, 2), generator=g).float() / 64
    else:
        qp = torch.rand((B, Nq, 2), generator=g)
        off = torch.randn((B, Nq, H, L, P, 2), generator=g) * off_sd
    att = torch.softmax(torch.randn((B, Nq, H, L * P), generator=g), -1).reshape(B, Nq, H, L, P)
    val = torch.randn((B, sum(sizes), H, C), generator=g)
    ls = [0, sizes[0], sizes[0] + sizes[1]]
    out, ki, kd = ms_deformable_attention(qp.to(dev), kv.to(dev), ls, off.to(dev), att.to(dev), val.to(dev),
                                          power=2.0, k=K, weighting="idw", return_knn=True)
    ro, ri = oracle_mod.deform(qp.numpy(), kv.numpy(), ls, off.numpy(), att.numpy(), val.numpy(), 2.0, K, "idw")
    np.testing.assert_array_equal(ki.cpu().numpy(), ri)
    _close(out, ro, torch.float32)


@pytest.mark.parametrize("L,P,K,dtype", [(8, 1, 5, torch.float32), (3, 3, 2, torch.float16), (1, 8, 8, torch.float32),
                                          (2, 16, 1, torch.bfloat16), (4, 4, 3, torch.float16)])
def test_level_point_neighbour_shapes(oracle_mod, dev, L, P, K, dtype):
    """Shapes off the cfg4 path: up to 8 levels, 1..16 points per level (1..16 lanes per
    row), K below the register slot count (no early stop), fp16 / bf16 / fp32 values."""
    print(f"[deform shapes] L={L} P={P} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(17 + L * 7 + P)
    B, Nq, H, C = 2, 160, 3, 16
    sizes = [max(K, 300 >> l) for l in range(L)]
    kv = torch.cat([torch.rand((B, n, 2), generator=g) for n in sizes], dim=1)
    ls = [0]
    for n in sizes:
        ls.append(ls[-1] + n)
    qp = torch.rand((B, Nq, 2), generator=g)
    off = (torch.randn((B, Nq, H, L, P, 2), generator=g) * 0.04).to(dtype)
    att = torch.softmax(torch.randn((B, Nq, H, L * P), generator=g), -1).reshape(B, Nq, H, L, P).to(dtype)
    val = torch.randn((B, ls[-1], H, C), generator=g).to(dtype)
    out, ki, _ = ms_deformable_attention(qp.to(dev), kv.to(dev), ls, off.to(dev), att.to(dev), val.to(dev),
                                         power=2.0, k=K, weighting="idw", return_knn=True)
    ro, ri = oracle_mod.deform(qp.numpy(), kv.numpy(), ls, _np(off), _np(att), _np(val), 2.0, K, "idw")
    np.testing.assert_array_equal(ki.cpu().numpy(), ri)
    _close(out, ro, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_given_index_kernels(oracle_mod, dev, dtype):
    g = torch.Generator().manual_seed(4)
    B, N, Nkv, K, C = 2, 300, 400, 4, 24
    sl = torch.rand((B, N, 2), generator=g)
    kv = torch.rand((B, Nkv, 2), generator=g)
    idx = knn(sl.to(dev), kv.to(dev), K)
    aw = torch.rand((B, N), generator=g).to(dtype)
    val = torch.randn((B, Nkv, C), generator=g).to(dtype)
    p = torch.tensor(2.5, device=dev)
    out = fused_deformable_attention(sl.to(dev), kv.to(dev), idx, p, aw.to(dev), val.to(dev))
    assert out.dtype == dtype
    rw, ro = oracle_mod.deform_sample(sl.numpy(), kv.numpy(), idx.cpu().numpy(), 2.5, 0, attn=_np(aw),
                                      values=_np(val))
    _close(out, ro, dtype)
    if dtype != torch.float32:
        return
    w = mssample(sl.to(dev), kv.to(dev), idx, p)
    assert w.shape == (B, N, K, 1)
    rw1, _ = oracle_mod.deform_sample(sl.numpy(), kv.numpy(), idx.cpu().numpy(), 2.5, 1)
    _close(w[..., 0], rw1, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_msdetrpc(oracle_mod, dev, dtype):
    g = torch.Generator().manual_seed(5)
    B, N, M, K, Nv, C = 2, 200, 16, 3, 500, 32
    idx = torch.randint(0, Nv, (B, N, M, K), generator=g)
    # softmaxed weights, as its callers pass (attention.py:381-399): outputs are
    # convex combinations of the values
    w = torch.softmax(torch.randn((B, N, M, K), generator=g), -1).to(dtype)
    a = torch.softmax(torch.randn((B, N, M), generator=g), -1).to(dtype)
    v = torch.randn((B, Nv, C), generator=g).to(dtype)
    out = MSDETRPCFunction.apply(idx.to(dev), w.to(dev), a.to(dev), v.to(dev))
    _close(out, oracle_mod.msdetrpc(idx.numpy(), _np(w), _np(a), _np(v)), dtype)


def test_deformable_modules_branches_agree(dev):
    """Fused (in-kernel K-NN) and unfused (knn + given-index / MSDETRPC) module
    branches compute the same function up to the reference's eps placement."""
    torch.manual_seed(0)
    m = DeformableCrossAttention(64, 4, 4).to(dev)
    with torch.no_grad():
        m.sampling_offsets.weight.normal_(0, 0.01)
        m.sampling_offsets.bias.mul_(0.01)
        m.attention_weights.weight.normal_(0, 0.1)
    q = torch.randn(2, 300, 64, device=dev)
    qp = torch.rand(2, 300, 2, device=dev)
    kv = torch.randn(2, 500, 64, device=dev)
    kp = torch.rand(2, 500, 2, device=dev)
    with torch.no_grad():
        a = m(q, qp, kv, kp)
        m.use_fused_knn, m.use_fused = False, True
        b = m(q, qp, kv, kp)
        m.use_fused = False
        c = m(q, qp, kv, kp)
    assert torch.allclose(a, b, atol=1e-5) and torch.allclose(a, c, atol=1e-4)
    s = DeformableSelfAttention(64, 4, 4).to(dev)
    with torch.no_grad():
        y = s(q, qp)
    assert y.shape == q.shape and torch.isfinite(y).all()


@pytest.mark.parametrize("self_attn", [False, True])
def test_deformable_module_against_oracle(oracle_mod, dev, self_attn):
    """DeformableCross/SelfAttention.forward (attention.py:275-404, 472-593) against the
    oracle: the module's own sampling_offsets / attention_weights (softmax over the 4
    points) / value_proj viewed [b, n_kv, h, c_] / output_proj, learnable Shepard power."""
    torch.manual_seed(4)
    d, h, p = 64, 4, 4
    m = (DeformableSelfAttention if self_attn else DeformableCrossAttention)(d, h, p).to(dev).eval()
    with torch.no_grad():
        m.sampling_offsets.weight.normal_(0, 0.02)
        m.attention_weights.weight.normal_(0, 0.2)
        m.shepard_power.fill_(1.3)
    g = torch.Generator().manual_seed(8)
    q = torch.randn((2, 300, d), generator=g).to(dev)
    qp = torch.rand((2, 300, 2), generator=g).to(dev)
    kv = q if self_attn else torch.randn((2, 450, d), generator=g).to(dev)
    kp = qp if self_attn else torch.rand((2, 450, 2), generator=g).to(dev)
    with torch.no_grad():
        out = m(q, qp) if self_attn else m(q, qp, kv, kp)
        b, n_q, n_kv = 2, 300, kv.shape[1]
        off = m.sampling_offsets(q).view(b, n_q, h, 1, p, 2)
        att = torch.softmax(m.attention_weights(q).view(b, n_q, h, p), -1).view(b, n_q, h, 1, p)
        val = m.value_proj(kv).view(b, n_kv, h, d // h)
        ro, _ = oracle_mod.deform(_np(qp), _np(kp), [0, n_kv], _np(off), _np(att), _np(val), 1.3, 4, "shepard")
        ref = m.output_proj(torch.from_numpy(ro.astype(np.float32)).to(dev).reshape(b, n_q, d))
    scale = float(ref.abs().max())
    assert float((out - ref).abs().max()) <= 1e-5 * max(scale, 1.0)


@pytest.mark.parametrize("self_attn", [False, True])
def test_deformable_module_bf16_autocast(oracle_mod, dev, self_attn):
    """The deformable modules under bf16 autocast: against the fp64 oracle on the module's
    own autocast offsets, attention weights and value projection, followed by the same
    autocast output projection."""
    torch.manual_seed(6)
    d, h, p = 64, 4, 4
    m = (DeformableSelfAttention if self_attn else DeformableCrossAttention)(d, h, p).to(dev).eval()
    with torch.no_grad():
        m.sampling_offsets.weight.normal_(0, 0.02)
        m.attention_weights.weight.normal_(0, 0.2)
        m.shepard_power.fill_(1.3)
    g = torch.Generator().manual_seed(12)
    q = torch.randn((2, 300, d), generator=g).to(dev)
    qp = torch.rand((2, 300, 2), generator=g).to(dev)
    kv = q if self_attn else torch.randn((2, 450, d), generator=g).to(dev)
    kp = qp if self_attn else torch.rand((2, 450, 2), generator=g).to(dev)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = m(q, qp) if self_attn else m(q, qp, kv, kp)
        b, n_q, n_kv = 2, 300, kv.shape[1]
        off = m.sampling_offsets(q).view(b, n_q, h, 1, p, 2)
        att = torch.softmax(m.attention_weights(q).float().view(b, n_q, h, p), -1).view(b, n_q, h, 1, p)
        val = m.value_proj(kv).view(b, n_kv, h, d // h)
        assert val.dtype == torch.bfloat16
        ro, _ = oracle_mod.deform(_np(qp), _np(kp), [0, n_kv], _np(off), _np(att), _np(val), 1.3, 4, "shepard")
        ref = m.output_proj(torch.from_numpy(ro.astype(np.float32)).to(dev).reshape(b, n_q, d))
    err = float((out.float() - ref.float()).abs().max())
    assert err <= 2e-2, f"abs err {err:.3e}"
