"""Neighbourhood attention backward (aff_nbhd_attn_bwd) on the GPU.

Reference: fp64 autograd of the reference's gathered PyTorch attention
(oracle/torch_path.py, local_attn.py:979-1006) on the same inputs (rounded to
the kernel's dtype first), whose gradients tests/test_oracle.py pins against
finite differences.  Every gradient the kernel returns is compared: dq, dk,
dv, the dense dbias (bias mode 1), the table gradient (modes 2 and 4) and
the blank tokens' gradients.

Tolerances: fp32 -> max|g - ref| <= 2e-5 * max|ref| and elementwise
1e-4 * |ref| + 2e-6 * max|ref|; bf16 / fp16 -> max|g - ref| <= 2e-2 *
max|ref| (the gradients are rounded to the 16-bit dtype and Delta uses the
16-bit forward output, as in the reference).  The backward forms every sum in
a fixed order, so two runs agree bit for bit.
"""
import numpy as np
import pytest
import torch

from affmae_amd import workloads
from affmae_amd.kernels import knn
from affmae_amd.kernels.local_attn import FlashLocalAttentionFunction, nbhd_attn_bwd, nbhd_attn_fwd
from affmae_amd.utils.pos_embed import pe_index, pre_table_fp32
from oracle import torch_path

pytestmark = pytest.mark.gpu


def _grid(B, N, seed):
    """Jittered points on a sqrt(2N)-wide grid, rounded to integers when asked (KNN neighbours are local)."""
    g = torch.Generator().manual_seed(seed)
    side = int(np.ceil(np.sqrt(2 * N)))
    out = torch.empty((B, N, 2))
    for b in range(B):
        cells = torch.randperm(side * side, generator=g)[:N].sort().values
        out[b] = torch.stack([cells % side, cells // side], -1).float() + torch.rand((N, 2), generator=g) - 0.5
    return out


def _table(H, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.rand((H, 5), generator=g) * 0.6 - 0.3
    b = torch.rand((H,), generator=g) * 0.2 - 0.1
    return (pre_table_fp32.double() @ w.double().T + b.double()).float()


def _close(got, ref, what, dtype):
    got = got.detach().double().cpu()
    scale = max(float(ref.abs().max()), 1e-30)
    err = float((got - ref).abs().max())
    if dtype == torch.float32:
        assert err <= 2e-5 * scale, f"{what}: rel err {err / scale:.3e}"
        bad = (got - ref).abs() > 1e-4 * ref.abs() + 2e-6 * scale
        assert not bool(bad.any()), f"{what}: elementwise err at {bad.nonzero()[:3].tolist()}"
    else:
        assert err <= 2e-2 * scale, f"{what}: rel err {err / scale:.3e}"


def _reference(q, k, v, idx, scale, dout, *, dense=None, table=None, pe=None, mask=None, bk=None, bv=None):
    """fp64 CPU autograd gradients of the gathered attention."""
    leaf = lambda t: None if t is None else t.detach().double().cpu().requires_grad_(True)
    q64, k64, v64 = leaf(q), leaf(k), leaf(v)
    d64, t64, bk64, bv64 = leaf(dense), leaf(table), leaf(bk), leaf(bv)
    bias = d64
    if t64 is not None:
        bias = torch_path.table_bias(pe.cpu(), t64)
    out = torch_path.gathered_attention(q64, k64, v64, idx.cpu(), scale, bias=bias,
                                        mask=None if mask is None else mask.cpu(), blank_k=bk64, blank_v=bv64)
    out.backward(dout.detach().double().cpu())
    grad = lambda t: None if t is None else t.grad
    return dict(dq=grad(q64), dk=grad(k64), dv=grad(v64), dbias=grad(d64), dtable=grad(t64), dbk=grad(bk64),
                dbv=grad(bv64))


def _case(B, H, N, D, M, dtype, seed, dev):
    pos = _grid(B, N, seed)
    idx = knn(pos.to(dev), pos.to(dev), M)
    g = torch.Generator().manual_seed(seed + 1)
    q, k, v, dout = (torch.randn((B, H, N, D), generator=g).to(dtype).to(dev) for _ in range(4))
    bk, bv = ((torch.randn((H, D), generator=g) * 0.5).to(dtype).to(dev) for _ in range(2))
    return pos, idx, q, k, v, dout, bk, bv


def _run_and_check(dev, dtype, q, k, v, idx, scale, dout, bk, bv, mask=None, **bias):
    out, lse = nbhd_attn_fwd(q, k, v, idx, scale, mask=mask, blank_k=bk, blank_v=bv, **bias)
    want_table = "pe_table" in bias
    dq, dk, dv, dbias, dtable, dbk, dbv = nbhd_attn_bwd(dout, q, k, v, idx, scale, out, lse, mask=mask, blank_k=bk,
                                                        blank_v=bv, want_dbias="bias" in bias,
                                                        want_dtable=want_table, **bias)
    torch.cuda.synchronize()
    pe = None
    if want_table:
        pe = bias["pe_idx"] if "pe_idx" in bias else pe_index(bias["pos"].cpu(), idx.cpu())
    ref = _reference(q, k, v, idx, scale, dout, dense=bias.get("bias"), table=bias.get("pe_table"), pe=pe,
                     mask=mask, bk=bk, bv=bv)
    _close(dq, ref["dq"], "dq", dtype)
    _close(dk, ref["dk"], "dk", dtype)
    _close(dv, ref["dv"], "dv", dtype)
    if "bias" in bias:
        _close(dbias, ref["dbias"], "dbias", torch.float32 if dtype == torch.float32 else dtype)
    if want_table:
        _close(dtable, ref["dtable"], "dtable", torch.float32 if dtype == torch.float32 else dtype)
    if bk is not None:
        _close(dbk, ref["dbk"], "dblank_k", dtype)
        _close(dbv, ref["dbv"], "dblank_v", dtype)
    return dq, dk, dv, dbias, dtable, dbk, dbv


@pytest.mark.parametrize("bias_mode", ["none", "dense", "table", "coords"])
@pytest.mark.parametrize("blank", [True, False])
def test_bwd_fp32_bias_modes(dev, bias_mode, blank):
    B, H, N, D, M = 2, 2, 300, 32, 16
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, torch.float32, seed=5, dev=dev)
    print(f"[bwd] fp32 {bias_mode} blank={blank}", flush=True)
    table = _table(H, seed=6).to(dev)
    gpos = pos.round().to(dev)
    bias = {}
    if bias_mode == "dense":
        bias = dict(bias=(torch.randn((B, H, N, M), generator=torch.Generator().manual_seed(7))).to(dev))
    elif bias_mode == "table":
        bias = dict(pe_idx=pe_index(gpos.cpu(), idx.cpu()).to(dev), pe_table=table)
    elif bias_mode == "coords":
        bias = dict(pos=gpos, pe_table=table)
    _run_and_check(dev, torch.float32, q, k, v, idx, D ** -0.5, dout, bk if blank else None, bv if blank else None,
                   **bias)


@pytest.mark.parametrize("per_head", [False, True])
def test_bwd_fp32_masks(dev, per_head):
    B, H, N, D, M = 2, 4, 256, 32, 24
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, torch.float32, seed=11, dev=dev)
    mask = torch.rand((B, H if per_head else 1, N, M), generator=torch.Generator().manual_seed(12)) > 0.3
    mask[..., 0] = True                      # every row keeps its first neighbour
    print(f"[bwd] fp32 mask per_head={per_head}", flush=True)
    _run_and_check(dev, torch.float32, q, k, v, idx, 0.3, dout, bk, bv, mask=mask.to(dev))


@pytest.mark.parametrize("D", [8, 16, 64, 128])
def test_bwd_fp32_head_dims(dev, D):
    B, H, N, M = 1, 2, 200, 12
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, torch.float32, seed=20 + D, dev=dev)
    print(f"[bwd] fp32 D={D}", flush=True)
    _run_and_check(dev, torch.float32, q, k, v, idx, D ** -0.5, dout, bk, bv)


def test_bwd_fp32_repeated_and_out_of_range(dev):
    """A key listed twice by one query gets both contributions; out-of-range indices get none
    (the reference is built with those entries masked)."""
    B, H, N, D, M = 1, 2, 200, 32, 16
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, torch.float32, seed=30, dev=dev)
    idx = idx.clone()
    idx[:, 3::7, 4] = idx[:, 3::7, 9]
    bad = idx.clone()
    bad[:, 5::11, 2] = N
    bad[:, 6::13, 7] = -1
    out, lse = nbhd_attn_fwd(q, k, v, bad, 0.3, blank_k=bk, blank_v=bv)
    got = nbhd_attn_bwd(dout, q, k, v, bad, 0.3, out, lse, blank_k=bk, blank_v=bv)
    torch.cuda.synchronize()
    valid = (bad >= 0) & (bad < N)
    ref = _reference(q, k, v, torch.where(valid, bad, torch.zeros_like(bad)), 0.3, dout,
                     mask=valid.unsqueeze(1), bk=bk, bv=bv)
    for name, g_ in zip(("dq", "dk", "dv"), got[:3]):
        _close(g_, ref[name], name, torch.float32)
    _close(got[5], ref["dbk"], "dblank_k", torch.float32)
    _close(got[6], ref["dbv"], "dblank_v", torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_bwd_16bit_mfma_forward(dev, dtype):
    """16-bit inputs at the cfg2 density (H=4, D=32, M=48, bias row from coordinates, blank):
    the forward runs on the wave kernel, the backward on its saved out / lse."""
    B, H, N, D, M = 1, 4, 2000, 32, 48
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, dtype, seed=40, dev=dev)
    print(f"[bwd] {dtype} N={N} M={M}", flush=True)
    _run_and_check(dev, dtype, q, k, v, idx, D ** -0.5, dout, bk, bv, pos=pos.to(dev), pe_table=_table(H, 41).to(dev))


def test_bwd_deterministic(dev):
    B, H, N, D, M = 2, 4, 3000, 32, 48
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, torch.bfloat16, seed=50, dev=dev)
    table = _table(H, 51).to(dev)
    out, lse = nbhd_attn_fwd(q, k, v, idx, 0.2, pos=pos.to(dev), pe_table=table, blank_k=bk, blank_v=bv)
    r1 = nbhd_attn_bwd(dout, q, k, v, idx, 0.2, out, lse, pos=pos.to(dev), pe_table=table, blank_k=bk, blank_v=bv,
                       want_dtable=True)
    r2 = nbhd_attn_bwd(dout, q, k, v, idx, 0.2, out, lse, pos=pos.to(dev), pe_table=table, blank_k=bk, blank_v=bv,
                       want_dtable=True)
    torch.cuda.synchronize()
    for a, b in zip(r1, r2):
        if a is not None:
            assert torch.equal(a, b)


def test_flash_local_attention_function_backward(dev):
    """The reference's autograd entry (local_attn.py:843-936): gradients of Q, K, V, the
    dense bias and the blank tokens, with a [B,1,N,M] mask."""
    B, H, N, D, M = 2, 2, 256, 32, 16
    pos, idx, q, k, v, dout, bk, bv = _case(B, H, N, D, M, torch.float32, seed=60, dev=dev)
    bias = torch.randn((B, H, N, M), generator=torch.Generator().manual_seed(61)).to(dev)
    mask = (torch.rand((B, 1, N, M), generator=torch.Generator().manual_seed(62)) > 0.2)
    mask[..., 0] = True
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, bias, bk, bv)]
    out = FlashLocalAttentionFunction.apply(leaves[0], leaves[1], leaves[2], idx.to(torch.int32), leaves[3],
                                            mask.to(dev), leaves[4], leaves[5], 0.25)
    out.backward(dout)
    torch.cuda.synchronize()
    ref = _reference(q, k, v, idx, 0.25, dout, dense=bias, mask=mask, bk=bk, bv=bv)
    for name, t in zip(("dq", "dk", "dv", "dbias", "dbk", "dbv"), leaves):
        _close(t.grad, ref[name], name, torch.float32)


def test_cluster_attention_module_backward(dev):
    """ClusterAttention with gradients: feat and every parameter (q, kv, proj, pos_embed through
    the table, blank tokens) against fp64 autograd of the module's composition."""
    import torch.nn.functional as F
    from affmae_amd.layers import ClusterAttention
    B, N, C, H, M = 2, 384, 64, 2, 24
    Ch = C // H
    pos = torch.floor(workloads.cfg1_coords(B, N, seed=8) * 24)
    idx = knn(pos.to(dev), pos.to(dev), M)
    pe = pe_index(pos, idx.cpu())
    torch.manual_seed(9)
    m = ClusterAttention(C, H).to(dev).train()
    cmask = torch.rand((B, N, M), generator=torch.Generator().manual_seed(10)) > 0.25
    cmask[..., 0] = True
    feat = torch.randn((B, N, C), generator=torch.Generator().manual_seed(11)).to(dev).requires_grad_(True)
    out = m(feat, idx, cmask.to(dev), pe.to(dev), False)
    gout = torch.randn(out.shape, generator=torch.Generator().manual_seed(12)).to(dev)
    out.backward(gout)
    torch.cuda.synchronize()

    p64 = {n: t.detach().double().cpu().requires_grad_(True) for n, t in m.named_parameters()}
    f64 = feat.detach().double().cpu().requires_grad_(True)
    q = F.linear(f64, p64["q.weight"], p64["q.bias"]).view(B, N, H, Ch).permute(0, 2, 1, 3)
    kv = F.linear(f64, p64["kv.weight"], p64["kv.bias"]).view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
    table = F.linear(pre_table_fp32.double(), p64["pos_embed.weight"], p64["pos_embed.bias"])
    o = torch_path.gathered_attention(q, kv[..., :Ch], kv[..., Ch:], idx.cpu(), m.scale,
                                      bias=torch_path.table_bias(pe, table), mask=cmask.unsqueeze(1),
                                      blank_k=p64["blank_k"].view(H, Ch), blank_v=p64["blank_v"].view(H, Ch))
    ref_out = F.linear(o.permute(0, 2, 1, 3).reshape(B, N, C), p64["proj.weight"], p64["proj.bias"])
    ref_out.backward(gout.double().cpu())
    _close(feat.grad, f64.grad, "feat", torch.float32)
    for n, t in m.named_parameters():
        _close(t.grad, p64[n].grad, n, torch.float32)
