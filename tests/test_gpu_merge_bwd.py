"""Backward of the weighted gathers (aff_weighted_features_bwd) on the GPU.

Reference: fp64 autograd of the reference's own torch expression of the op
(weighted_features_ref, weighted_features.py:440-457: gather, broadcast
multiply, sum over the neighbours), on the same inputs rounded to the
kernel's dtype.  Out-of-range indices contribute nothing: the reference is
built with their weights zeroed.  Tolerances: fp32 -> 2e-5 of the gradient's
scale (and elementwise 1e-4 plus a floor of 2e-6 of the scale); bf16 / fp16
-> 2e-2 of the scale.  d_feat is a fixed-order sum, so two runs agree bit for
bit.  The ClusterMerging module (aff.py:122-299) is checked end to end: the
gradients of its input features, its learned scores and every parameter.
"""
import pytest
import torch
import torch.nn.functional as F

from affmae_amd.kernels.weighted_features import weighted_features
from affmae_amd.kernels.weighted_gather import weighted_gather

pytestmark = pytest.mark.gpu


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


def _ref_features(w, f, idx):
    """weighted_features_ref (weighted_features.py:440-457)."""
    B, Nout, M, IC = w.shape
    C = f.shape[-1]
    g = f.gather(1, idx.reshape(B, Nout * M)[..., None].expand(-1, -1, C)).reshape(B, Nout, M, C)
    return (w[..., None] * g[:, :, :, None, :]).sum(dim=2)


def _case(B, N, Nout, M, C, IC, dtype, seed, dev, bad=True):
    g = torch.Generator().manual_seed(seed)
    w = torch.softmax(torch.randn((B, Nout, M, IC), generator=g), dim=2).to(dtype)
    f = torch.randn((B, N, C), generator=g).to(dtype)
    idx = torch.randint(0, N, (B, Nout, M), generator=g)
    idx[:, 1::5, 3] = idx[:, 1::5, 0]                       # repeated source rows
    if bad:
        idx[:, 2::7, 1] = N                                 # out of range: contributes nothing
        idx[:, 3::11, 2] = -1
    dout = torch.randn((B, Nout, IC, C), generator=g).to(dtype)
    return w.to(dev), f.to(dev), idx.to(dev), dout.to(dev)


def _reference(w, f, idx, dout, N):
    valid = (idx >= 0) & (idx < N)
    w64 = w.detach().double().cpu().requires_grad_(True)
    f64 = f.detach().double().cpu().requires_grad_(True)
    vi = valid.cpu()
    out = _ref_features(w64 * vi[..., None], f64, torch.where(vi, idx.cpu(), torch.zeros_like(idx.cpu())))
    out.backward(dout.detach().double().cpu())
    return w64.grad, f64.grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("C,IC", [(64, 4), (128, 4), (12, 4), (96, 3), (256, 2)])
def test_weighted_features_backward(dev, dtype, C, IC):
    B, N, Nout, M = 2, 400, 160, 48
    w, f, idx, dout = _case(B, N, Nout, M, C, IC, dtype, seed=C + IC, dev=dev)
    print(f"[wf bwd] {dtype} C={C} IC={IC}", flush=True)
    wl, fl = w.clone().requires_grad_(True), f.clone().requires_grad_(True)
    weighted_features(wl, fl, idx).backward(dout)
    torch.cuda.synchronize()
    rw, rf = _reference(w, f, idx, dout, N)
    _close(wl.grad, rw, "d_weights", dtype)
    _close(fl.grad, rf, "d_feat", dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_weighted_gather_backward(dev, dtype):
    B, N, Nout, M, C = 2, 500, 200, 24, 128
    w4, f, idx, dout4 = _case(B, N, Nout, M, C, 1, dtype, seed=3, dev=dev)
    w, dout = w4[..., 0].contiguous(), dout4[:, :, 0].contiguous()
    wl, fl = w.clone().requires_grad_(True), f.clone().requires_grad_(True)
    weighted_gather(idx, wl, fl).backward(dout)
    torch.cuda.synchronize()
    rw, rf = _reference(w.unsqueeze(-1), f, idx, dout.unsqueeze(2), N)
    _close(wl.grad, rw[..., 0], "d_weights", dtype)
    _close(fl.grad, rf, "d_feat", dtype)


def test_weighted_features_backward_deterministic(dev):
    B, N, Nout, M, C, IC = 4, 3000, 1200, 48, 128, 4
    w, f, idx, dout = _case(B, N, Nout, M, C, IC, torch.bfloat16, seed=9, dev=dev, bad=False)
    grads = []
    for _ in range(2):
        wl, fl = w.clone().requires_grad_(True), f.clone().requires_grad_(True)
        weighted_features(wl, fl, idx).backward(dout)
        grads.append((wl.grad, fl.grad))
    torch.cuda.synchronize()
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


def test_cluster_merging_module_backward(dev, oracle_mod):
    """ClusterMerging (reserve_on=False) with gradients through weighted_features: feat,
    the learned scores and every parameter against fp64 autograd of the module's
    composition, for the tokens the GPU kept (read back from pos_down)."""
    from affmae_amd.kernels.knn import knn
    from affmae_amd.layers import ClusterMerging
    from affmae_amd.utils.pos_embed import pe_index, pre_table_fp32
    B, side, c, M = 2, 24, 32, 24
    n = side * side
    g = torch.Generator().manual_seed(4)
    pos = torch.stack(torch.meshgrid(torch.arange(side), torch.arange(side), indexing="xy"), -1).reshape(1, n, 2)
    pos = pos.float().expand(B, -1, -1).contiguous()
    idx = knn(pos.to(dev), pos.to(dev), M)
    pe = pe_index(pos, idx.cpu())
    cmask = (torch.rand((B, n, M), generator=g) > 0.2).long()
    torch.manual_seed(5)
    m = ClusterMerging(c, 48, ds_rate=0.4, reserve_on=False).to(dev).train()
    feat = torch.randn((B, n, c), generator=g).to(dev).requires_grad_(True)
    prob = torch.rand((B, n, 1), generator=g).to(dev).requires_grad_(True)
    pos_down, feat_down = m(pos.to(dev), feat, idx, cmask.to(dev), prob, 2, pe.to(dev), 0)
    gout = torch.randn(feat_down.shape, generator=g).to(dev)
    feat_down.backward(gout)
    torch.cuda.synchronize()

    key = (pos[..., 0] * 4096 + pos[..., 1]).long()
    kd = (pos_down.cpu()[..., 0] * 4096 + pos_down.cpu()[..., 1]).long()
    order = key.argsort(dim=1)
    sel = order.gather(1, torch.searchsorted(key.gather(1, order), kd))
    p64 = {k: v.detach().double().cpu().requires_grad_(True) for k, v in m.named_parameters()}
    f64 = feat.detach().double().cpu().requires_grad_(True)
    pr64 = prob.detach().double().cpu().requires_grad_(True)
    mi = idx.cpu().gather(1, sel.unsqueeze(-1).expand(-1, -1, M))
    pes = pe.gather(1, sel.unsqueeze(-1).expand(-1, -1, M))
    cms = cmask.gather(1, sel.unsqueeze(-1).expand(-1, -1, M)).double()
    lp = pr64[..., 0].gather(1, mi.reshape(B, -1)).view(mi.shape) * cms
    t = F.linear(pre_table_fp32.double(), p64["weight_net.0.weight"], p64["weight_net.0.bias"])
    t = F.gelu(F.layer_norm(t, (4,), p64["weight_net.1.weight"], p64["weight_net.1.bias"]))
    w = t[pes] * lp.unsqueeze(-1)
    y = _ref_features(w, f64, mi).reshape(B, sel.shape[1], -1)
    y = F.linear(F.layer_norm(y, (4 * c,), p64["norm.weight"], p64["norm.bias"]), p64["linear.weight"],
                 p64["linear.bias"])
    y.backward(gout.double().cpu())
    _close(feat.grad, f64.grad, "feat", torch.float32)
    _close(prob.grad, pr64.grad, "learned_prob", torch.float32)
    for k, v in m.named_parameters():
        if p64[k].grad is not None:
            _close(v.grad, p64[k].grad, k, torch.float32)
