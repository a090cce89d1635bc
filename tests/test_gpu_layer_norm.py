"""LayerNorm kernels of the encoder's glue (aff_layer_norm_fwd, aff_layer_norm_map_fwd).

Reference: torch's F.layer_norm in fp64 on the CPU, on the same inputs (the
reference's nn.LayerNorm / LayerNorm2dImages, aff.py:514-526), with the
masked patch embedding's composition (aff.py:610-632: mask multiply,
LayerNorm over channels, exact GELU) restated in fp64.  Tolerances: fp32
output -> 2e-5 of max|ref| and elementwise 1e-4 relative plus a 2e-6 floor;
bf16 / fp16 output -> one rounding of the output format (2^-8 / 2^-11 relative
plus a 1e-2 / 2e-3 absolute floor).  The module-level checks compare the
fused inference path with the module's own torch path (the one that records
gradients) on the same weights.
"""
import pytest
import torch
import torch.nn.functional as F

from affmae_amd.kernels.layer_norm import layer_norm_map, layer_norm_rows, norm

pytestmark = pytest.mark.gpu


def _check(got, ref, out_dtype, what):
    got = got.detach().double().cpu()
    scale = max(float(ref.abs().max()), 1e-30)
    diff = (got - ref).abs()
    if out_dtype == torch.float32:
        assert float(diff.max()) <= 2e-5 * scale, f"{what}: rel err {float(diff.max()) / scale:.3e}"
        bad = diff > 1e-4 * ref.abs() + 2e-6 * scale
    else:
        rel, floor = (2.0 ** -8, 1e-2) if out_dtype == torch.bfloat16 else (2.0 ** -11, 2e-3)
        bad = diff > rel * ref.abs() + floor
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} elements off, first {bad.nonzero()[:3].tolist()}"


def _params(C, g):
    w = (1.0 + 0.3 * torch.randn(C, generator=g)).float()
    b = (0.2 * torch.randn(C, generator=g)).float()
    return w, b


@pytest.mark.parametrize("C", [8, 24, 64, 128, 256, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("in_dtype,out_dtype", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                                (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
                                                (torch.bfloat16, torch.float32)])
def test_rows(dev, C, in_dtype, out_dtype):
    g = torch.Generator().manual_seed(C)
    rows = 3000 if C <= 1024 else 300
    x = (torch.randn(rows, C, generator=g) * 3 + 1.5).to(in_dtype)
    w, b = _params(C, g)
    y = layer_norm_rows(x.to(dev), w.to(dev), b.to(dev), 1e-5, out_dtype)
    torch.cuda.synchronize()
    ref = F.layer_norm(x.double(), (C,), w.double(), b.double(), 1e-5)
    _check(y, ref, out_dtype, f"rows C={C} {in_dtype}->{out_dtype}")


def test_rows_strided_and_no_affine(dev):
    g = torch.Generator().manual_seed(7)
    base = torch.randn(2, 500, 96, generator=g)
    x = base[:, :, 16:80]                      # row stride 96, 64 channels
    y = layer_norm_rows(base.to(dev)[:, :, 16:80], None, None, 1e-6)
    torch.cuda.synchronize()
    ref = F.layer_norm(x.double(), (64,), None, None, 1e-6)
    _check(y, ref, torch.float32, "strided rows")
    assert y.shape == (2, 500, 64)


def test_rows_constant_rows_and_empty(dev):
    x = torch.full((64, 32), 3.25)
    x[1::2] = torch.arange(32.0)
    w, b = _params(32, torch.Generator().manual_seed(1))
    y = layer_norm_rows(x.to(dev), w.to(dev), b.to(dev), 1e-5)
    torch.cuda.synchronize()
    ref = F.layer_norm(x.double(), (32,), w.double(), b.double(), 1e-5)
    _check(y, ref, torch.float32, "constant rows")
    assert torch.equal(y[0].cpu(), b)          # a constant row normalises to the bias
    e = layer_norm_rows(torch.empty(0, 32, device=dev), w.to(dev), b.to(dev), 1e-5)
    assert e.shape == (0, 32)


def test_rows_rejects_unsupported(dev):
    with pytest.raises(ValueError):
        layer_norm_rows(torch.randn(4, 12, device=dev), None, None, 1e-5)      # C % 8 != 0
    with pytest.raises(NotImplementedError):
        layer_norm_rows(torch.randn(4, 4104, device=dev), None, None, 1e-5)    # C > 4096


def _map_ref(x, w, b, eps, keep, cell, gelu, token_major):
    B, C, H, W = x.shape
    v = x.double()
    if keep is not None:
        km = keep.double().view(B, 1, H // cell, 1, W // cell, 1)
        v = (v.view(B, C, H // cell, cell, W // cell, cell) * km).view(B, C, H, W)
    y = F.layer_norm(v.permute(0, 2, 3, 1), (C,), w.double() if w is not None else None,
                     b.double() if b is not None else None, eps)
    if gelu:
        y = F.gelu(y)
    return y.reshape(B, H * W, C) if token_major else y.permute(0, 3, 1, 2)


@pytest.mark.parametrize("C,H,W,cell", [(32, 64, 48, 2), (64, 32, 32, 1), (5, 24, 40, 4), (64, 16, 16, 8), (1, 8, 8, 2)])
@pytest.mark.parametrize("gelu,token_major", [(True, False), (False, True), (False, False)])
@pytest.mark.parametrize("in_dtype,out_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                                (torch.bfloat16, torch.float32)])
def test_map(dev, C, H, W, cell, gelu, token_major, in_dtype, out_dtype):
    g = torch.Generator().manual_seed(C * 7 + H)
    B = 3
    x = (torch.randn(B, C, H, W, generator=g) * 2 - 0.5).to(in_dtype)
    w, b = _params(C, g)
    keep = (torch.rand(B, (H // cell) * (W // cell), generator=g) > 0.4).float()
    y = layer_norm_map(x.to(dev), w.to(dev), b.to(dev), 1e-5, keep=keep.to(dev), cell=cell, gelu=gelu,
                       token_major=token_major, out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = _map_ref(x, w, b, 1e-5, keep, cell, gelu, token_major)
    assert tuple(y.shape) == tuple(ref.shape)
    _check(y, ref, out_dtype, f"map C={C} {H}x{W} cell={cell} gelu={gelu} tm={token_major}")


def test_map_without_mask(dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 32, 20, 12, generator=g)
    y = layer_norm_map(x.to(dev), None, None, 1e-5, gelu=True)
    torch.cuda.synchronize()
    _check(y, _map_ref(x, None, None, 1e-5, None, 1, True, False), torch.float32, "map no mask")


def test_map_rejects_bad_cell(dev):
    x = torch.randn(1, 8, 10, 10, device=dev)
    keep = torch.ones(1, 9, device=dev)
    with pytest.raises((ValueError, AssertionError)):
        layer_norm_map(x, None, None, 1e-5, keep=keep, cell=3)


def test_norm_dispatch_matches_module(dev):
    """norm(module, x): HIP kernel under no_grad, the module itself when a graph is recorded."""
    torch.manual_seed(0)
    ln = torch.nn.LayerNorm(128).to(dev)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.2)
        ln.bias.normal_(0.0, 0.2)
    x = torch.randn(4, 300, 128, device=dev)
    with torch.no_grad():
        y = norm(ln, x)
        ref = ln(x)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            ya = norm(ln, x)
            yl = norm(ln, x, to_autocast=True)
            ra = ln(x)
    assert y.dtype == ref.dtype and ya.dtype == ra.dtype == torch.float32 and yl.dtype == torch.bfloat16
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ya, ra, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(yl, ra.to(torch.bfloat16), rtol=2 ** -7, atol=1e-2)
    xr = x.clone().requires_grad_(True)
    yg = norm(ln, xr)
    assert yg.grad_fn is not None                # recorded by torch's own LayerNorm


@pytest.mark.parametrize("autocast", [False, True])
def test_patch_embed_fused_matches_torch_path(dev, autocast):
    """AFFPatchEmbed: the fused mask / LayerNorm / GELU inference path against the
    module's torch path (taken when the forward records gradients)."""
    from affmae_amd.layers import AFFPatchEmbed
    torch.manual_seed(1)
    pe = AFFPatchEmbed(img_size=64, patch_size=8, in_chans=1, embed_dim=64, norm_layer=torch.nn.LayerNorm).to(dev)
    with torch.no_grad():
        for ln in list(pe.lns) + [pe.norm]:
            m = ln.ln if hasattr(ln, "ln") else ln
            m.weight.normal_(1.0, 0.2)
            m.bias.normal_(0.0, 0.2)
    g = torch.Generator().manual_seed(2)
    B, th = 3, 8
    x = torch.randn(B, 1, 64, 64, generator=g).to(dev)
    ids_masked = torch.argsort(torch.rand(B, th * th, generator=g), dim=1)[:, : th * th // 2].contiguous().to(dev)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        with torch.no_grad():
            assert pe._fused(x)
            pos, feat, h, w = pe(x, ids_masked)
        xr = x.clone().requires_grad_(True)
        assert not pe._fused(xr)
        pos_r, feat_r, h_r, w_r = pe(xr, ids_masked)
    torch.cuda.synchronize()
    assert (h, w) == (h_r, w_r) == (th, th)
    assert feat.dtype == feat_r.dtype and feat.shape == feat_r.shape
    assert torch.equal(pos, pos_r.detach())
    tol = dict(rtol=2e-2, atol=2e-2) if autocast else dict(rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(feat, feat_r.detach(), **tol)
