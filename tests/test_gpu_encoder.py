"""Config 5: the AFF encoder (ClusterTransformerBlock, BasicLayer, ClusterMerging,
AFFEncoder; reference src/layers/aff.py:42-120, 122-299, 337-508, 642-736) on
the GPU.

The encoder's token selection (topk of a learned score) and clustering (a
float sort) make whole-network outputs discontinuous in their inputs, so the
composition is checked teacher-forced: forward hooks record what each stage,
block and merge received and returned on the GPU, and every one of them is
recomputed on the CPU in fp64 from those same inputs, with the oracle's KNN,
neighbourhood gathers, attention and weighted gather (oracle/) and torch fp64
for the dense layers (LayerNorm, Linear, GELU):

* stage index: member_idx, cluster_mask and pe_idx equal the oracle's KNN of
  the stage's cluster centres and its gathers, exactly;
* blocks: fp32 within 1e-4 of the output scale (and elementwise 1e-4 plus a
  floor of 1e-5 of the scale);
* merges: the kept tokens are the top int(0.4 n) of the GPU's learned scores,
  and the merged features match at the same tolerance;
* bf16 (autocast, as the reference trains): the attention kernel's output on
  the exact bf16 q / kv it received is within 2e-2 max-abs of the fp64
  oracle; every stage runs the wave kernel (stages 3-4, 8 and 16 heads, in
  workgroups of 4 heads; stages 1-2 with ClusterAttention's output
  projection fused, checked as the oracle's output times the bf16 weights).

The full config-5 forward (B=8, 1024^2, 32768 visible tokens, bf16) is
checked the same way at the attention-kernel boundary for image 0 of the
first block of every stage, plus its output shapes and finiteness.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from affmae_amd import workloads
from affmae_amd.kernels.local_attn import record_paths
from affmae_amd.layers.aff import BasicLayer, ClusterMerging, ClusterTransformerBlock
from affmae_amd.layers.attention import ClusterAttention
from affmae_amd.utils.geometry import space_filling_cluster

pytestmark = pytest.mark.gpu

FP32_REL = 1e-4
BF16_ABS = 2e-2
# stages 1-2 (2 and 4 heads) run the attention with the projection fused; stages 3-4 two steps
FUSED_PATHS = ["wave+proj"] * 4 + ["wave"] * 8


def _cpu64(t):
    return t.detach().double().cpu()


class Recorder:
    """Forward hooks on every BasicLayer, block, merge and attention of an encoder."""

    def __init__(self, enc):
        self.layers, self.blocks, self.merges, self.attn = [], [], [], []
        self.handles = []
        for li, layer in enumerate(enc.layers):
            self.handles.append(layer.register_forward_hook(self._layer(li)))
            for blk in layer.blocks:
                self.handles.append(blk.register_forward_hook(self._block(li, blk), with_kwargs=True))
                self._hook_attn(li, blk.attn)
            if isinstance(layer.downsample, ClusterMerging):
                self.handles.append(layer.downsample.register_forward_hook(self._merge(li, layer.downsample),
                                                                           with_kwargs=True))

    def _layer(self, li):
        def hook(mod, args, out):
            self.layers.append(dict(stage=li, pos_in=args[0].detach(), pos=out[0].detach(), feat_out=out[1].detach(),
                                    pos_down=out[2].detach(), feat_down=out[3].detach()))
        return hook

    def _block(self, li, blk):
        def hook(mod, args, kwargs, out):
            self.blocks.append(dict(stage=li, mod=blk, feat=kwargs["feat"].detach(), member_idx=kwargs["member_idx"],
                                    cluster_mask=kwargs["cluster_mask"], pe_idx=kwargs["pe_idx"],
                                    out=out.detach()))
        return hook

    def _merge(self, li, mod):
        def hook(m, args, kwargs, out):
            self.merges.append(dict(stage=li, mod=mod, out=(out[0].detach(), out[1].detach()),
                                    **{k: (v.detach() if torch.is_tensor(v) else v) for k, v in kwargs.items()}))
        return hook

    def _hook_attn(self, li, attn: ClusterAttention):
        rec = {"stage": li, "mod": attn}
        self.attn.append(rec)
        self.handles.append(attn.q.register_forward_hook(lambda m, a, o: rec.__setitem__("q", o.detach())))
        self.handles.append(attn.kv.register_forward_hook(lambda m, a, o: rec.__setitem__("kv", o.detach())))
        self.handles.append(attn.proj.register_forward_pre_hook(lambda m, a: rec.__setitem__("o", a[0].detach())))
        self.handles.append(attn.register_forward_hook(
            lambda m, a, kw, o: rec.update(member_idx=kw["member_idx"], cluster_mask=kw["cluster_mask"],
                                           pe_idx=kw["pe_idx"], y=o.detach()), with_kwargs=True))

    def close(self):
        for h in self.handles:
            h.remove()


def _table64(oracle_mod, attn):
    """pos_embed(pre_table) in fp64: the [T*T, H] bias table."""
    w = attn.pos_embed.weight.detach().double().cpu().numpy()
    b = attn.pos_embed.bias.detach().double().cpu().numpy()
    return oracle_mod.pre_table().astype(np.float64) @ w.T + b


def _attn_oracle(oracle_mod, attn, q, kv, member_idx, cluster_mask, pe_idx, images=None):
    """fp64 oracle attention on the given projections: [b, N, C] (before proj)."""
    H = attn.num_heads
    sel = slice(None) if images is None else images
    q64, kv64 = _cpu64(q[sel]), _cpu64(kv[sel])
    B, N, C = q64.shape
    Ch = C // H
    qh = q64.view(B, N, H, Ch).permute(0, 2, 1, 3).numpy()
    kvh = kv64.view(B, N, H, 2 * Ch).permute(0, 2, 1, 3)
    idx = member_idx[sel].cpu().numpy()
    dense = oracle_mod.table_bias(pe_idx[sel].cpu().numpy(), _table64(oracle_mod, attn))
    mask = None
    if cluster_mask is not None:
        mask = (cluster_mask[sel].cpu().numpy() > 0)[:, None]
    bk = attn.blank_k.detach().double().cpu().view(H, Ch).numpy()
    bv = attn.blank_v.detach().double().cpu().view(H, Ch).numpy()
    if q.dtype != torch.float32:                      # the kernel takes the blank tokens in q's dtype
        bk = attn.blank_k.detach().to(q.dtype).double().cpu().view(H, Ch).numpy()
        bv = attn.blank_v.detach().to(q.dtype).double().cpu().view(H, Ch).numpy()
    out, _ = oracle_mod.nbhd_attn(qh, kvh[..., :Ch].contiguous().numpy(), kvh[..., Ch:].contiguous().numpy(), idx,
                                  attn.scale, bias=dense, mask=mask, blank_k=bk, blank_v=bv)
    return torch.from_numpy(out).permute(0, 2, 1, 3).reshape(B, N, C)


def _lin(x, mod):
    return F.linear(x, _cpu64(mod.weight), _cpu64(mod.bias) if mod.bias is not None else None)


def _ln(x, mod):
    return F.layer_norm(x, mod.normalized_shape, _cpu64(mod.weight), _cpu64(mod.bias), mod.eps)


def _block_ref(oracle_mod, rec):
    """ClusterTransformerBlock.forward in fp64 (aff.py:86-115) from the recorded GPU input."""
    blk = rec["mod"]
    x = _cpu64(rec["feat"])
    h = _ln(x, blk.norm1)
    a = blk.attn
    q, kv = _lin(h, a.q), _lin(h, a.kv)
    o = _attn_oracle(oracle_mod, a, q, kv, rec["member_idx"], rec["cluster_mask"], rec["pe_idx"])
    x = x + _lin(o, a.proj)
    m = _lin(F.gelu(_lin(_ln(x, blk.norm2), blk.mlp.fc1)), blk.mlp.fc2)
    return x + m


def _merge_ref(oracle_mod, rec, sel):
    """ClusterMerging.forward in fp64 (aff.py:181-299, reserve_on=False) for the kept tokens `sel`."""
    mod = rec["mod"]
    feat, member_idx, pe_idx = _cpu64(rec["feat"]), rec["member_idx"].cpu(), rec["pe_idx"].cpu()
    cm = rec["cluster_mask"]
    lp_all = _cpu64(rec["learned_prob"])[..., 0]                       # [b, n]
    b, n, c = feat.shape
    mi = member_idx.gather(1, sel.unsqueeze(-1).expand(-1, -1, member_idx.shape[-1]))
    pe = pe_idx.gather(1, sel.unsqueeze(-1).expand(-1, -1, pe_idx.shape[-1]))
    lp = lp_all.gather(1, mi.reshape(b, -1)).view(mi.shape)
    if cm is not None:
        lp = lp * cm.cpu().double().gather(1, sel.unsqueeze(-1).expand(-1, -1, cm.shape[-1]))
    wn = mod.weight_net
    tab = F.gelu(_ln(_lin(torch.from_numpy(oracle_mod.pre_table()).double(), wn[0]), wn[1]))   # [T*T, 4]
    weights = tab[pe] * lp.unsqueeze(-1)                                                        # [b, n', M, 4]
    wf = oracle_mod.weighted_features(weights.numpy(), feat.numpy(), mi.numpy())                # [b, n', 4, c]
    y = torch.from_numpy(wf).reshape(b, sel.shape[1], -1)
    return _lin(_ln(y, mod.norm), mod.linear)


def _close(out, ref, what):
    out = _cpu64(out)
    scale = max(float(ref.abs().max()), 1e-30)
    err = float((out - ref).abs().max())
    assert err <= FP32_REL * scale, f"{what}: rel err {err / scale:.3e}"
    bad = (out - ref).abs() > FP32_REL * ref.abs() + 1e-5 * scale
    assert not bool(bad.any()), f"{what}: elementwise rel err at {bad.nonzero()[:3].tolist()}"


def _index_check(oracle_mod, layer_rec, blk_rec, cluster_size=8, nbhd=48):
    """member_idx / cluster_mask / pe_idx of a stage against the oracle's KNN and gathers
    on the stage's own clustering."""
    pos = layer_rec["pos_in"]
    b, n, _ = pos.shape
    pos_r, centres, members, cmask, _ = space_filling_cluster(pos, cluster_size, layer_rec["h"], layer_rec["w"])
    assert torch.equal(pos_r, layer_rec["pos"]), "stage tokens are not in the clustering's order"
    k = math.ceil(n / cluster_size)
    nnc = min(round(nbhd / cluster_size), k)
    near, _ = oracle_mod.knn(pos_r.cpu().numpy(), centres.cpu().numpy(), nnc)
    mi, mk, pe = oracle_mod.cluster_members(near, members.cpu().numpy(),
                                            None if cmask is None else cmask.cpu().numpy(), pos_r.cpu().numpy())
    assert np.array_equal(blk_rec["member_idx"].cpu().numpy(), mi)
    assert np.array_equal(blk_rec["pe_idx"].cpu().numpy(), pe)
    if cmask is None:
        assert blk_rec["cluster_mask"] is None
    else:
        assert np.array_equal(blk_rec["cluster_mask"].cpu().numpy() != 0, mk != 0)


def _small_encoder(dev):
    return workloads.cfg5_encoder(img_size=256).to(dev).eval()


def test_encoder_fp32_teacher_forced(oracle_mod, dev):
    """img 256^2, patch 4, 50% mask: 2048 visible tokens -> 819 -> 327 -> 130, every stage local."""
    enc = _small_encoder(dev)
    w = workloads.cfg5(B=2, img=256, seed=11)
    rec = Recorder(enc)
    with torch.no_grad():
        out = workloads.mae_encode(enc, w["images"].to(dev), w["ids_keep"].to(dev), w["ids_masked"].to(dev), 4)
    torch.cuda.synchronize()
    rec.close()
    assert [out[f"res{i}"].shape[1] for i in range(2, 6)] == [2048, 819, 327, 130]
    assert len(rec.blocks) == 12 and len(rec.merges) == 3
    for L in rec.layers:
        L["h"] = L["w"] = 64
    for li, L in enumerate(rec.layers):
        first = next(r for r in rec.blocks if r["stage"] == li)
        print(f"[enc fp32] stage {li} index n={L['pos_in'].shape[1]}", flush=True)
        _index_check(oracle_mod, L, first)
    for i, r in enumerate(rec.blocks):
        print(f"[enc fp32] block {i} stage {r['stage']}", flush=True)
        _close(r["out"], _block_ref(oracle_mod, r), f"block {i}")
    for r in rec.merges:
        pos, feat = r["pos"], r["feat"]
        pos_down, feat_down = r["out"]
        b, n, _ = pos.shape
        keep = int(n * r["mod"].ds_rate)
        # kept tokens, read back from the merged positions (grid positions are unique)
        key = (pos[..., 0] * 4096 + pos[..., 1]).long()
        kd = (pos_down[..., 0] * 4096 + pos_down[..., 1]).long()
        order = key.argsort(dim=1)
        sel = order.gather(1, torch.searchsorted(key.gather(1, order), kd))
        assert torch.equal(key.gather(1, sel), kd) and sel.shape[1] == keep
        prob = r["learned_prob"][..., 0]
        kept = torch.zeros_like(prob, dtype=torch.bool).scatter_(1, sel, True)
        lo = prob.masked_fill(~kept, float("inf")).min(1).values
        hi = prob.masked_fill(kept, float("-inf")).max(1).values
        assert bool((lo >= hi).all()), "kept tokens are not the top scores"
        print(f"[enc fp32] merge stage {r['stage']} n={n} -> {keep}", flush=True)
        _close(feat_down, _merge_ref(oracle_mod, r, sel.cpu()), f"merge stage {r['stage']}")
        assert torch.equal(pos_down, pos.gather(1, sel.unsqueeze(-1).expand(-1, -1, 2)))


def _bf16_attention_checks(oracle_mod, rec, images, expect_paths, paths):
    assert paths == expect_paths, f"attention paths {paths}"
    seen = set()
    for r in rec.attn:
        if r["stage"] in seen:
            continue
        seen.add(r["stage"])
        a = r["mod"]
        print(f"[enc bf16] stage {r['stage']} attention H={a.num_heads} N={r['q'].shape[1]}", flush=True)
        assert r["q"].dtype == torch.bfloat16 and r["kv"].dtype == torch.bfloat16 and r["y"].dtype == torch.bfloat16
        ref = _attn_oracle(oracle_mod, a, r["q"], r["kv"], r["member_idx"], r["cluster_mask"], r["pe_idx"],
                           images=images)
        if "o" in r:                      # two steps: the attention output itself
            err = float((_cpu64(r["o"][images]) - ref).abs().max())
            assert err <= BF16_ABS, f"stage {r['stage']}: attention abs err {err:.3e}"
        else:                             # projection fused in the kernel: y = O W^T + b
            w = a.proj.weight.detach().to(torch.bfloat16).double().cpu()
            yref = ref @ w.T + _cpu64(a.proj.bias.detach().to(torch.bfloat16))
            err = float((_cpu64(r["y"][images]) - yref).abs().max())
            assert err <= BF16_ABS * max(1.0, float(yref.abs().max())), f"stage {r['stage']}: fused proj err {err:.3e}"


def test_encoder_bf16_attention_parity(oracle_mod, dev):
    enc = _small_encoder(dev)
    w = workloads.cfg5(B=2, img=256, seed=12)
    rec = Recorder(enc)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16), record_paths() as paths:
        out = workloads.mae_encode(enc, w["images"].to(dev), w["ids_keep"].to(dev), w["ids_masked"].to(dev), 4)
    torch.cuda.synchronize()
    rec.close()
    _bf16_attention_checks(oracle_mod, rec, slice(None), FUSED_PATHS, list(paths))
    for i in range(2, 6):
        assert torch.isfinite(out[f"res{i}"]).all()


def test_encoder_bf16_stored_weights_match_autocast(dev):
    """cast_matmul_weights: the encoder with its Linear / convolution weights stored in bf16
    computes the autocast forward of the fp32-weight encoder (the same products on the same
    bf16 values; the attention bias table stays fp32)."""
    from affmae_amd.utils.precision import cast_matmul_weights
    w = workloads.cfg5(B=2, img=256, seed=13)
    args = (w["images"].to(dev), w["ids_keep"].to(dev), w["ids_masked"].to(dev), 4)
    ref_enc, enc16 = _small_encoder(dev), cast_matmul_weights(_small_encoder(dev))
    assert enc16.layers[0].blocks[0].attn.pos_embed.weight.dtype == torch.float32
    assert enc16.layers[0].blocks[0].attn.q.weight.dtype == torch.bfloat16
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        ref = workloads.mae_encode(ref_enc, *args)
        out = workloads.mae_encode(enc16, *args)
    for i in range(2, 6):
        a, b = out[f"res{i}"].float(), ref[f"res{i}"].float()
        assert torch.equal(out[f"res{i}_pos"], ref[f"res{i}_pos"])
        err = float((a - b).abs().max())
        assert err <= 1e-3 * max(1.0, float(b.abs().max())), f"res{i}: {err:.3e}"


def test_encoder_cfg5_full(oracle_mod, dev):
    """The full config: B=8, 1024^2, 65536 patches, 32768 visible tokens, bf16 autocast."""
    enc = workloads.cfg5_encoder().to(dev).eval()
    w = workloads.cfg5(B=8, img=1024, seed=0)
    rec = Recorder(enc)
    print("[enc cfg5] forward B=8 1024^2", flush=True)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16), record_paths() as paths:
        out = workloads.mae_encode(enc, w["images"].to(dev), w["ids_keep"].to(dev), w["ids_masked"].to(dev), 4)
    torch.cuda.synchronize()
    rec.close()
    dims = [64, 128, 256, 512]
    ns = [32768, 13107, 5242, 2096]
    for i in range(4):
        o = out[f"res{i + 2}"]
        assert tuple(o.shape) == (8, ns[i], dims[i]) and bool(torch.isfinite(o).all())
        p = out[f"res{i + 2}_pos"]
        assert tuple(p.shape) == (8, ns[i], 2)
        assert out[f"res{i + 2}_spatial_shape"] == (256, 256)
    for r in rec.attn:
        mi = r["member_idx"]
        assert int(mi.min()) >= 0 and int(mi.max()) < r["q"].shape[1]
    _bf16_attention_checks(oracle_mod, rec, slice(0, 1), FUSED_PATHS, list(paths))
