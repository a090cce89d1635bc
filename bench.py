#!/usr/bin/env python
"""Benchmark of the AFFMAE point-token hot path on one MI355X.

Workload: B=32 images of N=6272 visible tokens
(112x112 jittered grid, 50% kept), exact KNN with k=48 over the token
coordinates, then neighbourhood attention over those neighbours with H=4,
D=32, bf16 q/k/v ~ N(0,1), per-head blank tokens and the relative-position
bias (Linear(5,4) applied to the reference's offset table, the row chosen
in-kernel from the two coordinates).  One step = aff_knn + aff_nbhd_attn_fwd
over the whole batch with every input already resident in HBM.

Prints one JSON line.  ``value`` is tokens/s through the whole step, from
the wall clock around K steps (after W warm-up steps, synchronised on both
sides); ``roofline`` is for the attention kernel (the dominant one), with its
average launch duration measured by HIP events on the launch stream in a
second run of the same K steps (events recorded between the kernels would
add their host cost to the headline steps); ``cpu_baseline`` times the reference's own PyTorch path in
torch-CPU fp32 (oracle/torch_path.py) on the same images on this host.  The
HBM traffic and SQ-counter figures come from the committed rocprofv3
summaries under profiles/ and are null when the kernel source has changed
since they were measured.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
B, N, H, D, K_NN = 32, 6272, 4, 32, 48


def _metric_name() -> str:
    try:
        return json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    except Exception:
        return "neighbourhood-attn tokens/s + KNN queries/s @6272 tok, B=32; % HBM/MFMA roofline"


def attn_bytes(table_rows: int) -> int:
    """Algorithmic HBM bytes of one attention launch (every tensor once)."""
    qkvo = 4 * B * H * N * D * 2          # q, k, v read + out written, bf16
    idx = B * N * K_NN * 4                # member_idx int32
    pos = B * N * 2 * 4                   # coordinates fp32
    table = table_rows * H * 4            # bias table fp32
    blank = 2 * H * D * 2
    return qkvo + idx + pos + table + blank


def knn_bytes() -> int:
    return B * N * 2 * 4 + B * N * K_NN * 4


def cfg3_bytes(B3, N3, M3, C3, k) -> int:
    """Softmax merge: features, coordinates and indices in; features and coordinates out."""
    return B3 * N3 * C3 * 2 + B3 * M3 * k * 4 + B3 * N3 * 2 * 4 + B3 * M3 * 2 * 4 + B3 * M3 * C3 * 2 + B3 * M3 * 2 * 4


def cfg4_bytes(w) -> int:
    """Multi-level deformable attention: offsets, attention, query and level coordinates,
    values in; output out (every tensor once)."""
    el = lambda t: t.numel() * t.element_size()
    B4, Nq, H4, L4, P4, _ = w["offsets"].shape
    C4 = w["values"].shape[-1]
    return (el(w["offsets"]) + el(w["attn"]) + el(w["query_pos"]) + el(w["kv_pos"]) + el(w["values"])
            + B4 * Nq * H4 * C4 * w["values"].element_size())


def profile_figure(fname: str, tag: str, kernel: str, cast=float):
    """A figure from a committed rocprofv3 summary under profiles/ (lines
    "<tag>: <kernel> <value> <source>@<sha256 prefix>"), or None when there is no such line
    or the kernel source has changed since it was measured (the figure is stale)."""
    import hashlib
    f = ROOT / "profiles" / fname
    try:
        for line in f.read_text().splitlines():
            parts = line.split()
            if len(parts) == 4 and parts[0] == tag + ":" and parts[1] == kernel:
                src, _, sha = parts[3].partition("@")
                cur = hashlib.sha256((ROOT / src).read_bytes()).hexdigest()
                return cast(parts[2]) if sha and cur.startswith(sha) else None
    except OSError:
        pass
    return None


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the FETCH_SIZE / WRITE_SIZE summary, or None."""
    return profile_figure("hbm_traffic_fetch_write.md", "traffic", kernel, int)


def time_events(fn, reps: int):
    """Average duration (ms) of fn() over reps, HIP events on the current stream."""
    import torch
    fn()
    torch.cuda.synchronize()
    s = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    e = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    for i in range(reps):
        s[i].record()
        fn()
        e[i].record()
    torch.cuda.synchronize()
    return sum(s[i].elapsed_time(e[i]) for i in range(reps)) / reps


def other_configs(dev, reps: int):
    """Configs 3 and 4 at full size: kernel times and HBM fractions."""
    import torch
    from affmae_amd import workloads
    from affmae_amd.kernels.knn import knn_launch
    from affmae_amd.kernels.weighted_gather import softmax_merge_launch
    from affmae_amd.kernels.fused_deform_attn import ms_deformable_attention

    res = {}
    w3 = workloads.cfg3(B=32)
    sp, mp, f = w3["src_pos"].to(dev), w3["merged_pos"].to(dev), w3["feat"].to(dev)
    idx = knn_launch(mp, sp, 48, out_dtype=torch.int32)
    fo = torch.empty((32, 2509, 128), dtype=torch.bfloat16, device=dev)
    po = torch.empty((32, 2509, 2), dtype=torch.float32, device=dev)
    t_merge = time_events(lambda: softmax_merge_launch(mp, sp, f, idx, 0.1, out=fo, out_pos=po), reps)
    t_knn3 = time_events(lambda: knn_launch(mp, sp, 48, out_dtype=torch.int32), reps)
    b3 = cfg3_bytes(32, 6272, 2509, 128, 48)
    res["cfg3_softmax_merge"] = {"ms": t_merge, "algorithmic_bytes": b3,
                                 "hbm_frac": b3 / (t_merge * 1e-3) / HBM_PEAK,
                                 "merged_points_per_s": 32 * 2509 / (t_merge * 1e-3),
                                 "knn_k48_ms": t_knn3}
    del sp, mp, f, idx, fo, po
    w4 = workloads.cfg4(B=32)
    g4 = {n: (v.to(dev) if torch.is_tensor(v) else v) for n, v in w4.items()}
    t_def = time_events(lambda: ms_deformable_attention(g4["query_pos"], g4["kv_pos"], g4["level_start"],
                                                        g4["offsets"], g4["attn"], g4["values"], power=3.0, k=3,
                                                        weighting="idw"), reps)
    b4 = cfg4_bytes(w4)
    res["cfg4_ms_deform_idw"] = {"ms": t_def, "algorithmic_bytes": b4,
                                 "hbm_frac": b4 / (t_def * 1e-3) / HBM_PEAK,
                                 "queries_per_s": 32 * 12544 / (t_def * 1e-3)}
    del g4, w4
    res["cfg5_encoder"] = cfg5_encoder(dev, reps)
    return res


def cfg5_encoder(dev, reps: int):
    """Config 5: the AFF-small encoder forward (B=8, 1024^2, patch 4, 32768 visible tokens,
    bf16 autocast, random init).  Returns images/s of the whole forward and, per stage,
    the time and HBM fraction of each hot-path kernel call: every call of one forward is
    recorded (arguments kept), then replayed alone under HIP events."""
    import torch
    from affmae_amd import workloads
    from affmae_amd.layers import aff as aff_mod
    from affmae_amd.layers import attention as attn_mod
    from affmae_amd.kernels import local_attn

    enc = workloads.cfg5_encoder().to(dev).eval()
    w5 = workloads.cfg5(B=8, img=1024, seed=0)
    imgs, keep, masked = w5["images"].to(dev), w5["ids_keep"].to(dev), w5["ids_masked"].to(dev)

    def fwd():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return workloads.mae_encode(enc, imgs, keep, masked, 4)

    fwd()
    t_fwd = time_events(fwd, max(3, reps // 2))

    # one forward with the hot-path entry points wrapped to record their arguments
    calls = []
    stage = {"i": -1}
    orig = (aff_mod.knn, aff_mod.weighted_features, local_attn.nbhd_attn_fwd, attn_mod.nbhd_attn_proj_fwd)

    def rec_knn(q, r, k, *a, **kw):
        stage["i"] += 1
        calls.append(("knn", stage["i"], (q, r, k)))
        return orig[0](q, r, k, *a, **kw)

    def rec_wf(wts, feat, idx):
        calls.append(("merge", stage["i"], (wts, feat, idx)))
        return orig[1](wts, feat, idx)

    def rec_attn(*a, **kw):
        calls.append(("attn", stage["i"], (a, kw)))
        return orig[2](*a, **kw)

    def rec_proj(*a, **kw):
        y = orig[3](*a, **kw)
        if y is not None:                         # the attention ran with its projection fused
            calls.append(("attn_proj", stage["i"], (a, kw)))
        return y

    aff_mod.knn, aff_mod.weighted_features, local_attn.nbhd_attn_fwd = rec_knn, rec_wf, rec_attn
    attn_mod.nbhd_attn_proj_fwd = rec_proj
    try:
        fwd()
    finally:
        aff_mod.knn, aff_mod.weighted_features, local_attn.nbhd_attn_fwd = orig[:3]
        attn_mod.nbhd_attn_proj_fwd = orig[3]
    torch.cuda.synchronize()

    el = lambda t: t.numel() * t.element_size()
    stages = [dict(n=0, attn_ms=0.0, attn_calls=0, attn_bytes=0, knn_ms=0.0, merge_ms=0.0, merge_bytes=0)
              for _ in range(4)]
    for kind, si, args in calls:
        st = stages[si]
        if kind == "knn":
            q, r, k = args
            st["n"] = q.shape[1]
            st["knn_ms"] += time_events(lambda: orig[0](q, r, k), reps)
        elif kind == "merge":
            wts, feat, idx = args
            t = time_events(lambda: orig[1](wts, feat, idx), reps)
            B5, n2, M5, IC = wts.shape
            st["merge_ms"] += t
            # weights, indices and the source features in, [B, n', IC, C] out (every tensor once)
            st["merge_bytes"] += el(wts) + el(idx) + el(feat) + B5 * n2 * IC * feat.shape[-1] * feat.element_size()
        else:
            a, kw = args
            fused = kind == "attn_proj"
            t = time_events(lambda: (orig[3] if fused else orig[2])(*a, **kw), reps)
            q, kk, v, mi = a[0], a[1], a[2], a[3]
            mask, table, pe = kw.get("mask"), kw.get("pe_table"), kw.get("pe_idx")
            # q, k, v in, one [B, N, H*D] output (the projected rows when fused, plus the weight)
            by = 4 * el(q) + el(mi) + (el(pe) if pe is not None else 0) + (el(table) if table is not None else 0)
            if fused:
                by += a[5].numel() * q.element_size()
                st["proj_fused"] = True
            if mask is not None:
                by += mask.numel()                        # read as uint8
            st["attn_ms"] += t
            st["attn_calls"] += 1
            st["attn_bytes"] += by
            st["heads"] = q.shape[1]
    out = {"ms": t_fwd, "images_per_s": 8 / (t_fwd * 1e-3), "tokens_per_s": 8 * 32768 / (t_fwd * 1e-3),
           "hot_path_ms": sum(s_["attn_ms"] + s_["knn_ms"] + s_["merge_ms"] for s_ in stages), "stages": []}
    for i, st in enumerate(stages):
        e = {"tokens": st["n"], "heads": st.get("heads"), "attn_calls": st["attn_calls"],
             "attn_proj_fused": bool(st.get("proj_fused", False)),
             "attn_ms": st["attn_ms"], "knn_ms": st["knn_ms"], "merge_ms": st["merge_ms"]}
        if st["attn_ms"] > 0:
            e["attn_hbm_frac"] = st["attn_bytes"] / (st["attn_ms"] * 1e-3) / HBM_PEAK
        if st["merge_ms"] > 0:
            e["merge_hbm_frac"] = st["merge_bytes"] / (st["merge_ms"] * 1e-3) / HBM_PEAK
        out["stages"].append(e)
    out["hot_path_frac_of_forward"] = out["hot_path_ms"] / t_fwd
    return out


def host_cpu() -> dict:
    """CPU model, physical cores and logical CPUs of this host, and the CPUs this process may use."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    return {"model": model, "physical_cores": len(cores) or None, "logical_cpus": os.cpu_count(),
            "usable_cpus": len(os.sched_getaffinity(0))}


def cpu_baseline(w, table_cpu, budget_s: float):
    """The reference's own PyTorch path on this host's CPU, fp32, per image until the budget is
    spent: knn_pytorch_large (cdist^2 + topk, knn.py:1312-1332), the table bias gather
    (attention.py:117-124) and the gathered softmax attention (local_attn.py:979-1006)."""
    import torch
    from oracle import torch_path
    from affmae_amd.utils.pos_embed import pe_index

    threads = torch.get_num_threads()
    pos = w["pos"]
    q, k, v = (w[n].float() for n in ("q", "k", "v"))
    bk, bv = w["blank_k"].float(), w["blank_v"].float()
    done, t_total = 0, 0.0
    with torch.no_grad():
        while done < B and (t_total < budget_s or done == 0):
            b = done
            t0 = time.perf_counter()
            idx = torch_path.knn_cdist_topk(pos[b:b + 1], pos[b:b + 1], K_NN)
            bias = torch_path.table_bias(pe_index(pos[b:b + 1], idx), table_cpu)
            torch_path.gathered_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], idx, D ** -0.5, bias=bias,
                                          blank_k=bk, blank_v=bv)
            t_total += time.perf_counter() - t0
            done += 1
    host = host_cpu()
    return {
        "value": done * N / t_total,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} of {B} images ({done * N} tokens) of the reference's PyTorch path in torch-CPU fp32: "
                  f"cdist^2+topk KNN k=48, table bias gather, gathered softmax attention with blank token; "
                  f"{t_total:.2f} s on {threads} torch threads",
        "host": host,
    }


COPY_BYTES = 256 << 20     # size of the calibration copy of --only copy


def only_kernel(name: str, steps: int) -> int:
    """Launch one kernel family `steps` times on its full-size workload (inputs
    prepared first, one launch untimed), for counter runs under rocprofv3.
    `copy` is a plain device copy of COPY_BYTES (reads and writes COPY_BYTES):
    the calibration of FETCH_SIZE / WRITE_SIZE."""
    import torch
    import torch.nn.functional as F
    from affmae_amd import workloads
    from affmae_amd.kernels.knn import knn_launch

    dev = torch.device("cuda:0")
    if name == "copy":
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        fn = lambda: dst.copy_(src)
    elif name in ("attn", "knn"):
        from affmae_amd.kernels.local_attn import nbhd_attn_fwd
        from affmae_amd.utils.pos_embed import pre_table_fp32
        g = {n: t.to(dev) for n, t in workloads.cfg2(B=B, N=N, H=H, D=D).items()}
        if name == "knn":
            fn = lambda: knn_launch(g["pos"], g["pos"], K_NN, out_dtype=torch.int32)
        else:
            table = F.linear(pre_table_fp32.to(dev), g["pos_w"], g["pos_b"]).contiguous()
            idx = knn_launch(g["pos"], g["pos"], K_NN, out_dtype=torch.int32)
            out = torch.empty((B, H, N, D), dtype=torch.bfloat16, device=dev)
            fn = lambda: nbhd_attn_fwd(g["q"], g["k"], g["v"], idx, D ** -0.5, pos=g["pos"], pe_table=table,
                                       blank_k=g["blank_k"], blank_v=g["blank_v"], out=out, return_lse=False)
    elif name == "merge":
        from affmae_amd.kernels.weighted_gather import softmax_merge_launch
        w3 = workloads.cfg3(B=32)
        sp, mp, f = w3["src_pos"].to(dev), w3["merged_pos"].to(dev), w3["feat"].to(dev)
        idx = knn_launch(mp, sp, 48, out_dtype=torch.int32)
        fo = torch.empty((32, 2509, 128), dtype=torch.bfloat16, device=dev)
        po = torch.empty((32, 2509, 2), dtype=torch.float32, device=dev)
        fn = lambda: softmax_merge_launch(mp, sp, f, idx, 0.1, out=fo, out_pos=po)
    elif name == "encoder":
        from affmae_amd import workloads
        enc = workloads.cfg5_encoder().to(dev).eval()
        w5 = workloads.cfg5(B=8, img=1024, seed=0)
        imgs, keep, masked = w5["images"].to(dev), w5["ids_keep"].to(dev), w5["ids_masked"].to(dev)

        def fn():
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                return workloads.mae_encode(enc, imgs, keep, masked, 4)
    elif name == "deform":
        from affmae_amd.kernels.fused_deform_attn import ms_deformable_attention
        w4 = workloads.cfg4(B=32)
        g4 = {n: (v.to(dev) if torch.is_tensor(v) else v) for n, v in w4.items()}
        fn = lambda: ms_deformable_attention(g4["query_pos"], g4["kv_pos"], g4["level_start"], g4["offsets"],
                                             g4["attn"], g4["values"], power=3.0, k=3, weighting="idw")
    else:
        raise SystemExit(f"unknown --only kernel {name!r}")
    ms = time_events(fn, steps)
    print(json.dumps({"only": name, "launches": steps + 1, "ms_per_launch": ms}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-oracle work (0 = skip)")
    ap.add_argument("--no-other", action="store_true", help="skip the config-3/4 kernel timings")
    ap.add_argument("--only", choices=("attn", "knn", "merge", "deform", "encoder", "copy"),
                    help="launch only this kernel family --steps times (for rocprofv3 counter runs)")
    args = ap.parse_args()

    if args.only and args.gpus == 1:
        return only_kernel(args.only, args.steps)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested). Every hot-path op is "
              "independent per image, so the batch shards across GPUs with no exchange; multi-GPU runs are "
              "not part of this build.", file=sys.stderr)
        return 2

    import torch
    import torch.nn.functional as F
    from affmae_amd import workloads
    from affmae_amd.kernels.knn import knn_launch
    from affmae_amd.kernels.local_attn import nbhd_attn_fwd
    from affmae_amd.utils.pos_embed import pre_table_fp32

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    w = workloads.cfg2(B=B, N=N, H=H, D=D)
    g = {n: t.to(dev) for n, t in w.items()}
    table = F.linear(pre_table_fp32.to(dev), g["pos_w"], g["pos_b"]).contiguous()      # [65025, H] fp32
    out = torch.empty((B, H, N, D), dtype=torch.bfloat16, device=dev)
    scale = D ** -0.5

    K, W = args.steps, args.warmup
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(K)] for _ in range(3)]

    def step(i=None):
        if i is not None:
            ev[0][i].record()
        idx = knn_launch(g["pos"], g["pos"], K_NN, out_dtype=torch.int32)
        if i is not None:
            ev[1][i].record()
        nbhd_attn_fwd(g["q"], g["k"], g["v"], idx, scale, pos=g["pos"], pe_table=table,
                      blank_k=g["blank_k"], blank_v=g["blank_v"], out=out, return_lse=False)
        if i is not None:
            ev[2][i].record()

    for _ in range(W):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # the per-kernel HIP events go in a second run of the same K steps: recording them
    # inside the headline loop adds about 10 us of host work to each 0.23 ms step
    for i in range(K):
        step(i)
    torch.cuda.synchronize()

    sec = t1 - t0
    ms_step = sec / K * 1e3
    knn_ms = sum(ev[0][i].elapsed_time(ev[1][i]) for i in range(K)) / K
    attn_ms = sum(ev[1][i].elapsed_time(ev[2][i]) for i in range(K)) / K
    a_bytes = attn_bytes(table.shape[0])
    achieved = a_bytes / (attn_ms * 1e-3)

    # the same step on raster-ordered tokens (each 16-query tile's neighbour union is ~2x wider)
    wr = workloads.cfg2(B=B, N=N, H=H, D=D, order="raster")
    pos_r = wr["pos"].to(dev)
    idx_r = knn_launch(pos_r, pos_r, K_NN, out_dtype=torch.int32)
    attn_raster_ms = time_events(lambda: nbhd_attn_fwd(g["q"], g["k"], g["v"], idx_r, scale, pos=pos_r, pe_table=table,
                                                       blank_k=g["blank_k"], blank_v=g["blank_v"], out=out,
                                                       return_lse=False), 10)
    del wr, pos_r, idx_r

    other = None
    if not args.no_other:
        del w
        other = other_configs(dev, reps=10)
        w = workloads.cfg2(B=B, N=N, H=H, D=D)

    cpu = None
    if args.cpu_budget > 0:
        cpu = cpu_baseline(w, table.cpu(), args.cpu_budget)

    line = {
        "metric": _metric_name(),
        "value": B * N * K / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded 112x112 jittered grid (6272 of 12544 cells per image, tokens in the encoder's "
                "space-filling-cluster order), q/k/v ~ N(0,1) bf16, random-init Linear(5,4) bias table, "
                "blank tokens ~ N(0,0.2^2)",
        "config": {
            "workload": "cfg2: exact KNN k=48 + neighbourhood attention (bias table row from coordinates, blank token)",
            "global_batch": B, "seq_len": N, "heads": H, "head_dim": D, "k": K_NN,
        },
        "knn": {"ms": knn_ms, "queries_per_s": B * N / (knn_ms * 1e-3),
                "algorithmic_bytes": knn_bytes(),
                "hbm_frac": knn_bytes() / (knn_ms * 1e-3) / HBM_PEAK,
                "valu_busy": profile_figure("sq_counters_attn_knn_cfg2.md", "valu_busy", "knn")},
        "attention": {"ms": attn_ms, "tokens_per_s": B * N / (attn_ms * 1e-3),
                      "raster_order_ms": attn_raster_ms,
                      "valu_busy": profile_figure("sq_counters_attn_knn_cfg2.md", "valu_busy", "attn"),
                      "mfma_busy": profile_figure("sq_counters_attn_knn_cfg2.md", "mfma_busy", "attn"),
                      "lds_bank_conflict": profile_figure("sq_counters_attn_knn_cfg2.md", "lds_conflict", "attn")},
        "roofline": {
            "kernel": "nbhd_attn_wave_kernel<bf16_t, 4, false, true, false>",
            "bound": "hbm",
            "achieved": achieved / 1e9,
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK,
            "traffic": measured_traffic("attn"),
            "algorithmic_bytes": a_bytes,
        },
        "cpu_baseline": cpu,
        "other_configs": other,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
