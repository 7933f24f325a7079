#!/usr/bin/env python3
"""One sparse-attention decoder layer on one MI355X.

A step is one layer over synthetic, HBM-resident inputs (B=1, N=131072
tokens: 8 image blocks of 1024 + 122880 Morton-ordered voxel tokens in runs of
32-512, H=24, D=64, bf16, top-16 with the image blocks and the own block
forced):
  1. key and value block compression in one launch pair
     (lsrm_block_mean_pool2: keys in fp32, shared with the selection and
     rounded to bf16 for the compressed keys; values in bf16),
  2. per-query-block selection (pool Q in fp32, fp64 scores, top-k),
  3. selected-block attention forward (device plan + MFMA kernel).
`value` is the layer's effective TFLOP/s on the attended FLOPs
(4 * D * sum over heads and queries of the attended key count).  The
roofline object describes the attention forward kernel alone, timed with HIP
events on the stream it is launched on.  cpu_baseline times the CPU oracle
(PyTorch fp32) on a bounded sample of the same workload on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "large-sparse-reconstruction-model_amd"))
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

import lsrm_hip as H  # noqa: E402
from lsrm_hip import workloads as W  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def progress(msg: str) -> None:
    """A progress line on stderr (stdout carries only the result line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def event_time_ms(fn, reps: int) -> float:
    """Average ms per call of fn() measured with HIP events on torch's
    current stream (the stream every lsrm_hip call launches on), after one
    untimed call (first-call set-up of an operator stays outside)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def measured_traffic(config: int):
    """HBM bytes per attention-forward launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (already scaled by the plain-copy
    calibration recorded there); only config 3 has one, other configs and a
    missing summary give None."""
    if config != 3:
        return None
    path = ROOT / "profiles" / "attn_fwd_cfg3_hbm_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split()[1])
    return None


def cpu_baseline(w, q, k, v, topk_idx, flops_per_head_q, budget_s: float):
    """Times the CPU oracle head by head until the budget is spent."""
    from oracle.attention import sel_attn_ref  # the checker, timed as the CPU baseline

    # The GPU box grants one GPU's job a share of 16 host cores, whatever the
    # affinity mask lists; the thread count is held to that share and both
    # figures are reported.
    affinity = len(os.sched_getaffinity(0))
    cores = min(affinity, 16)
    torch.set_num_threads(cores)
    cu_sb, cu_blk, cu_q = w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens
    heads, flops, elapsed = 0, 0.0, 0.0
    g = w.hq // w.hkv
    for h in range(w.hkv):
        qh = q[:, h * g:(h + 1) * g].float().cpu()
        kh = k[:, h:h + 1].float().cpu()
        vh = v[:, h:h + 1].float().cpu()
        th = topk_idx[h:h + 1].cpu()
        t0 = time.perf_counter()
        with torch.no_grad():
            sel_attn_ref(qh, kh, vh, th, cu_sb, cu_blk, cu_q, w.scale)
        elapsed += time.perf_counter() - t0
        flops += flops_per_head_q[h]
        heads += 1
        if elapsed >= budget_s:
            break
    tflops = flops / elapsed / 1e12
    total_flops = sum(flops_per_head_q)
    return {
        "value": round(tflops, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{w.name}: attention forward of kv heads 0..{heads - 1} of {w.hkv} "
                   f"(all {w.n} queries, same selection) with the fp32 PyTorch oracle, "
                   f"{elapsed:.1f} s; extrapolated full-layer attention "
                   f"{total_flops / (tflops * 1e12) * 1e3:.0f} ms; {cores} threads = the box's "
                   f"16-core share per GPU (affinity mask lists {affinity} cores)"),
    }


def aware_rows_case(w, q, k, v, label):
    """Forward and backward over the 3D-aware rows of config 3's voxel tokens
    (each token's nearest 16 block centroids, built on the GPU) for the
    head layout of w / q / k / v: the key-centric plan and the grouped-tile
    plan, each built once (backward-capable) and timed apart."""
    dev = q.device
    n_img = w.n_image_tokens
    nb_img = w.n_image_blocks
    nv = w.n - n_img
    coords = torch.zeros(nv, 4, dtype=torch.int32)
    coords[:, 1:] = torch.from_numpy(w.voxel_coords)
    cu_v = (w.cu_block_tokens[nb_img:] - w.cu_block_tokens[nb_img]).to(dev)
    cu_sb_v = torch.tensor([0, cu_v.numel() - 1], dtype=torch.int32, device=dev)
    cu_q_v = torch.tensor([0, nv], dtype=torch.int32, device=dev)
    pts = H.volume_points(coords.to(dev), 64, 1.0)
    rows = H.nearest_blocks(pts, cu_v, cu_sb_v, cu_q_v, 16, w.hkv)
    qv, kv, vv = (t[n_img:].contiguous() for t in (q, k, v))
    lens = (cu_v[1:] - cu_v[:-1]).long()
    # every kv head carries the same rows; each of its hq / hkv query heads
    # attends them
    flops = 4.0 * w.d * w.hq * float(lens[rows[0].long().clamp(min=0)].masked_fill(
        rows[0] < 0, 0).sum())
    do = torch.randn(qv.shape, generator=torch.Generator(device=dev).manual_seed(7),
                     device=dev).to(qv.dtype)
    out = torch.empty_like(qv)
    lse = torch.empty(w.hq, nv, dtype=torch.float32, device=dev)
    times = {}
    for kc in (True, False):
        plan = H.SelAttnPlan(qv.shape, kv.shape, rows, cu_sb_v, cu_v, cu_q_v, backward=True,
                             key_centric=kc)
        ms_f = event_time_ms(lambda: plan.fwd(qv, kv, vv, w.scale, out, lse), 5)
        ms_b = event_time_ms(lambda: plan.bwd(do, qv, kv, vv, out, lse, w.scale), 3)
        del plan
        ms_p = event_time_ms(lambda: H.SelAttnPlan(qv.shape, kv.shape, rows, cu_sb_v, cu_v,
                                                   cu_q_v, backward=True, key_centric=kc), 2)
        times[kc] = (ms_f, ms_b, ms_p)
        torch.cuda.empty_cache()
    ms_f, ms_b, ms_p = times[True]
    tf = flops / (ms_f * 1e-3) / 1e12
    tb = 2.5 * flops / (ms_b * 1e-3) / 1e12
    return {
        f"attn_fwd_3d_aware_rows{label}": {
            "ms": round(ms_f, 4), "tflops": round(tf, 2),
            "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "plan": "key-centric", "plan_ms": round(ms_p, 4),
            "grouped_tiles_ms": round(times[False][0], 4),
            "grouped_tiles_plan_ms": round(times[False][2], 4),
            "workload": f"{nv} voxel tokens, {cu_v.numel() - 1} blocks, per-token nearest 16 "
                        f"block centroids, Hq={w.hq}, Hkv={w.hkv}, D={w.d}"},
        f"attn_bwd_3d_aware_rows{label}": {
            "ms": round(ms_b, 4), "tflops": round(tb, 2),
            "frac_bf16_peak": round(tb / PEAK_BF16_TFLOPS, 4),
            "plan": "key-centric", "grouped_tiles_ms": round(times[False][1], 4)},
    }


def per_token_paths(w, q, k, v, cu_sb, cu_blk, cu_q):
    """Config-3 paths with per-token selection rows (reported beside the
    headline, not part of it): the forward over the 3D-aware rows of the
    voxel tokens (nearest 16 block centroids, built on the GPU), and the
    learned selection (compressed attention + get_block_score, top-16)."""
    import sparse.ops as ops

    dev = q.device
    progress("3D-aware rows, H=24 D=64")
    res = aware_rows_case(w, q, k, v, "")
    progress("3D-aware rows, product heads (Hq=32, Hkv=2, D=32)")
    # LSRM's own decoder heads (main_lrm_vol_sparse.py:561-562): 32 query
    # heads over 2 kv heads, head dim 32, on the same tokens
    wp = W.product_shape()
    qp, kp, vp = W.tensors(wp, dev)
    res.update(aware_rows_case(wp, qp, kp, vp, "_product_heads"))
    del qp, kp, vp
    torch.cuda.empty_cache()

    progress("learned selection")
    ops.set_validation(False)
    ck = H.block_mean_pool(k.view(w.n, -1), cu_blk).view(-1, w.hkv, w.d)
    cv = H.block_mean_pool(v.view(w.n, -1), cu_blk).view(-1, w.hkv, w.d)
    _, lse = ops.compressed_attention(q, ck, cv, cu_q, cu_sb)
    ms_ca = event_time_ms(lambda: ops.compressed_attention(q, ck, cv, cu_q, cu_sb), 5)
    ms_bs = event_time_ms(lambda: ops.get_block_score(q, ck, lse, 16, cu_q, cu_sb, None, None), 5)
    ops.set_validation(True)
    # Selected attention on the learned rows (per-token, no locality on this
    # synthetic data): the key-centric plan; the plan is timed apart (it is
    # built once per selection and shared by forward and backward).
    rows_l = ops.get_block_score(q, ck, lse, 16, cu_q, cu_sb, None, None)
    lens = (cu_blk[1:] - cu_blk[:-1]).long()
    flops_l = 4.0 * w.d * (w.hq // w.hkv) * float(
        torch.where(rows_l >= 0, lens[rows_l.clamp(min=0).long()], 0).sum())
    plan_l = H.SelAttnPlan(q.shape, k.shape, rows_l, cu_sb, cu_blk, cu_q, backward=True,
                           key_centric=True)
    out_l = torch.empty_like(q)
    lse_l = torch.empty(w.hq, w.n, dtype=torch.float32, device=dev)
    ms_l = event_time_ms(lambda: plan_l.fwd(q, k, v, w.scale, out_l, lse_l), 3)
    do_l = torch.randn(q.shape, generator=torch.Generator(device=dev).manual_seed(8),
                       device=dev).to(q.dtype)
    ms_lb = event_time_ms(lambda: plan_l.bwd(do_l, q, k, v, out_l, lse_l, w.scale), 2)
    del plan_l, do_l
    ms_lp = event_time_ms(
        lambda: H.SelAttnPlan(q.shape, k.shape, rows_l, cu_sb, cu_blk, cu_q, backward=True,
                              key_centric=True), 2)
    del out_l, lse_l

    progress("gate merge")
    # gated merge of the three branch outputs at the layer shape (streams
    # gate [N, 3*hidden] and three [N, hidden] inputs, writes [N, hidden])
    hid = w.hq * w.d
    gen = torch.Generator(device=dev).manual_seed(11)
    gate = torch.rand(w.n, 3 * hid, generator=gen, device=dev).to(q.dtype)
    brs = [torch.randn(w.n, hid, generator=gen, device=dev).to(q.dtype) for _ in range(3)]
    ms_gm = event_time_ms(lambda: ops.gate_merge(gate, *brs), 10)
    gm_bytes = 7 * w.n * hid * q.element_size()
    del gate, brs
    return {
        **res,
        "learned_selection": {"compressed_attn_ms": round(ms_ca, 4),
                              "get_block_score_ms": round(ms_bs, 4), "topk": 16},
        "attn_fwd_learned_rows_key_centric": {
            "ms": round(ms_l, 4), "tflops": round(flops_l / (ms_l * 1e-3) / 1e12, 2),
            "plan_ms": round(ms_lp, 4),
            "bwd_ms": round(ms_lb, 4),
            "bwd_tflops": round(2.5 * flops_l / (ms_lb * 1e-3) / 1e12, 2),
            "workload": f"get_block_score rows (top-16 of {w.n_blocks} blocks per token), "
                        f"H={w.hq}"},
        "gate_merge": {"ms": round(ms_gm, 4), "bytes": gm_bytes,
                       "gbs": round(gm_bytes / (ms_gm * 1e-3) / 1e9, 1),
                       "frac_hbm_peak": round(gm_bytes / (ms_gm * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
    }


def stress_config5(dev, reps: int):
    """BASELINE config 5 (N=524288, 4 heads, top-32, heavy-tailed blocks,
    near-tie scores) measured beside the headline: the same layer (keys and
    values pooled in one launch pair, selection from the pooled keys, plan,
    attention forward), then the kernels one by one and the backward."""
    w = W.config(5)
    q, k, v = W.tensors(w, dev)
    cu_blk, cu_sb, cu_q = (t.to(dev) for t in (w.cu_block_tokens, w.cu_seqblocks, w.cu_seqlens))
    n, hkv, d = w.n, w.hkv, w.d
    k2, v2 = k.view(n, hkv * d), v.view(n, hkv * d)

    def layer():
        pk, _ = H.block_mean_pool2(k2, v2, cu_blk, torch.float32, None)
        topk_idx, _ = H.select_blocks(q, k, cu_sb, cu_blk, w.topk, None, True, pooled_k=pk)
        return H.sel_attn_fwd(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, w.scale)

    ms_layer = event_time_ms(layer, 5)
    pk, _ = H.block_mean_pool2(k2, v2, cu_blk, torch.float32, None)
    topk_idx, compact = H.select_blocks(q, k, cu_sb, cu_blk, w.topk, None, True, pooled_k=pk)
    flops = 4.0 * d * (w.hq // hkv) * W.attended_tokens(compact, w.cu_block_tokens,
                                                        w.cu_seqblocks)
    plan = H.SelAttnPlan(q.shape, k.shape, topk_idx, cu_sb, cu_blk, cu_q, backward=True)
    out = torch.empty_like(q)
    lse = torch.empty(w.hq, n, dtype=torch.float32, device=dev)
    ms_f = event_time_ms(lambda: plan.fwd(q, k, v, w.scale, out, lse), reps)
    do = torch.randn_like(q)
    ms_b = event_time_ms(lambda: plan.bwd(do, q, k, v, out, lse, w.scale), max(2, reps // 4))
    ms_sel = event_time_ms(lambda: H.select_blocks(q, k, cu_sb, cu_blk, w.topk, None, True,
                                                   pooled_k=pk), reps)
    ms_pool = event_time_ms(lambda: H.block_mean_pool(k2, cu_blk), reps)
    nb = w.n_blocks
    pool_bytes = n * hkv * d * 2 + nb * hkv * d * 2 + 4 * (nb + 1)
    del plan, do, out, lse
    torch.cuda.empty_cache()
    tf = flops / (ms_f * 1e-3) / 1e12
    tb = 2.5 * flops / (ms_b * 1e-3) / 1e12
    gbs = pool_bytes / (ms_pool * 1e-3) / 1e9
    return {
        "workload": f"cfg5: N={n}, H={w.hq}, D={d}, top-{w.topk}, {nb} lognormal blocks",
        "ms_per_layer": round(ms_layer, 4),
        "attn_fwd": {"ms": round(ms_f, 4), "tflops": round(tf, 2),
                     "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)},
        "attn_bwd": {"ms": round(ms_b, 4), "tflops": round(tb, 2),
                     "frac_bf16_peak": round(tb / PEAK_BF16_TFLOPS, 4)},
        "select": {"ms": round(ms_sel, 4)},
        "pool_k": {"ms": round(ms_pool, 4), "bytes": pool_bytes, "gbs": round(gbs, 1),
                   "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=[2, 3, 5])
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU oracle time for cpu_baseline (0 = skip)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run three 1 GiB device-to-device copies (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        x = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0").fill_(1)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print("copied 3 x 1 GiB")
        return 0

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the layer "
              "shards by kv head with no exchange); run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = W.config(args.config)
    q, k, v = W.tensors(w, dev)
    cu_blk = w.cu_block_tokens.to(dev)
    cu_sb = w.cu_seqblocks.to(dev)
    cu_q = w.cu_seqlens.to(dev)
    n, hq, hkv, d = w.n, w.hq, w.hkv, w.d
    k2 = k.view(n, hkv * d)
    v2 = v.view(n, hkv * d)
    # forced block ids resident on the device (no host copy inside a step)
    forced = torch.tensor(w.forced_blocks, dtype=torch.int32, device=dev)

    # Keys and values are pooled in one launch pair (keys in fp32: the
    # selection takes those means and the compressed keys are their rounding
    # to bf16, what block_mean_pool with a bf16 output returns).  Measured
    # slightly faster than pooling the values on a second stream beside the
    # selection.
    def layer():
        pk, cv = H.block_mean_pool2(k2, v2, cu_blk, torch.float32, None)
        ck = pk.to(k2.dtype)
        topk_idx, compact = H.select_blocks(q, k, cu_sb, cu_blk, w.topk, forced, True,
                                            pooled_k=pk)
        o, lse = H.sel_attn_fwd(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, w.scale)
        return ck, cv, topk_idx, compact, o, lse

    # Work count from the actual selection.
    _, _, topk_idx, compact, _, _ = layer()
    torch.cuda.synchronize()
    g = hq // hkv
    per_head = []
    cu_cpu = w.cu_block_tokens.long()
    lens = cu_cpu[1:] - cu_cpu[:-1]
    comp = compact.cpu().long()
    valid = comp >= 0
    att_per_block = torch.where(valid, lens[comp.clamp(min=0)], torch.zeros_like(comp)).sum(-1)
    for h in range(hkv):
        per_head.append(4.0 * d * g * float((att_per_block[h] * lens).sum()))
    flops = sum(per_head)

    progress(f"{w.name}: layer steps")
    for _ in range(args.warmup):
        layer()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        layer()
    torch.cuda.synchronize()
    ms_layer = (time.perf_counter() - t0) * 1e3 / args.steps

    progress("kernel timings")
    # Per-kernel times (HIP events on the launch stream).
    reps = args.kernel_reps
    plan = H.SelAttnPlan(q.shape, k.shape, topk_idx, cu_sb, cu_blk, cu_q)
    out = torch.empty_like(q)
    lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
    plan.fwd(q, k, v, w.scale, out, lse)
    ms_attn = event_time_ms(lambda: plan.fwd(q, k, v, w.scale, out, lse), reps)
    ms_plan = event_time_ms(
        lambda: H.SelAttnPlan(q.shape, k.shape, topk_idx, cu_sb, cu_blk, cu_q), reps)
    ms_pool = event_time_ms(lambda: H.block_mean_pool(k2, cu_blk), reps)
    ms_pool_kv = event_time_ms(lambda: H.block_mean_pool2(k2, v2, cu_blk, torch.float32, None),
                               reps)
    ms_select = event_time_ms(
        lambda: H.select_blocks(q, k, cu_sb, cu_blk, w.topk, forced, True), reps)
    # Backward (training path) on the same selection: dQ, reverse map, dK/dV.
    bplan = H.SelAttnPlan(q.shape, k.shape, topk_idx, cu_sb, cu_blk, cu_q, backward=True)
    do = torch.randn_like(q)
    bplan.bwd(do, q, k, v, out, lse, w.scale)
    ms_bwd = event_time_ms(lambda: bplan.bwd(do, q, k, v, out, lse, w.scale),
                           max(2, reps // 4))
    del bplan, do
    extra = per_token_paths(w, q, k, v, cu_sb, cu_blk, cu_q) if args.config == 3 else {}
    if args.config == 3:
        progress("cfg5 stress config")
        extra["cfg5_stress"] = stress_config5(dev, reps)
    nb = w.n_blocks
    pool_bytes = n * hkv * d * 2 + nb * hkv * d * 2 + 4 * (nb + 1)
    attn_tflops = flops / (ms_attn * 1e-3) / 1e12
    pool_gbs = pool_bytes / (ms_pool * 1e-3) / 1e9
    # keys (fp32 means) and values (bf16 means) in one launch pair
    pool_kv_bytes = 2 * n * hkv * d * 2 + nb * hkv * d * (4 + 2) + 4 * (nb + 1)
    pool_kv_gbs = pool_kv_bytes / (ms_pool_kv * 1e-3) / 1e9

    result = {
        "metric": "sparse-attn ms/layer + effective TFLOP/s @131K tok, H24 D64; % MFMA/HBM peak",
        "value": round(flops / (ms_layer * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_layer, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Q/K/V ~ 0.5 N(0,1), block metadata per the config)",
        "config": {
            "workload": f"{w.name}: sparse-attention layer (K/V compression + block "
                        f"selection + selected attention fwd)",
            "tokens": n, "heads_q": hq, "heads_kv": hkv, "head_dim": d, "topk": w.topk,
            "blocks": nb, "forced_blocks": len(w.forced_blocks),
            "attended_fwd_flops": flops,
        },
        "ms_per_layer": round(ms_layer, 4),
        "kernels": {
            "attn_fwd": {"ms": round(ms_attn, 4), "tflops": round(attn_tflops, 2),
                         "frac_bf16_peak": round(attn_tflops / PEAK_BF16_TFLOPS, 4)},
            "attn_plan": {"ms": round(ms_plan, 4)},
            "pool_k": {"ms": round(ms_pool, 4), "bytes": pool_bytes,
                       "gbs": round(pool_gbs, 1),
                       "frac_hbm_peak": round(pool_gbs / PEAK_HBM_GBS, 4)},
            "pool_kv": {"ms": round(ms_pool_kv, 4), "bytes": pool_kv_bytes,
                        "gbs": round(pool_kv_gbs, 1),
                        "frac_hbm_peak": round(pool_kv_gbs / PEAK_HBM_GBS, 4)},
            "select": {"ms": round(ms_select, 4)},
            "attn_bwd": {"ms": round(ms_bwd, 4),
                         "tflops": round(2.5 * flops / (ms_bwd * 1e-3) / 1e12, 2),
                         "frac_bf16_peak": round(2.5 * flops / (ms_bwd * 1e-3) / 1e12
                                                 / PEAK_BF16_TFLOPS, 4)},
            **extra,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(attn_tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(args.config),
        },
    }
    if args.cpu_budget > 0:
        progress("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(w, q, k, v, topk_idx, per_head, args.cpu_budget)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
