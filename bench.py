#!/usr/bin/env python3
"""Benchmark of the MXFP4 MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu]

A step is one MoE-layer forward (router -> bucketing -> gate_up+SwiGLU -> down ->
combine) over one batch of synthetic inputs already resident in HBM. The headline
workload is benchmark config 2 (GPT-OSS-20B-shape layer, decode batch 64, Zipf(1.1)
router skew). To keep the 256 MB Infinity Cache from serving weights, steps rotate
over enough device copies of the weights to exceed 1 GB. Prints ONE JSON line with
the throughput, the dominant kernel's roofline (timed live with HIP events on the
launch stream) and the CPU baseline (the oracle, timed on a bounded sample on this
host's cores). Without --config, the same line carries `by_config`: the same
measurements for configs 0 (decode B=1), 1 (standalone dequant), 3 (prefill 4096,
MFMA roofline) and 4 (GPT-OSS-120B shape, decode B=256), and `decode_batch_sweep`: the
config-2 layer at decode batches 1, 2, 4, ... 64 (tokens/s and HBM fraction each).
--config N runs config N alone (the profiling runs use that).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/sec + % HBM peak (decode) / % MFMA peak (prefill), 1 GPU"
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
MFMA_SUMMARY = os.path.join(ROOT, "profiles", "prefill_gemm_mfma_pmc.md")


def measured_traffic(cfg_index: int, kernel: str = "gate_up"):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel calibration)."""
    import re
    try:
        text = open(TRAFFIC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(r"^traffic\[config%d\.%s\]\s*=\s*(\d+)" % (cfg_index, kernel), text, re.M)
    return int(m.group(1)) if m else None


def measured_pmc(key: str, cfg_index: int, kernel: str = "gate_up"):
    """A counter-derived figure (`key[configN.kernel] = value`) from the committed
    rocprofv3 --pmc summary of the prefill GEMM: mfma_busy (matrix-core busy cycles over
    SIMD cycles), mfma_useful (algorithmic over executed MFMA FLOPs), lds_conflict (LDS
    bank-conflict cycles per CU over kernel cycles)."""
    import re
    try:
        text = open(MFMA_SUMMARY).read()
    except OSError:
        return None
    m = re.search(r"^%s\[config%d\.%s\]\s*=\s*([0-9.]+)" % (key, cfg_index, kernel), text, re.M)
    return float(m.group(1)) if m else None


HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=None, choices=[0, 1, 2, 3, 4],
                    help="run this config alone (default: config 2 plus by_config for 0, 1, 3, 4)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--batch", type=int, default=None,
                    help="with --config 0, 2, 3 or 4: the same layer at this many tokens (seeded inputs)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU-baseline budget of the headline config (by_config entries get half)")
    ap.add_argument("--hbm-probe", action="store_true",
                    help="time device copies of 12 MB .. 1 GB, cold (rotating over 4 GiB) and hot (the same bytes)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 512 MiB device-to-device copy three times (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings)")
    ap.add_argument("--graph", action="store_true",
                    help="time HIP-graph replays of the layer instead of eager C-ABI calls")
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on exactly one GPU (the MoE path has no multi-GPU code); "
              f"got --gpus {args.gpus}, WORLD_SIZE {world}", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.hbm_probe:
        hbm_probe()
        return
    if args.calibrate_copy:
        n = 512 * 1024 * 1024
        a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "launches": 3}))
        return

    if args.config is not None:
        res = bench_dequant(args, args.cpu_seconds) if args.config == 1 else bench_layer(args.config, args,
                                                                                           args.cpu_seconds)
        print(json.dumps(res), flush=True)
        return
    res = bench_layer(2, args, args.cpu_seconds)
    by = {}
    for c in (0, 1, 3, 4):
        free_device_memory()
        r = bench_dequant(args, args.cpu_seconds / 2) if c == 1 else bench_layer(c, args, args.cpu_seconds / 2)
        by[str(c)] = summarize(r)
        log(f"[bench] config {c}: {by[str(c)]['value']} {by[str(c)]['unit']}, "
            f"roofline {by[str(c)]['roofline']['frac']}")
    res["by_config"] = by
    print(json.dumps(res), flush=True)


def hbm_probe():
    """Device-to-device copies of n bytes (2n bytes moved): cold rotates the source over
    4 GiB, beyond the 256 MB Infinity Cache; hot copies the same bytes again. Median of 7
    copies each, timed alone between HIP events. Small cold copies show the start-up cost
    of a read from HBM that the small decode batches pay at every stage."""
    import torch

    pool = torch.empty(4 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(0)
    rows = []
    for mb in (12, 24, 48, 96, 240, 1000):
        n = (mb * 1000 * 1000) // 4096 * 4096
        for hot in (False, True):
            off, ts = 0, []
            for rep in range(8):
                if not hot:
                    off = (off + n + 37 * 4096) % (pool.numel() - n) // 4096 * 4096
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record()
                dst[:n].copy_(pool[off:off + n])
                e1.record()
                e1.synchronize()
                ts.append(e0.elapsed_time(e1))
            med = float(np.median(ts[1:]))
            rows.append({"mb": mb, "cache": "hot" if hot else "cold", "us": round(med * 1e3, 1),
                         "gbs_read_plus_write": round(2 * n / (med * 1e-3) / 1e9, 1)})
    print(json.dumps({"probe": "device copy", "rows": rows}), flush=True)


def free_device_memory():
    import gc
    import torch
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def timed_runs(stream, steps: int, call, runs: int = 21):
    """`runs` runs of `steps` back-to-back calls, each run between its own pair of events
    on the launch stream; returns each run's ms per step."""
    import torch
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(runs + 1)]
    out = []
    for r in range(runs):
        torch.cuda.synchronize()
        evs[0].record(stream)
        for i in range(steps):
            call(r * steps + i)
        evs[r + 1].record(stream)
        torch.cuda.synchronize()
        out.append(evs[0].elapsed_time(evs[r + 1]) / steps)
    return np.array(out)


def median_summary(runs_ms, steps: int) -> dict:
    return {"runs": int(len(runs_ms)), "steps_per_run": int(steps),
            "ms_per_step_median": round(float(np.median(runs_ms)), 5),
            "ms_per_step_min": round(float(np.min(runs_ms)), 5),
            "ms_per_step_max": round(float(np.max(runs_ms)), 5),
            "note": "value = K-step mean of the timed region; value_median = median over these runs of "
                    "(run time / K), the median of >= 20 runs the metric is quoted as; per_step_ms brackets every step "
                    "with its own events, which removes the launch overlap of back-to-back steps"}


def summarize(r: dict) -> dict:
    """The by_config entry of one config's result: throughput, time, roofline, CPU baseline."""
    keep = ("value", "value_median", "median_of_runs", "unit", "ms_per_step", "dtype", "config", "roofline",
            "cpu_baseline")
    out = {k: r[k] for k in keep}
    lay = r.get("layer", {})
    for k in ("per_step_ms", "stage_ms", "batch1_launch_ms", "hbm_gbs", "hbm_frac"):
        if k in lay:
            out[k] = lay[k]
    if "transpose" in r:
        out["transpose"] = r["transpose"]
    return out


def bench_layer(cfg_i: int, args, cpu_seconds: float) -> dict:
    """One MoE-layer config: K timed eager steps plus the per-step spread, the per-stage
    times, the block entry, the dominant kernel's roofline and the CPU baseline."""
    import torch
    from physllm_amd import ops
    from physllm_amd import synthetic as syn

    cfgd = syn.CONFIGS[cfg_i]
    log(f"[bench] generating config {cfg_i}: {cfgd['workload']}")
    layer, x = syn.make_config(cfg_i)
    if args.batch:
        x = syn.make_x(args.batch, layer.hidden, seed=cfgd["seed"])
    B, H, I, E, K = x.shape[0], layer.hidden, layer.intermediate, layer.num_experts, layer.top_k

    dl0 = ops.DeviceMoELayer.from_host(layer)
    xd = torch.from_numpy(x.view(np.int16)).cuda()
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream

    # touched experts (the device router; routing is deterministic)
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((B, K), dtype=torch.float32, device="cuda")
    ops.route_topk(xd, dl0.tensors["router_w"], dl0.tensors["router_b"], idx, wt, K, s)
    torch.cuda.synchronize()
    counts = np.bincount(idx.cpu().numpy().reshape(-1), minlength=E)
    e_touched = int((counts > 0).sum())
    layer_bytes = e_touched * layer.expert_bytes + E * H * 2 + E * 2 + B * H * 2 * 2

    # Steps rotate over device copies of the weights so that the bytes a step touches,
    # times the copies, exceed 1 GB: the 256 MB Infinity Cache cannot serve them.
    copies = [dl0]
    n_copies = 1 if cfg_i == 3 else max(1, math.ceil(1.1e9 / layer_bytes))
    for _ in range(n_copies - 1):
        t = {k: (v.clone() if v is not None else None) for k, v in dl0.tensors.items()}
        copies.append(ops.DeviceMoELayer.from_tensors(H, I, E, K, t, layer.alpha, layer.limit))
    log(f"[bench] {e_touched} experts touched ({layer_bytes / 1e6:.1f} MB/step); "
        f"{n_copies} weight copies x {layer.weight_bytes / 1e6:.1f} MB")

    out = torch.empty((B, H), dtype=torch.int16, device="cuda")
    ws = torch.empty(dl0.workspace_bytes(B), dtype=torch.uint8, device="cuda")

    def step(i):
        copies[i % n_copies].forward(xd, out, ws, stream=s)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ref_out = out.clone()

    # eager: one C-ABI call per step from the host
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    eager_ms = ev0.elapsed_time(ev1) / args.steps

    # graph: each weight copy's layer captured once (the layer has no host sync and
    # records no memset), then replayed; this is how a serving loop runs the layer
    graphs = []
    if args.graph:
        for c in range(n_copies):
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                copies[c].forward(xd, out, ws)
            graphs.append(gph)
        for i in range(max(args.warmup, n_copies)):
            graphs[i % n_copies].replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), "graph replay output differs from the eager output"

    # ---- timed region: K whole-layer steps ------------------------------------------
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        if graphs:
            graphs[i % n_copies].replay()
        else:
            step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    if graphs:
        assert torch.equal(out, ref_out), "timed replays changed the output"

    # ---- median of runs (the metric is quoted as the median of >= 20 runs): 21 more runs of K
    # back-to-back steps, each run between its own pair of events; the run's time / K
    runs_ms = timed_runs(stream, args.steps, lambda i: graphs[i % n_copies].replay() if graphs else step(i))

    # ---- per-step spread: K more steps, each between its own pair of events (after the
    # timed region, so the reported value is not affected); median and 10/90th percentiles.
    # An event between every two steps costs each step part of the launch overlap that
    # back-to-back steps have, so these per-step times sit above the run means.
    pev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    pev[0].record(stream)
    for i in range(args.steps):
        if graphs:
            graphs[i % n_copies].replay()
        else:
            step(i)
        pev[i + 1].record(stream)
    torch.cuda.synchronize()
    per_step = np.array([pev[i].elapsed_time(pev[i + 1]) for i in range(args.steps)])

    # ---- per-stage timing: each stage entry point launched K times back to back
    # (rotating weight copies) between two events on the launch stream; the stages
    # are idempotent given the routing state the route stage left in the workspace.
    from physllm_amd.capi import check, lib
    import ctypes
    L = lib()
    nbytes = ws.numel()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2)]

    def cw(i):
        d = copies[i % n_copies]
        return ctypes.byref(d.cfg), ctypes.byref(d.weights)

    stage_calls = [
        lambda i: L.physllm_moe_stage_route(*cw(i), xd.data_ptr(), B, None, None, ws.data_ptr(), nbytes, s),
        lambda i: L.physllm_moe_stage_gate_up(*cw(i), xd.data_ptr(), B, ws.data_ptr(), nbytes, s),
        lambda i: L.physllm_moe_stage_down(*cw(i), B, ws.data_ptr(), nbytes, s),
        lambda i: L.physllm_moe_stage_combine(cw(i)[0], B, out.data_ptr(), None, ws.data_ptr(), nbytes, s),
    ]
    stage_ms = np.zeros(4)
    for j, call in enumerate(stage_calls):
        check(call(0))
        torch.cuda.synchronize()
        evs[0].record(stream)
        for i in range(args.steps):
            check(call(i))
        evs[1].record(stream)
        torch.cuda.synchronize()
        stage_ms[j] = evs[0].elapsed_time(evs[1]) / args.steps
    assert torch.equal(out, ref_out), "staged entry points disagree with the layer entry point"

    # ---- the batch-1 launches (the layer at one or two tokens): logits, gate_up with the
    # in-kernel selection, down with the combine; each launched K times back to back
    b1_ms = None
    if B <= 2:
        def b1(i, launch):
            d = copies[i % n_copies]
            return L.physllm_moe_stage_batch1(ctypes.byref(d.cfg), ctypes.byref(d.weights), xd.data_ptr(), B,
                                              launch, out.data_ptr(), ws.data_ptr(), nbytes, s)
        if b1(0, 0) == 0:
            check(b1(0, 1))
            check(b1(0, 2))
            torch.cuda.synchronize()
            assert torch.equal(out, ref_out), "batch-1 stage launches disagree with the layer entry point"
            b1_ms = np.zeros(3)
            for j in range(3):
                torch.cuda.synchronize()
                evs[0].record(stream)
                for i in range(args.steps):
                    check(b1(i, j))
                evs[1].record(stream)
                torch.cuda.synchronize()
                b1_ms[j] = evs[0].elapsed_time(evs[1]) / args.steps
            assert torch.equal(out, ref_out), "batch-1 stage launches changed the output"

    # ---- the block around the layer (moe.rs:238-313): RMSNorm alone, then the fused
    # block entry (norm + layer + residual add) K times each, same weight rotation
    nw = torch.from_numpy(syn.bf16_from_f32(np.full(H, 1.0, np.float32)).view(np.int16)).cuda()
    hbuf = torch.empty_like(xd)
    out_blk = torch.empty_like(out)
    ws_blk = torch.empty(dl0.block_workspace_bytes(B), dtype=torch.uint8, device="cuda")
    block_calls = [
        lambda i: (L.launch_rms_norm(xd.data_ptr(), nw.data_ptr(), hbuf.data_ptr(), B, H, 1e-5, s), check()),
        lambda i: copies[i % n_copies].block_forward(xd, nw, 1e-5, out_blk, ws_blk, stream=s),
    ]
    block_ms = np.zeros(2)
    for j, call in enumerate(block_calls):
        call(0)
        torch.cuda.synchronize()
        evs[0].record(stream)
        for i in range(args.steps):
            call(i)
        evs[1].record(stream)
        torch.cuda.synchronize()
        block_ms[j] = evs[0].elapsed_time(evs[1]) / args.steps

    # ---- decode batch sweep (config 2's layer, its weight copies, seeded inputs): the
    # layer at B = 1 ... 64, eager, each batch's touched experts' bytes over its step time
    sweep = None
    if cfg_i == 2 and not args.batch:
        sweep = []
        for Bs in (1, 2, 4, 8, 16, 32, 64):
            xs_d = torch.from_numpy(syn.make_x(Bs, H, seed=cfgd["seed"]).view(np.int16)).cuda()
            idx_s = torch.empty((Bs, K), dtype=torch.int32, device="cuda")
            wt_s = torch.empty((Bs, K), dtype=torch.float32, device="cuda")
            ops.route_topk(xs_d, dl0.tensors["router_w"], dl0.tensors["router_b"], idx_s, wt_s, K, s)
            torch.cuda.synchronize()
            et = int((np.bincount(idx_s.cpu().numpy().reshape(-1), minlength=E) > 0).sum())
            by = et * layer.expert_bytes + E * H * 2 + E * 2 + Bs * H * 2 * 2
            out_s = torch.empty((Bs, H), dtype=torch.int16, device="cuda")
            ws_s = torch.empty(dl0.workspace_bytes(Bs), dtype=torch.uint8, device="cuda")
            # this batch's own rotation: its touched bytes x copies > 1.1 GB
            nc = max(1, math.ceil(1.1e9 / by))
            while len(copies) < nc:
                t = {k: (v.clone() if v is not None else None) for k, v in dl0.tensors.items()}
                copies.append(ops.DeviceMoELayer.from_tensors(H, I, E, K, t, layer.alpha, layer.limit))
            for i in range(args.warmup + nc):
                copies[i % nc].forward(xs_d, out_s, ws_s, stream=s)
            torch.cuda.synchronize()
            evs[0].record(stream)
            for i in range(args.steps):
                copies[i % nc].forward(xs_d, out_s, ws_s, stream=s)
            evs[1].record(stream)
            torch.cuda.synchronize()
            ms_s = evs[0].elapsed_time(evs[1]) / args.steps
            sweep.append({"batch": Bs, "experts_touched": et, "weight_copies_rotated": nc,
                          "us_per_step": round(ms_s * 1e3, 2),
                          "tokens_per_s": round(Bs / (ms_s * 1e-3), 1),
                          "hbm_frac": round(by / (ms_s * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})

    # ---- roofline of the dominant kernel (gate_up) ---------------------------------------
    gu_expert_bytes = (2 * I * H // 2) + (2 * I * H // 32) + 2 * (2 * I)
    gate_up_ms = float(stage_ms[1])
    if cfg_i == 3:
        flops = 2.0 * B * K * (2 * I) * H
        achieved = flops / (gate_up_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / BF16_MFMA_PEAK_TFLOPS, 4),
                "traffic": measured_traffic(cfg_i),
                "mfma_busy_pmc": measured_pmc("mfma_busy", cfg_i), "mfma_useful_pmc": measured_pmc("mfma_useful", cfg_i),
                "lds_conflict_pmc": measured_pmc("lds_conflict", cfg_i),
                "kernel": "gate_up grouped GEMM (k_mx_gemm3<0>)", "work_per_launch": flops}
    else:
        alg = e_touched * gu_expert_bytes + B * H * 2 + B * K * I * 2
        # the kernel the layer call runs: at one or two tokens the batch-1 gate_up
        if b1_ms is not None:
            gate_up_ms = float(b1_ms[1])
        achieved = alg / (gate_up_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(cfg_i),
                "kernel": ("k_b1_gate_up" if b1_ms is not None else "gate_up grouped GEMV (k_mx_gemv_stream<0>)"),
                "work_per_launch": alg}

    # ---- CPU baseline (oracle on this host's cores, bounded sample) ----------------------
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as orc
        nthr = orc.default_threads()
        xs = x if cfg_i != 3 else x[:64]
        n, tcpu = 0, 0.0
        while tcpu < cpu_seconds and n < 50:
            t1 = time.perf_counter()
            orc.moe_layer(layer, xs, nthreads=nthr)
            tcpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": round(xs.shape[0] * n / tcpu, 2), "unit": "tokens/s", "cores": nthr,
               "kind": "port",
               "sample": f"{n} full oracle layer call(s) on {xs.shape[0]} tokens of config {cfg_i} "
                         f"({tcpu:.1f} s, OpenMP over weight rows)"}

    res = {
        "metric": METRIC,
        "value": round(B / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "value_median": round(B / (float(np.median(runs_ms)) * 1e-3), 1),
        "median_of_runs": median_summary(runs_ms, args.steps),
        "dtype": "bf16",
        "data": "synthetic (seeded; MXFP4 e2m1 codes uniform, E8M0 scales 2^-8..2^-4, bf16 N(0,.02) biases/router, x N(0,1))",
        "config": {"workload": cfgd["workload"] + (f" (at batch {B})" if args.batch else ""),
                   "config_index": cfg_i, "batch": B, "hidden": H,
                   "intermediate": I, "experts": E, "top_k": K, "experts_touched": e_touched,
                   "weights": "MXFP4 (e2m1 + E8M0 per 32)", "weight_copies_rotated": n_copies},
        "roofline": roof,
        "layer": {"hbm_bytes_algorithmic": layer_bytes,
                  "hbm_gbs": round(layer_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                  "hbm_frac": round(layer_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "stage_ms": {"route": round(stage_ms[0], 5), "gate_up": round(stage_ms[1], 5),
                               "down": round(stage_ms[2], 5), "combine": round(stage_ms[3], 5)},
                  "batch1_launch_ms": (None if b1_ms is None else
                                       {"logits": round(float(b1_ms[0]), 5), "gate_up": round(float(b1_ms[1]), 5),
                                        "down_combine": round(float(b1_ms[2]), 5),
                                        "note": "the launches the layer call runs at this batch "
                                                "(physllm_moe_stage_batch1); stage_ms times the per-stage kernels"}),
                  "block_ms": {"rms_norm": round(block_ms[0], 5), "block_forward": round(block_ms[1], 5),
                               "note": "physllm_moe_block_forward = rms_norm + layer + residual add "
                                       "fused into the combine (eager, one call per step)"},
                  "per_step_ms": {"median": round(float(np.median(per_step)), 5),
                                  "p10": round(float(np.percentile(per_step, 10)), 5),
                                  "p90": round(float(np.percentile(per_step, 90)), 5),
                                  "steps": int(args.steps)},
                  "wall_s_timed_region": round(wall, 4),
                  "launch": "hip graph replay" if args.graph else "eager C-ABI call per step",
                  "eager_ms_per_step": round(eager_ms, 5)},
        "decode_batch_sweep": sweep,
        "cpu_baseline": cpu,
    }
    if sweep is None:
        del res["decode_batch_sweep"]
    return res


def bench_dequant(args, cpu_seconds: float) -> dict:
    """Config 1: standalone MXFP4 -> bf16 dequant of a [32, 5760, 2880] tensor through
    physllm_moe_mxfp4_dequant. A step is one whole-tensor launch; the 1.34 GB it moves
    is five times the Infinity Cache, so no rotation is needed. Value = algorithmic
    bytes (codes + scales read, bf16 written) per second."""
    import torch
    from physllm_amd import ops
    from physllm_amd import synthetic as syn

    cfgd = syn.CONFIGS[1]
    log(f"[bench] generating config 1: {cfgd['workload']}")
    packed, scales, numel = syn.make_dequant_input()
    pd = torch.from_numpy(packed).cuda()
    sd = torch.from_numpy(scales).cuda()
    out = torch.empty(numel, dtype=torch.int16, device="cuda")
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    alg = numel // 2 + numel // 32 + 2 * numel

    for _ in range(args.warmup):
        ops.mxfp4_dequant(pd, sd, out, s)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        ops.mxfp4_dequant(pd, sd, out, s)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    gbs = alg / (ms * 1e-3) / 1e9
    runs_ms = timed_runs(stream, args.steps, lambda i: ops.mxfp4_dequant(pd, sd, out, s))
    # per-launch spread (after the timed region): median and 10/90th percentiles
    pev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    pev[0].record(stream)
    for i in range(args.steps):
        ops.mxfp4_dequant(pd, sd, out, s)
        pev[i + 1].record(stream)
    torch.cuda.synchronize()
    per_step = np.array([pev[i].elapsed_time(pev[i + 1]) for i in range(args.steps)])

    # spot check: one expert's slab against the oracle (bit-exact)
    from oracle import oracle as orc
    per = 5760 * 2880
    e = 17
    got = out[e * per:(e + 1) * per].cpu().numpy().view(np.uint16)
    exp = orc.mxfp4_dequant(packed[e * per // 2:(e + 1) * per // 2], scales[e * per // 32:(e + 1) * per // 32], per)
    assert np.array_equal(got, exp), "dequant output differs from the oracle"

    # The transposing dequant (output [E, in, out]) on the same tensor: timed over the
    # same number of launches, one expert checked against the oracle.
    ev0.record(stream)
    for _ in range(args.steps):
        ops.mxfp4_dequant_transpose(pd, sd, out, 32, 5760, 2880, 32, s)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_t = ev0.elapsed_time(ev1) / args.steps
    got = out[e * per:(e + 1) * per].cpu().numpy().view(np.uint16).reshape(1, 2880, 5760)
    exp = orc.mxfp4_dequant_transpose(packed[e * per // 2:(e + 1) * per // 2],
                                      scales[e * per // 32:(e + 1) * per // 32], 1, 5760, 2880)
    assert np.array_equal(got, exp), "transposing dequant output differs from the oracle"
    gbs_t = alg / (ms_t * 1e-3) / 1e9
    transpose = {"ms_per_launch": round(ms_t, 5), "value": round(gbs_t, 1), "unit": "GB/s",
                 "frac": round(gbs_t / HBM_PEAK_GBS, 4), "kernel": "k_mxfp4_dequant_t32",
                 "output": "[32, 2880, 5760] bf16 (in, out transposed)"}

    cpu = None
    if not args.no_cpu:
        nthr = orc.default_threads()
        n, tcpu = 0, 0.0
        while tcpu < cpu_seconds and n < 4096:
            e = n % 32
            sl = slice(e * per // 2, (e + 1) * per // 2)
            ss = slice(e * per // 32, (e + 1) * per // 32)
            t1 = time.perf_counter()
            orc.mxfp4_dequant(packed[sl], scales[ss], per, nthreads=nthr)
            tcpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": round(n * (per // 2 + per // 32 + 2 * per) / tcpu / 1e9, 3), "unit": "GB/s",
               "cores": nthr, "kind": "port",
               "sample": f"{n} expert slabs [5760,2880] (cycling over the 32) through the oracle's "
                         f"dequant ({tcpu:.1f} s, OpenMP over blocks)"}

    res = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "value_median": round(alg / (float(np.median(runs_ms)) * 1e-3) / 1e9, 1),
        "median_of_runs": median_summary(runs_ms, args.steps),
        "dtype": "u8->bf16",
        "data": "synthetic (seeded; e2m1 codes uniform 0-15, E8M0 scales 2^-8..2^-4)",
        "config": {"workload": cfgd["workload"], "config_index": 1, "numel": numel,
                   "bytes_algorithmic": alg},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(1, "dequant"),
                     "kernel": "k_mxfp4_dequant32", "work_per_launch": alg},
        "layer": {"wall_s_timed_region": round(wall, 4), "launch": "eager C-ABI call per step",
                  "per_step_ms": {"median": round(float(np.median(per_step)), 5),
                                  "p10": round(float(np.percentile(per_step, 10)), 5),
                                  "p90": round(float(np.percentile(per_step, 90)), 5),
                                  "steps": int(args.steps)}},
        "transpose": transpose,
        "cpu_baseline": cpu,
    }
    return res


if __name__ == "__main__":
    main()
