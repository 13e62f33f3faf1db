#!/usr/bin/env python3
"""Benchmark of the MXFP4 MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu]

A step is one MoE-layer forward (router -> bucketing -> gate_up+SwiGLU -> down ->
combine) over one batch of synthetic inputs already resident in HBM. The default
workload is BASELINE config 2 (GPT-OSS-20B-shape layer, decode batch 64, Zipf(1.1)
router skew); --config picks another. To keep the 256 MB Infinity Cache from
serving weights, steps rotate over enough device copies of the weights to exceed
1 GB. Prints ONE JSON line with the throughput, the dominant kernel's roofline
(timed live with HIP events on the launch stream) and the CPU baseline (the
oracle, timed on a bounded sample on this host's cores).
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
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=[0, 2, 3, 4])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on exactly one GPU (the MoE path has no multi-GPU code); "
              f"got --gpus {args.gpus}, WORLD_SIZE {world}", file=sys.stderr)
        sys.exit(2)

    import torch

    from physllm_amd import ops
    from physllm_amd import synthetic as syn

    cfg_i = args.config
    cfgd = syn.CONFIGS[cfg_i]
    log(f"[bench] generating config {cfg_i}: {cfgd['workload']}")
    layer, x = syn.make_config(cfg_i)
    B, H, I, E, K = x.shape[0], layer.hidden, layer.intermediate, layer.num_experts, layer.top_k

    dl0 = ops.DeviceMoELayer.from_host(layer)
    copies = [dl0]
    n_copies = 1 if cfg_i == 3 else max(1, math.ceil(1.1e9 / layer.weight_bytes))
    for _ in range(n_copies - 1):
        t = {k: (v.clone() if v is not None else None) for k, v in dl0.tensors.items()}
        copies.append(ops.DeviceMoELayer.from_tensors(H, I, E, K, t, layer.alpha, layer.limit))
    log(f"[bench] {n_copies} weight copies x {layer.weight_bytes / 1e6:.1f} MB")

    xd = torch.from_numpy(x.view(np.int16)).cuda()
    out = torch.empty((B, H), dtype=torch.int16, device="cuda")
    ws = torch.empty(dl0.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream

    def step(i):
        copies[i % n_copies].forward(xd, out, ws, stream=s)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K whole-layer steps ------------------------------------------
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / args.steps

    # ---- per-stage timing (events between the stage entry points, same stream) -------
    from physllm_amd.capi import check, lib
    import ctypes
    L = lib()
    nbytes = ws.numel()
    stage_ms = np.zeros(4)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    for i in range(args.steps):
        d = copies[i % n_copies]
        c, w = ctypes.byref(d.cfg), ctypes.byref(d.weights)
        evs[0].record(stream)
        check(L.physllm_moe_stage_route(c, w, xd.data_ptr(), B, None, None, ws.data_ptr(), nbytes, s))
        evs[1].record(stream)
        check(L.physllm_moe_stage_gate_up(c, w, xd.data_ptr(), B, ws.data_ptr(), nbytes, s))
        evs[2].record(stream)
        check(L.physllm_moe_stage_down(c, w, B, ws.data_ptr(), nbytes, s))
        evs[3].record(stream)
        check(L.physllm_moe_stage_combine(c, B, out.data_ptr(), None, ws.data_ptr(), nbytes, s))
        evs[4].record(stream)
        torch.cuda.synchronize()
        stage_ms += [evs[j].elapsed_time(evs[j + 1]) for j in range(4)]
    stage_ms /= args.steps

    # touched experts (routing is deterministic; read once, outside the timed region)
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((B, K), dtype=torch.float32, device="cuda")
    ops.route_topk(xd, dl0.tensors["router_w"], dl0.tensors["router_b"], idx, wt, K, s)
    torch.cuda.synchronize()
    counts = np.bincount(idx.cpu().numpy().reshape(-1), minlength=E)
    e_touched = int((counts > 0).sum())

    # ---- roofline of the dominant kernel (gate_up) ---------------------------------------
    gu_expert_bytes = (2 * I * H // 2) + (2 * I * H // 32) + 2 * (2 * I)
    gate_up_ms = float(stage_ms[1])
    if cfg_i == 3:
        flops = 2.0 * B * K * (2 * I) * H
        achieved = flops / (gate_up_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                "kernel": "gate_up grouped GEMM", "work_per_launch": flops}
    else:
        alg = e_touched * gu_expert_bytes + B * H * 2 + B * K * I * 2
        achieved = alg / (gate_up_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "gate_up grouped GEMV (k_mx_gemv<0>)", "work_per_launch": alg}
    layer_bytes = e_touched * layer.expert_bytes + E * H * 2 + E * 2 + B * H * 2 * 2

    # ---- CPU baseline (oracle on this host's cores, bounded sample) ----------------------
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as orc
        nthr = orc.default_threads()
        xs = x if cfg_i != 3 else x[:64]
        n, tcpu = 0, 0.0
        while tcpu < args.cpu_seconds and n < 50:
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
        "dtype": "bf16",
        "data": "synthetic (seeded; MXFP4 e2m1 codes uniform, E8M0 scales 2^-8..2^-4, bf16 N(0,.02) biases/router, x N(0,1))",
        "config": {"workload": cfgd["workload"], "config_index": cfg_i, "batch": B, "hidden": H,
                   "intermediate": I, "experts": E, "top_k": K, "experts_touched": e_touched,
                   "weights": "MXFP4 (e2m1 + E8M0 per 32)", "weight_copies_rotated": n_copies},
        "roofline": roof,
        "layer": {"hbm_bytes_algorithmic": layer_bytes,
                  "hbm_gbs": round(layer_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                  "hbm_frac": round(layer_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "stage_ms": {"route": round(stage_ms[0], 5), "gate_up": round(stage_ms[1], 5),
                               "down": round(stage_ms[2], 5), "combine": round(stage_ms[3], 5)},
                  "wall_s_timed_region": round(wall, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
