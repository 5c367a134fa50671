#!/usr/bin/env python3
"""Benchmark of the routed-expert SwiGLU FFN on one MI355X.

Default workload (the config the metric is quoted
on): a Mixtral-8x7B-shaped MoE stack, 32 layers x 8 Q4_0 experts
(d_model 4096, d_ff 14336; 256 experts = 25.4 GB resident in HBM), top-2
routing from N(0,1) logits per token per layer (softmax, top-2,
renormalised), decode batch 1.  One step = one token through all 32 layers:
layer l reads its own N(0,1) input vector x_l (standing in for the normed
residual stream, which keeps magnitudes bounded without a norm kernel) and
accumulates out += sum_i w_i y_i (the engine's WeightedInto accumulate).  Weights are synthetic (this library's
counter-based generator: nibbles uniform, d = f16(U(0.005, 0.02))).

Prints one JSON line (rank 0).  The CPU baseline leg times the C oracle's
restatement of the reference's Q4_0 CPU path (dequantise + f32 GEMV,
q4_0_cpu_reference_forward) on a bounded sample of the same experts.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG = "micro-expert-router-ssd-streamed-moe-mer_amd"

HBM_PEAK_GBPS = 8000.0
Q4_BLOCK = 18
METRIC = "expert-FFN tokens/s + achieved HBM GB/s (% of peak), Mixtral-shape Q4_0 top-2"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(mer, blob_dev, x_np, dm, dff, experts_per_token, budget_s, gpu_y):
    """Oracle (checker) timing on host cores: a bounded sample of expert FFNs.

    Cycles through the sampled experts until `budget_s` of CPU work is
    timed; each expert's first CPU result is also compared with the GPU's."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import mer_oracle  # noqa: E402  (test infrastructure, used as the checker)

    threads = max(1, min(16, os.cpu_count() or 1))
    hosts = [blob.cpu().numpy() for blob in blob_dev]
    times, max_err = [], 0.0
    spent = 0.0
    i = 0
    while spent < budget_s or i < len(hosts):
        host = hosts[i % len(hosts)]
        t0 = time.perf_counter()
        y = mer_oracle.q4_0_reference_forward(host, x_np, dm, dff, nthreads=threads)
        dt = time.perf_counter() - t0
        times.append(dt)
        spent += dt
        if i < len(hosts):
            err = np.abs(y.astype(np.float64) - gpu_y[i]) / (1e-3 + 1e-3 * np.abs(y))
            max_err = max(max_err, float(err.max()))
        i += 1
    per_expert = float(np.mean(times))
    return {
        "value": 1.0 / (per_expert * experts_per_token),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{len(times)} Mixtral-shape Q4_0 expert FFNs ({len(hosts)} distinct experts, cycled) with the "
                   f"reference's q4_0_cpu_reference_forward (dequantise + f32 GEMV) restated in C on {threads} "
                   f"threads: {spent:.1f} s, mean {per_expert * 1e3:.1f} ms/expert, scaled to "
                   f"{experts_per_token} experts/token"),
        "ms_per_expert": per_expert * 1e3,
        "parity_worst_ratio": max_err,
    }


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_kernel_mixtral_q4_0_traffic.md")


def read_traffic(dominant: str):
    """HBM bytes per decode launch measured with rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes (scaled by a copy kernel), as committed under profiles/."""
    if dominant != "decode" or not os.path.exists(TRAFFIC_FILE):
        return None
    import re

    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", open(TRAFFIC_FILE).read())
    if not m:
        return None
    return {"bytes": int(m.group(1)), "source": os.path.relpath(TRAFFIC_FILE, ROOT)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0xC0FFEE)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the run, launch a plain elementwise kernel that reads and writes MIB MiB "
                         "(counter calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--route-after-prev", action="store_true",
                    help="layer l's routing is read and its experts streamed only after layer l-1's output is "
                         "complete (MER_MOE_ROUTE_AFTER_PREV), as when routing is computed from that output")
    ap.add_argument("--per-layer", action="store_true",
                    help="one mer_hip_moe_forward call per layer instead of one multi-layer launch per token")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(experts would shard id % n_gpu; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    mer = importlib.import_module(PKG)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mer.init(0)
    lib = mer._lib.lib()

    L, E, K, dm, dff = args.layers, 8, 2, 4096, 14336
    ebytes = mer.expert_weight_bytes_for(dm, dff, mer.WeightDtype.Q4_0)
    assert ebytes == 99_090_432
    nb = ebytes // Q4_BLOCK
    log(f"allocating {L * E} experts x {ebytes} B = {L * E * ebytes / 1e9:.2f} GB")
    weights = torch.empty(L * E * ebytes, dtype=torch.uint8, device=dev)
    for e in range(L * E):
        mer.fill_synthetic(mer.WeightDtype.Q4_0, args.seed, e, nb, 0.005, 0.02, weights[e * ebytes:(e + 1) * ebytes])
    torch.cuda.synchronize()
    base = weights.data_ptr()
    table = torch.tensor([[base + (l * E + e) * ebytes for e in range(E)] for l in range(L)],
                         dtype=torch.int64, device=dev)

    routing = importlib.import_module(PKG + ".routing")
    total_steps = args.warmup + args.steps
    rng = np.random.default_rng(args.seed + 2)
    logits = rng.standard_normal((total_steps, L, E)).astype(np.float32)
    ids = np.zeros((total_steps, L, 1, K), np.int32)
    wts = np.zeros((total_steps, L, 1, K), np.float32)
    for s in range(total_steps):
        for l in range(L):
            i, w = routing.route_scores(logits[s, l], K)
            ids[s, l, 0], wts[s, l, 0] = i, w
    ids_d = torch.from_numpy(ids).to(dev)
    wts_d = torch.from_numpy(wts).to(dev)
    xs = np.random.default_rng(args.seed + 1).standard_normal((L, 1, dm)).astype(np.float32)
    x0 = xs[0]
    xs_d = torch.from_numpy(xs).to(dev)
    out = torch.zeros((1, dm), dtype=torch.float32, device=dev)

    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.mer_hip_moe_forward

    # Pre-bound C-ABI arguments per (step, layer): the timed loop is pure launches.
    def step_args(s):
        return [(4, dm, dff, 1, K, table[l].data_ptr(), E, ids_d[s, l].data_ptr(), wts_d[s, l].data_ptr(),
                 xs_d[l].data_ptr(), out.data_ptr(), 2, stream) for l in range(L)]

    # one multi-layer launch per token: prebuilt mer_layer_args arrays
    fn_layers = lib.mer_hip_moe_forward_layers

    def layer_array(s):
        arr = (mer._lib.MerLayerArgs * L)()
        for l in range(L):
            arr[l] = mer._lib.MerLayerArgs(table[l].data_ptr(), E, ids_d[s, l].data_ptr(), wts_d[s, l].data_ptr(),
                                           xs_d[l].data_ptr(), out.data_ptr())
        return arr

    if args.per_layer:
        all_args = [step_args(s) for s in range(total_steps)]
    else:
        flags = 2 | (8 if args.route_after_prev else 0)  # ACCUMULATE [| ROUTE_AFTER_PREV]
        all_args = [(4, dm, dff, L, 1, K, layer_array(s), flags, stream) for s in range(total_steps)]

    def run_step(s):
        if args.per_layer:
            for a in all_args[s]:
                rc = fn(*a)
                if rc:
                    mer.errors.raise_for_status(rc)
        else:
            rc = fn_layers(*all_args[s])
            if rc:
                mer.errors.raise_for_status(rc)

    log("warmup")
    for s in range(args.warmup):
        run_step(s)
    torch.cuda.synchronize()
    mer.take_device_status()

    log(f"timing {args.steps} steps")
    mer.stage_timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.warmup, total_steps):
        run_step(s)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    stages = mer.stage_timing_read()
    mer.stage_timing_enable(False)
    mer.take_device_status()
    elapsed = t1 - t0
    ms_per_step = elapsed * 1e3 / args.steps
    tokens_per_s = args.steps / elapsed

    # Algorithmic bytes (packed weights of each distinct expert touched + f32
    # activations in/out).  Per launch of each stage (K experts per launch):
    proj = ebytes // 3
    gate_up_bytes = K * 2 * proj + dm // 32 * 100 + K * dff // 32 * 100  # weights + x digits in + h digits out
    down_bytes = K * proj + K * dff // 32 * 100 + K * 4 * dm * 4  # weights + h digits in + 4 slice partials
    combine_bytes = K * 4 * dm * 4 + 2 * dm * 4                   # partial slices + out read/write
    per_layer_bytes = K * ebytes + 3 * dm * 4  # + x_l in, out read + written
    token_bytes = L * per_layer_bytes
    prep_bytes = dm * 4 + dm // 32 * 100 + K * 12                 # x in, digit planes out, slot pointers
    decode_bytes = per_layer_bytes if args.per_layer else token_bytes   # one decode_kernel launch
    stage_bytes = {"gate_up": gate_up_bytes, "down": down_bytes, "combine": combine_bytes, "prep": prep_bytes,
                   "decode": decode_bytes}
    stage_info = {}
    for name, (ms, cnt) in stages.items():
        if cnt:
            avg = ms / cnt
            stage_info[name] = {"avg_us": avg * 1e3, "launches": cnt,
                                "gbps": stage_bytes[name] / (avg * 1e-3) / 1e9}
    dominant = max(stage_info, key=lambda k: stage_info[k]["avg_us"] * stage_info[k]["launches"])
    dom = stage_info[dominant]

    # Parity of the sampled experts: GPU single-expert forward on x0.
    sample = [(0, l, int(ids[0, l, 0, i])) for l in range(min(L, 8)) for i in range(K)]
    blobs = [weights[(l * E + e) * ebytes:(l * E + e + 1) * ebytes] for _, l, e in sample]
    xdev = torch.from_numpy(x0[0]).to(dev)
    gpu_y = [mer.q4_0_forward(b, xdev, dm, dff).cpu().numpy().astype(np.float64) for b in blobs]

    result = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "mixtral-8x7b-moe-decode-q4_0-top2", "layers": L, "experts_per_layer": E,
                   "top_k": K, "d_model": dm, "d_ff": dff, "batch": 1, "resident_bytes": L * E * ebytes,
                   "bytes_per_token": token_bytes, "parallelism": "single-gpu",
                   "launch": "per-layer" if args.per_layer else "all-layers",
                   "routing": ("each layer's routing used only after the previous layer's output is complete"
                               if args.per_layer or args.route_after_prev else
                               "every layer's routing is a launch input (exogenous N(0,1) logits)")},
        "hbm_gbps": token_bytes * tokens_per_s / 1e9,
        "hbm_frac_of_peak": token_bytes * tokens_per_s / 1e9 / HBM_PEAK_GBPS,
        "roofline": {"bound": "hbm", "kernel": "decode_kernel" if dominant == "decode" else f"proj_kernel ({dominant})",
                     "achieved": dom["gbps"],
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": dom["gbps"] / HBM_PEAK_GBPS,
                     "traffic": None, "algorithmic_bytes_per_launch": stage_bytes[dominant],
                     "avg_launch_us": dom["avg_us"]},
        "stages": stage_info,
    }
    traffic = read_traffic(dominant)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic["bytes"]
        result["roofline"]["traffic_source"] = traffic["source"]
    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.add(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 launches of add(src, 1) over {args.copy_calibration} MiB in, same out")
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(mer, blobs, x0[0], dm, dff, L * K, args.cpu_seconds, gpu_y)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
