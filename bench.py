#!/usr/bin/env python3
"""Benchmark of the routed-expert SwiGLU FFN on one MI355X.

Default workload (the config the metric is quoted
on): a Mixtral-8x7B-shaped MoE stack, 32 layers x 8 Q4_0 experts
(d_model 4096, d_ff 14336; 256 experts = 25.4 GB resident in HBM), top-2
routing from N(0,1) logits per token per layer (softmax over the selected
two), decode batch 1.  One step = one token through all 32 layers in one
mer_hip_moe_forward_layers launch: layer l reads its own N(0,1) input x_l
(standing in for the normed residual stream) and accumulates
out += sum_i w_i y_i; layer l+1 starts packing its input only after layer
l's output is complete.  Weights come from this library's counter-based
generator (nibbles uniform, d = f16(U(0.005, 0.02))).

--config 0: one Mixtral-shape Q4_0 expert per step (expert-FFN/s), cycling
  over 32 distinct resident experts so no step re-reads a cached expert.
--config 2: the Qwen3-30B-A3B shape, 48 layers x 128 Q8_0 experts
  (d_model 2048, d_ff 768; 30.8 GB resident), top-8 from a per-layer
  LinearGate [128 x 2048] ~ N(0, 0.02) applied to a fresh N(0,1) hidden
  state per step and layer (routed on the host).
--config 4: DeepSeek-V3-shaped routed experts under cache pressure: 256
  Q4_0 experts (d_model 7168, d_ff 2048; 6.34 GB) in pinned host RAM, a
  64-slot VRAM SlotCache (25%), decode batch 4 x top-8 from
  SkewedStream(Zipf 1.0, stay 0.7) with uniform 1/k weights.  Each step
  prepares its distinct experts (misses uploaded on the cache's copy stream,
  overlapping the previous step's kernel) and runs one mer_hip_moe_forward.
--config 3: the batched grouped-expert case, 64 tokens x 128 Qwen3-shaped
  Q8_0 experts, top-8 from N(0,1) logits plus a Zipf(1.1) popularity skew
  (routing.zipf_skewed_routes), one mer_hip_moe_grouped call per step.  Steps
  cycle over 8 copies of the 128-expert layer (5.1 GB) with fresh routing and
  inputs, so no step finds its experts in the memory-side cache.

Prints one JSON line.  Every timed step writes outputs of its own; the
outputs of the last timed launch are read back and checked against the
oracle (cpu_baseline.parity_worst_ratio).  The CPU baseline leg times the C
oracle's restatement of the reference's CPU path over whole steps of the
same workload, starting with that last timed step, on the host's cores (up
to the 16-thread share of a one-GPU job; host fields in the line):
q4_0_cpu_reference_forward (dequantise + f32 GEMV) for Q4_0,
forward_q8_0_direct_into's AVX2 kernel for Q8_0.  Configs 1 and 2 also
report the same steps under MER_MOE_ROUTE_AFTER_PREV (route_after_prev)
and as one call per layer (per_layer).  Configs 0 and 1 also report the same
steps with MER_MOE_QMM (qmm): Q4_0 through Candle's QMatMul arithmetic, the
reference engine's default Q4_0 arm, checked against the oracle's
restatement of it under the bar of tests/test_gpu_qmm.py.  `value` and
`roofline` stay on q4_0_cpu_reference_forward's semantics.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG = "micro-expert-router-ssd-streamed-moe-mer_amd"

HBM_PEAK_GBPS = 8000.0
Q4, Q8 = 4, 5
BLOCK_BYTES = {Q4: 18, Q8: 34}
METRIC = "expert-FFN tokens/s + achieved HBM GB/s (% of peak), Mixtral-shape Q4_0 top-2"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_kernel_mixtral_q4_0_traffic.md")
# What the kernels compute in: packed GGUF weights against block fixed-point
# activations (integer digit planes), accumulated in f32.
DTYPE_LABEL = {
    Q4: "q4_0 weights x 22-bit block fixed-point activations, f32 accumulate",
    Q8: "q8_0 weights x 22-bit block fixed-point activations, f32 accumulate",
}
DTYPE_LABEL_GROUPED = "q8_0/q4_0 weights x 24-bit block fixed-point activations (int8 MFMA), f32 accumulate"

CONFIGS = {
    0: dict(workload="mixtral-expert-q4_0", dtype=Q4, d_model=4096, d_ff=14336, layers=1, experts=32, top_k=1,
            scale=(0.005, 0.02), metric="expert-FFN/s, one Mixtral-shape Q4_0 expert per step", unit="expert-FFN/s"),
    1: dict(workload="mixtral-8x7b-moe-decode-q4_0-top2", dtype=Q4, d_model=4096, d_ff=14336, layers=32, experts=8,
            top_k=2, scale=(0.005, 0.02), metric=METRIC, unit="tokens/s"),
    2: dict(workload="qwen3-30b-a3b-moe-decode-q8_0-top8", dtype=Q8, d_model=2048, d_ff=768, layers=48, experts=128,
            top_k=8, scale=(0.002, 0.01), metric="expert-FFN tokens/s + achieved HBM GB/s, Qwen3-30B-A3B-shape Q8_0 top-8",
            unit="tokens/s"),
    3: dict(workload="qwen3-moe-grouped-64tok-q8_0-top8-zipf1.1", dtype=Q8, d_model=2048, d_ff=768, layers=8,
            experts=128, top_k=8, tokens=64, scale=(0.002, 0.01),
            metric="expert-FFN tokens/s + achieved HBM GB/s, 64-token Qwen3-shape Q8_0 top-8 grouped batch",
            unit="tokens/s"),
    4: dict(workload="deepseek-v3-experts-q4_0-top8-batch4-cache25pct", dtype=Q4, d_model=7168, d_ff=2048, layers=1,
            experts=256, top_k=8, tokens=4, slots=64, scale=(0.005, 0.02),
            metric="expert-FFN tokens/s under cache pressure (25% of experts in VRAM, misses over PCIe), "
                   "DeepSeek-V3-shape Q4_0 top-8 batch 4", unit="tokens/s"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_info(threads: int) -> dict:
    """The host the CPU baseline ran on: its thread count, the CPUs the OS
    reports and may schedule this process on, and the CPU model string."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return {"cores": threads, "host_cpus": os.cpu_count(), "affinity_cpus": affinity, "cpu_model": model}


def baseline_threads() -> int:
    """Threads for the oracle: every CPU this process may run on, capped at
    16, the host-CPU share of a one-GPU job on the GPU boxes (more threads
    than that share would time the scheduler, not the kernel)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(dtype, dm, dff, steps, blob_of, gpu_rows, budget_s, units_per_step, unit, what):
    """The oracle (checker) timed on host cores over whole steps of the
    timed workload, and the parity leg of the timed launch.

    `steps` lists steps, the first being the last timed step; a step is a
    list of output rows, a row a list of layers, a layer (x, expert keys,
    slot weights): the row's value is the sum over its layers of the
    slot-order combine (combine_outputs_into, inference.rs:4472-4491) of the
    layer's experts on x.  blob_of(key) gives an expert's host bytes (fetched
    before each step's clock starts).  The first step's rows are compared
    with gpu_rows, the outputs the timed launch wrote.  Steps run, cycling
    through the list, until `budget_s` of CPU work is timed (at least one)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import mer_oracle  # noqa: E402  (test infrastructure, used as the checker)

    threads = baseline_threads()

    def expert(blob, x):
        if dtype == Q4:
            return mer_oracle.q4_0_reference_forward(blob, x, dm, dff, nthreads=threads)
        rc, y = mer_oracle.q8_0_direct_forward(blob, x, dm, dff, kernel=1, nthreads=threads)
        assert rc == 0
        return y

    spent, n_steps, n_experts, worst = 0.0, 0, 0, None
    for si in range(1 << 30):  # the steps again and again until the budget is spent
        if n_steps and spent >= budget_s:
            break
        step = steps[si % len(steps)]
        blobs = {key: blob_of(key) for row in step for _, keys, _ in row for key in keys}
        t0 = time.perf_counter()
        rows = []
        for row in step:
            acc = np.zeros(dm, np.float64)
            for x, keys, wts in row:
                ys = np.stack([expert(blobs[k], x) for k in keys])
                acc += mer_oracle.combine_outputs(ys, np.asarray(wts, np.float32)).astype(np.float64)
                n_experts += len(keys)
            rows.append(acc)
        spent += time.perf_counter() - t0
        n_steps += 1
        if si == 0:
            # the parity tests' bar: |gpu - ref| <= 1e-3 |ref| + 1e-3 max(1, 1e-3 max|ref|)
            ref = np.stack(rows)
            got = np.asarray(gpu_rows, np.float64).reshape(ref.shape)
            allowed = 1e-3 * np.abs(ref) + 1e-3 * max(1.0, 1e-3 * float(np.abs(ref).max()))
            worst = float((np.abs(ref - got) / allowed).max())
    out = {
        "value": n_steps * units_per_step / spent,
        "unit": unit,
        **host_info(threads),
        "kind": "port",
        "sample": (f"{n_steps} whole step(s) of the timed workload ({n_experts} expert FFNs, starting with the "
                   f"last timed step, cycling over {len(steps)} timed steps) with {what} restated in C on {threads} "
                   f"threads: {spent:.1f} s"),
        "ms_per_expert": spent / max(n_experts, 1) * 1e3,
        "parity_worst_ratio": worst,
        "parity_of": "the outputs the last timed launch wrote, against the oracle on the same step",
    }
    return out


def read_traffic(cfg_id: int):
    """HBM bytes per decode launch measured with rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes (scaled by a copy kernel), as committed under profiles/."""
    if cfg_id != 1 or not os.path.exists(TRAFFIC_FILE):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", open(TRAFFIC_FILE).read())
    if not m:
        return None
    return {"bytes": int(m.group(1)), "source": os.path.relpath(TRAFFIC_FILE, ROOT)}


def run_cache_pressure(args, cfg, mer, routing, dev, stream):
    """Config 4: decode through a VRAM SlotCache fed from pinned host RAM."""
    import torch

    dtype, dm, dff, K, T = cfg["dtype"], cfg["d_model"], cfg["d_ff"], cfg["top_k"], cfg["tokens"]
    E, n_slots = cfg["experts"], cfg["slots"]
    wd = mer.WeightDtype(dtype)
    ebytes = mer.expert_weight_bytes_for(dm, dff, wd)
    nb = ebytes // BLOCK_BYTES[dtype]
    log(f"config 4: {E} experts x {ebytes} B = {E * ebytes / 1e9:.2f} GB in pinned host RAM, {n_slots} VRAM slots")
    host = torch.empty(E * ebytes, dtype=torch.uint8, pin_memory=True)
    stage = torch.empty(ebytes, dtype=torch.uint8, device=dev)
    lo, hi = cfg["scale"]
    for e in range(E):
        mer.fill_synthetic(wd, args.seed, e, nb, lo, hi, stage)
        host[e * ebytes:(e + 1) * ebytes].copy_(stage)
    torch.cuda.synchronize()
    blobs = [host[e * ebytes:(e + 1) * ebytes] for e in range(E)]

    # plain pinned H2D rate on this box (the copy roofline of a miss)
    t0 = time.perf_counter()
    for e in range(8):
        stage.copy_(blobs[e], non_blocking=True)
    torch.cuda.synchronize()
    h2d_peak = 8 * ebytes / (time.perf_counter() - t0) / 1e9

    total_steps = args.warmup + args.steps
    stream_gen = routing.SkewedStream(E, K, 1.0, 0.7, args.seed + 2)
    ids = np.array([[stream_gen.next_experts() for _ in range(T)] for _ in range(total_steps)], np.int32)
    wts = np.full((total_steps, T, K), 1.0 / K, np.float32)  # uniform, as Router::Markov (gating.rs:494-503)
    xs = np.random.default_rng(args.seed + 1).standard_normal((total_steps, T, dm)).astype(np.float32)
    ids_d, wts_d, xs_d = (torch.from_numpy(a).to(dev) for a in (ids, wts, xs))
    outs = torch.zeros((total_steps, T, dm), dtype=torch.float32, device=dev)
    cache = mer.SlotCache(wd, dm, dff, n_slots, E)
    distinct = [list(dict.fromkeys(int(v) for v in ids[s].reshape(-1))) for s in range(total_steps)]

    def run_step(s):
        cache.prepare(distinct[s], host_blobs=[blobs[e] for e in distinct[s]])
        mer.moe_forward(wd, dm, dff, cache, ids_d[s], wts_d[s], xs_d[s], out=outs[s])

    log("warmup")
    for s in range(args.warmup):
        run_step(s)
    torch.cuda.synchronize()
    mer.take_device_status()
    st0 = cache.stats()
    log(f"timing {args.steps} steps")
    mer.stage_timing_enable(True)
    t0 = time.perf_counter()
    for s in range(args.warmup, total_steps):
        run_step(s)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    stages = mer.stage_timing_read()
    mer.stage_timing_enable(False)
    mer.take_device_status()
    st1 = cache.stats()
    hits, misses = st1["hits"] - st0["hits"], st1["misses"] - st0["misses"]
    up_bytes = st1["bytes_uploaded"] - st0["bytes_uploaded"]
    dec_ms, dec_n = stages["decode"]
    timed_u = np.array([len(distinct[s]) for s in range(args.warmup, total_steps)])
    kernel_bytes = float(np.mean(timed_u)) * ebytes + 2 * T * dm * 4
    dec_avg_us = dec_ms / max(dec_n, 1) * 1e3
    t_copy = up_bytes / (h2d_peak * 1e9)
    t_comp = dec_ms * 1e-3
    overlap = (t_copy + t_comp - elapsed) / min(t_copy, t_comp) if min(t_copy, t_comp) > 0 else None

    s_last = total_steps - 1
    gpu_last = outs[s_last].cpu().numpy()

    value = args.steps * T / elapsed
    result = {
        "metric": cfg["metric"], "value": value, "unit": cfg["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "data": "synthetic",
        "config": {"workload": cfg["workload"], "experts": E, "vram_slots": n_slots, "top_k": K, "batch": T,
                   "d_model": dm, "d_ff": dff, "weights": "Q4_0", "host_bytes": E * ebytes,
                   "parallelism": "single-gpu",
                   "routing": "SkewedStream(Zipf s=1.0, stay 0.7) per token, uniform 1/k weights",
                   "launch": "per step: SlotCache.prepare(distinct ids) + mer_hip_moe_forward (4 tokens)"},
        "cache": {"hits": hits, "misses": misses, "hit_rate": hits / max(hits + misses, 1),
                  "distinct_experts_per_step": float(np.mean(timed_u)), "bytes_uploaded": up_bytes,
                  "h2d_gbps": up_bytes / elapsed / 1e9, "h2d_peak_gbps": h2d_peak,
                  "h2d_busy_frac": t_copy / elapsed, "compute_busy_frac": t_comp / elapsed,
                  "overlap_frac": overlap},
        "roofline": {"bound": "hbm", "kernel": "decode_kernel", "achieved": kernel_bytes / (dec_avg_us * 1e-6) / 1e9,
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": kernel_bytes / (dec_avg_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, "traffic": None,
                     "algorithmic_bytes_per_launch": int(kernel_bytes), "avg_launch_us": dec_avg_us,
                     "note": "the step is bound by PCIe uploads of misses (see cache.h2d_*), not by this kernel"},
    }
    result["dtype"] = DTYPE_LABEL[dtype]
    if not args.no_cpu_baseline:
        log("cpu baseline")
        steps = [[[(xs[s, t], [int(e) for e in ids[s, t]], wts[s, t])] for t in range(T)]
                 for s in range(s_last, args.warmup - 1, -1)]
        result["cpu_baseline"] = cpu_baseline(dtype, dm, dff, steps, lambda e: blobs[e].numpy(), gpu_last,
                                              args.cpu_seconds, T, cfg["unit"],
                                              "the reference's q4_0_cpu_reference_forward (dequantise + f32 GEMV)")
        result["cpu_baseline"]["sample"] += "; experts read from host RAM (no PCIe)"
    cache.close()
    return result


def qmm_parity(dm, dff, step, blob_of, gpu_rows):
    """Parity of a QMatMul-mode launch: the oracle's restatement of
    run_inference_q4_0_qmm (Q8_0-quantised activations, inference.rs:
    4159-4243) on the same step, worst |gpu - ref| / allowed under the bar
    of tests/test_gpu_qmm.py (the FFN bar plus the oracle's flip bound).
    `step` is a list of rows as in cpu_baseline."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import mer_oracle  # noqa: E402  (test infrastructure, used as the checker)

    threads = baseline_threads()
    rows, bounds, flagged = [], [], 0
    blobs = {k: blob_of(k) for row in step for _, keys, _ in row for k in keys}  # fetched before the clock
    n_experts = sum(len(keys) for row in step for _, keys, _ in row)
    t0 = time.perf_counter()
    for row in step:
        acc = np.zeros(dm, np.float64)
        bnd = np.zeros(dm, np.float64)
        for x, keys, wts in row:
            res = [mer_oracle.q4_0_qmm_forward_bounded(blobs[k], x, dm, dff, nthreads=threads) for k in keys]
            acc += mer_oracle.combine_outputs(np.stack([r[0] for r in res]), np.asarray(wts, np.float32)).astype(
                np.float64)
            bnd += sum(abs(float(w)) * r[1].astype(np.float64) for w, r in zip(wts, res))
            flagged += sum(r[2] for r in res)
        rows.append(acc)
        bounds.append(bnd)
    spent = time.perf_counter() - t0
    ref = np.stack(rows)
    got = np.asarray(gpu_rows, np.float64).reshape(ref.shape)
    bar = 1e-3 * np.abs(ref) + 1e-3 * max(1.0, 1e-3 * float(np.abs(ref).max()))
    err = np.abs(ref - got)
    return {"cpu_ms_per_expert": spent / max(n_experts, 1) * 1e3, "cpu_threads": threads,
            "cpu_note": "the oracle's scalar-C restatement of the QMatMul arithmetic on the same step, flip bound "
                        "included (Candle's own AVX kernels are faster; ~27 ms per Mixtral expert in the "
                        "reference's notes, 16 cores)",
            "parity_worst_ratio": float((err / (bar + np.stack(bounds))).max()),
            "rows_beyond_ffn_bar": int((err > bar).sum()), "h_elements_flagged": int(flagged),
            "parity_bar": "1e-3 |ref| + 1e-3 max(1, 1e-3 max|ref|) + the oracle's flip bound (h elements within "
                          "1e-3 steps of a Q8_0 rounding midpoint may round either way in another f32 order)"}


def router_pass(gates, xs_d, ids, L, E, K, dm, first_step, n_steps):
    """The GPU LinearGate router (mer_hip_route_linear_gate, row a19) on the
    config-2 steps' hidden states, one call per layer (logits kernel + select
    kernel), all calls enqueued back to back between one pair of HIP events
    on the current stream, so the figure is GPU time per call.  Reported
    beside the expert path, not part of `value` (the timed steps route on the
    host); `agreement` is the fraction of (step, layer) whose GPU top-k id set
    equals the host routing's."""
    import ctypes

    import torch

    mer = importlib.import_module(PKG)
    dev = xs_d.device
    lib = mer._lib.lib()
    gates_d = torch.from_numpy(gates).to(dev)
    stream = torch.cuda.current_stream().cuda_stream
    opts = mer._lib.MerGateOptions(0, 1, 0, 1, 1, 1.0)
    calls = [(s, l) for s in range(first_step, first_step + n_steps) for l in range(L)]
    ids_out = torch.empty((len(calls), K), dtype=torch.int32, device=dev)
    w_out = torch.empty((len(calls), K), dtype=torch.float32, device=dev)
    args = [(gates_d[l].data_ptr(), E, dm, xs_d[s, l].data_ptr(), 1, K, ctypes.byref(opts),
             ids_out[i].data_ptr(), w_out[i].data_ptr(), None, stream) for i, (s, l) in enumerate(calls)]
    fn = lib.mer_hip_route_linear_gate
    for a in args[:L]:  # warm
        fn(*a)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for a in args:
        rc = fn(*a)
        if rc:
            mer.errors.raise_for_status(rc)
    t1.record()
    torch.cuda.synchronize()
    avg = t0.elapsed_time(t1) * 1e3 / len(args)
    got = ids_out.cpu().numpy()
    agree = np.mean([set(got[i].tolist()) == set(ids[s, l, 0].tolist()) for i, (s, l) in enumerate(calls)])
    nbytes = E * dm * 4 + dm * 4 + K * 8
    return {"kernels": "router_logits_kernel + router_kernel", "calls": len(args), "avg_us_per_call": avg,
            "bytes_per_call": nbytes, "gbps": nbytes / (avg * 1e-6) / 1e9,
            "frac": nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBPS, "agreement": float(agree)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=1, choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=None, help="override the config's layer count")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0xC0FFEE)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the run, launch a plain elementwise kernel that reads and writes MIB MiB "
                         "(counter calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--route-after-prev", action="store_true",
                    help="layer l's routing is read and its experts streamed only after layer l-1's output is "
                         "complete (MER_MOE_ROUTE_AFTER_PREV), as when routing is computed from that output")
    ap.add_argument("--no-route-after-prev-pass", action="store_true",
                    help="skip the second pass of configs 1 and 2 under MER_MOE_ROUTE_AFTER_PREV (for profiler runs "
                         "whose per-kernel averages should cover the timed launches only)")
    ap.add_argument("--no-qmm-pass", action="store_true",
                    help="skip the Q4_0 QMatMul-mode pass (MER_MOE_QMM) reported as `qmm` on configs 0 and 1")
    ap.add_argument("--per-layer", action="store_true",
                    help="one mer_hip_moe_forward call per layer instead of one multi-layer launch per token")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(experts would shard by id % n_gpu across GPUs). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    mer = importlib.import_module(PKG)
    routing = importlib.import_module(PKG + ".routing")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    mer.init(0)
    lib = mer._lib.lib()
    stream = torch.cuda.current_stream().cuda_stream

    cfg = CONFIGS[args.config]
    if args.config == 4:
        print(json.dumps(run_cache_pressure(args, cfg, mer, routing, dev, stream)), flush=True)
        return 0
    dtype, dm, dff, K = cfg["dtype"], cfg["d_model"], cfg["d_ff"], cfg["top_k"]
    L = args.layers if args.layers is not None else cfg["layers"]
    E = cfg["experts"]
    ebytes = mer.expert_weight_bytes_for(dm, dff, mer.WeightDtype(dtype))
    nb = ebytes // BLOCK_BYTES[dtype]
    n_exp = L * E
    log(f"config {args.config}: allocating {n_exp} experts x {ebytes} B = {n_exp * ebytes / 1e9:.2f} GB")
    weights = torch.empty(n_exp * ebytes, dtype=torch.uint8, device=dev)
    lo, hi = cfg["scale"]
    for e in range(n_exp):
        mer.fill_synthetic(mer.WeightDtype(dtype), args.seed, e, nb, lo, hi, weights[e * ebytes:(e + 1) * ebytes])
    torch.cuda.synchronize()
    base = weights.data_ptr()

    def blob(e):
        return weights[e * ebytes:(e + 1) * ebytes]

    total_steps = args.warmup + args.steps
    rng_x = np.random.default_rng(args.seed + 1)
    rng_r = np.random.default_rng(args.seed + 2)

    # Every step writes outputs of its own, so the outputs of the last timed
    # launch can be read back and checked against the oracle (parity leg).
    if args.config == 0:
        # one expert per step, cycling over E distinct resident experts
        xs = rng_x.standard_normal((1, dm)).astype(np.float32)
        xs_d = torch.from_numpy(xs).to(dev)
        outs = torch.zeros((total_steps, dm), dtype=torch.float32, device=dev)
        fn = lib.mer_hip_expert_forward
        all_args = [(dtype, base + (s % E) * ebytes, ebytes, xs_d.data_ptr(), dm, dm, dff, outs[s].data_ptr(), dm,
                     stream) for s in range(total_steps)]
        step_bytes = ebytes + 2 * dm * 4
        launch_bytes = step_bytes

        def run_step(s):
            rc = fn(*all_args[s])
            if rc:
                mer.errors.raise_for_status(rc)

        def step_rows(s):
            return [[(xs[0], [s % E], np.ones(1, np.float32))]]

        experts_per_step = 1
        routing_desc = "none (one expert per step)"
    elif args.config == 3:
        T = cfg["tokens"]
        table = torch.tensor([[base + (l * E + e) * ebytes for e in range(E)] for l in range(L)],
                             dtype=torch.int64, device=dev)
        ids = np.zeros((total_steps, T, K), np.int32)
        wts = np.zeros((total_steps, T, K), np.float32)
        for s in range(total_steps):
            ids[s], wts[s] = routing.zipf_skewed_routes(T, E, K, 1.1, seed=args.seed + 2 + s)
        xs = rng_x.standard_normal((total_steps, T, dm)).astype(np.float32)
        ids_d = torch.from_numpy(ids).to(dev)
        wts_d = torch.from_numpy(wts).to(dev)
        xs_d = torch.from_numpy(xs).to(dev)
        outs = torch.zeros((total_steps, T, dm), dtype=torch.float32, device=dev)
        distinct = np.array([len(np.unique(ids[s])) for s in range(total_steps)])
        step_bytes_list = distinct * ebytes + 2 * T * dm * 4  # distinct experts' weights + x in + out
        fn = lib.mer_hip_moe_grouped
        all_args = [(dtype, dm, dff, T, K, table[s % L].data_ptr(), E, ids_d[s].data_ptr(), wts_d[s].data_ptr(),
                     xs_d[s].data_ptr(), outs[s].data_ptr(), 0, stream) for s in range(total_steps)]
        timed_u = distinct[args.warmup:]
        step_bytes = int(np.mean(step_bytes_list[args.warmup:]))
        launch_bytes = step_bytes

        def run_step(s):
            rc = fn(*all_args[s])
            if rc:
                mer.errors.raise_for_status(rc)

        def step_rows(s):
            return [[(xs[s, t], [(s % L) * E + int(e) for e in ids[s, t]], wts[s, t])] for t in range(T)]

        experts_per_step = T * K
        routing_desc = ("N(0,1) logits + ln p_zipf(rank; s=1.1) over a seeded rank permutation, softmax top-8 "
                        f"renormalised; distinct experts per step {timed_u.min()}..{timed_u.max()} "
                        f"(mean {timed_u.mean():.1f})")
    else:
        table = torch.tensor([[base + (l * E + e) * ebytes for e in range(E)] for l in range(L)],
                             dtype=torch.int64, device=dev)
        ids = np.zeros((total_steps, L, 1, K), np.int32)
        wts = np.zeros((total_steps, L, 1, K), np.float32)
        if args.config == 1:
            xs = rng_x.standard_normal((1, L, 1, dm)).astype(np.float32)   # one x_l per layer
            logits = rng_r.standard_normal((total_steps, L, E)).astype(np.float32)
            for s in range(total_steps):
                for l in range(L):
                    ids[s, l, 0], wts[s, l, 0] = routing.route_scores(logits[s, l], K)
            routing_desc = "N(0,1) logits per token and layer, softmax over the selected top-k"
        else:
            xs = rng_x.standard_normal((total_steps, L, 1, dm)).astype(np.float32)  # fresh hidden state per step
            gates = (rng_r.standard_normal((L, E, dm)) * 0.02).astype(np.float32)
            for s in range(total_steps):
                for l in range(L):
                    ids[s, l, 0], wts[s, l, 0] = routing.route_linear_gate(gates[l], xs[s, l, 0], K)
            routing_desc = "LinearGate [E x d_model] ~ N(0, 0.02) per layer on the step's hidden state (host)"
        ids_d = torch.from_numpy(ids).to(dev)
        wts_d = torch.from_numpy(wts).to(dev)
        xs_d = torch.from_numpy(xs).to(dev)
        outs = torch.zeros((total_steps, 1, dm), dtype=torch.float32, device=dev)
        x_of = (lambda s, l: xs[0, l, 0]) if args.config == 1 else (lambda s, l: xs[s, l, 0])
        xsel = (lambda s, l: xs_d[0, l]) if args.config == 1 else (lambda s, l: xs_d[s, l])
        per_layer_bytes = K * ebytes + 3 * dm * 4  # distinct routed experts + x in, out read + written
        step_bytes = L * per_layer_bytes
        flags = 2 | (8 if args.route_after_prev else 0)  # ACCUMULATE [| ROUTE_AFTER_PREV]
        if args.per_layer:
            fn = lib.mer_hip_moe_forward
            all_args = [[(dtype, dm, dff, 1, K, table[l].data_ptr(), E, ids_d[s, l].data_ptr(), wts_d[s, l].data_ptr(),
                          xsel(s, l).data_ptr(), outs[s].data_ptr(), 2, stream) for l in range(L)]
                        for s in range(total_steps)]
            launch_bytes = per_layer_bytes

            def run_step(s):
                for a in all_args[s]:
                    rc = fn(*a)
                    if rc:
                        mer.errors.raise_for_status(rc)
        else:
            fn = lib.mer_hip_moe_forward_layers

            def layer_array(s):
                arr = (mer._lib.MerLayerArgs * L)()
                for l in range(L):
                    arr[l] = mer._lib.MerLayerArgs(table[l].data_ptr(), E, ids_d[s, l].data_ptr(),
                                                   wts_d[s, l].data_ptr(), xsel(s, l).data_ptr(), outs[s].data_ptr())
                return arr

            all_args = [(dtype, dm, dff, L, 1, K, layer_array(s), flags, stream) for s in range(total_steps)]
            launch_bytes = step_bytes

            def run_step(s):
                rc = fn(*all_args[s])
                if rc:
                    mer.errors.raise_for_status(rc)

        def step_rows(s):
            return [[(x_of(s, l), [l * E + int(e) for e in ids[s, l, 0]], wts[s, l, 0]) for l in range(L)]]

        experts_per_step = L * K

    log("warmup")
    for s in range(args.warmup):
        run_step(s)
    torch.cuda.synchronize()
    mer.take_device_status()
    outs[args.warmup:].zero_()
    torch.cuda.synchronize()

    # The timed steps run with no per-launch events: events recorded around
    # every launch delay each dispatch (a one-expert launch measured 43.3 us
    # between its own events, against 40.3 us per launch back to back).  One
    # pair of HIP events on the launch stream brackets the timed region; the
    # per-launch stage events then run over a second pass of the same steps.
    log(f"timing {args.steps} steps")
    mer.stage_timing_enable(False)
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_a.record()
    for s in range(args.warmup, total_steps):
        run_step(s)
    ev_b.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    region_us = ev_a.elapsed_time(ev_b) * 1e3
    gpu_last = outs[total_steps - 1].cpu().numpy().copy()  # what the last timed launch wrote
    mer.stage_timing_enable(True)
    for s in range(args.warmup, total_steps):
        run_step(s)
    torch.cuda.synchronize()
    stages = mer.stage_timing_read()
    mer.stage_timing_enable(False)
    mer.take_device_status()
    elapsed = t1 - t0
    ms_per_step = elapsed * 1e3 / args.steps
    steps_per_s = args.steps / elapsed

    # Per-launch algorithmic bytes of each stage (packed weights of each
    # distinct expert touched + f32 activations in/out).
    proj = ebytes // 3
    if args.config == 3:
        u = float(np.mean(timed_u))
        n_pairs = cfg["tokens"] * K
        stage_bytes = {
            "prep": n_pairs * 8 + cfg["tokens"] * dm * 4 + cfg["tokens"] * dm // 32 * 100,
            "gate_up": int(u * 2 * proj) + cfg["tokens"] * dm // 32 * 100 + n_pairs * dff // 32 * 100,
            "down": int(u * proj) + n_pairs * dff // 32 * 100 + n_pairs * dm * 4,
            "combine": n_pairs * dm * 4 + cfg["tokens"] * dm * 4,
        }
    else:
        stage_bytes = {
            "decode": launch_bytes,  # the persistent decode kernel
            "gate_up": K * 2 * proj + dm // 32 * 100 + K * dff // 32 * 100,
            "down": K * proj + K * dff // 32 * 100 + K * 4 * dm * 4,
            "combine": K * 4 * dm * 4 + 2 * dm * 4,
            "prep": dm * 4 + dm // 32 * 100 + K * 12,
        }
    stage_info = {}
    for name, (ms, cnt) in stages.items():
        if cnt:
            avg = ms / cnt
            stage_info[name] = {"avg_us": avg * 1e3, "launches": cnt, "gbps": stage_bytes[name] / (avg * 1e-3) / 1e9}
    dominant = max(stage_info, key=lambda k: stage_info[k]["avg_us"] * stage_info[k]["launches"])
    dom = dict(stage_info[dominant])
    timing_note = "avg_launch_us from HIP events around the instrumented second pass, one pair per launch"
    if dominant == "decode":
        # one decode launch per step: the timed region's own events, per launch
        dom["avg_us"] = region_us / args.steps
        dom["gbps"] = launch_bytes / (dom["avg_us"] * 1e-6) / 1e9
        timing_note = ("avg_launch_us = HIP events around the timed region on the launch stream / launches "
                       "(launches back to back, no events between them)")

    config = {"workload": cfg["workload"], "layers": L, "experts_per_layer": E if args.config else 1,
              "top_k": K, "d_model": dm, "d_ff": dff, "weights": "Q4_0" if dtype == Q4 else "Q8_0",
              "batch": cfg.get("tokens", 1),
              "resident_bytes": n_exp * ebytes, "bytes_per_step": step_bytes, "parallelism": "single-gpu",
              "routing": routing_desc}
    if args.config == 3:
        config["launch"] = "mer_hip_moe_grouped per step (group, gate/up, down, combine)"
        config["layer_copies"] = "steps cycle over the 8 copies; each step reads one copy's routed experts"
    elif args.config:
        config["launch"] = "per-layer" if args.per_layer else "all-layers"
        config["routing_use"] = ("each layer's routing used only after the previous layer's output is complete"
                                 if args.per_layer or args.route_after_prev else
                                 "every layer's routing is a launch input")
    result = {
        "metric": cfg["metric"],
        "value": steps_per_s * cfg.get("tokens", 1),
        "unit": cfg["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_LABEL_GROUPED if args.config == 3 else DTYPE_LABEL[dtype],
        "data": "synthetic",
        "config": config,
        "hbm_gbps": step_bytes * steps_per_s / 1e9,  # algorithmic bytes per step x steps/s
        "hbm_frac_of_peak": step_bytes * steps_per_s / 1e9 / HBM_PEAK_GBPS,
        "roofline": {"bound": "hbm", "kernel": "decode_kernel" if dominant == "decode" else
                     (f"gproj_kernel ({dominant})" if args.config == 3 else f"proj_kernel ({dominant})"),
                     "achieved": dom["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": dom["gbps"] / HBM_PEAK_GBPS, "traffic": None,
                     "algorithmic_bytes_per_launch": stage_bytes[dominant], "avg_launch_us": dom["avg_us"],
                     "timing": timing_note},
        "stages": stage_info,
    }
    if args.config in (1, 2) and not args.per_layer and not args.route_after_prev and not args.no_route_after_prev_pass:
        # The same steps again with MER_MOE_ROUTE_AFTER_PREV: layer l reads its
        # routing and streams its experts only once layer l-1 is complete, as
        # a model whose routing is computed from that output must.
        all_rap = [(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7] | 8, a[8]) for a in all_args]
        torch.cuda.synchronize()
        r0 = time.perf_counter()
        ev_a.record()
        for s in range(args.warmup, total_steps):
            rc = fn(*all_rap[s])
            if rc:
                mer.errors.raise_for_status(rc)
        ev_b.record()
        torch.cuda.synchronize()
        r1 = time.perf_counter()
        mer.take_device_status()
        rap_us = ev_a.elapsed_time(ev_b) * 1e3 / args.steps
        result["route_after_prev"] = {
            "value": args.steps / (r1 - r0) * cfg.get("tokens", 1), "unit": cfg["unit"],
            "ms_per_step": (r1 - r0) * 1e3 / args.steps, "avg_launch_us": rap_us,
            "frac": launch_bytes / (rap_us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "note": "the same steps with MER_MOE_ROUTE_AFTER_PREV (routing known only after the previous layer)"}
    if args.config in (1, 2) and not args.per_layer and not args.route_after_prev and not args.no_route_after_prev_pass:
        # The same steps as one mer_hip_moe_forward call per layer, MER's own
        # call pattern (moe_step_inner's WeightedInto, engine.rs:5206,
        # :5548-5639): each call reads its layer's routing and input when the
        # stream reaches it, after the previous layer's call has finished.
        pl_fn = lib.mer_hip_moe_forward
        pl_args = [[(dtype, dm, dff, 1, K, table[l].data_ptr(), E, ids_d[s, l].data_ptr(), wts_d[s, l].data_ptr(),
                     xsel(s, l).data_ptr(), outs[s].data_ptr(), 2, stream) for l in range(L)]
                   for s in range(total_steps)]
        for s in range(args.warmup):
            for a in pl_args[s]:
                pl_fn(*a)
        torch.cuda.synchronize()
        p0 = time.perf_counter()
        ev_a.record()
        for s in range(args.warmup, total_steps):
            for a in pl_args[s]:
                rc = pl_fn(*a)
                if rc:
                    mer.errors.raise_for_status(rc)
        ev_b.record()
        torch.cuda.synchronize()
        p1 = time.perf_counter()
        mer.take_device_status()
        pl_us = ev_a.elapsed_time(ev_b) * 1e3 / (args.steps * L)
        pl_ms = (p1 - p0) * 1e3 / args.steps
        result["per_layer"] = {
            "value": args.steps / (p1 - p0) * cfg.get("tokens", 1), "unit": cfg["unit"],
            "ms_per_step": pl_ms, "launches_per_step": L, "avg_launch_us": pl_us,
            "frac": step_bytes / (pl_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "kernel_frac": per_layer_bytes / (pl_us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "note": "the same steps as one mer_hip_moe_forward per layer (MER's call pattern), launched back to "
                    "back; avg_launch_us = HIP events around the pass / launches; frac counts the whole step by "
                    "the host clock, kernel_frac the average launch"}
        if dtype == Q4 and not args.no_qmm_pass:
            # the engine's default: one call per layer, Q4_0 through QMatMul
            q_pl = [[a[:11] + (a[11] | 16,) + a[12:] for a in row] for row in pl_args]
            torch.cuda.synchronize()
            p0 = time.perf_counter()
            ev_a.record()
            for s in range(args.warmup, total_steps):
                for a in q_pl[s]:
                    rc = pl_fn(*a)
                    if rc:
                        mer.errors.raise_for_status(rc)
            ev_b.record()
            torch.cuda.synchronize()
            p1 = time.perf_counter()
            mer.take_device_status()
            q_us = ev_a.elapsed_time(ev_b) * 1e3 / (args.steps * L)
            result["per_layer"]["qmm"] = {
                "value": args.steps / (p1 - p0) * cfg.get("tokens", 1), "ms_per_step": (p1 - p0) * 1e3 / args.steps,
                "avg_launch_us": q_us, "kernel_frac": per_layer_bytes / (q_us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
                "note": "the same per-layer calls with MER_MOE_QMM (the engine's default Q4_0 arm)"}
    if dtype == Q4 and args.config in (0, 1) and not args.per_layer and not args.route_after_prev \
            and not args.no_qmm_pass:
        # The same steps with Candle's QMatMul arithmetic (MER_MOE_QMM): the
        # engine's default Q4_0 arm (use_qmm_for_q4, engine.rs:1144, :1825),
        # activations quantised to Q8_0 per block as QMatMul does.
        if args.config == 0:
            q_fn = lib.mer_hip_expert_forward_qmm
            q_args = [a[1:] for a in all_args]
        else:
            q_fn = fn
            q_args = [a[:7] + (a[7] | 16,) + a[8:] for a in all_args]
        outs.zero_()
        for s in range(args.warmup):
            q_fn(*q_args[s])
        torch.cuda.synchronize()
        q0 = time.perf_counter()
        ev_a.record()
        for s in range(args.warmup, total_steps):
            rc = q_fn(*q_args[s])
            if rc:
                mer.errors.raise_for_status(rc)
        ev_b.record()
        torch.cuda.synchronize()
        q1 = time.perf_counter()
        mer.take_device_status()
        q_us = ev_a.elapsed_time(ev_b) * 1e3 / args.steps
        result["qmm"] = {
            "value": args.steps / (q1 - q0) * cfg.get("tokens", 1), "unit": cfg["unit"],
            "ms_per_step": (q1 - q0) * 1e3 / args.steps, "avg_launch_us": q_us,
            "frac": launch_bytes / (q_us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "dtype": "q4_0 weights x Q8_0 activations (Candle QMatMul), int32 block dots, f32 accumulate",
            "note": "the same steps with MER_MOE_QMM: Q4_0 through Candle's QMatMul arithmetic, the reference "
                    "engine's default Q4_0 arm; avg_launch_us = HIP events around the pass / launches"}
        if not args.no_cpu_baseline:
            q_last = outs[total_steps - 1].cpu().numpy().copy()
            q_blobs = {}

            def q_blob(e):
                if e not in q_blobs:
                    q_blobs[e] = weights[e * ebytes:(e + 1) * ebytes].cpu().numpy()
                return q_blobs[e]

            result["qmm"].update(qmm_parity(dm, dff, step_rows(total_steps - 1), q_blob, q_last))
            q_blobs.clear()
    if args.config == 2:
        result["router"] = router_pass(gates, xs_d, ids, L, E, K, dm, args.warmup, min(5, args.steps))
    traffic = read_traffic(args.config) if dominant == "decode" and not args.per_layer else None
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
        what = ("the reference's q4_0_cpu_reference_forward (dequantise + f32 GEMV)" if dtype == Q4 else
                "the reference's forward_q8_0_direct_into AVX2 row kernels")
        host_blobs = {}

        def blob_of(e):
            if e not in host_blobs:
                host_blobs[e] = weights[e * ebytes:(e + 1) * ebytes].cpu().numpy()
            return host_blobs[e]

        steps = [step_rows(s) for s in range(total_steps - 1, args.warmup - 1, -1)]
        result["cpu_baseline"] = cpu_baseline(dtype, dm, dff, steps, blob_of, gpu_last, args.cpu_seconds,
                                              cfg.get("tokens", 1) if args.config else 1, cfg["unit"], what)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
