"""bench.py's command-line contract that needs no GPU: more than one GPU is
refused with a message (this build measures one GPU), before torch or the
HIP library is touched."""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env=env)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2", "--steps", "1")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="4")
    r = _bench("--steps", "1", env=env)
    assert r.returncode == 2
    assert "--gpus 1" in r.stderr


def test_cpu_baseline_checks_rows_and_reports_host(oracle):
    """bench.cpu_baseline on a two-layer step of two tiny Q4_0 experts: the
    rows it recomputes equal the oracle's slot-order combine summed over
    layers, so outputs equal to that score a worst ratio of 0 and perturbed
    ones exceed 1; the line names the host's CPUs and the threads used."""
    import numpy as np

    sys.path.insert(0, ROOT)
    import bench

    dm, dff = 64, 64
    nb = oracle.expert_weight_bytes(4, dm, dff) // 18
    blobs = {e: oracle.bench_fill(4, 3, e, 0, nb, 0.005, 0.02) for e in range(3)}
    rng = np.random.default_rng(0)
    xs = rng.standard_normal((2, dm)).astype(np.float32)
    w = [np.array([0.7, 0.3], np.float32), np.array([0.5, 0.5], np.float32)]
    step = [[(xs[0], [0, 1], w[0]), (xs[1], [2, 0], w[1])]]
    want = np.zeros(dm)
    for l, keys in enumerate(([0, 1], [2, 0])):
        ys = np.stack([oracle.q4_0_reference_forward(blobs[k], xs[l], dm, dff) for k in keys])
        want += oracle.combine_outputs(ys, w[l])
    r = bench.cpu_baseline(4, dm, dff, [step], blobs.__getitem__, want, 0.0, 1, "tokens/s", "q4 oracle")
    assert r["parity_worst_ratio"] < 1e-3
    assert r["cores"] >= 1 and r["host_cpus"] >= r["cores"] and r["affinity_cpus"] >= 1 and "cpu_model" in r
    bad = want + 0.05 * np.abs(want).max()
    assert bench.cpu_baseline(4, dm, dff, [step], blobs.__getitem__, bad, 0.0, 1, "tokens/s", "q4")[
        "parity_worst_ratio"] > 1.0


def test_qmm_parity_uses_the_flip_aware_bar(oracle):
    """bench.qmm_parity on a two-layer step of two tiny Q4_0 experts: the
    oracle's own QMatMul rows score 0, rows moved by more than the bar plus
    the flip bound score above 1."""
    import numpy as np

    sys.path.insert(0, ROOT)
    import bench

    dm, dff = 64, 96
    nb = oracle.expert_weight_bytes(4, dm, dff) // 18
    blobs = {e: oracle.bench_fill(4, 5, e, 0, nb, 0.005, 0.02) for e in range(3)}
    rng = np.random.default_rng(1)
    xs = rng.standard_normal((2, dm)).astype(np.float32)
    w = [np.array([0.7, 0.3], np.float32), np.array([0.5, 0.5], np.float32)]
    step = [[(xs[0], [0, 1], w[0]), (xs[1], [2, 0], w[1])]]
    want = np.zeros(dm)
    for l, keys in enumerate(([0, 1], [2, 0])):
        ys = np.stack([oracle.q4_0_qmm_forward(blobs[k], xs[l], dm, dff) for k in keys])
        want += oracle.combine_outputs(ys, w[l])
    r = bench.qmm_parity(dm, dff, step, blobs.__getitem__, want)
    assert r["parity_worst_ratio"] < 1e-3 and r["rows_beyond_ffn_bar"] == 0
    bad = want + 0.5 * np.abs(want).max() + 1.0
    assert bench.qmm_parity(dm, dff, step, blobs.__getitem__, bad)["parity_worst_ratio"] > 1.0
