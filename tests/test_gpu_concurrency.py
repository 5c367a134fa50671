"""Re-entrancy of the C ABI and HIP-graph replay of the decode kernel.

The reference runs its expert kernels from parallel workers and lets the
GPU backend run up to four dispatches at once, each with a workspace of its
own (engine.rs:985-993, backend/mod.rs:1346-1432, :2685-2697); its CPU
kernels are pinned as re-entrant on one resident expert
(inference.rs:6247-6277).  Here four host threads drive four streams
through the C ABI at once, on the same resident experts; every output must
be bit-identical to the serial run of the same call (scheduling never
changes a sum's order) and within the 1e-3 bar of the oracle.  Four
full-grid persistent decode launches on four streams cannot all be
resident at once: the library orders every decode launch of the device
after the previous one, whatever its stream, so these cases also check
that no two persistent grids stall each other.
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from test_gpu_parity import Q4, Q8, _oracle_moe, _table, assert_ffn_close, make_expert, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu

N_WORKERS = 4
ITERS = 6


def _worker_inputs(n_exp, n_tok, k, dm, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    return ids, w, x


def _run_threads(fns):
    errors = []

    def wrap(fn):
        try:
            fn()
        except BaseException as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=wrap, args=(f,)) for f in fns]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    if errors:
        raise errors[0]


@pytest.mark.parametrize("dtype,dm,dff,n_tok", [(Q4, 1024, 2048, 1), (Q8, 2048, 768, 2), (Q4, 96, 160, 2)])
def test_concurrent_moe_forward_on_four_streams(mer, oracle, gpu, dtype, dm, dff, n_tok):
    """mer_hip_moe_forward from 4 threads on 4 streams (decode kernel, and
    the generic path for the unaligned shape)."""
    say(f"concurrent moe_forward dtype={dtype} dm={dm} dff={dff} n_tok={n_tok}")
    n_exp, k = 6, 2
    blobs = [make_expert(oracle, dtype, dm, dff, e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    lib = mer._lib.lib()
    inputs = [_worker_inputs(n_exp, n_tok, k, dm, 100 + i) for i in range(N_WORKERS)]
    dev_in = [tuple(to_dev(a, gpu) for a in inp) for inp in inputs]
    # serial reference on the default stream
    serial = []
    for ids, w, x in dev_in:
        serial.append(mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, ids, w, x).cpu().numpy())
    torch.cuda.synchronize()
    for i, (ids, w, x) in enumerate(inputs):
        assert_ffn_close(serial[i], _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff), f"serial worker {i}")

    # worker 0 runs on the stream of the serial calls, the others on new
    # streams; the library orders their decode launches on the GPU
    streams = [torch.cuda.current_stream(gpu)] + [torch.cuda.Stream(device=gpu) for _ in range(N_WORKERS - 1)]
    outs = [[torch.full((n_tok, dm), float("nan"), device=gpu) for _ in range(ITERS)] for _ in range(N_WORKERS)]
    torch.cuda.synchronize()

    def worker(i):
        ids, w, x = dev_in[i]
        s = streams[i].cuda_stream

        def run():
            for it in range(ITERS):
                rc = lib.mer_hip_moe_forward(dtype, dm, dff, n_tok, k, table.data_ptr(), n_exp, ids.data_ptr(),
                                             w.data_ptr(), x.data_ptr(), outs[i][it].data_ptr(), 0, s)
                assert rc == 0, mer._lib.last_error()
        return run

    _run_threads([worker(i) for i in range(N_WORKERS)])
    for s in streams:
        s.synchronize()
    mer.take_device_status()
    for i in range(N_WORKERS):
        for it in range(ITERS):
            got = outs[i][it].cpu().numpy()
            assert np.array_equal(got, serial[i]), f"worker {i} iteration {it} differs from the serial run"
    for s in streams[1:]:
        mer.stream_release(s)


def test_concurrent_expert_forward_same_resident(mer, oracle, gpu):
    """mer_hip_expert_forward on ONE resident Q8_0 expert from 4 threads,
    each on its own stream, with different inputs (inference.rs:6247-6277)."""
    say("concurrent expert_forward on one resident expert")
    dm, dff = 512, 1024
    blob = make_expert(oracle, Q8, dm, dff, 3)
    dblob = to_dev(blob, gpu)
    lib = mer._lib.lib()
    xs = [np.random.default_rng(7 + i).standard_normal(dm).astype(np.float32) for i in range(N_WORKERS)]
    dxs = [to_dev(x, gpu) for x in xs]
    serial = [mer.dispatch_expert_forward(mer.WeightDtype.Q8_0, dblob, dx, dm, dff).cpu().numpy() for dx in dxs]
    for i in range(N_WORKERS):
        rc, want = oracle.q8_0_direct_forward(blob, xs[i], dm, dff)
        assert rc == 0
        assert_ffn_close(serial[i], want, f"serial {i}")
    streams = [torch.cuda.Stream(device=gpu) for _ in range(N_WORKERS)]
    outs = [[torch.empty(dm, device=gpu) for _ in range(ITERS)] for _ in range(N_WORKERS)]
    torch.cuda.synchronize()

    def worker(i):
        def run():
            for it in range(ITERS):
                rc = lib.mer_hip_expert_forward(Q8, dblob.data_ptr(), dblob.numel(), dxs[i].data_ptr(), dm, dm, dff,
                                                outs[i][it].data_ptr(), dm, streams[i].cuda_stream)
                assert rc == 0, mer._lib.last_error()
        return run

    _run_threads([worker(i) for i in range(N_WORKERS)])
    torch.cuda.synchronize()
    for i in range(N_WORKERS):
        for it in range(ITERS):
            assert np.array_equal(outs[i][it].cpu().numpy(), serial[i]), f"worker {i} iteration {it}"
    for s in streams:
        mer.stream_release(s)


def test_concurrent_layers_and_one_shared_stream(mer, oracle, gpu):
    """Two threads run 3-layer mer_hip_moe_forward_layers launches on two
    streams while two more threads share a third stream (serialised by the
    stream's workspace lock, ordered by the stream)."""
    say("concurrent moe_forward_layers + shared stream")
    dm, dff, n_layers, n_exp, k = 512, 1024, 3, 4, 2
    blobs = [[make_expert(oracle, Q4, dm, dff, l * n_exp + e) for e in range(n_exp)] for l in range(n_layers)]
    tables = [_table(b, gpu) for b in blobs]
    lib = mer._lib.lib()
    n_jobs = 4
    jobs = []
    for j in range(n_jobs):
        rng = np.random.default_rng(40 + j)
        ids = [np.stack([rng.choice(n_exp, k, replace=False)]).astype(np.int32) for _ in range(n_layers)]
        ws = [rng.random((1, k)).astype(np.float32) for _ in range(n_layers)]
        xs = [rng.standard_normal((1, dm)).astype(np.float32) for _ in range(n_layers)]
        want = np.zeros((1, dm), np.float32)
        for l in range(n_layers):  # accumulate: out += sum_i w_i y_i per layer
            want = want + _oracle_moe(oracle, Q4, blobs[l], ids[l], ws[l], xs[l], dm, dff)
        jobs.append(dict(ids=[to_dev(a, gpu) for a in ids], ws=[to_dev(a, gpu) for a in ws],
                         xs=[to_dev(a, gpu) for a in xs], want=want))

    def layer_args(j, out):
        arr = (mer._lib.MerLayerArgs * n_layers)()
        for l in range(n_layers):
            arr[l] = mer._lib.MerLayerArgs(tables[l][1].data_ptr(), n_exp, jobs[j]["ids"][l].data_ptr(),
                                           jobs[j]["ws"][l].data_ptr(), jobs[j]["xs"][l].data_ptr(), out.data_ptr())
        return arr

    outs = [[torch.zeros((1, dm), device=gpu) for _ in range(ITERS)] for _ in range(n_jobs)]
    args = [[layer_args(j, outs[j][it]) for it in range(ITERS)] for j in range(n_jobs)]
    streams = [torch.cuda.Stream(device=gpu) for _ in range(3)]
    stream_of = [0, 1, 2, 2]
    torch.cuda.synchronize()

    def worker(j):
        def run():
            s = streams[stream_of[j]].cuda_stream
            for it in range(ITERS):
                rc = lib.mer_hip_moe_forward_layers(Q4, dm, dff, n_layers, 1, k, args[j][it], 2, s)
                assert rc == 0, mer._lib.last_error()
        return run

    _run_threads([worker(j) for j in range(n_jobs)])
    torch.cuda.synchronize()
    mer.take_device_status()
    for j in range(n_jobs):
        first = outs[j][0].cpu().numpy()
        assert_ffn_close(first, jobs[j]["want"], f"job {j}")
        for it in range(1, ITERS):
            assert np.array_equal(outs[j][it].cpu().numpy(), first), f"job {j} iteration {it}"
    for s in streams:
        mer.stream_release(s)


def test_decode_graph_replay(mer, oracle, gpu):
    """A captured mer_hip_moe_forward_layers launch replays correctly: each
    replay runs with a fresh epoch from device memory, so release flags and
    digit lines of the previous replay are never taken as current.  New
    inputs are copied in between replays (eager work + synchronisation), and
    every replay is checked against an eager launch on the same inputs."""
    say("decode graph replay")
    dm, dff, n_layers, n_exp, k = 512, 1024, 2, 4, 2
    blobs = [[make_expert(oracle, Q4, dm, dff, 50 + l * n_exp + e) for e in range(n_exp)] for l in range(n_layers)]
    tables = [_table(b, gpu) for b in blobs]
    ids = [torch.zeros((1, k), dtype=torch.int32, device=gpu) for _ in range(n_layers)]
    ws = [torch.zeros((1, k), device=gpu) for _ in range(n_layers)]
    xs = [torch.zeros((1, dm), device=gpu) for _ in range(n_layers)]
    outs = [torch.zeros((1, dm), device=gpu) for _ in range(n_layers)]
    layers = [dict(table=tables[l][1], ids=ids[l], weights=ws[l], x=xs[l], out=outs[l]) for l in range(n_layers)]

    def load(seed):
        rng = np.random.default_rng(seed)
        for l in range(n_layers):
            ids[l].copy_(torch.from_numpy(rng.choice(n_exp, k, replace=False).astype(np.int32).reshape(1, k)))
            ws[l].copy_(torch.from_numpy(rng.random((1, k)).astype(np.float32)))
            xs[l].copy_(torch.from_numpy(rng.standard_normal((1, dm)).astype(np.float32)))

    s = torch.cuda.Stream(device=gpu)
    with torch.cuda.stream(s):
        load(1)
        mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers)  # grows the workspace before capture
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers)
    for rep in range(4):
        load(10 + rep)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [o.cpu().numpy().copy() for o in outs]
        with torch.cuda.stream(s):
            mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers)  # eager, same inputs
        s.synchronize()
        for l in range(n_layers):
            assert np.array_equal(got[l], outs[l].cpu().numpy()), f"replay {rep} layer {l} differs from eager"
        if rep == 0:
            for l in range(n_layers):
                want = _oracle_moe(oracle, Q4, blobs[l], ids[l].cpu().numpy(), ws[l].cpu().numpy(),
                                   xs[l].cpu().numpy(), dm, dff)
                assert_ffn_close(got[l], want, f"replay 0 layer {l}")
    mer.take_device_status()
    del g
    mer.stream_release(s)


def test_decode_beside_busy_device(mer, oracle, gpu):
    """Decode launches while ordinary kernels keep the device busy from
    another stream (large matrix products, as an engine's attention would):
    the persistent grid shares the CUs with them, gets its remaining
    workgroups as they finish, and every output matches the serial run.
    (No kernel of the caller spin-waits here: beside such kernels the
    library makes no progress guarantee.)"""
    say("decode beside a busy device")
    dm, dff, n_layers, n_exp, k = 1024, 2048, 4, 6, 2
    blobs = [[make_expert(oracle, Q4, dm, dff, 900 + l * n_exp + e) for e in range(n_exp)] for l in range(n_layers)]
    tables = [_table(b, gpu) for b in blobs]
    rng = np.random.default_rng(31)
    ids = [to_dev(np.stack([rng.choice(n_exp, k, replace=False)]).astype(np.int32), gpu) for _ in range(n_layers)]
    ws = [to_dev(rng.random((1, k)).astype(np.float32), gpu) for _ in range(n_layers)]
    xs = [to_dev(rng.standard_normal((1, dm)).astype(np.float32), gpu) for _ in range(n_layers)]

    def layers(out):
        return [dict(table=tables[l][1], ids=ids[l], weights=ws[l], x=xs[l], out=out) for l in range(n_layers)]

    ref = torch.zeros((1, dm), device=gpu)
    mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers(ref))
    torch.cuda.synchronize()
    busy = torch.cuda.Stream(device=gpu)
    mine = torch.cuda.Stream(device=gpu)
    a = torch.randn((4096, 4096), device=gpu)
    outs = [torch.zeros((1, dm), device=gpu) for _ in range(8)]
    with torch.cuda.stream(busy):
        for _ in range(20):
            a = torch.tanh(a @ a.T * 1e-3)
    with torch.cuda.stream(mine):
        for o in outs:
            mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers(o))
    torch.cuda.synchronize()
    mer.take_device_status()  # raises if a decode wait timed out
    want = ref.cpu().numpy()
    for i, o in enumerate(outs):
        assert np.array_equal(o.cpu().numpy(), want), f"launch {i} beside the busy stream"
    assert torch.isfinite(a).all()
    mer.stream_release(mine)
