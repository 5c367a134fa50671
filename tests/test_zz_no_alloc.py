"""mer_hip_moe_forward_noalloc (the entry point for callers that cannot
allocate) against mer_hip_moe_forward, through the C ABI: the same decode
kernel on a static scratch array instead of a workspace, so outputs must be
bit-identical.  Calls in a row with different shapes, the later ones
smaller, reuse the array that keeps the previous call's contents."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from test_gpu_parity import Q4, Q8, _oracle_moe, _table, assert_ffn_close, make_expert, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu


def _call(mer, name, dtype, dm, dff, table, n_exp, ids, w, x, out, flags, stream=None):
    lib = mer._lib.lib()
    n_tok, k = ids.shape
    st = (stream or torch.cuda.current_stream()).cuda_stream
    return getattr(lib, name)(dtype, dm, dff, n_tok, k, table.data_ptr(), n_exp, ids.data_ptr(), w.data_ptr(),
                              x.data_ptr(), out.data_ptr(), flags, st)


def test_noalloc_matches_moe_forward(mer, oracle, gpu):
    cases = [(Q4, 1024, 2048, 4, 2, 2), (Q8, 2048, 768, 1, 8, 0), (Q4, 512, 1024, 1, 1, 1), (Q4, 1024, 2048, 2, 2, 0)]
    for i, (dtype, dm, dff, n_tok, k, flags) in enumerate(cases):
        say(f"noalloc call {i}: dtype={dtype} dm={dm} dff={dff} n_tok={n_tok} k={k} flags={flags}")
        n_exp = max(k, 4)
        blobs = [make_expert(oracle, dtype, dm, dff, 300 + e) for e in range(n_exp)]
        devs, table = _table(blobs, gpu)
        rng = np.random.default_rng(70 + i)
        ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
        w = rng.random((n_tok, k)).astype(np.float32)
        x = rng.standard_normal((n_tok, dm)).astype(np.float32)
        base = rng.standard_normal((n_tok, dm)).astype(np.float32)
        ids_d, w_d, x_d = to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu)
        ref = to_dev(base, gpu)
        got = to_dev(base, gpu)
        assert _call(mer, "mer_hip_moe_forward", dtype, dm, dff, table, n_exp, ids_d, w_d, x_d, ref, flags) == 0
        assert _call(mer, "mer_hip_moe_forward_noalloc", dtype, dm, dff, table, n_exp, ids_d, w_d, x_d, got,
                     flags) == 0, mer._lib.last_error()
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), f"call {i} differs from mer_hip_moe_forward"
        want = _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
        if flags == 1:
            want = want + x
        elif flags == 2:
            want = want + base
        assert_ffn_close(got.cpu().numpy(), want, f"call {i}")
        mer.take_device_status()
        del devs


def test_noalloc_rejects_oversized_and_unaligned(mer, oracle, gpu):
    say("noalloc limits")
    lib = mer._lib.lib()
    dummy = torch.zeros(16, dtype=torch.int64, device=gpu)
    # 64 Mixtral-shape tokens x top-2 need ~15 MiB of scratch (> 8 MiB)
    rc = lib.mer_hip_moe_forward_noalloc(Q4, 4096, 14336, 64, 2, dummy.data_ptr(), 16, dummy.data_ptr(),
                                         dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), 0, 0)
    assert rc == 33 and "static scratch" in mer._lib.last_error()[1]
    rc = lib.mer_hip_moe_forward_noalloc(Q4, 96, 160, 1, 1, dummy.data_ptr(), 16, dummy.data_ptr(),
                                         dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), 0, 0)
    assert rc == 4 and "multiples of 64" in mer._lib.last_error()[1]


def test_noalloc_two_streams_back_to_back(mer, oracle, gpu):
    """Two streams issue no-alloc calls back to back with no host
    synchronisation in between, on different inputs and shapes: the calls
    share the GPU's one scratch array, and the library orders every decode
    launch of a device after the previous one, so each output must equal
    mer_hip_moe_forward's bit for bit."""
    say("noalloc on two streams")
    cases = [(Q4, 1024, 2048, 2, 2), (Q4, 512, 1024, 1, 2)]
    runs = []
    for i, (dtype, dm, dff, n_tok, k) in enumerate(cases):
        n_exp = 4
        blobs = [make_expert(oracle, dtype, dm, dff, 400 + 10 * i + e) for e in range(n_exp)]
        devs, table = _table(blobs, gpu)
        calls = []
        for c in range(3):
            rng = np.random.default_rng(90 + 10 * i + c)
            ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
            w = rng.random((n_tok, k)).astype(np.float32)
            x = rng.standard_normal((n_tok, dm)).astype(np.float32)
            ids_d, w_d, x_d = to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu)
            ref = torch.zeros((n_tok, dm), device=gpu)
            assert _call(mer, "mer_hip_moe_forward", dtype, dm, dff, table, n_exp, ids_d, w_d, x_d, ref, 0) == 0
            calls.append((ids_d, w_d, x_d, ref, torch.full((n_tok, dm), float("nan"), device=gpu)))
        runs.append((dtype, dm, dff, n_exp, devs, table, calls))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=gpu) for _ in range(2)]
    for c in range(3):  # interleave: stream 0 runs case 0, stream 1 case 1, no host sync
        for s_idx, (dtype, dm, dff, n_exp, devs, table, calls) in enumerate(runs):
            ids_d, w_d, x_d, ref, got = calls[c]
            rc = _call(mer, "mer_hip_moe_forward_noalloc", dtype, dm, dff, table, n_exp, ids_d, w_d, x_d, got, 0,
                       stream=streams[s_idx])
            assert rc == 0, mer._lib.last_error()
    torch.cuda.synchronize()
    for s_idx, (dtype, dm, dff, n_exp, devs, table, calls) in enumerate(runs):
        for c, (_, _, _, ref, got) in enumerate(calls):
            assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), f"stream {s_idx} call {c}"
    mer.take_device_status()
    for s in streams:
        mer.stream_release(s)
