"""Parity of the grouped multi-token path (mer_hip_moe_grouped: pairs
grouped by expert, int8 MFMA over token tiles) against the CPU oracle, run
pair by pair and combined in slot order.  Bar: the north-star 1e-3
abs/rel, in the same combined form as the other FFN parity tests."""
from __future__ import annotations

import importlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from test_gpu_parity import Q4, Q8, _table, assert_ffn_close, make_expert, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu

routing = importlib.import_module("micro-expert-router-ssd-streamed-moe-mer_amd.routing")


def oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff, table_ok=None):
    n_tok, k = ids.shape
    want = np.zeros((n_tok, dm), np.float32)
    cache = {}
    for t in range(n_tok):
        ys, ws = [], []
        for i in range(k):
            e = int(ids[t, i])
            if w[t, i] == 0.0 or e < 0 or e >= len(blobs) or (table_ok is not None and not table_ok[e]):
                continue
            key = (t, e)
            if key not in cache:
                if dtype == Q4:
                    cache[key] = oracle.q4_0_reference_forward(blobs[e], x[t], dm, dff)
                else:
                    cache[key] = oracle.q8_0_direct_forward(blobs[e], x[t], dm, dff)[1]
            ys.append(cache[key])
            ws.append(w[t, i])
        if ys:
            want[t] = oracle.combine_outputs(np.stack(ys), np.array(ws, np.float32))
    return want


@pytest.mark.parametrize("dtype,dm,dff,n_exp,n_tok,k", [
    (Q8, 256, 192, 6, 40, 3),     # popular experts span several 16-pair tiles
    (Q4, 256, 192, 6, 40, 3),
    (Q8, 128, 64, 3, 1, 2),       # one token
    (Q4, 512, 1024, 16, 24, 4),   # gate/up K over two LDS stages
    (Q8, 192, 128, 5, 20, 2),     # d_model % 128 != 0: 64-row down workgroups
    (Q4, 320, 64, 4, 9, 3),       # the same for Q4_0, one h block per pair
    (Q4, 128, 128, 16, 256, 8),   # 2048 pairs: 128-row gate/up workgroups
    (Q8, 256, 192, 12, 300, 7),   # 2100 pairs, the same for Q8_0
])
def test_grouped_vs_oracle(mer, oracle, gpu, dtype, dm, dff, n_exp, n_tok, k):
    say(f"grouped dtype={dtype} dm={dm} dff={dff} experts={n_exp} tokens={n_tok} k={k}")
    blobs = [make_expert(oracle, dtype, dm, dff, e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids, w = routing.zipf_skewed_routes(n_tok, n_exp, k, 1.1, seed=5)
    if n_tok > 3:
        w[2, 1] = 0.0  # zero-weight slot: skipped (engine.rs:5575-5580)
        ids[3, 1] = ids[3, 0]  # the same expert twice for one token
    x = np.random.default_rng(7).standard_normal((n_tok, dm)).astype(np.float32)
    want = oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
    args = (mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu))
    got = mer.moe_grouped(*args).cpu().numpy()
    assert_ffn_close(got, want, "grouped")
    got_r = mer.moe_grouped(*args, residual=True).cpu().numpy()
    assert_ffn_close(got_r, want + x, "grouped residual")
    out = to_dev(np.full((n_tok, dm), 0.5, np.float32), gpu)
    mer.moe_grouped(*args, out=out, accumulate=True)
    assert_ffn_close(out.cpu().numpy(), want + 0.5, "grouped accumulate")
    # repeatable bit for bit
    assert np.array_equal(mer.moe_grouped(*args).cpu().numpy(), got)
    mer.take_device_status()
    del devs


def test_grouped_qwen3_batch_config(mer, oracle, gpu):
    """The batched grouped-expert workload at full size: 64 tokens, 128
    Qwen3-shaped Q8_0 experts, top-8, Zipf(1.1) popularity."""
    dm, dff, n_exp, n_tok, k = 2048, 768, 128, 64, 8
    say("grouped qwen3 64 tokens x 128 experts top-8")
    blobs = [make_expert(oracle, Q8, dm, dff, e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids, w = routing.zipf_skewed_routes(n_tok, n_exp, k, 1.1, seed=3)
    counts = np.bincount(ids.ravel(), minlength=n_exp)
    assert counts.max() > 16  # at least one expert spans several token tiles
    x = np.random.default_rng(9).standard_normal((n_tok, dm)).astype(np.float32)
    want = oracle_moe(oracle, Q8, blobs, ids, w, x, dm, dff)
    got = mer.moe_grouped(mer.WeightDtype.Q8_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu)).cpu().numpy()
    assert_ffn_close(got, want, "grouped qwen3")
    # the decode path agrees on the same batch
    dec = mer.moe_forward(mer.WeightDtype.Q8_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu)).cpu().numpy()
    assert_ffn_close(got, dec, "grouped vs decode")
    mer.take_device_status()
    del devs


@pytest.mark.parametrize("name,dm,dff,n_exp,n_tok,k", [
    ("mixtral", 4096, 14336, 8, 12, 2),    # Mixtral-shape Q4_0 prefill chunk
    ("deepseek", 7168, 2048, 16, 16, 8),   # DeepSeek-V3 routed-expert shape
])
def test_grouped_q4_model_shapes(mer, oracle, gpu, name, dm, dff, n_exp, n_tok, k):
    """The grouped path at the Q4_0 model shapes of the decode configs, with
    residual: K of 4096 and 7168 (16 and 28 gate/up stages, 56 and 16 down
    stages), more pairs per expert than one 16-pair tile for the popular
    ones, and the decode path on the same batch as a second opinion."""
    say(f"grouped {name} Q4_0 {n_tok} tokens x {n_exp} experts top-{k}")
    blobs = [make_expert(oracle, Q4, dm, dff, 40 + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids, w = routing.zipf_skewed_routes(n_tok, n_exp, k, 1.0, seed=11)
    x = np.random.default_rng(21).standard_normal((n_tok, dm)).astype(np.float32)
    want = oracle_moe(oracle, Q4, blobs, ids, w, x, dm, dff) + x
    got = mer.moe_grouped(mer.WeightDtype.Q4_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu), residual=True).cpu().numpy()
    assert_ffn_close(got, want, f"grouped {name}")
    dec = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu), residual=True).cpu().numpy()
    assert_ffn_close(got, dec, f"grouped vs decode {name}")
    mer.take_device_status()
    del devs


def test_grouped_missing_expert_records_residency_miss(mer, oracle, gpu):
    dm, dff = 128, 128
    say("grouped missing expert")
    blobs = [make_expert(oracle, Q8, dm, dff, e) for e in range(3)]
    devs, table = _table(blobs, gpu)
    table[1] = 0  # expert 1 not resident
    ids = np.array([[0, 1], [2, 9], [1, 0]], np.int32)  # 9 is outside the table
    w = np.array([[0.5, 0.5], [0.25, 0.75], [0.0, 1.0]], np.float32)  # [2,0]: zero weight, no miss
    x = np.random.default_rng(1).standard_normal((3, dm)).astype(np.float32)
    got = mer.moe_grouped(mer.WeightDtype.Q8_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu)).cpu().numpy()
    want = oracle_moe(oracle, Q8, blobs, ids, w, x, dm, dff, table_ok=[True, False, True])
    assert_ffn_close(got, want, "grouped with misses")
    with pytest.raises(mer.GpuExpertDispatchError) as e:
        mer.take_device_status()
    assert e.value.kind == mer.GpuExpertDispatchErrorKind.ResidencyMiss
    del devs


def test_grouped_rejects_unsupported_shapes(mer, oracle, gpu):
    say("grouped shape errors")
    blobs = [make_expert(oracle, Q8, 96, 128, 0)]
    devs, table = _table(blobs, gpu)
    ids = torch.zeros((2, 1), dtype=torch.int32, device=gpu)
    w = torch.ones((2, 1), dtype=torch.float32, device=gpu)
    x = torch.zeros((2, 96), dtype=torch.float32, device=gpu)
    with pytest.raises(mer.ExpertWeightsError):
        mer.moe_grouped(mer.WeightDtype.Q8_0, 96, 128, table, ids, w, x)  # d_model not a multiple of 64
    big = torch.zeros((5000, 1), dtype=torch.int32, device=gpu)
    with pytest.raises(mer.RoutedExpertGpuIncompatibility):  # more than 4096 routed pairs
        mer.moe_grouped(mer.WeightDtype.Q8_0, 128, 128, table, big, big.float(),
                        torch.zeros((5000, 128), device=gpu))
    del devs
