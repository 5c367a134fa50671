"""The LinearGate router on the GPU (mer_hip_route_linear_gate) against the
oracle's restatement of gating.rs:395-476 and the reference's own known
answers.  Logits are f32 dot products in a different summation order, so
they are compared within f32 rounding; the selection is checked exactly by
running the oracle's scoring and top-k on the GPU's own logits."""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def routing(mer):
    import importlib

    return importlib.import_module(mer.__name__ + ".routing")


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu)


def test_router_reference_known_answers(mer, gpu):
    r = routing(mer)
    g = GOLDEN["gate_routing_surface_known_answers"]
    for c in g["cases"]:
        say(f"router known answer {c['name']}")
        w = np.eye(c["n"], dtype=np.float32)
        bias = None if c["bias"] is None else dev(c["bias"], gpu)
        ids, ws = r.route_linear_gate_gpu(dev(w, gpu), dev(np.array([c["x"]], np.float32), gpu), c["top_k"],
                                          sigmoid=c["sigmoid"], normalise=c["normalise"], bias=bias,
                                          n_group=c["n_group"], topk_group=c["topk_group"], scaling=c["scaling"])
        ids, ws = ids.cpu().numpy()[0], ws.cpu().numpy()[0]
        if "experts" in c:
            assert list(ids) == c["experts"], c["name"]
        if "weights" in c:
            assert np.allclose(ws, c["weights"], atol=c["weight_tol"]), c["name"]
        if "weight_sum" in c:
            assert abs(float(ws.sum()) - c["weight_sum"]) < c["weight_tol"], c["name"]
        if "experts_min" in c:
            assert (ids >= c["experts_min"]).all() and len(ids) == c["count"], c["name"]
    t = g["ties"]
    ids, ws = r.route_linear_gate_gpu(torch.zeros((t["num_experts"], t["d_model"]), device=gpu),
                                      dev(np.array([t["x"]], np.float32), gpu), t["top_k"])
    assert list(ids.cpu().numpy()[0]) == t["experts"]
    assert np.allclose(ws.cpu().numpy(), t["weight"], atol=1e-6)


ROUTER_CASES = [
    # (n_experts, d_model, top_k, options, n_tokens); logits run in groups of 4 tokens,
    # with 16-byte loads when d_model % 4 == 0 and scalar loads otherwise
    (8, 64, 2, {}, 3),
    (128, 2048, 8, {}, 3),
    (128, 2048, 8, {}, 37),
    (256, 7168, 8, dict(sigmoid=True, bias=True, n_group=8, topk_group=4, scaling=2.5), 3),
    (160, 1000, 6, dict(sigmoid=True, normalise=False), 3),
    (1024, 512, 64, {}, 3),
    (64, 96, 4, dict(bias=True), 3),
    (48, 99, 3, {}, 6),
]


@pytest.mark.parametrize("n_experts,d_model,top_k,opts,n_tok", ROUTER_CASES)
def test_router_matches_oracle(mer, oracle, gpu, n_experts, d_model, top_k, opts, n_tok):
    say(f"router E={n_experts} dm={d_model} k={top_k} {opts} tokens={n_tok}")
    r = routing(mer)
    rng = np.random.default_rng(n_experts * 31 + d_model)
    w = (rng.standard_normal((n_experts, d_model)) * 0.02).astype(np.float32)
    x = rng.standard_normal((n_tok, d_model)).astype(np.float32)
    o = dict(opts)
    bias = (rng.standard_normal(n_experts) * 0.1).astype(np.float32) if o.pop("bias", False) else None
    ids, ws, lg = r.route_linear_gate_gpu(dev(w, gpu), dev(x, gpu), top_k, bias=None if bias is None else dev(bias, gpu),
                                          return_logits=True, **o)
    ids, ws, lg = ids.cpu().numpy(), ws.cpu().numpy(), lg.cpu().numpy()
    for t in range(n_tok):
        _, _, lo = oracle.linear_gate_route_ex(w, x[t], top_k, bias=bias, **o)
        scale = np.abs(w).astype(np.float64) @ np.abs(x[t]).astype(np.float64)
        assert (np.abs(lg[t].astype(np.float64) - lo) <= 1e-5 * scale + 1e-7).all(), f"logits token {t}"
        want_ids, want_ws = oracle.gate_route_ex(lg[t], top_k, bias=bias, **o)
        assert list(ids[t][:len(want_ids)]) == list(want_ids), f"ids token {t}"
        assert (ids[t][len(want_ids):] == -1).all()
        assert np.allclose(ws[t][:len(want_ws)], want_ws, rtol=1e-5, atol=1e-7), f"weights token {t}"


def test_router_misaligned_input_takes_scalar_loads(mer, oracle, gpu):
    """x one float past a 16-byte boundary (a valid contiguous view) routes
    exactly as the aligned copy does, without logits requested."""
    say("router misaligned x")
    r = routing(mer)
    rng = np.random.default_rng(3)
    w = dev((rng.standard_normal((128, 2048)) * 0.02).astype(np.float32), gpu)
    x = rng.standard_normal((5, 2048)).astype(np.float32)
    flat = dev(np.concatenate([np.zeros(1, np.float32), x.ravel()]), gpu)
    xm = flat[1:].view(5, 2048)
    assert xm.data_ptr() % 16 != 0
    ids_m, ws_m = r.route_linear_gate_gpu(w, xm, 8)
    ids_a, ws_a = r.route_linear_gate_gpu(w, dev(x, gpu), 8)
    assert torch.equal(ids_m, ids_a)
    assert np.allclose(ws_m.cpu().numpy(), ws_a.cpu().numpy(), rtol=1e-5, atol=1e-7)


def test_router_nonfinite_row_is_uniform(mer, gpu):
    """A NaN logit makes softmax_inplace fall back to the uniform row
    (transformer.rs:2807-2819): the top-k are then the lowest ids."""
    say("router NaN row")
    r = routing(mer)
    w = np.ones((16, 8), np.float32)
    x = np.full((1, 8), np.nan, np.float32)
    ids, ws = r.route_linear_gate_gpu(dev(w, gpu), dev(x, gpu), 4)
    assert list(ids.cpu().numpy()[0]) == [0, 1, 2, 3]
    assert np.allclose(ws.cpu().numpy(), 0.25)


def test_router_feeds_moe_forward(mer, oracle, gpu):
    """Route on the GPU, then run the routed experts with those ids and
    weights; slots without a qualifying expert (id -1, weight 0) are skipped
    without a residency miss."""
    say("router -> moe_forward")
    r = routing(mer)
    dm, dff, n_exp, k, n_tok = 256, 512, 6, 4, 2
    rng = np.random.default_rng(5)
    blobs = []
    for e in range(n_exp):
        nb = oracle.expert_weight_bytes(4, dm, dff) // 18
        blobs.append(oracle.bench_fill(4, 3, e, 0, nb, 0.005, 0.02))
    devs = [torch.from_numpy(b).to(gpu) for b in blobs]
    table = torch.tensor([d.data_ptr() for d in devs], dtype=torch.int64, device=gpu)
    w = (rng.standard_normal((n_exp, dm)) * 0.05).astype(np.float32)
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    # experts 3..5 can never be selected (their sigmoid selection is -inf)
    bias = np.array([0, 0, 0, -np.inf, -np.inf, -np.inf], np.float32)
    ids, ws = r.route_linear_gate_gpu(dev(w, gpu), dev(x, gpu), k, sigmoid=True, bias=dev(bias, gpu))
    ids_np, ws_np = ids.cpu().numpy(), ws.cpu().numpy()
    assert (ids_np[:, 3] == -1).all() and (ws_np[:, 3] == 0).all()
    mer.take_device_status()
    got = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, table, ids, ws, dev(x, gpu)).cpu().numpy()
    mer.take_device_status()  # raises if a residency miss was recorded
    for t in range(n_tok):
        valid = ids_np[t] >= 0
        ys = np.stack([oracle.q4_0_reference_forward(blobs[i], x[t], dm, dff) for i in ids_np[t][valid]])
        want = oracle.combine_outputs(ys, ws_np[t][valid])
        err = np.abs(got[t] - want)
        assert (err <= 1e-3 + 1e-3 * np.abs(want)).all()
    del devs
