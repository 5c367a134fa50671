"""The Q4_0 QMatMul mode (MER_MOE_QMM, mer_hip_expert_forward_qmm: Candle's
Q8_0-activation arithmetic, run_inference_q4_0_qmm, inference.rs:
4159-4243) against the oracle's restatement (mo_q4_0_qmm_forward).  The
integer block dots are exact on both sides; the f32 sums differ in order,
and h, formed in f32 in another order, can round a block element to the
neighbouring Q8_0 step, so the bar is the FFN bar of test_gpu_parity.  Each
case also checks that the GPU result sits far closer to the QMM oracle than
to the dequant oracle, i.e. that the mode really quantises its inputs.

The bar: quantising h per block makes the output a step function of h.
GPU and oracle form h in different f32 orders, so an h element lying within
~1e-4 of a Q8_0 rounding midpoint may round to the neighbouring step on one
side (Candle's own AVX and scalar codes would differ the same way).  Such a
flip moves row r by |W_d[r, j]| d_j.  The oracle flags every element within
1e-3 steps of a midpoint (and every block whose f16 scale is that close to
an f16 midpoint) and adds what each could move to its row (the flip bound).
The bar is the FFN bar of test_gpu_parity plus that bound."""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_parity import ABS_TOL, REL_TOL, _table, assert_ffn_close, make_expert, say, to_dev

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

Q4, Q8 = 4, 5


def assert_qmm_close(got, ref, bound, label):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    bound = np.asarray(bound, np.float64).ravel()
    assert np.isfinite(got).all(), label
    abs_bar = ABS_TOL * max(1.0, 1e-3 * float(np.abs(ref).max()))
    allowed = REL_TOL * np.abs(ref) + abs_bar + bound
    err = np.abs(got - ref)
    worst = int(np.argmax(err / allowed))
    say(f"{label}: worst err {err[worst]:.3g} allowed {allowed[worst]:.3g} (flip bound {bound[worst]:.3g}); "
        f"{int((err > REL_TOL * np.abs(ref) + abs_bar).sum())} rows beyond the FFN bar")
    assert (err <= allowed).all(), f"{label}: worst index {worst} gpu={got[worst]} ref={ref[worst]}"


def _closer_to_qmm(got, qmm, deq, label):
    e_q = float(np.abs(np.asarray(got, np.float64) - qmm).max())
    e_d = float(np.abs(np.asarray(got, np.float64) - deq).max())
    say(f"{label}: max|gpu - qmm oracle| {e_q:.3g}, max|gpu - dequant oracle| {e_d:.3g}")
    assert e_q < 0.05 * e_d, label


@pytest.mark.parametrize("dm,dff", [(64, 128), (512, 1024), (2048, 768), (7168, 2048), (4096, 14336)])
def test_expert_forward_qmm_vs_oracle(mer, oracle, gpu, dm, dff):
    say(f"qmm expert dm={dm} dff={dff}")
    blob = make_expert(oracle, Q4, dm, dff, 3)
    x = np.random.default_rng(dm + dff).standard_normal(dm).astype(np.float32)
    got = mer.q4_0_qmm_forward(to_dev(blob, gpu), to_dev(x, gpu), dm, dff).cpu().numpy()
    want, bound, flagged = oracle.q4_0_qmm_forward_bounded(blob, x, dm, dff)
    say(f"qmm {dm}x{dff}: {flagged} h elements flagged")
    assert_qmm_close(got, want, bound, f"qmm {dm}x{dff}")
    _closer_to_qmm(got, want, oracle.q4_0_reference_forward(blob, x, dm, dff), f"qmm {dm}x{dff}")
    # the engine's dispatch with use_qmm takes the same arm
    got2 = mer.dispatch_expert_forward(mer.WeightDtype.Q4_0, to_dev(blob, gpu), to_dev(x, gpu), dm, dff,
                                       use_qmm=True).cpu().numpy()
    assert np.array_equal(got, got2)


def test_moe_forward_qmm_vs_oracle_combine(mer, oracle, gpu):
    dm, dff = 1024, 2048
    say(f"qmm moe dm={dm} dff={dff}")
    n_exp, n_tok, k = 6, 3, 2
    blobs = [make_expert(oracle, Q4, dm, dff, e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    rng = np.random.default_rng(5)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    w[2, 0] = 0.0
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = np.zeros((n_tok, dm), np.float32)
    bound = np.zeros((n_tok, dm), np.float64)
    deq = np.zeros((n_tok, dm), np.float32)
    for t in range(n_tok):
        res = [oracle.q4_0_qmm_forward_bounded(blobs[i], x[t], dm, dff) for i in ids[t]]
        want[t] = oracle.combine_outputs(np.stack([r[0] for r in res]), w[t])
        bound[t] = sum(float(w[t, i]) * res[i][1].astype(np.float64) for i in range(k))
        deq[t] = oracle.combine_outputs(
            np.stack([oracle.q4_0_reference_forward(blobs[i], x[t], dm, dff) for i in ids[t]]), w[t])
    args = (mer.WeightDtype.Q4_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu))
    got = mer.moe_forward(*args, qmm=True).cpu().numpy()
    assert_qmm_close(got, want, bound, "qmm moe")
    _closer_to_qmm(got, want, deq, "qmm moe")
    got_r = mer.moe_forward(*args, residual=True, qmm=True).cpu().numpy()
    assert_qmm_close(got_r, want + x, bound, "qmm moe residual")
    # the no-alloc entry point runs the same kernels: bit-identical
    out = torch.empty((n_tok, dm), dtype=torch.float32, device=gpu)
    rc = mer._lib.lib().mer_hip_moe_forward_noalloc(
        Q4, dm, dff, n_tok, k, table.data_ptr(), table.numel(), args[4].data_ptr(), args[5].data_ptr(),
        args[6].data_ptr(), out.data_ptr(), 16, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    assert np.array_equal(out.cpu().numpy(), got)
    mer.take_device_status()
    del devs


def test_moe_forward_layers_qmm_chained(mer, oracle, gpu):
    dm, dff, L, E, k = 512, 1024, 3, 4, 2
    say(f"qmm layers chained L={L}")
    blobs = [[make_expert(oracle, Q4, dm, dff, l * E + e) for e in range(E)] for l in range(L)]
    keep, layers = [], []
    rng = np.random.default_rng(9)
    x0 = rng.standard_normal((1, dm)).astype(np.float32)
    ids = [rng.choice(E, k, replace=False).astype(np.int32).reshape(1, k) for _ in range(L)]
    ws = [rng.random((1, k)).astype(np.float32) for _ in range(L)]
    for l in range(L):
        devs, table = _table(blobs[l], gpu)
        keep.append(devs)
        layers.append({"table": table, "ids": to_dev(ids[l], gpu), "weights": to_dev(ws[l], gpu),
                       "x": to_dev(x0, gpu) if l == 0 else None,
                       "out": torch.zeros((1, dm), dtype=torch.float32, device=gpu)})
    mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers, residual=True, chain=True, qmm=True)
    torch.cuda.synchronize()
    x = x0[0]
    for l in range(L):
        res = [oracle.q4_0_qmm_forward_bounded(blobs[l][i], x, dm, dff) for i in ids[l][0]]
        want = x + oracle.combine_outputs(np.stack([r[0] for r in res]), ws[l][0])
        bound = sum(float(ws[l][0][i]) * res[i][1].astype(np.float64) for i in range(k))
        got = layers[l]["out"].cpu().numpy()[0]
        assert_qmm_close(got, want, bound, f"qmm chained layer {l}")
        x = got  # the next layer's oracle input is the GPU's own output of this layer
    mer.take_device_status()
    del keep


def test_qmm_flag_leaves_q8_0_unchanged(mer, oracle, gpu):
    """use_qmm switches only the Q4_0 arm (engine.rs:1825-1830)."""
    dm, dff = 512, 768
    say("qmm flag on Q8_0")
    blobs = [make_expert(oracle, Q8, dm, dff, e) for e in range(3)]
    devs, table = _table(blobs, gpu)
    ids = to_dev(np.array([[0, 2]], np.int32), gpu)
    w = to_dev(np.array([[0.25, 0.75]], np.float32), gpu)
    x = to_dev(np.random.default_rng(1).standard_normal((1, dm)).astype(np.float32), gpu)
    a = mer.moe_forward(mer.WeightDtype.Q8_0, dm, dff, table, ids, w, x).cpu().numpy()
    b = mer.moe_forward(mer.WeightDtype.Q8_0, dm, dff, table, ids, w, x, qmm=True).cpu().numpy()
    assert np.array_equal(a, b)
    del devs


def test_qmm_layout_errors(mer, oracle, gpu):
    say("qmm layout errors")
    blob = make_expert(oracle, Q4, 96, 64, 0)  # multiples of 32, not of 64
    with pytest.raises(mer.errors.InvalidLayout):
        mer.q4_0_qmm_forward(to_dev(blob, gpu), to_dev(np.zeros(96, np.float32), gpu), 96, 64)
    # dispatch with use_qmm on dims that are not multiples of 32 takes the dequant arm, as the engine does
    dm, dff = 80, 48
    blob = make_expert(oracle, Q4, dm, dff, 1)
    x = np.random.default_rng(2).standard_normal(dm).astype(np.float32)
    got = mer.dispatch_expert_forward(mer.WeightDtype.Q4_0, to_dev(blob, gpu), to_dev(x, gpu), dm, dff,
                                      use_qmm=True).cpu().numpy()
    assert_ffn_close(got, oracle.q4_0_reference_forward(blob, x, dm, dff), "qmm fallback")


def test_qmm_non_finite_inputs_follow_the_oracle(mer, oracle, gpu):
    """Candle's quantisation ignores a NaN in the block maximum and turns the
    NaN element into 0; an infinite element makes the block scale infinite,
    so the outputs become NaN.  The GPU mode agrees on which outputs are NaN
    and on the finite ones."""
    dm, dff = 128, 256
    blob = make_expert(oracle, Q4, dm, dff, 5)
    for label, bad in (("nan", np.nan), ("inf", np.inf)):
        say(f"qmm non-finite input {label}")
        x = np.random.default_rng(3).standard_normal(dm).astype(np.float32)
        x[37] = bad
        want, bound, _ = oracle.q4_0_qmm_forward_bounded(blob, x, dm, dff)
        got = mer.q4_0_qmm_forward(to_dev(blob, gpu), to_dev(x, gpu), dm, dff).cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want)), label
        ok = ~np.isnan(want)
        if ok.any():
            assert_qmm_close(got[ok], want[ok], bound[ok], f"qmm {label}")


def test_grouped_qmm_vs_oracle(mer, oracle, gpu):
    """The grouped int8-MFMA path under MER_MOE_QMM: Candle's Q8_0 value sits
    in the first of its three digit planes, so the contraction is the same
    and only the input quantisation changes."""
    dm, dff, n_exp, n_tok, k = 512, 1024, 6, 24, 2
    say(f"qmm grouped dm={dm} dff={dff} tokens={n_tok}")
    blobs = [make_expert(oracle, Q4, dm, dff, 20 + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    rng = np.random.default_rng(21)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = np.zeros((n_tok, dm), np.float32)
    bound = np.zeros((n_tok, dm), np.float64)
    deq = np.zeros((n_tok, dm), np.float32)
    for t in range(n_tok):
        res = [oracle.q4_0_qmm_forward_bounded(blobs[i], x[t], dm, dff) for i in ids[t]]
        want[t] = oracle.combine_outputs(np.stack([r[0] for r in res]), w[t])
        bound[t] = sum(float(w[t, i]) * res[i][1].astype(np.float64) for i in range(k))
        deq[t] = oracle.combine_outputs(
            np.stack([oracle.q4_0_reference_forward(blobs[i], x[t], dm, dff) for i in ids[t]]), w[t])
    got = mer.moe_grouped(mer.WeightDtype.Q4_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu),
                          qmm=True).cpu().numpy()
    assert_qmm_close(got, want, bound, "qmm grouped")
    _closer_to_qmm(got, want, deq, "qmm grouped")
    mer.take_device_status()
    del devs


@pytest.mark.parametrize("path", ["decode", "grouped"])
def test_qmm_swiglu_limit_matches_oracle(mer, oracle, gpu, path):
    """forward_qmm clamps the gate before SiLU as well (clamp_swiglu_gate,
    inference.rs:4119); the limit binds on a good part of the rows."""
    dm, dff = 512, 1024
    say(f"qmm swiglu limit path={path}")
    blobs = [make_expert(oracle, Q4, dm, dff, 90 + e) for e in range(3)]
    devs, table = _table(blobs, gpu)
    rng = np.random.default_rng(41)
    n_tok, k = 3, 2
    ids = np.stack([rng.choice(3, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    x = (rng.standard_normal((n_tok, dm)) * 3).astype(np.float32)
    fn = mer.moe_grouped if path == "grouped" else mer.moe_forward
    try:
        mer.set_swiglu_limit(0.5)
        oracle.set_swiglu_limit(0.5)
        want = np.zeros((n_tok, dm), np.float32)
        bound = np.zeros((n_tok, dm), np.float64)
        for t in range(n_tok):
            res = [oracle.q4_0_qmm_forward_bounded(blobs[i], x[t], dm, dff) for i in ids[t]]
            want[t] = oracle.combine_outputs(np.stack([r[0] for r in res]), w[t])
            bound[t] = sum(float(w[t, i]) * res[i][1].astype(np.float64) for i in range(k))
        got = fn(mer.WeightDtype.Q4_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu),
                 qmm=True).cpu().numpy()
    finally:
        mer.set_swiglu_limit(None)
        oracle.set_swiglu_limit(float("inf"))
    assert_qmm_close(got, want, bound, f"qmm swiglu limit {path}")
    unclamped = np.stack([oracle.combine_outputs(np.stack([oracle.q4_0_qmm_forward(blobs[i], x[t], dm, dff)
                                                           for i in ids[t]]), w[t]) for t in range(n_tok)])
    assert np.abs(unclamped - want).max() > 100 * np.abs(got - want).max()  # the clamp bound
    mer.take_device_status()
    del devs
