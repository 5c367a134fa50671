"""Pin the CPU oracle against the reference's own known answers, closed
forms and float64 brute force.  CPU only."""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
Q4, Q8 = 4, 5


# ---- f16 conversions -----------------------------------------------------

def test_f16_to_f32_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(c)) for c in codes], np.float32)
    finite = ~np.isnan(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.isnan(got[~finite]).all()


def test_f32_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_rust_round_semantics(oracle):
    # f32::round is half away from zero; `as i32` saturates, NaN -> 0.
    for v, want in [(0.5, 1), (-0.5, -1), (1.5, 2), (2.5, 3), (-2.5, -3), (1e20, 2**31 - 1),
                    (-1e20, -2**31), (float("nan"), 0)]:
        assert oracle.lib().mo_round_to_i32(v) == want


# ---- block formats (reference known answers) ----------------------------

def test_q4_0_ramp_block_known_answer(oracle):
    g = GOLDEN["q4_0_ramp_block"]
    blk = oracle.canonical_block(g["scale"], g["nibbles"])
    assert np.array_equal(oracle.dequantize_block(Q4, blk), np.array(g["expected"], np.float32))


def test_q4_0_extrema_and_negative_scale(oracle):
    for case in GOLDEN["q4_0_extrema_blocks"]["cases"]:
        blk = oracle.canonical_block(case["scale"], case["nibbles"])
        assert np.array_equal(oracle.dequantize_block(Q4, blk), np.array(case["expected"], np.float32))


def test_q4_0_writer_emits_exact_ggml_nibbles(oracle):
    g = GOLDEN["q4_0_writer_bytes"]
    blk = oracle.quantize_block(Q4, g["src"])
    assert int(blk[0]) | (int(blk[1]) << 8) == g["expected_scale_f16"]
    assert list(blk[2:]) == g["expected_qs"]


def test_q4_0_zero_block(oracle):
    blk = oracle.quantize_block(Q4, np.zeros(32, np.float32))
    assert blk[0] == 0 and blk[1] == 0
    assert all(b == GOLDEN["q4_0_zero_block"]["qs_byte"] for b in blk[2:])
    assert (oracle.dequantize_block(Q4, blk) == 0).all()


def _xorshift_block(state: int, n: int, scale: float):
    out = []
    mask = (1 << 64) - 1
    for _ in range(n):
        state ^= (state << 13) & mask
        state ^= state >> 7
        state ^= (state << 17) & mask
        u = (state >> 40) & 0xFFFFFFFF
        out.append((np.float32(u) / np.float32(1 << 23) - np.float32(1.0)) * np.float32(scale))
    return np.array(out, np.float32)


@pytest.mark.parametrize("dtype,div", [(Q4, 7.0), (Q8, 127.0)])
def test_round_trip_error_bound(oracle, dtype, div):
    # inference.rs:5664-5732 / :5761-5783: |x - dq(q(x))| <= d * 1.01
    cases = [np.zeros(32, np.float32), (np.arange(32, dtype=np.float32) - 15.5) / 3,
             np.where(np.arange(32) % 2 == 0, -7.0, 7.0).astype(np.float32),
             _xorshift_block(0xCAFEBABE, 32, 2.5), _xorshift_block(0xC0FFEE, 32, 1.5),
             np.array([-1e4] + [i * 1e-3 for i in range(1, 32)], np.float32)]
    for src in cases:
        dq = oracle.dequantize_block(dtype, oracle.quantize_block(dtype, src))
        d = np.abs(src).max() / div
        assert (np.abs(dq - src) <= d * 1.01 + np.finfo(np.float32).eps).all()


def test_q8_0_constant_block_is_exact(oracle):
    # inference.rs:5819-5845: constant 1.0 lands exactly on q=127
    dq = oracle.dequantize_block(Q8, oracle.quantize_block(Q8, np.ones(32, np.float32)))
    assert (np.abs(dq - 1.0) < 1e-3).all()


def test_q4_dequant_closed_form_random(oracle):
    rng = np.random.default_rng(1)
    blocks = rng.integers(0, 256, (500, 18), dtype=np.uint8)
    blocks[:, 1] &= 0x7B  # finite scales
    for b in blocks:
        d = np.float32(np.frombuffer(b[:2].tobytes(), np.float16)[0])
        q = np.concatenate([b[2:] & 15, b[2:] >> 4]).astype(np.int32) - 8
        want = (d * q.astype(np.float32)).astype(np.float32)
        assert np.array_equal(oracle.dequantize_block(Q4, b).view(np.uint32), want.view(np.uint32))


def test_q8_dequant_closed_form_random(oracle):
    rng = np.random.default_rng(2)
    blocks = rng.integers(0, 256, (500, 34), dtype=np.uint8)
    blocks[:, 1] &= 0x7B
    for b in blocks:
        d = np.float32(np.frombuffer(b[:2].tobytes(), np.float16)[0])
        want = (d * b[2:].view(np.int8).astype(np.float32)).astype(np.float32)
        assert np.array_equal(oracle.dequantize_block(Q8, b).view(np.uint32), want.view(np.uint32))


def test_stream_decode_truncates_tail(oracle):
    blk = oracle.canonical_block(0.5, GOLDEN["q4_0_ramp_block"]["nibbles"])
    two = np.concatenate([blk, blk])
    out = oracle.dequantize_to_f32(Q4, two, 40)
    assert out.size == 40 and np.array_equal(out[32:], out[:8])


def test_expert_weight_bytes(oracle):
    for c in GOLDEN["expert_bytes"]["cases"]:
        assert oracle.expert_weight_bytes(c["dtype"], c["d_model"], c["d_ff"]) == c["bytes"]


# ---- raw Q4 matvec ------------------------------------------------------

def canonical_cases(oracle):
    nib = GOLDEN["q4_canonical_nibbles"]
    cases = []
    for c in GOLDEN["q4_canonical_raw_cases"]["cases"]:
        w = np.concatenate([oracle.canonical_block(s, nib[n]) for s, n in c["blocks"]])
        x = oracle.deterministic_input(c["columns"], c["input_seed"])
        cases.append((c, w, x))
    return cases


def _brute_raw(w, off, rows, cols, x):
    out = []
    for r in range(rows):
        s = 0.0
        for k in range(cols // 32):
            b = w[(off + r * (cols // 32) + k) * 18:][:18]
            d = float(np.frombuffer(b[:2].tobytes(), np.float16)[0])
            q = [int(b[2 + (j % 16)] & 15) if j < 16 else int(b[2 + (j % 16)] >> 4) for j in range(32)]
            s += sum(d * (q[j] - 8) * float(x[k * 32 + j]) for j in range(32))
        out.append(s)
    return np.array(out)


def test_deterministic_input_closed_form(oracle):
    for seed in range(1, 9):
        x = oracle.deterministic_input(64, seed)
        want = np.array([((i * (seed * 2 + 3) + seed) % 31 - 15) / 32 for i in range(64)], np.float32)
        assert np.array_equal(x, want)


def test_canonical_raw_cases_exact(oracle):
    cases = canonical_cases(oracle)
    assert len(cases) == 8
    for c, w, x in cases:
        got = oracle.cpu_q4_matvec(w, c["w_block_off"], c["rows"], c["columns"], x)
        want = _brute_raw(w, c["w_block_off"], c["rows"], c["columns"], x)
        # every product and partial sum is a short dyadic rational: exact
        assert np.array_equal(got.astype(np.float64), want), c["name"]
    zero = [g for g in cases if g[0]["name"] == "zero-scale-extrema"][0]
    assert list(oracle.cpu_q4_matvec(zero[1], 0, 1, 32, zero[2])) == GOLDEN["q4_canonical_raw_cases"]["zero_scale_output"]
    multi = [g for g in cases if g[0]["rows"] >= 2][0]
    out = oracle.cpu_q4_matvec(multi[1], multi[0]["w_block_off"], 2, 32, multi[2])
    assert out[0] != out[1]
    unaligned = [g for g in cases if "unaligned" in g[0]["name"]][0]
    assert (unaligned[0]["w_block_off"] * 18) % 4 != 0


# ---- expert forward -----------------------------------------------------

def _brute_forward(dtype, blob, x, dm, dff, limit=None):
    n = dm * dff
    nb = -(-n // 32)
    pb = nb * (18 if dtype == Q4 else 34)
    mats = []
    for p in range(3):
        vals = []
        for b in range(nb):
            off = p * pb + b * (18 if dtype == Q4 else 34)
            vals.append(np.asarray(_dq64(dtype, blob[off:off + (18 if dtype == Q4 else 34)])))
        mats.append(np.concatenate(vals)[:n])
    g = mats[0].reshape(dff, dm) @ x.astype(np.float64)
    u = mats[1].reshape(dff, dm) @ x.astype(np.float64)
    if limit is not None:
        g = np.clip(g, -limit, limit)
    h = g / (1 + np.exp(-g)) * u
    return mats[2].reshape(dm, dff) @ h


def _dq64(dtype, b):
    d = float(np.frombuffer(b[:2].tobytes(), np.float16)[0])
    if dtype == Q4:
        q = np.concatenate([b[2:] & 15, b[2:] >> 4]).astype(np.float64) - 8
    else:
        q = b[2:].view(np.int8).astype(np.float64)
    return d * q


def _close(got, want, rel=1e-5, abs_=1e-5):
    return np.all(np.abs(got - want) <= abs_ + rel * np.abs(want))


@pytest.mark.parametrize("dm,dff", [(32, 32), (64, 96), (37, 45), (128, 64), (10, 10)])
def test_q4_reference_forward_vs_float64(oracle, dm, dff):
    blob = oracle.generate_synthetic_expert(Q4, 3, dm, dff)
    x = oracle.synth_hidden_state(5, dm, 9)
    got = oracle.q4_0_reference_forward(blob, x, dm, dff)
    want = _brute_forward(Q4, blob, x, dm, dff)
    scale = np.abs(want).max()
    assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-6)


def test_q4_complete_fixture_is_finite_nonzero(oracle):
    g = GOLDEN["q4_complete_fixture"]
    blk = oracle.canonical_block(g["scale"], GOLDEN["q4_canonical_nibbles"]["ramp"])
    blocks = oracle.expert_weight_bytes(Q4, g["d_model"], g["d_ff"]) // 18
    blob = np.tile(blk, blocks)
    x = oracle.deterministic_input(g["d_model"], g["input_seed"])
    y = oracle.q4_0_reference_forward(blob, x, g["d_model"], g["d_ff"])
    assert np.isfinite(y).all() and (y != 0).any()


@pytest.mark.parametrize("dm,dff", [(32, 32), (64, 96), (37, 45), (64, 45), (37, 64)])
def test_q8_direct_vs_float64(oracle, dm, dff):
    blob = oracle.randomized_q8_expert(dm, dff, dm ^ dff)
    x = oracle.synth_hidden_state(19, dm, 7)
    want = _brute_forward(Q8, blob, x, dm, dff)
    for kernel in (0, 1):
        rc, got = oracle.q8_0_direct_forward(blob, x, dm, dff, kernel=kernel)
        assert rc == 0
        tol = 3e-3 * np.maximum(np.abs(want), 1.0) + 3e-5  # inference.rs:5962-5980
        assert np.all(np.abs(got - want) <= tol)
        assert _close(got, want, rel=1e-4, abs_=1e-6 * np.abs(want).max())


def _gate_f64(dtype, blob, x, dm, dff):
    n = dm * dff
    vals = [_dq64(dtype, blob[b * (18 if dtype == Q4 else 34):(b + 1) * (18 if dtype == Q4 else 34)])
            for b in range(-(-n // 32))]
    return np.concatenate(vals)[:n].reshape(dff, dm) @ x.astype(np.float64)


@pytest.mark.parametrize("dtype,dm,dff", [(Q4, 64, 96), (Q4, 37, 45), (Q8, 64, 96), (Q8, 37, 45)])
def test_swiglu_limit_clamp_vs_float64(oracle, dtype, dm, dff):
    """set_swiglu_limit / clamp_swiglu_gate (inference.rs:86-123): with a
    limit between the median and the largest |gate| the clamp binds on part
    of the rows, and the forward equals float64 brute force with
    silu(clip(g, -l, l)) * u; a non-positive or non-finite limit removes it."""
    blob = oracle.generate_synthetic_expert(Q4, 3, dm, dff) if dtype == Q4 else oracle.randomized_q8_expert(dm, dff, 77)
    x = (oracle.synth_hidden_state(5, dm, 9) * 4).astype(np.float32)
    g = np.abs(_gate_f64(dtype, blob, x, dm, dff))
    limit = float(np.float32(np.quantile(g, 0.8)))
    assert (g > limit).sum() >= dff // 8 and (g < limit).sum() >= dff // 2
    fwd = (lambda: oracle.q4_0_reference_forward(blob, x, dm, dff)) if dtype == Q4 else \
        (lambda: oracle.q8_0_direct_forward(blob, x, dm, dff)[1])
    plain = fwd()
    try:
        oracle.set_swiglu_limit(limit)
        assert oracle.swiglu_limit() == limit
        got = fwd()
        want = _brute_forward(dtype, blob, x, dm, dff, limit)
        scale = np.abs(want).max()
        assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-6)
        assert np.abs(got - plain).max() > 1e-3 * scale  # the clamp changed the result
        for off in (0.0, -1.0, float("nan"), float("inf")):
            oracle.set_swiglu_limit(off)
            assert oracle.swiglu_limit() is None
            assert np.array_equal(fwd(), plain)
    finally:
        oracle.set_swiglu_limit(None)


def test_q8_direct_matches_dequant_reference(oracle):
    dm, dff = 37, 45
    blob = oracle.randomized_q8_expert(dm, dff, 0x51A1A11E)
    x = oracle.synth_hidden_state(9, dm, 3)
    want = oracle.q8_0_dequant_forward(blob, x, dm, dff)
    rc, got = oracle.q8_0_direct_forward(blob, x, dm, dff)
    assert rc == 0
    assert np.all(np.abs(got - want) <= 3e-3 * np.maximum(np.abs(want), 1.0) + 3e-5)


def test_q8_avx2_order_vs_scalar_qwen(oracle):
    # inference.rs:6138-6161: AVX2 vs scalar at 2048x768 within 2e-5
    dm, dff = 2048, 768
    blob = oracle.randomized_q8_expert(dm, dff, 0x20480768)
    x = oracle.synth_hidden_state(23, dm, 11)
    rc0, s = oracle.q8_0_direct_forward(blob, x, dm, dff, kernel=0)
    rc1, a = oracle.q8_0_direct_forward(blob, x, dm, dff, kernel=1)
    assert rc0 == rc1 == 0
    assert np.all(np.abs(s - a) <= 2e-5 * np.maximum(np.abs(s), 1.0) + 3e-5)
    assert not np.array_equal(s, a)  # the two orders really differ


def _q8_row(width, case, seed, oracle):
    # kernels/avx2.rs:193-223 row generator
    mask = (1 << 64) - 1
    blocks = width // 32
    out = np.zeros(blocks * 34, np.uint8)
    state = seed
    for b in range(blocks):
        sb = {0: 0, 1: 1, 2: 0x7BFF, 6: 0x0400}.get(case, oracle.f32_to_f16(np.float32(0.003 + b * 0.00001)))
        out[b * 34] = sb & 0xFF
        out[b * 34 + 1] = sb >> 8
        for i in range(32):
            if case == 3:
                q = 0
            elif case == 4:
                q = -128 if (i + b) % 2 == 0 else 127
            elif case == 5:
                q = -1 if (i + b) % 2 == 0 else 1
            else:
                state ^= (state << 13) & mask
                state ^= state >> 7
                state ^= (state << 17) & mask
                q = np.int64(state & 0xFF).astype(np.uint8).view(np.int8)
            out[b * 34 + 2 + i] = np.int8(q).view(np.uint8)
    return out


def test_q8_row_kernels_known_cases(oracle):
    g = GOLDEN["q8_row_cases"]
    for width in g["widths"]:
        x = np.sin(np.arange(width, dtype=np.float32) * np.float32(0.013)).astype(np.float32) * np.float32(0.01)
        for case in g["cases"]:
            for seed in g["seeds"]:
                row = _q8_row(width, case, seed, oracle)
                exact = float(np.dot(_dq64(Q8, row[:34]) if False else np.concatenate(
                    [_dq64(Q8, row[b * 34:(b + 1) * 34]) for b in range(width // 32)]), x.astype(np.float64)))
                for kernel in (0, 1):
                    got = oracle.q8_0_row_dot(kernel, row, x)
                    assert abs(got - exact) <= 2e-4 + 2e-5 * abs(exact), (width, case, seed, kernel)


def test_q8_validation_taxonomy(oracle):
    # inference.rs:6193-6244
    assert oracle.validate_q8_direct(0, 0, 0, 0, 2) == 4  # zero dims -> InvalidLayout
    assert oracle.validate_q8_direct(10, 31, 32, 32, 32) == 4  # x mismatch
    need = oracle.expert_weight_bytes(Q8, 32, 64)
    assert oracle.validate_q8_direct(need - 1, 32, 32, 32, 64) == 5  # truncated within a page
    assert oracle.validate_q8_direct(need, 32, 32, 32, 64) == 0
    small = oracle.expert_weight_bytes(Q8, 32, 32)  # <= 4096 -> BufferTooSmall
    assert oracle.validate_q8_direct(small - 1, 32, 32, 32, 32) == 1
    assert oracle.validate_q8_direct(0, 2**63, 2**63, 2**63, 2) == 4  # overflow


def test_q4_validation_taxonomy(oracle):
    need = oracle.expert_weight_bytes(Q4, 4096, 14336)
    assert oracle.validate_q4_0(need, 4096, 14336) == 0
    assert oracle.validate_q4_0(need - 4096, 4096, 14336) == 5
    assert oracle.validate_q4_0(need - 4097, 4096, 14336) == 1
    assert oracle.validate_q4_0(need - 100, 4096, 14336, tolerance=4096) == 0
    assert oracle.validate_q4_0(107, 8, 8) == 1


def test_q8_nonfinite_propagates(oracle):
    blob = oracle.randomized_q8_expert(32, 32, 5)
    x = np.full(32, 0.25, np.float32)
    x[3], x[17] = np.nan, np.inf
    rc, y = oracle.q8_0_direct_forward(blob, x, 32, 32)
    assert rc == 0 and not np.isfinite(y).all()


def test_combine_closed_form(oracle):
    rng = np.random.default_rng(3)
    outs = rng.standard_normal((4, 64)).astype(np.float32)
    s = rng.random(4).astype(np.float32)
    got = oracle.combine_outputs(outs, s)
    acc = np.zeros(64, np.float32)
    for i in range(4):
        acc = (acc + s[i] * outs[i]).astype(np.float32)
    assert np.array_equal(got, acc)


# ---- generators ----------------------------------------------------------

def test_synth_hidden_state_matches_splitmix_vector(oracle):
    x = oracle.synth_hidden_state(0, 4, 0)
    vec = [int(v, 16) for v in GOLDEN["splitmix64_seed0"]["outputs"]]
    want = np.array([np.float32(v >> 40) / np.float32(1 << 23) - np.float32(1) for v in vec], np.float32)
    assert np.array_equal(x, want)


def test_xorshift_generator_first_value(oracle):
    # xorshift64(13,7,17) from state 1 gives 1082269761 (brute force by hand)
    blob = oracle.randomized_q8_expert(1, 1, 1)
    u = 1082269761 >> 40
    v0 = (np.float32(u) / np.float32(16777215.0) - np.float32(0.5)) * np.float32(0.08)
    blk = oracle.quantize_block(Q8, np.array([v0], np.float32))
    assert np.array_equal(blob[:34], blk)


def test_bench_fill_properties(oracle):
    q4 = oracle.bench_fill(Q4, 7, 3, 0, 20000, 0.005, 0.02).reshape(-1, 18)
    d = q4[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    assert d.min() >= np.float16(0.005) and d.max() <= np.float16(0.02)
    nib = np.concatenate([q4[:, 2:] & 15, q4[:, 2:] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    q8 = oracle.bench_fill(Q8, 7, 3, 0, 5000, 0.002, 0.01).reshape(-1, 34)
    q = q8[:, 2:].view(np.int8).ravel().astype(np.int32)
    assert q.min() == -127 and q.max() == 127
    # a sub-range of blocks equals the same blocks of a full fill
    part = oracle.bench_fill(Q4, 7, 3, 100, 50, 0.005, 0.02).reshape(-1, 18)
    assert np.array_equal(part, q4[100:150])


def test_output_digest_closed_form(oracle):
    y = np.zeros(3, np.float32)
    d, norm = oracle.output_digest(5, 2, y)
    want = 0xcbf29ce484222325 ^ 5 ^ 2
    for _ in range(3):
        want = (want * 0x100000001b3) & ((1 << 64) - 1)
    assert d == want and norm == 0.0


# ---- routing ---------------------------------------------------------------

def test_linear_gate_known_answers(oracle):
    g = GOLDEN["gate_known_answers"]["largest_logit_first"]
    w = np.repeat(np.arange(1, 5, dtype=np.float32), 3).reshape(4, 3)
    ids, ws = oracle.linear_gate_route(w, np.array(g["x"], np.float32), g["top_k"])
    assert list(ids) == g["experts"]
    assert abs(ws.sum() - 1) < 1e-5 and ws[0] > ws[1]
    u = GOLDEN["gate_known_answers"]["top_k_all_uniform"]
    ids, ws = oracle.linear_gate_route(np.zeros((4, 2), np.float32), np.zeros(2, np.float32), 4)
    assert list(ids) == [0, 1, 2, 3]  # ties resolve to the lower id
    assert np.allclose(ws, u["weight"], atol=1e-5)


def test_softmax_closed_form_and_fallback(oracle):
    v = oracle.softmax([1.0, 2.0, 3.0])
    e = np.exp(np.array([1, 2, 3], np.float64) - 3)
    assert np.allclose(v, e / e.sum(), rtol=1e-6)
    assert np.allclose(oracle.softmax([np.nan, 1.0]), [0.5, 0.5])


def test_topk_matches_sorted_selection(oracle):
    rng = np.random.default_rng(4)
    for _ in range(200):
        logits = rng.standard_normal(8).astype(np.float32)
        ids, ws = oracle.topk_softmax_logits(logits, 2)
        order = sorted(range(8), key=lambda i: (-logits[i], i))[:2]
        assert list(ids) == order
        e = np.exp(logits.astype(np.float64) - logits.max())
        p = e / e.sum()
        assert np.allclose(ws, p[order] / p[order].sum(), rtol=1e-5)


def test_skewed_stream_properties(oracle):
    # workload.rs:284-343
    s = oracle.SkewedStream(32, 4, 1.0, 0.0, 7)
    for _ in range(1000):
        e = s.next_experts()
        assert len(e) == 4 and len(set(e)) == 4
    s = oracle.SkewedStream(64, 2, 1.2, 0.0, 0xABCD)
    counts = np.zeros(64, np.int64)
    for _ in range(20000):
        for i in s.next_experts():
            counts[i] += 1
    assert counts.max() > 5 * np.median(counts)

    def repeats(rho):
        st = oracle.SkewedStream(128, 2, 0.8, rho, 99)
        prev, n = st.next_experts(), 0
        for _ in range(5000):
            cur = st.next_experts()
            n += cur == prev
            prev = cur
        return n

    assert repeats(0.9) > 3 * repeats(0.0)


def test_gate_routing_surface_known_answers(oracle):
    """The reference's own LinearGate tests with an identity gate (logit[i] =
    x[i]): sigmoid scoring, selection-only bias, group-limited selection,
    routed scaling and the default softmax gate."""
    g = GOLDEN["gate_routing_surface_known_answers"]
    for c in g["cases"]:
        w = np.eye(c["n"], dtype=np.float32)
        ids, ws, _ = oracle.linear_gate_route_ex(w, np.array(c["x"], np.float32), c["top_k"], sigmoid=c["sigmoid"],
                                                 normalise=c["normalise"], bias=c["bias"], n_group=c["n_group"],
                                                 topk_group=c["topk_group"], scaling=c["scaling"])
        if "experts" in c:
            assert list(ids) == c["experts"], c["name"]
        if "weights" in c:
            assert np.allclose(ws, c["weights"], atol=c["weight_tol"]), c["name"]
        if "weight_sum" in c:
            assert abs(float(ws.sum()) - c["weight_sum"]) < c["weight_tol"], c["name"]
        if "experts_min" in c:
            assert len(ids) == c["count"] and all(int(e) >= c["experts_min"] for e in ids), c["name"]
    t = g["ties"]
    ids, ws, _ = oracle.linear_gate_route_ex(np.zeros((t["num_experts"], t["d_model"]), np.float32),
                                             np.array(t["x"], np.float32), t["top_k"])
    assert list(ids) == t["experts"] and np.allclose(ws, t["weight"], atol=1e-6)


def test_gate_route_ex_default_equals_default_gate(oracle):
    """With the default options the full routing surface is the default
    gate (pinned above by its own known answers)."""
    rng = np.random.default_rng(12)
    for _ in range(50):
        w = rng.standard_normal((16, 24)).astype(np.float32)
        x = rng.standard_normal(24).astype(np.float32)
        ids0, ws0 = oracle.linear_gate_route(w, x, 4)
        ids1, ws1, _ = oracle.linear_gate_route_ex(w, x, 4)
        assert list(ids0) == list(ids1) and np.array_equal(ws0, ws1)


def test_gate_group_filter_brute_force(oracle):
    """Group-limited selection against brute force on small cases: the
    chosen experts are the top-k (score desc, id asc) among the experts of
    the topk_group groups with the largest top-2 sums."""
    rng = np.random.default_rng(13)
    for _ in range(200):
        n, n_group, topk_group, k = 16, 4, 2, 3
        logits = rng.standard_normal(n).astype(np.float32)
        bias = rng.standard_normal(n).astype(np.float32) * 0.5
        ids, _ = oracle.gate_route_ex(logits, k, sigmoid=True, normalise=False, bias=bias, n_group=n_group,
                                      topk_group=topk_group)
        sel = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))) + bias
        gs = n // n_group
        gsum = [sorted(sel[g * gs:(g + 1) * gs])[-1] + sorted(sel[g * gs:(g + 1) * gs])[-2] for g in range(n_group)]
        groups = sorted(range(n_group), key=lambda g: (-gsum[g], g))[:topk_group]
        cand = [e for e in range(n) if e // gs in groups]
        want = sorted(cand, key=lambda e: (-sel[e], e))[:k]
        assert list(ids) == want
