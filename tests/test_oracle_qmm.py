"""Pin the oracle's Candle-QMatMul Q4_0 path (mo_q4_0_qmm_forward,
run_inference_q4_0_qmm, inference.rs:4159-4243) on the CPU: the reference's
own QMM-vs-dequant test, a float64 brute force built from the closed forms
of the Q4_0 decode and the Q8_0 activation quantisation, and the half-way
rounding that separates `f32::round` from round-half-even.  CPU only."""
from __future__ import annotations

import numpy as np
import pytest

Q4 = 4


def _np_quantize_q8_0(x: np.ndarray):
    """BlockQ8_0::from_float (candle-core 0.10.2) in numpy, f32 throughout."""
    xb = x.astype(np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (xb * inv[:, None]).astype(np.float32)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)  # round half away from zero
    q = np.clip(q, -128, 127).astype(np.int64)
    d16 = d.astype(np.float16).astype(np.float32)
    return q.reshape(-1), d16


def _brute_qmm(oracle, blob, x, dm, dff):
    """Float64 forward from the closed forms: weights from the pinned Q4_0
    decode (value = d * (nibble - 8)), activations from the numpy Q8_0
    quantisation; each block contributes d_w d_x sum(w_int q)."""
    per = dm * dff // 32 * 18

    def proj(k, vec, rows, cols):
        w = oracle.dequantize_to_f32(Q4, blob[k * per:(k + 1) * per], rows * cols).astype(np.float64)
        q, d = _np_quantize_q8_0(vec)
        xq = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
        return w.reshape(rows, cols) @ xq, np.abs(w.reshape(rows, cols)) @ np.abs(xq)

    g, gm = proj(0, x, dff, dm)
    u, um = proj(1, x, dff, dm)
    g32, u32 = g.astype(np.float32), u.astype(np.float32)
    h = (g32 / (np.float32(1) + np.exp(-g32)) * u32).astype(np.float32)
    return proj(2, h, dm, dff)


def test_qmm_matches_dequant_like_the_reference(oracle):
    """run_inference_q4_0_qmm_matches_dequant_baseline (inference.rs:
    6547-6594): d_model 32, d_ff 64, the test's own weight generator,
    synth_hidden_state(0, 32, 1), |a - b| <= 5e-2 max(|a|, 1) + 1e-5."""
    dm, dff = 32, 64
    blocks = dm * dff // 32
    parts = []
    for projection in range(3):
        for b in range(blocks):
            w = [(1.0 if (i + b + projection) % 2 == 0 else -1.0) * ((i * 11 + b * 7 + projection * 5) % 17) / 20.0
                 for i in range(32)]
            parts.append(oracle.quantize_block(Q4, np.array(w, np.float32)))
    blob = np.concatenate(parts)
    x = oracle.synth_hidden_state(0, dm, 1)
    base = oracle.q4_0_reference_forward(blob, x, dm, dff)
    qmm = oracle.q4_0_qmm_forward(blob, x, dm, dff)
    assert np.isfinite(base).all() and np.isfinite(qmm).all()
    tol = 5e-2 * np.maximum(np.abs(base), 1.0) + 1e-5
    assert (np.abs(base - qmm) <= tol).all()
    assert not np.array_equal(base, qmm)  # the activations really were quantised


def test_q8_0_activation_quantisation_closed_form(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(32 * 40).astype(np.float32) * np.float32(10.0) ** rng.integers(-4, 4),
                        np.zeros(32, np.float32)])
    q, d = oracle.quantize_row_q8_0_candle(x)
    qw, dw = _np_quantize_q8_0(x)
    assert np.array_equal(q.astype(np.int64), qw)
    assert np.array_equal(d.view(np.uint32), dw.view(np.uint32))
    assert (d[-1] == 0) and not q[-32:].any()


def test_q8_0_quantisation_rounds_half_away_from_zero(oracle):
    # amax = 127 -> d = 1, id = 1: the values themselves are rounded
    x = np.zeros(32, np.float32)
    x[:6] = [127.0, 2.5, -2.5, 0.5, -0.5, 3.5]
    q, d = oracle.quantize_row_q8_0_candle(x)
    assert d[0] == 1.0
    assert q[:6].tolist() == [127, 3, -3, 1, -1, 4]  # round-half-even would give 2, -2, 0, 0, 4


@pytest.mark.parametrize("dm,dff,seed", [(64, 96, 1), (128, 64, 2), (256, 320, 3), (1024, 4096, 4)])
def test_qmm_forward_float64_brute_force(oracle, dm, dff, seed):
    """The brute force forms h in float64, the oracle in f32, so h elements
    next to a rounding midpoint may quantise differently: the difference must
    lie within f32 rounding of the magnitudes summed plus the oracle's flip
    bound (which the oracle computes from its own h)."""
    blob = oracle.generate_synthetic_expert(Q4, seed, dm, dff)
    x = (np.random.default_rng(seed).standard_normal(dm) * 2).astype(np.float32)
    got, bound, flagged = oracle.q4_0_qmm_forward_bounded(blob, x, dm, dff)
    assert np.array_equal(got, oracle.q4_0_qmm_forward(blob, x, dm, dff))
    want, mag = _brute_qmm(oracle, blob, x, dm, dff)
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= 2e-6 * mag + 1e-7 + bound).all()
    assert flagged < dff * 0.01 + 2  # the margin flags a few elements, not a fraction of h


def test_qmm_flip_bound_covers_a_real_flip(oracle):
    """An element moved across a rounding midpoint changes the output by
    exactly what the bound allows for it: the oracle run on x and on a copy
    of x whose h lands on the other side of a midpoint differ by no more than
    the bound of either, and the bound is zero without flagged elements."""
    dm, dff = 128, 64
    blob = oracle.generate_synthetic_expert(Q4, 7, dm, dff)
    x = (np.random.default_rng(7).standard_normal(dm)).astype(np.float32)
    y0, b0, n0 = oracle.q4_0_qmm_forward_bounded(blob, x, dm, dff, margin=0.0)
    assert n0 == 0 and not b0.any()
    # a margin of half a step flags every element: the bound then covers any
    # change of the h quantisation by one step per element
    y1, b1, n1 = oracle.q4_0_qmm_forward_bounded(blob, x, dm, dff, margin=0.5)
    assert n1 >= dff and (b1 > 0).all()
    assert np.array_equal(y0, y1)


def test_qmm_rejects_unaligned_dimensions(oracle):
    """q4_0_qmm_rejects_unaligned_dimensions (inference.rs:6597):
    InvalidLayout when d_model or d_ff is not a multiple of 32."""
    blob = np.zeros(oracle.expert_weight_bytes(Q4, 31, 32), np.uint8)
    with pytest.raises(ValueError, match="status 4"):
        oracle.q4_0_qmm_forward(blob, np.zeros(31, np.float32), 31, 32)
