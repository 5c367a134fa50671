"""Every instantiation of the persistent decode kernel against the oracle.

The decode kernel is compiled per (weight format, gate/up lane-group width
GG, down lane-group width GD), 2 x 3 x 3 = 18 one-wave variants, plus the
paired two-wave variants for gate/up rows cut into two column slices of
at most 32 chunks (GG 16 or 32), 2 x 2 x 3 = 12 more; the planner picks one
from the shape (column chunks per slice <= 16, <= 32 or <= 64 lanes), the
number of routed instances (narrow layers split gate/up rows into two
column slices) and the down rows' length (32-chunk slices when they
divide).  The paired cases also cross the padding of the item list (the
gate/up items start at an even index of an even-length layer).  Each case below is built to land on one variant; `_plan` mirrors
the planner's rule so a change of the rule shows up here as a failed
geometry assertion rather than as silently lost coverage.  Bar:
assert_ffn_close against the oracle's routed forward and slot-order combine.  The
Q4_0 instances of the QMatMul mode (15 more) run the same shapes."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from test_gpu_parity import Q4, Q8, _oracle_moe, _table, assert_ffn_close, make_expert, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu


def _group_width(chunks: int, min_slices: int = 1) -> int:
    slices = max(-(-chunks // 64), min_slices)
    cps = -(-chunks // slices)
    return 16 if cps <= 16 else (32 if cps <= 32 else 64)


def _plan(dm: int, dff: int, n_tok: int, k: int) -> tuple[int, int, bool]:
    """(GG, GD, paired) as plan_decode chooses them (mer_abi.hip)."""
    g_chunks, d_chunks = dm // 64, dff // 64
    narrow = n_tok * k * (dff // 32) < 512 and g_chunks >= 32
    d32 = d_chunks > 64 and d_chunks % 32 == 0 and k * (d_chunks // 32) <= 16
    g_slices = max(-(-g_chunks // 64), 2 if narrow else 1)
    gg = _group_width(g_chunks, 2 if narrow else 1)
    return gg, _group_width(d_chunks, d_chunks // 32 if d32 else 1), g_slices == 2 and gg <= 32


# (d_model, d_ff, tokens, top_k) -> (GG, GD, paired)
SHAPES = {
    (1024, 1024, 2, 2): (16, 16, False),
    (1024, 2048, 2, 2): (16, 32, False),
    (1024, 4096, 1, 2): (16, 64, False),
    (2048, 1024, 8, 2): (32, 16, False),
    (2048, 2048, 4, 2): (32, 32, False),
    (2048, 4096, 4, 2): (32, 64, False),
    (4096, 1024, 8, 2): (64, 16, False),
    (4096, 2048, 4, 2): (64, 32, False),
    (4096, 4096, 2, 2): (64, 64, False),
    # narrow layers: two gate/up column slices, paired workgroups
    (2048, 1024, 2, 2): (16, 16, True),
    (2048, 2048, 1, 2): (16, 32, True),
    (2048, 4096, 1, 2): (16, 64, True),
    (4096, 1024, 1, 2): (32, 16, True),
    (4096, 2048, 3, 1): (32, 32, True),
    (4096, 4096, 1, 2): (32, 64, True),
}
CASES = [(dt, *shape) for dt in (Q4, Q8) for shape in SHAPES]


@pytest.mark.parametrize("dtype,dm,dff,n_tok,k", CASES)
def test_decode_variant_vs_oracle(mer, oracle, gpu, dtype, dm, dff, n_tok, k):
    gg, gd, paired = SHAPES[(dm, dff, n_tok, k)]
    assert _plan(dm, dff, n_tok, k) == (gg, gd, paired)
    say(f"decode variant fmt={dtype} GG={gg} GD={gd} paired={paired}: dm={dm} dff={dff} tokens={n_tok} top_k={k}")
    rng = np.random.default_rng(dm * 7 + dff + 13 * n_tok + dtype)
    n_exp = 3
    blobs = [make_expert(oracle, dtype, dm, dff, 700 + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
    got = mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu)).cpu().numpy()
    torch.cuda.synchronize()
    mer.take_device_status()
    assert_ffn_close(got, want, f"decode variant fmt={dtype} GG={gg} GD={gd} paired={paired}")
    del devs


@pytest.mark.parametrize("dm,dff,n_tok,k", list(SHAPES))
def test_decode_qmm_variant_vs_oracle(mer, oracle, gpu, dm, dff, n_tok, k):
    """The 15 Q4_0 instances of the QMatMul mode (MER_MOE_QMM, Candle's
    Q8_0 activations), one per shape above, against the oracle's restatement
    of run_inference_q4_0_qmm under the bar of test_gpu_qmm (the FFN bar plus
    the oracle's flip bound)."""
    from test_gpu_qmm import assert_qmm_close

    gg, gd, paired = SHAPES[(dm, dff, n_tok, k)]
    say(f"decode qmm variant GG={gg} GD={gd} paired={paired}: dm={dm} dff={dff} tokens={n_tok} top_k={k}")
    rng = np.random.default_rng(dm * 5 + dff + 11 * n_tok)
    n_exp = 3
    blobs = [make_expert(oracle, Q4, dm, dff, 800 + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = np.zeros((n_tok, dm), np.float32)
    bound = np.zeros((n_tok, dm), np.float64)
    for t in range(n_tok):
        res = [oracle.q4_0_qmm_forward_bounded(blobs[i], x[t], dm, dff) for i in ids[t]]
        want[t] = oracle.combine_outputs(np.stack([r[0] for r in res]), w[t])
        bound[t] = sum(float(w[t, i]) * res[i][1].astype(np.float64) for i in range(k))
    got = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu),
                          qmm=True).cpu().numpy()
    torch.cuda.synchronize()
    mer.take_device_status()
    assert_qmm_close(got, want, bound, f"decode qmm variant GG={gg} GD={gd} paired={paired}")
    del devs
