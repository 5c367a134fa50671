"""Seeded sweeps of the routed forward (mer_hip_moe_forward, and the grouped
mer_hip_moe_grouped) over shapes,
batch sizes, top-k, weight formats and combine flags, against the oracle.

Each case draws its shape from lists that cross the kernel-selection rules:
d_model and d_ff multiples of 32 that take the persistent decode kernel
(with one or two gate/up column slices, 32-chunk or wider down slices),
and shapes with d_model * d_ff not a multiple of 64 that take the generic
path.  Routing picks distinct experts per token; some slots get weight 0
(skipped by the combine, engine.rs:5575-5580).  Bar: assert_ffn_close."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from test_gpu_parity import Q4, Q8, _oracle_moe, _table, assert_ffn_close, make_expert, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu

DMS = [64, 96, 128, 256, 512, 1024, 2048, 4096]
DFFS = [32, 64, 160, 256, 768, 1024, 1408, 2048]
UNALIGNED = [(37, 45), (45, 96), (96, 37)]
N_CASES = 24


def _case(i):
    rng = np.random.default_rng(1000 + i)
    dtype = Q4 if i % 2 == 0 else Q8
    if i % 8 == 7:
        dm, dff = UNALIGNED[(i // 8) % len(UNALIGNED)]
    else:
        dm, dff = int(rng.choice(DMS)), int(rng.choice(DFFS))
        while dm * dff > 4096 * 2048:
            dff //= 2
    n_exp = int(rng.integers(2, 10))
    k = int(rng.integers(1, min(n_exp, 8) + 1))
    n_tok = int(rng.integers(1, 9))
    mode = ("plain", "residual", "accumulate")[i % 3]
    return rng, dtype, dm, dff, n_exp, k, n_tok, mode


@pytest.mark.parametrize("i", range(N_CASES))
def test_moe_forward_sweep(mer, oracle, gpu, i):
    rng, dtype, dm, dff, n_exp, k, n_tok, mode = _case(i)
    say(f"sweep case {i}: dtype={dtype} dm={dm} dff={dff} experts={n_exp} top_k={k} tokens={n_tok} mode={mode}")
    blobs = [make_expert(oracle, dtype, dm, dff, 100 * i + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    w[rng.random((n_tok, k)) < 0.15] = 0.0
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
    if mode == "accumulate":
        base = rng.standard_normal((n_tok, dm)).astype(np.float32)
        out = to_dev(base, gpu)
        mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu),
                        out=out, accumulate=True)
        got, want = out.cpu().numpy(), want + base
    else:
        residual = mode == "residual"
        got = mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                              to_dev(x, gpu), residual=residual).cpu().numpy()
        if residual:
            want = want + x
    torch.cuda.synchronize()
    mer.take_device_status()
    assert_ffn_close(got, want, f"sweep case {i}")
    del devs


# ---- the grouped int8-MFMA path (mer_hip_moe_grouped) ---------------------

G_DMS = [64, 128, 256, 512, 1024, 2048, 4096]
G_DFFS = [64, 128, 192, 256, 768, 1024, 2048]
N_GROUPED = 16


@pytest.mark.parametrize("i", range(N_GROUPED))
def test_moe_grouped_sweep(mer, oracle, gpu, i):
    """Zipf-skewed routing (several pairs of one expert share a 16-pair
    tile), d_model a multiple of 64 as the grouped path requires."""
    from test_gpu_grouped import oracle_moe, routing
    rng = np.random.default_rng(2000 + i)
    dtype = Q8 if i % 2 == 0 else Q4
    dm, dff = int(rng.choice(G_DMS)), int(rng.choice(G_DFFS))
    while dm * dff > 2048 * 1024:
        dff //= 2
    n_exp = int(rng.integers(2, 17))
    k = int(rng.integers(1, min(n_exp, 8) + 1))
    n_tok = int(rng.integers(1, 65))
    mode = ("plain", "residual", "accumulate")[i % 3]
    say(f"grouped sweep case {i}: dtype={dtype} dm={dm} dff={dff} experts={n_exp} top_k={k} tokens={n_tok} mode={mode}")
    blobs = [make_expert(oracle, dtype, dm, dff, 300 * i + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    ids, w = routing.zipf_skewed_routes(n_tok, n_exp, k, 1.1, seed=40 + i)
    w[rng.random((n_tok, k)) < 0.1] = 0.0
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
    args = (mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu))
    if mode == "accumulate":
        base = rng.standard_normal((n_tok, dm)).astype(np.float32)
        out = to_dev(base, gpu)
        mer.moe_grouped(*args, out=out, accumulate=True)
        got, want = out.cpu().numpy(), want + base
    else:
        got = mer.moe_grouped(*args, residual=mode == "residual").cpu().numpy()
        if mode == "residual":
            want = want + x
    torch.cuda.synchronize()
    mer.take_device_status()
    assert_ffn_close(got, want, f"grouped sweep case {i}")
    del devs
