"""Parity of the gfx950 path (through the C ABI) against the CPU oracle.

Bars: dequantised weights, raw Q4 matvec on dyadic fixtures, and the
synthetic generator are bit-exact; FFN outputs satisfy the north-star
max-abs/rel 1e-3 bar in the combined form of the reference's
compare_vectors (q4_parity.rs:677-737):
    |gpu - ref| <= 1e-3 * |ref| + 1e-3 * max(1, 1e-3 * max|ref|).
For outputs up to magnitude 1000 the absolute term is exactly 1e-3.  For
larger outputs it is 1e-6 of the output scale: an entry that cancels to
near zero inside a sum of terms of size max|ref| carries fp32 reordering
noise of ~1e-7 of that scale whatever the summation order, so a fixed
1e-3 floor would test the summation order rather than the kernel.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

Q4, Q8 = 4, 5
ABS_TOL = 1e-3
REL_TOL = 1e-3
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def assert_ffn_close(got, ref, label):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, label
    got, ref = got.ravel(), ref.ravel()
    assert np.isfinite(got).all(), label
    err = np.abs(got - ref)
    scale = max(1.0, float(np.abs(ref).max()))
    abs_bar = ABS_TOL * max(1.0, 1e-3 * scale)
    if abs_bar > ABS_TOL:
        # outputs reaching thousands: the absolute floor scales with the largest |ref|
        say(f"{label}: absolute floor {abs_bar:.3g} (max|ref| {scale:.3g}), relative {REL_TOL}")
    allowed = REL_TOL * np.abs(ref) + abs_bar
    worst = int(np.argmax(err / allowed))
    assert (err <= allowed).all(), (
        f"{label}: worst index {worst} gpu={got[worst]} ref={ref[worst]} err={err[worst]} allowed={allowed[worst]}")


def make_expert(oracle, dtype, dm, dff, expert_index=0, seed=0xC0FFEE):
    """Synthetic expert with the bench generator (oracle side)."""
    nb = oracle.expert_weight_bytes(dtype, dm, dff) // oracle.BLOCK_BYTES[dtype]
    lo, hi = (0.005, 0.02) if dtype == Q4 else (0.002, 0.01)
    return oracle.bench_fill(dtype, seed, expert_index, 0, nb, lo, hi)


def randn(n, seed):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


# ---- bit-exact pieces ----------------------------------------------------

@pytest.mark.parametrize("dtype", [Q4, Q8])
def test_dequant_bit_exact(mer, oracle, gpu, dtype):
    say(f"dequant dtype={dtype}")
    bb = oracle.BLOCK_BYTES[dtype]
    rng = np.random.default_rng(dtype)
    blocks = rng.integers(0, 256, (4099, bb), dtype=np.uint8)
    blocks[:, 1] &= 0x7B  # finite scales
    edge = [0x0000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF, 0x3C00]
    for i, s in enumerate(edge):
        blocks[i, 0], blocks[i, 1] = s & 0xFF, s >> 8
    src = blocks.ravel()
    n_weights = 4099 * 32 - 13  # tail block truncated
    want = oracle.dequantize_to_f32(dtype, src, n_weights)
    got = mer.dequantize_to_f32(mer.WeightDtype(dtype), to_dev(src, gpu), n_weights).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_raw_q4_canonical_cases_exact(mer, oracle, gpu):
    nib = GOLDEN["q4_canonical_nibbles"]
    for c in GOLDEN["q4_canonical_raw_cases"]["cases"]:
        say(f"raw q4 case {c['name']}")
        w = np.concatenate([oracle.canonical_block(s, nib[n]) for s, n in c["blocks"]])
        x = oracle.deterministic_input(c["columns"], c["input_seed"])
        want = oracle.cpu_q4_matvec(w, c["w_block_off"], c["rows"], c["columns"], x)
        got = mer.q4_0_matvec(to_dev(w, gpu), c["w_block_off"], c["rows"], c["columns"], to_dev(x, gpu))
        got = got.cpu().numpy()
        # the reference reports raw max error 0 on GPU hardware
        assert np.array_equal(got, want), c["name"]


def test_raw_q4_rejects_bad_geometry(mer, gpu):
    w = torch.zeros(18 * 3, dtype=torch.uint8, device=gpu)
    x = torch.zeros(32, dtype=torch.float32, device=gpu)
    with pytest.raises(mer.InvalidLayout):
        mer.q4_0_matvec(w, 2, 2, 32, x)  # needs 4 blocks, has 3
    with pytest.raises(mer.InvalidLayout):
        mer.q4_0_matvec(w, 0, 1, 48, x)


@pytest.mark.parametrize("dtype", [Q4, Q8])
def test_fill_synthetic_matches_oracle(mer, oracle, gpu, dtype):
    say(f"fill dtype={dtype}")
    bb = oracle.BLOCK_BYTES[dtype]
    n = 5000
    want = oracle.bench_fill(dtype, 0xC0FFEE, 17, 1234, n, 0.005, 0.02)
    out = torch.empty(n * bb, dtype=torch.uint8, device=gpu)
    mer.fill_synthetic(mer.WeightDtype(dtype), 0xC0FFEE, 17, n, 0.005, 0.02, out, block_begin=1234)
    assert np.array_equal(out.cpu().numpy(), want)


# ---- expert forward --------------------------------------------------------

Q4_SHAPES = [(32, 32), (64, 96), (37, 45), (128, 128), (256, 1024), (1024, 256), (7168, 2048), (4096, 14336)]
Q8_SHAPES = [(32, 32), (64, 96), (37, 45), (64, 45), (37, 64), (2048, 768), (512, 4096)]


@pytest.mark.parametrize("dm,dff", Q4_SHAPES)
def test_expert_forward_q4_vs_oracle(mer, oracle, gpu, dm, dff):
    say(f"q4 expert forward dm={dm} dff={dff}")
    blob = make_expert(oracle, Q4, dm, dff)
    x = randn(dm, dm + dff)
    want = oracle.q4_0_reference_forward(blob, x, dm, dff, nthreads=16)
    got = mer.q4_0_forward(to_dev(blob, gpu), to_dev(x, gpu), dm, dff).cpu().numpy()
    assert_ffn_close(got, want, f"q4 {dm}x{dff}")


@pytest.mark.parametrize("dm,dff", Q8_SHAPES)
def test_expert_forward_q8_vs_oracle(mer, oracle, gpu, dm, dff):
    say(f"q8 expert forward dm={dm} dff={dff}")
    blob = make_expert(oracle, Q8, dm, dff)
    x = randn(dm, 3 * dm + dff)
    rc, want = oracle.q8_0_direct_forward(blob, x, dm, dff, kernel=1, nthreads=16)
    assert rc == 0
    y = torch.empty(dm, dtype=torch.float32, device=gpu)
    mer.forward_q8_0_direct_into(to_dev(blob, gpu), to_dev(x, gpu), dm, dff, y)
    assert_ffn_close(y.cpu().numpy(), want, f"q8 {dm}x{dff}")


def test_q8_reference_generator_expert(mer, oracle, gpu):
    # randomized_q8_expert + synth_hidden_state at the Qwen shape
    # (inference.rs:6138-6161 inputs), against the scalar-order oracle.
    dm, dff = 2048, 768
    say("q8 randomized reference expert 2048x768")
    blob = oracle.randomized_q8_expert(dm, dff, 0x20480768)
    x = oracle.synth_hidden_state(23, dm, 11)
    rc, want = oracle.q8_0_direct_forward(blob, x, dm, dff, kernel=0)
    assert rc == 0
    got = mer.dispatch_expert_forward(mer.WeightDtype.Q8_0, to_dev(blob, gpu), to_dev(x, gpu), dm, dff)
    assert_ffn_close(got.cpu().numpy(), want, "q8 randomized")


def test_q4_reference_generator_expert(mer, oracle, gpu):
    # io_provider.rs synthetic experts (max-abs quantised U(-1/sqrt(d),..))
    dm, dff = 1024, 2048
    say("q4 io_provider synthetic expert 1024x2048")
    blob = oracle.generate_synthetic_expert(Q4, 5, dm, dff)
    x = oracle.synth_hidden_state(3, dm, 1)
    want = oracle.q4_0_reference_forward(blob, x, dm, dff)
    got = mer.q4_0_forward(to_dev(blob, gpu), to_dev(x, gpu), dm, dff)
    assert_ffn_close(got.cpu().numpy(), want, "q4 io_provider")


def test_q4_complete_fixture(mer, oracle, gpu):
    g = GOLDEN["q4_complete_fixture"]
    say("q4 complete fixture 32x32")
    blk = oracle.canonical_block(g["scale"], GOLDEN["q4_canonical_nibbles"]["ramp"])
    blob = np.tile(blk, oracle.expert_weight_bytes(Q4, 32, 32) // 18)
    x = oracle.deterministic_input(32, g["input_seed"])
    want = oracle.q4_0_reference_forward(blob, x, 32, 32)
    got = mer.q4_0_forward(to_dev(blob, gpu), to_dev(x, gpu), 32, 32).cpu().numpy()
    assert np.isfinite(got).all() and (got != 0).any()
    assert_ffn_close(got, want, "complete fixture")


def test_expert_forward_is_deterministic(mer, oracle, gpu):
    dm, dff = 4096, 14336
    say("determinism 4096x14336")
    blob = to_dev(make_expert(oracle, Q4, dm, dff, 3), gpu)
    x = to_dev(randn(dm, 5), gpu)
    a = mer.q4_0_forward(blob, x, dm, dff).cpu().numpy()
    b = mer.q4_0_forward(blob, x, dm, dff).cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_expert_forward_unaligned_pointer_uses_generic_path(mer, oracle, gpu):
    dm, dff = 128, 128
    say("unaligned device pointer 128x128")
    blob = make_expert(oracle, Q4, dm, dff)
    buf = torch.zeros(blob.size + 2, dtype=torch.uint8, device=gpu)
    buf[2:] = to_dev(blob, gpu)
    x = randn(dm, 9)
    want = oracle.q4_0_reference_forward(blob, x, dm, dff)
    got = mer.q4_0_forward(buf[2:], to_dev(x, gpu), dm, dff).cpu().numpy()
    assert_ffn_close(got, want, "unaligned")


def test_expert_forward_host_entry(mer, oracle, gpu):
    dm, dff = 2048, 768
    say("host entry q8 2048x768")
    blob = make_expert(oracle, Q8, dm, dff, 2)
    x = randn(dm, 4)
    rc, want = oracle.q8_0_direct_forward(blob, x, dm, dff)
    got = mer.expert_forward_host(mer.WeightDtype.Q8_0, blob, x, dm, dff)
    assert_ffn_close(got, want, "host entry")


def test_expert_forward_errors(mer, oracle, gpu):
    dm, dff = 4096, 14336
    need = oracle.expert_weight_bytes(Q4, dm, dff)
    say("error paths")
    buf = torch.zeros(need, dtype=torch.uint8, device=gpu)
    x = torch.zeros(dm, dtype=torch.float32, device=gpu)
    with pytest.raises(mer.TruncatedPayload) as e:
        mer.q4_0_forward(buf[: need - 100], x, dm, dff)
    assert (e.value.have, e.value.need) == (need - 100, need)
    with pytest.raises(mer.BufferTooSmall):
        mer.q4_0_forward(buf[:1000], x, dm, dff)
    with pytest.raises(mer.Candle):
        mer.q4_0_forward(buf, x[:10], dm, dff)
    with pytest.raises(mer.InvalidLayout):
        mer.dispatch_expert_forward(mer.WeightDtype.Q8_0, buf, x[:31], 32, 32)
    with pytest.raises(mer.RoutedExpertGpuIncompatibility):
        mer.dispatch_expert_forward(3, buf, x, 32, 32)


def test_q8_nonfinite_activation_propagates(mer, oracle, gpu):
    say("q8 non-finite propagation")
    blob = oracle.randomized_q8_expert(32, 32, 5)
    x = np.full(32, 0.25, np.float32)
    x[3], x[17] = np.nan, np.inf
    y = mer.dispatch_expert_forward(mer.WeightDtype.Q8_0, to_dev(blob, gpu), to_dev(x, gpu), 32, 32)
    assert not np.isfinite(y.cpu().numpy()).all()


def test_q4_zero_dff_returns_zeros(mer, gpu):
    say("q4 d_ff=0")
    y = torch.full((8,), 7.0, device=gpu)
    mer.dispatch_expert_forward(mer.WeightDtype.Q4_0, torch.zeros(0, dtype=torch.uint8, device=gpu),
                                torch.zeros(8, device=gpu), 8, 0, out=y)
    assert (y.cpu() == 0).all()


# ---- routed experts + combine -----------------------------------------------

def _table(blobs, gpu):
    devs = [to_dev(b, gpu) for b in blobs]
    table = torch.tensor([d.data_ptr() for d in devs], dtype=torch.int64, device=gpu)
    return devs, table


@pytest.mark.parametrize("dtype,dm,dff", [(Q4, 256, 512), (Q8, 256, 512), (Q4, 96, 160), (Q8, 2048, 768)])
def test_moe_forward_vs_oracle_combine(mer, oracle, gpu, dtype, dm, dff):
    say(f"moe forward dtype={dtype} dm={dm} dff={dff}")
    n_exp, n_tok, k = 6, 3, 2
    blobs = [make_expert(oracle, dtype, dm, dff, e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    rng = np.random.default_rng(11)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    w[1, 1] = 0.0  # zero weight slot is skipped (engine.rs:5575-5580)
    x = rng.standard_normal((n_tok, dm)).astype(np.float32)
    want = np.zeros((n_tok, dm), np.float32)
    for t in range(n_tok):
        ys = []
        for i in range(k):
            if dtype == Q4:
                ys.append(oracle.q4_0_reference_forward(blobs[ids[t, i]], x[t], dm, dff))
            else:
                ys.append(oracle.q8_0_direct_forward(blobs[ids[t, i]], x[t], dm, dff)[1])
        want[t] = oracle.combine_outputs(np.stack(ys), w[t])
    got = mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                          to_dev(x, gpu)).cpu().numpy()
    assert_ffn_close(got, want, "moe")
    got_r = mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu),
                            to_dev(x, gpu), residual=True).cpu().numpy()
    assert_ffn_close(got_r, want + x, "moe residual")
    out = to_dev(np.ones((n_tok, dm), np.float32), gpu)
    mer.moe_forward(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu),
                    out=out, accumulate=True)
    assert_ffn_close(out.cpu().numpy(), want + 1, "moe accumulate")
    mer.take_device_status()
    del devs


def test_moe_forward_missing_expert_records_residency_miss(mer, oracle, gpu):
    dm, dff = 128, 256
    say("moe missing expert")
    blobs = [make_expert(oracle, Q4, dm, dff, e) for e in range(2)]
    devs, table = _table(blobs, gpu)
    table = torch.cat([table, torch.zeros(1, dtype=torch.int64, device=gpu)])  # id 2 not resident
    ids = torch.tensor([[0, 2], [1, 7]], dtype=torch.int32, device=gpu)  # 7 out of table
    w = torch.tensor([[0.5, 0.5], [0.25, 0.75]], dtype=torch.float32, device=gpu)
    x = to_dev(randn(2 * dm, 1).reshape(2, dm), gpu)
    got = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, table, ids, w, x).cpu().numpy()
    xs = x.cpu().numpy()
    want0 = 0.5 * oracle.q4_0_reference_forward(blobs[0], xs[0], dm, dff)
    want1 = 0.25 * oracle.q4_0_reference_forward(blobs[1], xs[1], dm, dff)
    assert_ffn_close(got[0], want0, "miss row 0")
    assert_ffn_close(got[1], want1, "miss row 1")
    with pytest.raises(mer.GpuExpertDispatchError) as e:
        mer.take_device_status()
    assert e.value.kind == mer.GpuExpertDispatchErrorKind.ResidencyMiss
    mer.take_device_status()  # cleared
    del devs


def test_moe_forward_full_mixtral_top2(mer, oracle, gpu):
    """Full-size property: fused top-2 + combine equals the weighted sum
    of two single-expert forwards, and the oracle."""
    dm, dff = 4096, 14336
    say("moe full mixtral top-2")
    blobs = [make_expert(oracle, Q4, dm, dff, e) for e in (4, 9)]
    devs, table = _table(blobs, gpu)
    x = randn(dm, 77)
    ids_np, w_np = oracle.topk_softmax_logits(randn(8, 78), 2)
    ids = torch.tensor([[0, 1]], dtype=torch.int32, device=gpu)
    w = to_dev(w_np.reshape(1, 2), gpu)
    got = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, table, ids, w, to_dev(x.reshape(1, dm), gpu))
    got = got.cpu().numpy()[0]
    y0 = mer.q4_0_forward(devs[0], to_dev(x, gpu), dm, dff).cpu().numpy()
    y1 = mer.q4_0_forward(devs[1], to_dev(x, gpu), dm, dff).cpu().numpy()
    assert_ffn_close(got, w_np[0] * y0 + w_np[1] * y1, "fused vs separate")
    want = oracle.combine_outputs(np.stack([oracle.q4_0_reference_forward(b, x, dm, dff, 16) for b in blobs]), w_np)
    assert_ffn_close(got, want, "fused vs oracle")


# ---- all layers of a decode step in one launch ----------------------------

def _oracle_expert(oracle, dtype, blob, x, dm, dff):
    if dtype == Q4:
        return oracle.q4_0_reference_forward(blob, x, dm, dff)
    rc, y = oracle.q8_0_direct_forward(blob, x, dm, dff)
    assert rc == 0
    return y


def _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff):
    out = np.zeros_like(x)
    for t in range(x.shape[0]):
        ys = np.stack([_oracle_expert(oracle, dtype, blobs[ids[t, i]], x[t], dm, dff) for i in range(ids.shape[1])])
        out[t] = oracle.combine_outputs(ys, w[t])
    return out


LAYER_MODES = [("accumulate", Q4), ("residual", Q4), ("plain", Q4), ("chain", Q4), ("chain_residual", Q4),
               ("accumulate_strict", Q4), ("chain_residual_strict", Q4), ("accumulate", Q8), ("residual", Q8)]


@pytest.mark.parametrize("mode,dtype", LAYER_MODES)
def test_moe_forward_layers_vs_oracle(mer, oracle, gpu, mode, dtype):
    """mer_hip_moe_forward_layers against the oracle run layer by layer, for
    every flag combination; a second launch with new inputs reuses the
    library's scratch and must not see the first launch's data."""
    dm, dff, n_layers, n_exp, n_tok, k = 256, 512, 3, 4, 2, 2
    chain, residual = "chain" in mode, "residual" in mode
    accumulate, strict = "accumulate" in mode, "strict" in mode
    say(f"moe layers mode={mode} dtype={dtype}")
    blobs = [[make_expert(oracle, dtype, dm, dff, l * n_exp + e) for e in range(n_exp)] for l in range(n_layers)]
    tables = [_table(b, gpu) for b in blobs]
    rng = np.random.default_rng(31)
    ids = [np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
           for _ in range(n_layers)]
    w = [rng.random((n_tok, k)).astype(np.float32) for _ in range(n_layers)]
    for launch in range(2):
        xs = [rng.standard_normal((n_tok, dm)).astype(np.float32) for _ in range(n_layers)]
        acc0 = rng.standard_normal((n_tok, dm)).astype(np.float32)
        shared = to_dev(acc0, gpu) if accumulate else None
        layers = []
        for l in range(n_layers):
            layers.append(dict(table=tables[l][1], ids=to_dev(ids[l], gpu), weights=to_dev(w[l], gpu),
                               x=None if chain and l > 0 else to_dev(xs[l], gpu),
                               out=shared if accumulate else torch.zeros((n_tok, dm), device=gpu)))
        mer.moe_forward_layers(mer.WeightDtype(dtype), dm, dff, layers, residual=residual, accumulate=accumulate,
                               chain=chain, route_after_prev=strict)
        torch.cuda.synchronize()
        acc = acc0.copy()
        prev = None
        for l in range(n_layers):
            xin = prev if chain and l > 0 else xs[l]
            y = _oracle_moe(oracle, dtype, blobs[l], ids[l], w[l], xin, dm, dff)
            if accumulate:
                acc = acc + y
                continue
            want = xin + y if residual else y
            assert_ffn_close(layers[l]["out"].cpu().numpy(), want, f"launch {launch} layer {l}")
            prev = layers[l]["out"].cpu().numpy() if chain else None
        if accumulate:
            assert_ffn_close(shared.cpu().numpy(), acc, f"launch {launch} accumulated")
    mer.take_device_status()
    del tables


def test_null_device_pointers_rejected_before_launch(mer, gpu):
    """Every entry point that takes device buffers refuses a null one with
    MER_ERR_INVALID_LAYOUT before any kernel is launched."""
    say("null device pointers")
    lib = mer._lib.lib()
    bad = mer._lib.Status.INVALID_LAYOUT
    buf = torch.zeros(4096, dtype=torch.uint8, device=gpu)
    f = torch.zeros(256, dtype=torch.float32, device=gpu)
    assert lib.mer_hip_q4_0_matvec(None, 18, 0, 1, 32, f.data_ptr(), f.data_ptr(), None) == bad
    assert lib.mer_hip_q4_0_matvec(buf.data_ptr(), 18, 0, 1, 32, None, f.data_ptr(), None) == bad
    assert lib.mer_hip_q4_0_matvec(buf.data_ptr(), 18, 0, 1, 32, f.data_ptr(), None, None) == bad
    assert lib.mer_hip_fill_synthetic(4, 1, 0, 0, 4, 0.01, 0.02, None, None) == bad
    assert lib.mer_hip_fill_synthetic(4, 1, 0, 0, 0, 0.01, 0.02, None, None) == 0  # nothing to fill
    assert lib.mer_hip_dequantize(4, None, 18, 32, f.data_ptr(), None) == bad
    assert lib.mer_hip_expert_forward(4, None, 0, f.data_ptr(), 64, 64, 64, f.data_ptr(), 64, None) != 0
    ids = torch.zeros((1, 1), dtype=torch.int32, device=gpu)
    for args in ((None, 1, ids.data_ptr(), f.data_ptr(), f.data_ptr(), f.data_ptr()),
                 (buf.data_ptr(), 1, None, f.data_ptr(), f.data_ptr(), f.data_ptr()),
                 (buf.data_ptr(), 1, ids.data_ptr(), f.data_ptr(), None, f.data_ptr())):
        table, n, i, w, x, o = args
        assert lib.mer_hip_moe_forward(4, 64, 64, 1, 1, table, n, i, w, x, o, 0, None) == bad
        assert lib.mer_hip_moe_grouped(4, 64, 64, 1, 1, table, n, i, w, x, o, 0, None) == bad
    assert lib.mer_hip_expert_batch_f16(4, 64, 64, 1, buf.data_ptr(), 1, ids.data_ptr(), None, f.data_ptr(), None) == bad
    torch.cuda.synchronize()
    mer.take_device_status()


@pytest.mark.parametrize("path,dtype,dm,dff", [("decode", Q4, 512, 1024), ("decode", Q8, 2048, 768),
                                               ("generic", Q4, 96, 160), ("grouped", Q8, 256, 512),
                                               ("layers", Q4, 256, 512)])
def test_swiglu_limit_matches_oracle(mer, oracle, gpu, path, dtype, dm, dff):
    """mer_set_swiglu_limit: every kernel family clamps the gate before SiLU
    as clamp_swiglu_gate does (inference.rs:86-123, :3689-3702); the limit
    is chosen so it binds on a good part of the rows.  Removing it restores
    the unclamped outputs bit for bit."""
    say(f"swiglu limit path={path} dtype={dtype} dm={dm} dff={dff}")
    n_exp, n_tok, k = 4, 3, 2
    blobs = [make_expert(oracle, dtype, dm, dff, 60 + e) for e in range(n_exp)]
    devs, table = _table(blobs, gpu)
    rng = np.random.default_rng(31)
    ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, k)).astype(np.float32)
    x = (rng.standard_normal((n_tok, dm)) * 3).astype(np.float32)
    limit = 0.5 if dtype == Q4 else 2.0
    wd = mer.WeightDtype(dtype)

    def run():
        if path == "grouped":
            return mer.moe_grouped(wd, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu)).cpu().numpy()
        if path == "layers":
            outs = [torch.zeros((n_tok, dm), device=gpu) for _ in range(2)]
            layers = [dict(table=table, ids=to_dev(ids, gpu), weights=to_dev(w, gpu), x=to_dev(x, gpu), out=outs[l])
                      for l in range(2)]
            mer.moe_forward_layers(wd, dm, dff, layers)
            return outs[1].cpu().numpy()
        return mer.moe_forward(wd, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu)).cpu().numpy()

    plain = run()
    try:
        mer.set_swiglu_limit(limit)
        oracle.set_swiglu_limit(limit)
        assert mer.swiglu_limit() == limit
        got = run()
        want = _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
    finally:
        mer.set_swiglu_limit(None)
        oracle.set_swiglu_limit(None)
    assert_ffn_close(got, want, f"{path} clamped")
    assert np.abs(got - plain).max() > 10 * ABS_TOL, "the clamp did not bind"
    assert mer.swiglu_limit() is None
    assert np.array_equal(run(), plain)
    mer.take_device_status()
    del devs
