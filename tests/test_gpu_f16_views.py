"""The GPU backend's f16-view entry points (mer_hip_expert_batch_f16):
routed_expert_matmul_batch_q4 and expert_matmul on an f16 hidden state,
one uncombined f16 output row per expert, against the oracle run on the
same (f16-exact) input.

Bar: the north-star 1e-3 of assert_ffn_close plus the f16 output rounding,
|got - ref| <= 1e-3 |ref| + 1e-3 max(1, 1e-3 max|ref|) + 2^-11 |ref|."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from test_gpu_parity import Q4, Q8, _oracle_expert, _table, make_expert, randn, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu


def assert_f16_close(got16, ref, label):
    got = np.asarray(got16, np.float32).ravel()
    ref = np.asarray(ref, np.float32).ravel()
    assert np.isfinite(got).all(), label
    floor = 1e-3 * max(1.0, 1e-3 * float(np.abs(ref).max()))
    allowed = 1e-3 * np.abs(ref) + floor + np.abs(ref) * 2.0 ** -11
    err = np.abs(got - ref)
    worst = int(np.argmax(err / allowed))
    assert (err <= allowed).all(), f"{label}: worst {worst} gpu={got[worst]} ref={ref[worst]} err={err[worst]}"


@pytest.mark.parametrize("dtype,dm,dff,n", [(Q4, 512, 1024, 8), (Q8, 512, 256, 8), (Q8, 96, 160, 3), (Q4, 4096, 14336, 2)])
def test_expert_batch_f16_vs_oracle(mer, oracle, gpu, dtype, dm, dff, n):
    """Layer batch of n experts (8 = the reference's batch size) on one
    hidden state; the 96 x 160 shape takes the generic kernels, 4096 x 14336
    is a Mixtral expert."""
    say(f"f16 batch dtype={dtype} {dm}x{dff} n={n}")
    blobs = [make_expert(oracle, dtype, dm, dff, 40 + e) for e in range(n + 1)]
    devs, table = _table(blobs, gpu)
    ids = np.array([(3 * i + 1) % (n + 1) for i in range(n)], np.int32)
    x16 = (randn(dm, 5) * 0.5).astype(np.float16)
    out = mer.routed_expert_matmul_batch(mer.WeightDtype(dtype), dm, dff, table, to_dev(ids, gpu),
                                         to_dev(x16, gpu))
    torch.cuda.synchronize()
    mer.take_device_status()
    assert out.dtype == torch.float16 and tuple(out.shape) == (n, dm)
    got = out.cpu().numpy()
    x32 = x16.astype(np.float32)
    for i in range(n):
        assert_f16_close(got[i], _oracle_expert(oracle, dtype, blobs[ids[i]], x32, dm, dff), f"expert row {i}")
    del devs


def test_expert_matmul_single_equals_batch_row(mer, oracle, gpu):
    dm, dff = 256, 512
    say("f16 expert_matmul")
    blobs = [make_expert(oracle, Q4, dm, dff, e) for e in range(3)]
    devs, table = _table(blobs, gpu)
    x16 = to_dev(randn(dm, 9).astype(np.float16), gpu)
    one = mer.expert_matmul(mer.WeightDtype.Q4_0, dm, dff, table, 2, x16)
    batch = mer.routed_expert_matmul_batch(mer.WeightDtype.Q4_0, dm, dff, table,
                                           torch.tensor([0, 2], dtype=torch.int32, device=gpu), x16)
    torch.cuda.synchronize()
    assert tuple(one.shape) == (dm,)
    assert torch.equal(one, batch[1])
    assert_f16_close(one.cpu().numpy(), _oracle_expert(oracle, Q4, blobs[2], x16.cpu().numpy().astype(np.float32), dm, dff),
                     "single")
    mer.take_device_status()
    del devs


def test_expert_batch_f16_missing_expert(mer, oracle, gpu):
    """A non-resident expert gives a zero row and a residency miss; the
    other rows are unaffected."""
    dm, dff = 128, 256
    say("f16 batch missing expert")
    blobs = [make_expert(oracle, Q8, dm, dff, e) for e in range(2)]
    devs, table = _table(blobs, gpu)
    ids = torch.tensor([1, 5, 0], dtype=torch.int32, device=gpu)
    x16 = (randn(dm, 3)).astype(np.float16)
    got = mer.routed_expert_matmul_batch(mer.WeightDtype.Q8_0, dm, dff, table, ids, to_dev(x16, gpu)).cpu().numpy()
    assert not got[1].any()
    x32 = x16.astype(np.float32)
    assert_f16_close(got[0], _oracle_expert(oracle, Q8, blobs[1], x32, dm, dff), "row 0")
    assert_f16_close(got[2], _oracle_expert(oracle, Q8, blobs[0], x32, dm, dff), "row 2")
    with pytest.raises(mer.GpuExpertDispatchError) as e:
        mer.take_device_status()
    assert e.value.kind == mer.GpuExpertDispatchErrorKind.ResidencyMiss
    mer.take_device_status()
    del devs


def test_expert_batch_f16_rejects_bad_arguments(mer, gpu):
    table = torch.zeros(1, dtype=torch.int64, device=gpu)
    ids = torch.zeros(1, dtype=torch.int32, device=gpu)
    x = torch.zeros(64, dtype=torch.float16, device=gpu)
    with pytest.raises(mer.RoutedExpertGpuIncompatibility):
        mer.routed_expert_matmul_batch(3, 64, 64, table, ids, x)  # Q4K: not on this path
    with pytest.raises(ValueError):
        mer.routed_expert_matmul_batch(mer.WeightDtype.Q4_0, 128, 64, table, ids, x)
    with pytest.raises(TypeError):
        mer.routed_expert_matmul_batch(mer.WeightDtype.Q4_0, 64, 64, table, ids, x.float())
