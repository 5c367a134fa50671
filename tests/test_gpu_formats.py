"""End to end from the on-disk formats: experts read out of a GGUF file
(and out of UTH1-headed blobs) into pinned host buffers, made resident
through the slot cache and run by the decode path, against the oracle on
the same bytes.  Bar: the north-star 1e-3 of assert_ffn_close."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import gguf_synth as gs  # noqa: E402
from test_gpu_parity import Q4, Q8, _oracle_moe, assert_ffn_close, say, to_dev  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ggml,dtype,per_expert", [(gs.GGML_Q4_0, Q4, False), (gs.GGML_Q8_0, Q8, True)])
def test_gguf_experts_through_slot_cache(mer, oracle, gpu, tmp_path, ggml, dtype, per_expert):
    dm, dff, ne, k, T = 512, 1024, 8, 2, 3
    say(f"gguf e2e ggml={ggml} per_expert={per_expert}")
    path = tmp_path / "moe.gguf"
    gs.moe_model(path, ggml, dm, dff, ne, layers=(0, 1), per_expert=per_expert, seed=ggml)
    rng = np.random.default_rng(3)
    with mer.GgufExperts(path) as g:
        for layer in (0, 1):
            info = g.moe_layer(layer)
            assert (info.d_model, info.d_ff, info.n_experts, int(info.dtype)) == (dm, dff, ne, dtype)
            host = [g.read_expert(layer, e, mer.pinned_expert_buffer(info.expert_bytes)) for e in range(ne)]
            blobs = [h.numpy().copy() for h in host]
            cache = mer.SlotCache(info.dtype, dm, dff, n_slots=2 * T, n_experts=ne)  # T tokens x top-2 touch at most 2T experts
            ids = np.stack([rng.choice(ne, k, replace=False) for _ in range(T)]).astype(np.int32)
            w = rng.random((T, k)).astype(np.float32)
            x = rng.standard_normal((T, dm)).astype(np.float32)
            distinct = list(dict.fromkeys(int(v) for v in ids.reshape(-1)))
            cache.prepare(distinct, host_blobs=[host[e] for e in distinct])
            out = mer.moe_forward(info.dtype, dm, dff, cache, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu))
            torch.cuda.synchronize()
            mer.take_device_status()
            want = _oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff)
            assert_ffn_close(out.cpu().numpy(), want, f"layer {layer}")
            cache.close()


def test_uth_headed_blobs_strip_to_the_device_path(mer, oracle, gpu):
    """Blobs written with the UTH1 SwiGLU header (page-aligned payload)
    dispatch from the stripped payload, as a resident expert does."""
    dm, dff, ne = 256, 512, 3
    say("uth strip e2e")
    rng = np.random.default_rng(9)
    nb = dm * dff // 32
    raw = [np.concatenate([gs.q_blocks(gs.GGML_Q8_0, nb, rng) for _ in range(3)]) for _ in range(ne)]
    headed = [np.frombuffer(mer.swiglu_expert_header(mer.UthDtype.Q8_0, dm, dff) + r.tobytes(), np.uint8)
              for r in raw]
    payloads = []
    for hb in headed:
        h, p = mer.strip_uth(hb)
        assert h.kind == 1 and (h.d_model, h.d_ff) == (dm, dff) and h.payload_offset == 4096
        payloads.append(to_dev(np.ascontiguousarray(p), gpu))
    table = torch.tensor([p.data_ptr() for p in payloads], dtype=torch.int64, device=gpu)
    ids = np.array([[0, 2], [1, 0]], np.int32)
    w = np.array([[0.7, 0.3], [0.5, 0.5]], np.float32)
    x = rng.standard_normal((2, dm)).astype(np.float32)
    out = mer.moe_forward(mer.WeightDtype.Q8_0, dm, dff, table, to_dev(ids, gpu), to_dev(w, gpu), to_dev(x, gpu))
    torch.cuda.synchronize()
    mer.take_device_status()
    assert_ffn_close(out.cpu().numpy(), _oracle_moe(oracle, Q8, raw, ids, w, x, dm, dff), "uth")
