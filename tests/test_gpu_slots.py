"""The VRAM expert-slot cache (mer_slot_cache_*): routed forwards through
its slot table against the CPU oracle, LRU eviction, the directional
generation rule of the physical registry (backend/mod.rs:709-741, tests at
backend/mod.rs:6160-6250), capacity failures that change nothing, and
prefetch.  Every step's compute is enqueued without host waits, so a slot
reused by a later step checks that uploads wait for earlier compute."""
from __future__ import annotations

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

Q4, Q8 = 4, 5
ABS_TOL = 1e-3
REL_TOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def assert_ffn_close(got, ref, label):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, label
    assert np.isfinite(got).all(), label
    err = np.abs(got - ref)
    scale = max(1.0, float(np.abs(ref).max()))
    allowed = REL_TOL * np.abs(ref) + ABS_TOL * max(1.0, 1e-3 * scale)
    worst = int(np.argmax(err / allowed))
    assert (err <= allowed).all(), (
        f"{label}: worst index {worst} gpu={got[worst]} ref={ref[worst]} err={err[worst]} allowed={allowed[worst]}")


def make_expert(oracle, dtype, dm, dff, expert_index, seed=0x51075):
    nb = oracle.expert_weight_bytes(dtype, dm, dff) // oracle.BLOCK_BYTES[dtype]
    lo, hi = (0.005, 0.02) if dtype == Q4 else (0.002, 0.01)
    return oracle.bench_fill(dtype, seed, expert_index, 0, nb, lo, hi)


def pinned(mer, blob):
    t = mer.pinned_expert_buffer(blob.nbytes)
    t.numpy()[:] = blob
    return t


def oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff):
    out = np.zeros_like(x)
    for t in range(x.shape[0]):
        ys = []
        for i in range(ids.shape[1]):
            b = blobs[ids[t, i]]
            if dtype == Q4:
                ys.append(oracle.q4_0_reference_forward(b, x[t], dm, dff))
            else:
                rc, y = oracle.q8_0_direct_forward(b, x[t], dm, dff)
                assert rc == 0
                ys.append(y)
        out[t] = oracle.combine_outputs(np.stack(ys), w[t])
    return out


class LruModel:
    """Expected slot bookkeeping: hits touched first, then each miss takes a
    free slot (lowest index) or the least recently used slot not needed by
    the same call."""

    def __init__(self, n_slots):
        self.expert = [None] * n_slots
        self.last = [0] * n_slots
        self.tick = 0
        self.hits = self.misses = self.evictions = 0

    def prepare(self, ids):
        needed = set()
        for e in ids:
            if e in self.expert:
                s = self.expert.index(e)
                if s not in needed:
                    self.hits += 1
                needed.add(s)
                self.tick += 1
                self.last[s] = self.tick
        for e in ids:
            if e in self.expert:
                continue
            free = [s for s in range(len(self.expert)) if self.expert[s] is None and s not in needed]
            if free:
                v = free[0]
            else:
                v = min((s for s in range(len(self.expert)) if s not in needed), key=lambda s: self.last[s])
                self.evictions += 1
            self.expert[v] = e
            self.tick += 1
            self.last[v] = self.tick
            needed.add(v)
            self.misses += 1


@pytest.mark.parametrize("dtype,dm,dff", [(Q4, 256, 512), (Q8, 256, 512)])
def test_slot_cache_steps_vs_oracle(mer, oracle, gpu, dtype, dm, dff):
    """A stream of routed steps over 10 experts through 4 slots, all steps
    enqueued before any host wait; every output against the oracle and the
    hit/miss/eviction counts against the LRU rule."""
    say(f"slot cache steps dtype={dtype} dm={dm} dff={dff}")
    n_exp, n_slots, n_tok, k = 10, 4, 2, 2
    blobs = [make_expert(oracle, dtype, dm, dff, e) for e in range(n_exp)]
    host = [pinned(mer, b) for b in blobs]
    rng = np.random.default_rng(7)
    model = LruModel(n_slots)
    cache = mer.SlotCache(mer.WeightDtype(dtype), dm, dff, n_slots, n_exp)
    assert cache.expert_bytes == blobs[0].nbytes
    steps = []
    for step in range(12):
        if step % 4 == 3:
            ids = steps[-1][0].copy()  # a repeated set: all hits
        else:
            ids = np.stack([rng.choice(n_exp, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
        w = rng.random((n_tok, k)).astype(np.float32)
        x = rng.standard_normal((n_tok, dm)).astype(np.float32)
        flat = [int(e) for e in ids.reshape(-1)]
        distinct = list(dict.fromkeys(flat))
        cache.prepare(distinct, host_blobs=[host[e] for e in distinct])
        model.prepare(distinct)
        out = mer.moe_forward(mer.WeightDtype(dtype), dm, dff, cache, torch.from_numpy(ids).to(gpu),
                              torch.from_numpy(w).to(gpu), torch.from_numpy(x).to(gpu))
        steps.append((ids, w, x, out))
    torch.cuda.synchronize()
    mer.take_device_status()
    for i, (ids, w, x, out) in enumerate(steps):
        assert_ffn_close(out.cpu().numpy(), oracle_moe(oracle, dtype, blobs, ids, w, x, dm, dff), f"step {i}")
    st = cache.stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (model.hits, model.misses, model.evictions), st
    assert st["evictions"] > 0 and st["hits"] > 0
    assert st["resident"] == n_slots
    assert st["bytes_uploaded"] == st["misses"] * cache.expert_bytes
    cache.close()


def test_slot_cache_generations(mer, oracle, gpu):
    """Equal generation = hit; an older requester is refused without
    disturbing the entry; a newer one retires and reinstalls the expert."""
    dm, dff = 128, 256
    say("slot cache generations")
    a, b = make_expert(oracle, Q4, dm, dff, 1), make_expert(oracle, Q4, dm, dff, 2)
    ha, hb = pinned(mer, a), pinned(mer, b)
    x = np.random.default_rng(3).standard_normal((1, dm)).astype(np.float32)
    ids = torch.tensor([[3]], dtype=torch.int32, device=gpu)
    w = torch.tensor([[1.0]], dtype=torch.float32, device=gpu)
    xd = torch.from_numpy(x).to(gpu)
    with mer.SlotCache(mer.WeightDtype.Q4_0, dm, dff, 2, 8) as cache:
        cache.prepare([3], generations=[5], host_blobs=[ha])
        y5 = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, cache, ids, w, xd).cpu().numpy()
        cache.prepare([3], generations=[5])  # hit: no blob needed
        assert cache.stats()["hits"] == 1
        before = cache.stats()
        with pytest.raises(mer.GpuExpertDispatchError) as e:
            cache.prepare([3], generations=[4], host_blobs=[hb])
        assert e.value.kind == mer.GpuExpertDispatchErrorKind.ResidencyMiss
        assert cache.stats() == before
        y5b = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, cache, ids, w, xd).cpu().numpy()
        cache.prepare([3], generations=[6], host_blobs=[hb])
        y6 = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, cache, ids, w, xd).cpu().numpy()
        st = cache.stats()
        assert st["stale_retirements"] == 1 and st["misses"] == 2 and st["resident"] == 1
    assert_ffn_close(y5[0], oracle.q4_0_reference_forward(a, x[0], dm, dff), "generation 5")
    assert_ffn_close(y5b[0], y5[0], "generation 5 after refused older request")
    assert_ffn_close(y6[0], oracle.q4_0_reference_forward(b, x[0], dm, dff), "generation 6")


def test_slot_cache_failures_change_nothing(mer, oracle, gpu):
    dm, dff = 64, 64
    say("slot cache failures")
    blobs = [make_expert(oracle, Q4, dm, dff, e) for e in range(4)]
    host = [pinned(mer, bl) for bl in blobs]
    with mer.SlotCache(mer.WeightDtype.Q4_0, dm, dff, 2, 4) as cache:
        cache.prepare([0, 1], host_blobs=host[:2])
        before = cache.stats()
        with pytest.raises(mer.GpuExpertDispatchError) as e:
            cache.prepare([0, 2, 3], host_blobs=[host[0], host[2], host[3]])
        assert e.value.kind == mer.GpuExpertDispatchErrorKind.PhysicalCapacity
        with pytest.raises(mer.GpuExpertDispatchError) as e:
            cache.prepare([2])  # not resident, no blob
        assert e.value.kind == mer.GpuExpertDispatchErrorKind.ResidencyMiss
        with pytest.raises(mer.GpuExpertDispatchError) as e:
            cache.prepare([9], host_blobs=[host[0]])  # beyond the table
        assert e.value.kind == mer.GpuExpertDispatchErrorKind.ResidencyMiss
        with pytest.raises(mer.InvalidLayout):
            cache.prepare([1, 1], generations=[0, 1], host_blobs=[host[1], host[1]])
        assert cache.stats() == before
        # the table still serves the two resident experts
        x = np.random.default_rng(5).standard_normal((1, dm)).astype(np.float32)
        ids = torch.tensor([[0, 1]], dtype=torch.int32, device=gpu)
        w = torch.tensor([[0.5, 0.5]], dtype=torch.float32, device=gpu)
        got = mer.moe_forward(mer.WeightDtype.Q4_0, dm, dff, cache, ids, w, torch.from_numpy(x).to(gpu))
        want = oracle_moe(oracle, Q4, blobs, np.array([[0, 1]]), np.array([[0.5, 0.5]], np.float32), x, dm, dff)
        assert_ffn_close(got.cpu().numpy(), want, "after failures")
        with pytest.raises(ValueError):
            cache.prepare([2], host_blobs=[torch.zeros(3, dtype=torch.uint8)])


def test_slot_cache_prefetch_then_prepare(mer, oracle, gpu):
    """Prefetched experts become hits; the last prepare's slots survive a
    prefetch; a table entry of a prefetched expert is published only by
    prepare."""
    dm, dff = 128, 128
    say("slot cache prefetch")
    blobs = [make_expert(oracle, Q8, dm, dff, e) for e in range(6)]
    host = [pinned(mer, bl) for bl in blobs]
    x = np.random.default_rng(9).standard_normal((1, dm)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    w = torch.tensor([[0.75, 0.25]], dtype=torch.float32, device=gpu)
    with mer.SlotCache(mer.WeightDtype.Q8_0, dm, dff, 4, 6) as cache:
        cache.prepare([0, 1], host_blobs=host[:2])
        y01 = mer.moe_forward(mer.WeightDtype.Q8_0, dm, dff, cache,
                              torch.tensor([[0, 1]], dtype=torch.int32, device=gpu), w, xd)
        cache.prefetch([2, 3, 4], host_blobs=host[2:5])  # two free slots: 4 is dropped, 0 and 1 stay
        st = cache.stats()
        assert st["prefetches"] == 2 and st["evictions"] == 0 and st["misses"] == 2 and st["resident"] == 4
        cache.prepare([0, 1])  # both survived the prefetch
        cache.prefetch([4], host_blobs=[host[4]])  # evicts the older prefetched expert (2), never 0 or 1
        st = cache.stats()
        assert st["prefetches"] == 3 and st["evictions"] == 1
        cache.prepare([3, 4])  # prefetched: hits, no uploads
        st2 = cache.stats()
        assert st2["misses"] == 2 and st2["bytes_uploaded"] == st["bytes_uploaded"] and st2["hits"] == 4
        with pytest.raises(mer.GpuExpertDispatchError):
            cache.prepare([2])  # evicted, no blob
        y34 = mer.moe_forward(mer.WeightDtype.Q8_0, dm, dff, cache,
                              torch.tensor([[3, 4]], dtype=torch.int32, device=gpu), w, xd)
        torch.cuda.synchronize()
    wn = np.array([[0.75, 0.25]], np.float32)
    assert_ffn_close(y01.cpu().numpy(), oracle_moe(oracle, Q8, blobs, np.array([[0, 1]]), wn, x, dm, dff), "0,1")
    assert_ffn_close(y34.cpu().numpy(), oracle_moe(oracle, Q8, blobs, np.array([[3, 4]]), wn, x, dm, dff), "3,4")


def test_slot_cache_feeds_layers_launch(mer, oracle, gpu):
    """The slot table as the expert table of the persistent all-layers
    launch (two layers share the cache; ids are global expert ids)."""
    dm, dff, n_exp = 256, 256, 8
    say("slot cache layers launch")
    blobs = [make_expert(oracle, Q4, dm, dff, e) for e in range(n_exp)]
    host = [pinned(mer, bl) for bl in blobs]
    rng = np.random.default_rng(21)
    ids = [np.array([[1, 6]], np.int32), np.array([[2, 5]], np.int32)]
    ws = [rng.random((1, 2)).astype(np.float32) for _ in range(2)]
    x = rng.standard_normal((1, dm)).astype(np.float32)
    with mer.SlotCache(mer.WeightDtype.Q4_0, dm, dff, 4, n_exp) as cache:
        cache.prepare([1, 6, 2, 5], host_blobs=[host[e] for e in (1, 6, 2, 5)])
        outs = [torch.zeros((1, dm), dtype=torch.float32, device=gpu) for _ in range(2)]
        layers = [dict(table=cache, ids=torch.from_numpy(ids[l]).to(gpu), weights=torch.from_numpy(ws[l]).to(gpu),
                       x=torch.from_numpy(x).to(gpu) if l == 0 else None, out=outs[l]) for l in range(2)]
        mer.moe_forward_layers(mer.WeightDtype.Q4_0, dm, dff, layers, residual=True, chain=True)
        got = [o.cpu().numpy() for o in outs]
    h = x
    for l in range(2):
        h = h + oracle_moe(oracle, Q4, blobs, ids[l], ws[l], h, dm, dff)
        assert_ffn_close(got[l], h, f"layer {l}")
