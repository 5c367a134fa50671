"""Host-side routing inputs: LinearGate-style top-k selection and the
Zipf / Markov SkewedStream workload (numpy; these produce the expert ids and
mixing weights the device path consumes).
"""
from __future__ import annotations

import numpy as np

_MASK = (1 << 64) - 1


def softmax_inplace(v: np.ndarray) -> np.ndarray:
    """transformer.rs:2747-2819: stable softmax over the non-NaN maximum; a
    NaN or non-finite maximum yields the uniform distribution."""
    v = np.asarray(v, np.float32)
    if v.size == 0:
        return v
    if np.isnan(v).any() or not np.isfinite(np.max(v)):
        v[...] = np.float32(1.0) / np.float32(v.size)
        return v
    e = np.exp(v - np.max(v)).astype(np.float32)
    s = np.float32(0.0)
    for val in e:  # sequential f32 sum, as the reference's loop
        s = np.float32(s + val)
    if s > 0:
        e = (e / s).astype(np.float32)
    v[...] = e
    return v


def _total_key(x: np.float32) -> int:
    b = int(np.float32(x).view(np.int32))
    return b ^ 0x7FFFFFFF if b < 0 else b


def route_scores(logits, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """gating.rs:395-476 for the default gate, given raw logits: softmax,
    top-k by (score desc, id asc) over finite scores, weights = the chosen
    softmax scores renormalised when their sum is finite and positive."""
    scores = softmax_inplace(np.array(logits, np.float32, copy=True))
    cand = [i for i in range(scores.size) if np.isfinite(scores[i])]
    cand.sort(key=lambda i: (-_total_key(scores[i]), i))
    ids = np.array(cand[:top_k], np.int32)
    w = scores[ids].astype(np.float32)
    s = np.float32(0.0)
    for val in w:
        s = np.float32(s + val)
    if np.isfinite(s) and s > 0:
        w = (w / s).astype(np.float32)
    return ids, w


def route_linear_gate(w_gate: np.ndarray, x: np.ndarray, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """LinearGate::route: logits = W x, then route_scores."""
    logits = (np.asarray(w_gate, np.float32) @ np.asarray(x, np.float32)).astype(np.float32)
    return route_scores(logits, top_k)


def _splitmix64(state: int) -> tuple[int, int]:
    state = (state + 0x9E3779B97F4A7C15) & _MASK
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK
    return state, z ^ (z >> 31)


class SkewedStream:
    """workload.rs:54-175: Zipf(s) popularity over a seeded rank->id
    permutation plus a Markov stay probability rho."""

    def __init__(self, num_experts: int, top_k: int, zipf_s: float, correlation: float, seed: int):
        n = max(num_experts, 1)
        self.top_k = min(max(top_k, 1), n)
        s = max(zipf_s, 0.0)
        self.rho = min(max(correlation, 0.0), 1.0)
        w = [1.0 / float((r + 1.0) ** s) for r in range(n)]
        total = 0.0
        for x in w:
            total += x
        acc, cdf = 0.0, []
        for x in w:
            acc += x / total
            cdf.append(acc)
        cdf[-1] = 1.0
        self.cdf = np.array(cdf, np.float64)
        st = (seed ^ 0xD1B54A32D192ED03) & _MASK
        perm = list(range(n))
        for i in range(n - 1, 0, -1):
            st, z = _splitmix64(st)
            j = z % (i + 1)
            perm[i], perm[j] = perm[j], perm[i]
        self.rank_to_id = perm
        self.state = (seed + 0x12345678) & _MASK
        self.prev: list[int] = []

    def _unit(self) -> float:
        self.state, z = _splitmix64(self.state)
        return float(z >> 11) / float(1 << 53)

    def sample_rank(self, u: float) -> int:
        i = int(np.searchsorted(self.cdf, u, side="left"))
        return min(i, self.cdf.size - 1)

    def next_experts(self) -> list[int]:
        if self.prev and self._unit() < self.rho:
            return list(self.prev)
        chosen: list[int] = []
        guard, guard_max = 0, max(self.top_k * 64, 64)
        while len(chosen) < self.top_k and guard < guard_max:
            eid = self.rank_to_id[self.sample_rank(self._unit())]
            if eid not in chosen:
                chosen.append(eid)
            guard += 1
        r = 0
        while len(chosen) < self.top_k and r < len(self.rank_to_id):
            if self.rank_to_id[r] not in chosen:
                chosen.append(self.rank_to_id[r])
            r += 1
        self.prev = list(chosen)
        return chosen


def route_linear_gate_gpu(gate, x, top_k: int, *, sigmoid: bool = False, normalise: bool = True, bias=None,
                          n_group: int = 1, topk_group: int = 1, scaling: float = 1.0, return_logits: bool = False):
    """LinearGate::route_with_scratch (gating.rs:395-476) on the GPU through
    mer_hip_route_linear_gate.  gate: f32 [n_experts, d_model] and x: f32
    [n_tokens, d_model] device tensors; returns device tensors ids (int32,
    -1 for slots no expert qualifies for), weights (f32) [n_tokens, top_k]
    and, when asked, the logits [n_tokens, n_experts]."""
    import ctypes

    import torch

    from . import _lib, errors
    from .expert import _init_for, _ptr, _stream

    if gate.dim() != 2 or x.dim() != 2 or gate.shape[1] != x.shape[1]:
        raise ValueError("gate must be [n_experts, d_model] and x [n_tokens, d_model]")
    _init_for(x)
    n_experts, d_model = gate.shape
    n_tokens = x.shape[0]
    ids = torch.empty((n_tokens, top_k), dtype=torch.int32, device=x.device)
    weights = torch.empty((n_tokens, top_k), dtype=torch.float32, device=x.device)
    logits = torch.empty((n_tokens, n_experts), dtype=torch.float32, device=x.device) if return_logits else None
    opts = _lib.MerGateOptions(1 if sigmoid else 0, 1 if normalise else 0,
                               0 if bias is None else _ptr(bias, torch.float32), n_group, topk_group, scaling)
    rc = _lib.lib().mer_hip_route_linear_gate(_ptr(gate, torch.float32), n_experts, d_model, _ptr(x, torch.float32),
                                              n_tokens, top_k, ctypes.byref(opts), ids.data_ptr(), weights.data_ptr(),
                                              0 if logits is None else logits.data_ptr(), _stream())
    if rc:
        errors.raise_for_status(rc)
    return (ids, weights, logits) if return_logits else (ids, weights)


def zipf_skewed_routes(n_tokens: int, n_experts: int, top_k: int, zipf_s: float, seed: int):
    """Routing of the batched grouped-expert workload: per token, logits
    N(0,1) + ln p_zipf(rank(e); s), where rank is a seeded permutation of the
    experts and p_zipf(r) is proportional to 1 / (r + 1)^s; then the default
    gate's softmax, top-k and renormalisation (route_scores, gating.rs:395-476).
    Returns ids int32 [n_tokens, top_k] and weights f32 [n_tokens, top_k]."""
    rng = np.random.default_rng(seed)
    rank = rng.permutation(n_experts)
    p = 1.0 / np.power(np.arange(1, n_experts + 1, dtype=np.float64), zipf_s)
    bias = np.log(p / p.sum())[rank].astype(np.float32)
    ids = np.zeros((n_tokens, top_k), np.int32)
    w = np.zeros((n_tokens, top_k), np.float32)
    for t in range(n_tokens):
        logits = rng.standard_normal(n_experts).astype(np.float32) + bias
        ids[t], w[t] = route_scores(logits, top_k)
    return ids, w
