"""ctypes binding of the CPU oracle (libmer_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product package never
imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmer_oracle.so")

Q4_0, Q8_0 = 4, 5
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34}

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_sz = ctypes.c_size_t

_SIG = {
    "mo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "mo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "mo_round_to_i32": (ctypes.c_int32, [ctypes.c_float]),
    "mo_dequantize_q4_0_block": (None, [_u8p, _f32p]),
    "mo_dequantize_q8_0_block": (None, [_u8p, _f32p]),
    "mo_quantize_q4_0_block": (None, [_f32p, _sz, _u8p]),
    "mo_quantize_q8_0_block": (None, [_f32p, _sz, _u8p]),
    "mo_dequantize_to_f32": (ctypes.c_int, [ctypes.c_int, _u8p, _sz, _sz, _f32p]),
    "mo_expert_weight_bytes": (_sz, [ctypes.c_int, _sz, _sz]),
    "mo_validate_q4_0": (ctypes.c_int, [_sz, _sz, _sz, _sz, ctypes.POINTER(_sz)]),
    "mo_validate_q8_direct": (ctypes.c_int, [_sz, _sz, _sz, _sz, _sz, ctypes.POINTER(_sz)]),
    "mo_q4_0_reference_forward": (ctypes.c_int, [_u8p, _sz, _f32p, _sz, _sz, _f32p, ctypes.c_int]),
    "mo_q4_0_qmm_forward": (ctypes.c_int, [_u8p, _sz, _f32p, _sz, _sz, _f32p, ctypes.c_int]),
    "mo_q4_0_qmm_forward_ex": (ctypes.c_int, [_u8p, _sz, _f32p, _sz, _sz, _f32p, _f32p, ctypes.c_float,
                                              ctypes.POINTER(_sz), ctypes.c_int]),
    "mo_quantize_row_q8_0_candle": (None, [_f32p, _sz, ctypes.POINTER(ctypes.c_int8), _f32p]),
    "mo_q8_0_dequant_forward": (ctypes.c_int, [_u8p, _sz, _f32p, _sz, _sz, _f32p, ctypes.c_int]),
    "mo_q8_0_direct_forward": (
        ctypes.c_int, [_u8p, _sz, _f32p, _sz, _sz, _sz, _f32p, _sz, ctypes.c_int, ctypes.c_int]),
    "mo_q8_0_row_dot": (ctypes.c_float, [ctypes.c_int, _u8p, _f32p, _sz]),
    "mo_have_avx2_fma": (ctypes.c_int, []),
    "mo_silu": (ctypes.c_float, [ctypes.c_float]),
    "mo_set_swiglu_limit": (None, [ctypes.c_float]),
    "mo_get_swiglu_limit": (ctypes.c_float, []),
    "mo_combine_outputs": (None, [_f32p, _f32p, _sz, _sz, _f32p]),
    "mo_synth_hidden_state": (None, [ctypes.c_uint64, _sz, ctypes.c_uint64, _f32p]),
    "mo_deterministic_input": (None, [_sz, _sz, _f32p]),
    "mo_canonical_block": (None, [ctypes.c_float, _u8p, _u8p]),
    "mo_cpu_q4_matvec": (ctypes.c_int, [_u8p, _sz, _sz, _sz, _sz, _f32p, _f32p]),
    "mo_randomized_q8_expert": (None, [_sz, _sz, ctypes.c_uint64, _u8p]),
    "mo_generate_synthetic_expert": (None, [ctypes.c_int, ctypes.c_uint32, _sz, _sz, _u8p]),
    "mo_output_digest": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint32, _f32p, _sz, _f32p]),
    "mo_bench_fill_q4_0": (None, [ctypes.c_uint64] * 4 + [ctypes.c_float, ctypes.c_float, _u8p]),
    "mo_bench_fill_q8_0": (None, [ctypes.c_uint64] * 4 + [ctypes.c_float, ctypes.c_float, _u8p]),
    "mo_softmax_inplace": (None, [_f32p, _sz]),
    "mo_linear_gate_route": (ctypes.c_int, [_f32p, _sz, _sz, _f32p, _sz, _u32p, _f32p]),
    "mo_topk_softmax_logits": (None, [_f32p, _sz, _sz, _u32p, _f32p]),
    "mo_gate_route_ex": (_sz, [_f32p, _sz, _sz, ctypes.c_int, ctypes.c_int, _f32p, _sz, _sz, ctypes.c_float,
                               _u32p, _f32p]),
    "mo_linear_gate_route_ex": (_sz, [_f32p, _sz, _sz, _f32p, _sz, ctypes.c_int, ctypes.c_int, _f32p, _sz, _sz,
                                      ctypes.c_float, _u32p, _f32p, _f32p]),
    "mo_skewed_new": (ctypes.c_void_p, [ctypes.c_uint32, _sz, ctypes.c_double, ctypes.c_double, ctypes.c_uint64]),
    "mo_skewed_next": (_sz, [ctypes.c_void_p, _u32p]),
    "mo_skewed_free": (None, [ctypes.c_void_p]),
}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def _u8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


def _u32(a: np.ndarray):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_u32p)


def f16_to_f32(h: int) -> float:
    return lib().mo_f16_to_f32(h)


def f32_to_f16(x: float) -> int:
    return lib().mo_f32_to_f16(x)


def dequantize_block(dtype: int, block: np.ndarray) -> np.ndarray:
    out = np.zeros(32, np.float32)
    blk = np.ascontiguousarray(block, np.uint8)
    if dtype == Q4_0:
        lib().mo_dequantize_q4_0_block(_u8(blk), _f(out))
    else:
        lib().mo_dequantize_q8_0_block(_u8(blk), _f(out))
    return out


def quantize_block(dtype: int, values) -> np.ndarray:
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(BLOCK_BYTES[dtype], np.uint8)
    fn = lib().mo_quantize_q4_0_block if dtype == Q4_0 else lib().mo_quantize_q8_0_block
    fn(_f(v), v.size, _u8(out))
    return out


def dequantize_to_f32(dtype: int, src: np.ndarray, n_weights: int) -> np.ndarray:
    out = np.zeros(n_weights, np.float32)
    rc = lib().mo_dequantize_to_f32(dtype, _u8(src), src.size, n_weights, _f(out))
    if rc:
        raise ValueError(f"oracle dequantize status {rc}")
    return out


def expert_weight_bytes(dtype: int, d_model: int, d_ff: int) -> int:
    return lib().mo_expert_weight_bytes(dtype, d_model, d_ff)


def validate_q4_0(length: int, d_model: int, d_ff: int, tolerance: int = 0) -> int:
    need = _sz(0)
    return lib().mo_validate_q4_0(length, d_model, d_ff, tolerance, ctypes.byref(need))


def validate_q8_direct(length: int, x_len: int, y_len: int, d_model: int, d_ff: int) -> int:
    need = _sz(0)
    return lib().mo_validate_q8_direct(length, x_len, y_len, d_model, d_ff, ctypes.byref(need))


def q4_0_reference_forward(blob: np.ndarray, x: np.ndarray, d_model: int, d_ff: int,
                           nthreads: int = 8) -> np.ndarray:
    y = np.zeros(d_model, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    rc = lib().mo_q4_0_reference_forward(_u8(blob), blob.size, _f(xa), d_model, d_ff, _f(y), nthreads)
    if rc:
        raise ValueError(f"oracle q4_0 forward status {rc}")
    return y


def q4_0_qmm_forward(blob: np.ndarray, x: np.ndarray, d_model: int, d_ff: int,
                     nthreads: int = 8) -> np.ndarray:
    """run_inference_q4_0_qmm (inference.rs:4159-4243): Candle QMatMul with
    Q8_0-quantised activations (mo_q4_0_qmm_forward)."""
    y = np.zeros(d_model, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    rc = lib().mo_q4_0_qmm_forward(_u8(blob), blob.size, _f(xa), d_model, d_ff, _f(y), nthreads)
    if rc:
        raise ValueError(f"oracle q4_0 qmm forward status {rc}")
    return y


# Distance from a Q8_0 rounding midpoint, in quantisation steps, within which
# two f32 evaluation orders of h may round an element differently (a few
# times the f32 noise of h measured in steps, ~1e-4).
QMM_FLIP_MARGIN = 1e-3


def q4_0_qmm_forward_bounded(blob: np.ndarray, x: np.ndarray, d_model: int, d_ff: int,
                             margin: float = QMM_FLIP_MARGIN, nthreads: int = 8):
    """q4_0_qmm_forward plus its flip bound (mo_q4_0_qmm_forward_ex):
    returns (y, bound[d_model], n_flagged)."""
    y = np.zeros(d_model, np.float32)
    bound = np.zeros(d_model, np.float32)
    n = _sz(0)
    xa = np.ascontiguousarray(x, np.float32)
    rc = lib().mo_q4_0_qmm_forward_ex(_u8(blob), blob.size, _f(xa), d_model, d_ff, _f(y), _f(bound), margin,
                                      ctypes.byref(n), nthreads)
    if rc:
        raise ValueError(f"oracle q4_0 qmm forward status {rc}")
    return y, bound, n.value


def quantize_row_q8_0_candle(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Candle's BlockQ8_0::from_float over a row (len a multiple of 32):
    int8 values and the f16-rounded block scales as f32."""
    xa = np.ascontiguousarray(x, np.float32)
    q = np.zeros(xa.size, np.int8)
    d = np.zeros(xa.size // 32, np.float32)
    lib().mo_quantize_row_q8_0_candle(_f(xa), xa.size, q.ctypes.data_as(ctypes.POINTER(ctypes.c_int8)), _f(d))
    return q, d


def q8_0_dequant_forward(blob: np.ndarray, x: np.ndarray, d_model: int, d_ff: int,
                         nthreads: int = 8) -> np.ndarray:
    y = np.zeros(d_model, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    rc = lib().mo_q8_0_dequant_forward(_u8(blob), blob.size, _f(xa), d_model, d_ff, _f(y), nthreads)
    if rc:
        raise ValueError(f"oracle q8_0 dequant forward status {rc}")
    return y


def q8_0_direct_forward(blob: np.ndarray, x: np.ndarray, d_model: int, d_ff: int, kernel: int = 1,
                        nthreads: int = 8, y_len: int | None = None) -> tuple[int, np.ndarray]:
    y = np.zeros(d_model if y_len is None else y_len, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    rc = lib().mo_q8_0_direct_forward(_u8(blob), blob.size, _f(xa), xa.size, d_model, d_ff, _f(y), y.size,
                                      kernel, nthreads)
    return rc, y


def q8_0_row_dot(kernel: int, row: np.ndarray, x: np.ndarray) -> float:
    xa = np.ascontiguousarray(x, np.float32)
    return lib().mo_q8_0_row_dot(kernel, _u8(np.ascontiguousarray(row, np.uint8)), _f(xa), xa.size)


def set_swiglu_limit(limit) -> None:
    """set_swiglu_limit (inference.rs:90-99); None or a non-positive /
    non-finite limit removes the clamp."""
    lib().mo_set_swiglu_limit(float("inf") if limit is None else float(limit))


def swiglu_limit():
    v = lib().mo_get_swiglu_limit()
    return None if v == float("inf") else v


def combine_outputs(outputs: np.ndarray, scores: np.ndarray) -> np.ndarray:
    o = np.ascontiguousarray(outputs, np.float32)
    s = np.ascontiguousarray(scores, np.float32)
    k, d = o.shape
    out = np.zeros(d, np.float32)
    lib().mo_combine_outputs(_f(o), _f(s), k, d, _f(out))
    return out


def synth_hidden_state(token_idx: int, d_model: int, seed: int) -> np.ndarray:
    out = np.zeros(d_model, np.float32)
    lib().mo_synth_hidden_state(token_idx, d_model, seed, _f(out))
    return out


def deterministic_input(length: int, seed: int) -> np.ndarray:
    out = np.zeros(length, np.float32)
    lib().mo_deterministic_input(length, seed, _f(out))
    return out


def canonical_block(scale: float, nibbles) -> np.ndarray:
    nb = np.ascontiguousarray(nibbles, np.uint8)
    out = np.zeros(18, np.uint8)
    lib().mo_canonical_block(scale, _u8(nb), _u8(out))
    return out


def cpu_q4_matvec(weights: np.ndarray, w_block_off: int, rows: int, columns: int, x: np.ndarray) -> np.ndarray:
    out = np.zeros(rows, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    rc = lib().mo_cpu_q4_matvec(_u8(weights), weights.size, w_block_off, rows, columns, _f(xa), _f(out))
    if rc:
        raise ValueError(f"oracle raw matvec status {rc}")
    return out


def randomized_q8_expert(d_model: int, d_ff: int, state: int) -> np.ndarray:
    out = np.zeros(expert_weight_bytes(Q8_0, d_model, d_ff), np.uint8)
    lib().mo_randomized_q8_expert(d_model, d_ff, state, _u8(out))
    return out


def generate_synthetic_expert(dtype: int, expert_id: int, d_model: int, d_ff: int) -> np.ndarray:
    out = np.zeros(expert_weight_bytes(dtype, d_model, d_ff), np.uint8)
    lib().mo_generate_synthetic_expert(dtype, expert_id, d_model, d_ff, _u8(out))
    return out


def output_digest(token_idx: int, expert_id: int, y: np.ndarray) -> tuple[int, float]:
    norm = ctypes.c_float(0)
    ya = np.ascontiguousarray(y, np.float32)
    d = lib().mo_output_digest(token_idx, expert_id, _f(ya), ya.size, ctypes.byref(norm))
    return d, norm.value


def bench_fill(dtype: int, seed: int, expert_index: int, block_begin: int, n_blocks: int, lo: float,
               hi: float) -> np.ndarray:
    out = np.zeros(n_blocks * BLOCK_BYTES[dtype], np.uint8)
    fn = lib().mo_bench_fill_q4_0 if dtype == Q4_0 else lib().mo_bench_fill_q8_0
    fn(seed, expert_index, block_begin, n_blocks, lo, hi, _u8(out))
    return out


def softmax(v) -> np.ndarray:
    a = np.array(v, np.float32)
    lib().mo_softmax_inplace(_f(a), a.size)
    return a


def linear_gate_route(w: np.ndarray, x: np.ndarray, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    wa = np.ascontiguousarray(w, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    ids = np.zeros(top_k, np.uint32)
    ws = np.zeros(top_k, np.float32)
    n = lib().mo_linear_gate_route(_f(wa), wa.shape[0], wa.shape[1], _f(xa), top_k, _u32(ids), _f(ws))
    return ids[:n], ws[:n]


def topk_softmax_logits(logits, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    la = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(top_k, np.uint32)
    ws = np.zeros(top_k, np.float32)
    lib().mo_topk_softmax_logits(_f(la), la.size, top_k, _u32(ids), _f(ws))
    return ids, ws


def gate_route_ex(logits, top_k: int, *, sigmoid: bool = False, normalise: bool = True, bias=None,
                  n_group: int = 1, topk_group: int = 1, scaling: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """LinearGate scoring + selection (gating.rs:395-476) on given logits."""
    la = np.ascontiguousarray(logits, np.float32)
    ba = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ids = np.zeros(max(top_k, 1), np.uint32)
    ws = np.zeros(max(top_k, 1), np.float32)
    n = lib().mo_gate_route_ex(_f(la), la.size, top_k, int(sigmoid), int(normalise), None if ba is None else _f(ba),
                               n_group, topk_group, scaling, _u32(ids), _f(ws))
    return ids[:n], ws[:n]


def linear_gate_route_ex(w: np.ndarray, x: np.ndarray, top_k: int, **opts) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """logits = W x (dot_f32 order), then gate_route_ex; also returns the logits."""
    wa = np.ascontiguousarray(w, np.float32)
    xa = np.ascontiguousarray(x, np.float32)
    bias = opts.get("bias")
    ba = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ids = np.zeros(max(top_k, 1), np.uint32)
    ws = np.zeros(max(top_k, 1), np.float32)
    lo = np.zeros(wa.shape[0], np.float32)
    n = lib().mo_linear_gate_route_ex(_f(wa), wa.shape[0], wa.shape[1], _f(xa), top_k, int(opts.get("sigmoid", False)),
                                      int(opts.get("normalise", True)), None if ba is None else _f(ba),
                                      opts.get("n_group", 1), opts.get("topk_group", 1), opts.get("scaling", 1.0),
                                      _u32(ids), _f(ws), _f(lo))
    return ids[:n], ws[:n], lo


class SkewedStream:
    """workload.rs:54-175 through the C restatement."""

    def __init__(self, num_experts: int, top_k: int, zipf_s: float, rho: float, seed: int):
        self._h = lib().mo_skewed_new(num_experts, top_k, zipf_s, rho, seed)
        self._buf = np.zeros(max(1, min(top_k, max(num_experts, 1))), np.uint32)

    def next_experts(self) -> list[int]:
        n = lib().mo_skewed_next(self._h, _u32(self._buf))
        return [int(v) for v in self._buf[:n]]

    def __del__(self):
        if getattr(self, "_h", None):
            lib().mo_skewed_free(self._h)
            self._h = None
