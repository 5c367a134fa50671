"""Routed-expert execution: host-side mirror of MER's expert interface.

Each function names the reference entry point it stands in for (paths
relative to rust-engine/src/).  Device tensors are torch tensors on the
current HIP device; all compute runs in libmer_hip.so on the caller's
current stream.
"""
from __future__ import annotations

import ctypes
import enum

import torch

from . import _lib
from .errors import raise_for_status


class WeightDtype(enum.IntEnum):
    """WeightDtype ordinals (inference.rs:138-236) of the GGUF formats."""

    Q4_0 = 4
    Q8_0 = 5


# inference.rs:731-750, kernels/mod.rs:74-75
Q4_0_BLOCK_ELEMS = 32
Q4_0_BLOCK_BYTES = 18
Q4_0_LAYOUT_STANDARD_V1 = "ggml-standard-v1"
Q8_0_BLOCK_ELEMS = 32
Q8_0_BLOCK_BYTES = 34
EXPERT_SIZE_TOLERANCE_BYTES = 4096  # inference.rs:3962

MOE_RESIDUAL = 1
MOE_ACCUMULATE = 2
MOE_CHAIN = 4
MOE_ROUTE_AFTER_PREV = 8
MOE_QMM = 16  # Q4_0 through Candle QMatMul arithmetic (Q8_0 activations)


def _device_index(t: torch.Tensor) -> int:
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _ptr(t: torch.Tensor, dtype: torch.dtype | None = None) -> int:
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


def _table(table) -> tuple[int, int]:
    """(device pointer, length) of an expert table: an int64 device tensor of
    blob pointers, or an object exposing table_ptr / table_len (SlotCache)."""
    if isinstance(table, torch.Tensor):
        return _ptr(table, torch.int64), table.numel()
    return int(table.table_ptr), int(table.table_len)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _call(name: str, *args, layer: int = 0, expert_id: int = 0) -> None:
    rc = getattr(_lib.lib(), name)(*args)
    if rc != 0:
        raise_for_status(rc, layer, expert_id)


def init(device: int | None = None) -> None:
    """mer_hip_init for `device` (default: torch's current device)."""
    _lib.ensure_init(torch.cuda.current_device() if device is None else device)


def _init_for(t: torch.Tensor) -> None:
    _lib.ensure_init(_device_index(t))


# ---- host-only ---------------------------------------------------------

def expert_weight_bytes_for(d_model: int, d_ff: int, dtype: WeightDtype) -> int:
    """expert_weight_bytes_for (inference.rs:1089-1146)."""
    return int(_lib.lib().mer_expert_weight_bytes(int(dtype), d_model, d_ff))


def summarise_output(token_idx: int, expert_id: int, y) -> tuple[int, float]:
    """summarise_output (inference.rs:3087-3106): the (digest, out_norm) of an
    expert output, as InferenceOutput carries them (inference.rs:984-994).
    y: host float32 array or a torch tensor (copied to the host)."""
    import numpy as np

    if isinstance(y, torch.Tensor):
        y = y.detach().to("cpu")
        y = y.numpy()
    ya = np.ascontiguousarray(np.asarray(y, np.float32).ravel())
    d = ctypes.c_uint64()
    n = ctypes.c_float()
    _call("mer_output_digest", token_idx, expert_id, ya.ctypes.data if ya.size else None, ya.size, ctypes.byref(d),
          ctypes.byref(n))
    return int(d.value), float(n.value)


def validate_expert(dtype: WeightDtype, length: int, x_len: int, y_len: int, d_model: int, d_ff: int,
                    tolerance: int = 0) -> None:
    """Raises the reference's typed error for an invalid expert call."""
    _call("mer_validate_expert", int(dtype), length, x_len, y_len, d_model, d_ff, tolerance)


def routed_expert_gpu_compatibility(dtype: WeightDtype, d_model: int, d_ff: int) -> None:
    """routed_expert_gpu_compatibility (backend/mod.rs:4691-4719)."""
    _call("mer_routed_expert_gpu_compatibility", int(dtype), d_model, d_ff)


# ---- device ------------------------------------------------------------

def dequantize_to_f32(dtype: WeightDtype, src: torch.Tensor, n_weights: int,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """dequantize_q4_0_to_f32 / dequantize_q8_0_to_f32 (inference.rs:852, :963)."""
    _init_for(src)
    if out is None:
        out = torch.empty(n_weights, dtype=torch.float32, device=src.device)
    _call("mer_hip_dequantize", int(dtype), _ptr(src, torch.uint8), src.numel(), n_weights,
          _ptr(out, torch.float32), _stream())
    return out


def q4_0_matvec(weights: torch.Tensor, w_block_off: int, rows: int, columns: int, x: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Raw Q4_0 qualification matvec (backend/mod.rs:3532-3768)."""
    _init_for(weights)
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=weights.device)
    _call("mer_hip_q4_0_matvec", _ptr(weights, torch.uint8), weights.numel(), w_block_off, rows, columns,
          _ptr(x, torch.float32), _ptr(out, torch.float32), _stream())
    return out


def dispatch_expert_forward(dtype: WeightDtype, resident: torch.Tensor, x: torch.Tensor, d_model: int,
                            d_ff: int, out: torch.Tensor | None = None, use_qmm: bool = False) -> torch.Tensor:
    """dispatch_expert_forward's Q4_0 / Q8_0 arms (engine.rs:1761-1848) on
    VRAM-resident expert bytes: y = W_down (silu(W_gate x) * (W_up x)).

    use_qmm: as the engine's flag, Q4_0 runs Candle's QMatMul arithmetic
    (run_inference_q4_0_qmm, Q8_0-quantised activations) when both dims are
    multiples of 32, and the dequant reference otherwise (engine.rs:1825-1830);
    Q8_0 ignores it."""
    _init_for(resident)
    if out is None:
        out = torch.empty(d_model, dtype=torch.float32, device=resident.device)
    if use_qmm and dtype == WeightDtype.Q4_0 and d_model % 32 == 0 and d_ff % 32 == 0:
        _call("mer_hip_expert_forward_qmm", _ptr(resident, torch.uint8), resident.numel(), _ptr(x, torch.float32),
              x.numel(), d_model, d_ff, _ptr(out, torch.float32), out.numel(), _stream())
        return out
    _call("mer_hip_expert_forward", int(dtype), _ptr(resident, torch.uint8), resident.numel(),
          _ptr(x, torch.float32), x.numel(), d_model, d_ff, _ptr(out, torch.float32), out.numel(), _stream())
    return out


def q4_0_qmm_forward(resident: torch.Tensor, x: torch.Tensor, d_model: int, d_ff: int,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """The device twin of run_inference_q4_0_qmm (inference.rs:4159-4243)."""
    _init_for(resident)
    if out is None:
        out = torch.empty(d_model, dtype=torch.float32, device=resident.device)
    _call("mer_hip_expert_forward_qmm", _ptr(resident, torch.uint8), resident.numel(), _ptr(x, torch.float32),
          x.numel(), d_model, d_ff, _ptr(out, torch.float32), out.numel(), _stream())
    return out


def forward_q8_0_direct_into(resident: torch.Tensor, x: torch.Tensor, d_model: int, d_ff: int,
                             y: torch.Tensor) -> None:
    """forward_q8_0_direct_into (inference.rs:3636-3644): caller-owned y."""
    dispatch_expert_forward(WeightDtype.Q8_0, resident, x, d_model, d_ff, out=y)


def q4_0_forward(resident: torch.Tensor, x: torch.Tensor, d_model: int, d_ff: int) -> torch.Tensor:
    """The device twin of q4_0_cpu_reference_forward (inference.rs:3291-3306)."""
    return dispatch_expert_forward(WeightDtype.Q4_0, resident, x, d_model, d_ff)


def expert_forward_host(dtype: WeightDtype, resident: bytes | bytearray | memoryview, x, d_model: int,
                        d_ff: int):
    """Host buffers in, host vector out (synchronous, PCIe-inclusive).

    `resident` is a bytes-like object, `x` a float32 numpy array."""
    import numpy as np

    init()
    xa = np.ascontiguousarray(x, dtype=np.float32)
    buf = (ctypes.c_uint8 * len(resident)).from_buffer_copy(resident) if not isinstance(
        resident, np.ndarray) else resident.ctypes.data_as(ctypes.c_void_p)
    y = np.zeros(d_model, dtype=np.float32)
    _call("mer_hip_expert_forward_host", int(dtype), ctypes.cast(buf, ctypes.c_void_p), len(resident),
          xa.ctypes.data, xa.size, d_model, d_ff, y.ctypes.data, y.size)
    return y


def moe_forward(dtype: WeightDtype, d_model: int, d_ff: int, table: torch.Tensor, expert_ids: torch.Tensor,
                weights: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None, *,
                residual: bool = False, accumulate: bool = False, qmm: bool = False) -> torch.Tensor:
    """Routed experts + top-k weighted combine for a decode batch: the
    WeightedInto loop of moe_step_inner (engine.rs:5548-5639).  qmm: Q4_0
    experts with Candle's QMatMul arithmetic (MER_MOE_QMM).

    table      int64 [E] device pointers of resident expert blobs (0 = absent),
               or a SlotCache (its device slot table)
    expert_ids int32 [n_tokens, top_k]
    weights    float32 [n_tokens, top_k]
    x          float32 [n_tokens, d_model]
    """
    _init_for(x)
    n_tokens, top_k = expert_ids.shape
    if weights.shape != expert_ids.shape or x.shape != (n_tokens, d_model):
        raise ValueError("shape mismatch between expert_ids, weights and x")
    if out is None:
        out = torch.empty_like(x)
    flags = (MOE_RESIDUAL if residual else 0) | (MOE_ACCUMULATE if accumulate else 0) | (MOE_QMM if qmm else 0)
    _call("mer_hip_moe_forward", int(dtype), d_model, d_ff, n_tokens, top_k, *_table(table),
          _ptr(expert_ids, torch.int32), _ptr(weights, torch.float32), _ptr(x, torch.float32),
          _ptr(out, torch.float32), flags, _stream())
    return out


def routed_expert_matmul_batch(dtype: WeightDtype, d_model: int, d_ff: int, table: torch.Tensor,
                               expert_ids: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The GPU backend's f16-view batch: routed_expert_matmul_batch_q4
    (backend/mod.rs:3770-3850, :4401-4418).  Every expert of expert_ids
    (int32 [n]) runs on the same f16 hidden state x [d_model]; returns
    f16 [n, d_model], row i = y of expert expert_ids[i] (not combined).
    The reference takes exactly 8 experts; any n >= 1 is accepted here."""
    _init_for(x)
    n = expert_ids.numel()
    if x.numel() != d_model:
        raise ValueError("x must hold d_model elements")
    if out is None:
        out = torch.empty((n, d_model), dtype=torch.float16, device=x.device)
    if out.numel() != n * d_model:
        raise ValueError("out must hold n * d_model elements")
    _call("mer_hip_expert_batch_f16", int(dtype), d_model, d_ff, n, *_table(table), _ptr(expert_ids, torch.int32),
          _ptr(x, torch.float16), _ptr(out, torch.float16), _stream())
    return out


def expert_matmul(dtype: WeightDtype, d_model: int, d_ff: int, table: torch.Tensor, expert_id: int,
                  x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Backend::expert_matmul / routed_expert_matmul (backend/mod.rs:1095-1103,
    :4421-4441): one resident expert on an f16 hidden state, f16 [d_model] out."""
    ids = torch.tensor([expert_id], dtype=torch.int32, device=x.device)
    y = routed_expert_matmul_batch(dtype, d_model, d_ff, table, ids, x, None if out is None else out.view(1, d_model))
    return y.view(d_model)


def moe_grouped(dtype: WeightDtype, d_model: int, d_ff: int, table: torch.Tensor, expert_ids: torch.Tensor,
                weights: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None, *,
                residual: bool = False, accumulate: bool = False, qmm: bool = False) -> torch.Tensor:
    """moe_forward for a multi-token batch on the grouped int8-MFMA path:
    pairs grouped by expert on the device, each expert's weights read once
    for all of its tokens (the batched routed_expert_matmul_batch_q4,
    backend/mod.rs:4401-4418).  Same arguments and combine as moe_forward;
    qmm: Q4_0 experts with Candle's QMatMul arithmetic (MER_MOE_QMM)."""
    _init_for(x)
    n_tokens, top_k = expert_ids.shape
    if weights.shape != expert_ids.shape or x.shape != (n_tokens, d_model):
        raise ValueError("shape mismatch between expert_ids, weights and x")
    if out is None:
        out = torch.empty_like(x)
    flags = (MOE_RESIDUAL if residual else 0) | (MOE_ACCUMULATE if accumulate else 0) | (MOE_QMM if qmm else 0)
    _call("mer_hip_moe_grouped", int(dtype), d_model, d_ff, n_tokens, top_k, *_table(table),
          _ptr(expert_ids, torch.int32), _ptr(weights, torch.float32), _ptr(x, torch.float32),
          _ptr(out, torch.float32), flags, _stream())
    return out


def moe_forward_layers(dtype: WeightDtype, d_model: int, d_ff: int, layers, *, residual: bool = False,
                       accumulate: bool = False, chain: bool = False, route_after_prev: bool = False,
                       qmm: bool = False) -> None:
    """All MoE layers of one decode step in a single persistent launch: the
    per-layer WeightedInto step of moe_step_inner (engine.rs:5548-5639) for
    every layer (model.rs:2715-2741), layers in order.

    `layers` is a sequence of dicts with device tensors: table (int64 [E]),
    ids (int32 [n_tokens, top_k]), weights (f32 [n_tokens, top_k]),
    x (f32 [n_tokens, d_model]; may be None for layers > 0 with chain=True)
    and out (f32 [n_tokens, d_model]).  route_after_prev: layer l > 0 reads
    its routing and streams its experts only after layer l-1's output is
    complete (as when routing is computed from that output).  qmm: Q4_0
    experts with Candle's QMatMul arithmetic (MER_MOE_QMM).
    """
    if not layers:
        return
    first = layers[0]
    _init_for(first["out"])
    n_tokens, top_k = first["ids"].shape
    arr = (_lib.MerLayerArgs * len(layers))()
    for i, la in enumerate(layers):
        if la["ids"].shape != (n_tokens, top_k) or la["weights"].shape != (n_tokens, top_k):
            raise ValueError("every layer needs the same [n_tokens, top_k] routing shape")
        if la["out"].shape != (n_tokens, d_model):
            raise ValueError("out must be [n_tokens, d_model]")
        x = la.get("x")
        arr[i] = _lib.MerLayerArgs(*_table(la["table"]), _ptr(la["ids"], torch.int32),
                                   _ptr(la["weights"], torch.float32), 0 if x is None else _ptr(x, torch.float32),
                                   _ptr(la["out"], torch.float32))
    flags = ((MOE_RESIDUAL if residual else 0) | (MOE_ACCUMULATE if accumulate else 0) | (MOE_CHAIN if chain else 0)
             | (MOE_ROUTE_AFTER_PREV if route_after_prev else 0) | (MOE_QMM if qmm else 0))
    _call("mer_hip_moe_forward_layers", int(dtype), d_model, d_ff, len(layers), n_tokens, top_k, arr, flags, _stream())


def fill_synthetic(dtype: WeightDtype, seed: int, expert_index: int, n_blocks: int, scale_lo: float,
                   scale_hi: float, out: torch.Tensor, block_begin: int = 0) -> torch.Tensor:
    """This library's counter-based synthetic GGUF block generator."""
    _init_for(out)
    bb = Q4_0_BLOCK_BYTES if dtype == WeightDtype.Q4_0 else Q8_0_BLOCK_BYTES
    if out.numel() < n_blocks * bb:
        raise ValueError("output buffer too small")
    _call("mer_hip_fill_synthetic", int(dtype), seed, expert_index, block_begin, n_blocks, scale_lo, scale_hi,
          _ptr(out, torch.uint8), _stream())
    return out


def set_swiglu_limit(limit: float | None) -> None:
    """set_swiglu_limit (inference.rs:90-99): install the GPT-OSS SwiGLU gate
    clamp for every later expert forward of this process (silu(clamp(g,
    -limit, limit)) * u); None, or a non-positive / non-finite limit, removes
    it."""
    _call("mer_set_swiglu_limit", float("inf") if limit is None else float(limit))


def swiglu_limit() -> float | None:
    """swiglu_limit (inference.rs:103-112): the installed clamp, or None."""
    v = _lib.lib().mer_get_swiglu_limit()
    return None if v == float("inf") else v


def stream_release(stream: "torch.cuda.Stream | int | None" = None) -> None:
    """Free the library's workspace of `stream` (default: the current
    stream); call before destroying a stream the library has used."""
    init()
    handle = _stream() if stream is None else (stream if isinstance(stream, int) else stream.cuda_stream)
    _call("mer_hip_stream_release", handle)


def take_device_status() -> None:
    """Raise the first device-side fault recorded since the last call."""
    init()
    _call("mer_hip_take_device_status")


STAGES = ("gate_up", "down", "combine", "prep", "decode")


def stage_timing_enable(enable: bool = True) -> None:
    """Start (or stop) GPU stage timing of every expert launch."""
    init()
    _call("mer_hip_stage_timing_enable", 1 if enable else 0)


def stage_timing_read() -> dict[str, tuple[float, int]]:
    """{stage: (total_ms, launches)} since the last enable/read (syncs)."""
    init()
    ms = (ctypes.c_double * len(STAGES))()
    counts = (ctypes.c_uint64 * len(STAGES))()
    _call("mer_hip_stage_timing_read", ms, counts)
    return {name: (ms[i], int(counts[i])) for i, name in enumerate(STAGES)}
