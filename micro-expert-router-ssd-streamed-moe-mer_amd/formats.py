"""On-disk expert formats: UTH expert-blob headers and the GGUF MoE reader.

Host-side mirror of the reference's TensorHeader / MixedExpertHeader
(tensor_header.rs:189-536), of ExpertResident's header strip
(expert_cache.rs:103-143) and of its GGUF native-quant expert extraction
(gguf_loader.rs:2880-3010), over the mer_uth_* / mer_gguf_* C ABI.  The
parsing itself runs in the library (mer_format.cpp); this module only
moves buffers across the boundary.

A GGUF Q4_0 / Q8_0 expert is copied byte for byte into MER's
gate || up || down blob, so read_expert's output goes straight into a
pinned host buffer, a SlotCache upload or an expert table.
"""
from __future__ import annotations

import ctypes
import dataclasses
import enum
import os

import numpy as np

from . import _lib
from .errors import raise_for_status
from .expert import WeightDtype

# ExpertResident's default block alignment (expert_cache.rs:103).
DEFAULT_BLOCK_ALIGN = 4096


class UthDtype(enum.IntEnum):
    """UthDtypeId (tensor_header.rs:78-90)."""
    F32 = 0
    F16 = 1
    INT8 = 2
    Q4K = 3
    Q4_0 = 4
    Q8_0 = 5
    BF16 = 6
    MXFP4 = 7
    Q5K = 8
    Q6K = 9
    MIXED = 10


@dataclasses.dataclass(frozen=True)
class ProjectionRange:
    """One UTH2 projection range, payload-relative (tensor_header.rs:140-170)."""
    dtype: UthDtype
    offset: int
    len: int
    weights: int


@dataclasses.dataclass(frozen=True)
class UthHeader:
    """A parsed UTH1 or UTH2 header and where its payload starts."""
    kind: int  # 1 = UTH1, 2 = UTH2
    version: int
    dtype: UthDtype
    flags: int
    shape: tuple
    quant_scale_offset: int
    quant_scale_count: int
    d_model: int
    d_ff: int
    projections: tuple  # UTH2 gate, up, down ranges; () for UTH1
    payload_offset: int
    payload_len: int


def _host_buffer(buf):
    """(address, length, keep-alive) of a host byte buffer: bytes-like,
    numpy array or CPU torch tensor."""
    if hasattr(buf, "data_ptr") and hasattr(buf, "is_cuda"):
        if buf.is_cuda:
            raise ValueError("expected a host buffer, got a device tensor")
        if not buf.is_contiguous():
            raise ValueError("host buffer must be contiguous")
        return buf.data_ptr(), buf.numel() * buf.element_size(), buf
    arr = np.frombuffer(buf, dtype=np.uint8) if not isinstance(buf, np.ndarray) else buf
    if not arr.flags.c_contiguous:
        raise ValueError("host buffer must be contiguous")
    return arr.ctypes.data if arr.size else None, arr.nbytes, arr


def probe_uth(blob, block_align: int = DEFAULT_BLOCK_ALIGN) -> UthHeader | None:
    """The blob's UTH2 header if it carries a valid one, else its UTH1
    header, else None (a headerless legacy blob), as
    ExpertResident::new_with_block_align strips (expert_cache.rs:110-143)."""
    ptr, n, _keep = _host_buffer(blob)
    info = _lib.MerUthInfo()
    rc = _lib.lib().mer_uth_probe(ptr, n, block_align, ctypes.byref(info))
    if rc:
        raise_for_status(rc)
    if info.kind == 0:
        return None
    projs = ()
    if info.kind == 2:
        projs = tuple(ProjectionRange(UthDtype(p.dtype), p.offset, p.len, p.weights) for p in info.proj)
    return UthHeader(kind=info.kind, version=info.version, dtype=UthDtype(info.dtype), flags=info.flags,
                     shape=tuple(info.shape[:info.shape_rank]), quant_scale_offset=info.quant_scale_offset,
                     quant_scale_count=info.quant_scale_count, d_model=info.d_model, d_ff=info.d_ff,
                     projections=projs, payload_offset=info.payload_offset, payload_len=info.payload_len)


def strip_uth(blob, block_align: int = DEFAULT_BLOCK_ALIGN):
    """(header or None, payload view): the weights a resident expert
    dispatches from; a legacy blob comes back whole, unchanged."""
    h = probe_uth(blob, block_align)
    # numpy arrays and tensors are sliced as themselves, bytes-likes as a memoryview
    view = blob if isinstance(blob, np.ndarray) or hasattr(blob, "data_ptr") else memoryview(blob).cast("B")
    if h is None:
        return None, view
    return h, view[h.payload_offset:h.payload_offset + h.payload_len]


def swiglu_expert_header(dtype: UthDtype | WeightDtype | int, d_model: int, d_ff: int,
                         block_align: int = DEFAULT_BLOCK_ALIGN) -> bytes:
    """TensorHeader::for_swiglu_expert(...).write_padded(block_align)
    (tensor_header.rs:398-470): the UTH1 header of a gate || up || down
    blob, zero-padded so the weights start block-aligned."""
    lib = _lib.lib()
    need = ctypes.c_size_t()
    rc = lib.mer_uth_write_expert_header(int(dtype), d_model, d_ff, block_align, None, 0, ctypes.byref(need))
    if rc:
        raise_for_status(rc)
    out = ctypes.create_string_buffer(need.value)
    rc = lib.mer_uth_write_expert_header(int(dtype), d_model, d_ff, block_align, out, need.value, ctypes.byref(need))
    if rc:
        raise_for_status(rc)
    return out.raw[:need.value]


class StackedLayout(enum.IntEnum):
    STACKED = 0     # blk.L.ffn_{gate,up,down}_exps.weight
    PER_EXPERT = 1  # blk.L.ffn_{gate,up,down}.e.weight


@dataclasses.dataclass(frozen=True)
class MoeLayer:
    """A layer's routed-expert geometry as the GGUF file holds it."""
    dtype: WeightDtype
    layout: StackedLayout
    d_model: int
    d_ff: int
    n_experts: int
    expert_bytes: int


class GgufExperts:
    """A GGUF file's MoE expert tensors (versions 1-3, Q4_0 / Q8_0),
    read with positioned reads: nothing but the header is held in memory.

    Mirrors load_layer_expert_native_quant (gguf_loader.rs:2880-3010): a
    stacked tensor's expert e is the byte run at e * projection_bytes; a
    per-expert tensor's whole body is the expert's projection."""

    def __init__(self, path: str | os.PathLike):
        h = ctypes.c_void_p()
        rc = _lib.lib().mer_gguf_open(os.fsencode(path), ctypes.byref(h))
        if rc:
            raise_for_status(rc)
        self._h = h

    def close(self) -> None:
        if self._h:
            _lib.lib().mer_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _handle(self):
        if not self._h:
            raise ValueError("GgufExperts is closed")
        return self._h

    def moe_layer(self, layer: int) -> MoeLayer:
        info = _lib.MerGgufMoeInfo()
        rc = _lib.lib().mer_gguf_moe_layer(self._handle(), layer, ctypes.byref(info))
        if rc:
            raise_for_status(rc, layer=layer)
        return MoeLayer(WeightDtype(info.dtype), StackedLayout(info.layout), info.d_model, info.d_ff,
                        info.n_experts, info.expert_bytes)

    def read_expert(self, layer: int, expert: int, out=None):
        """Expert `expert` of `layer` as MER's gate || up || down blob.
        `out` (numpy uint8 array or CPU tensor, e.g. a pinned buffer) is
        filled and returned; without it a new numpy array is returned."""
        if out is None:
            out = np.empty(self.moe_layer(layer).expert_bytes, np.uint8)
        ptr, n, _keep = _host_buffer(out)
        rc = _lib.lib().mer_gguf_read_expert(self._handle(), layer, expert, ptr, n)
        if rc:
            raise_for_status(rc, layer=layer, expert_id=expert)
        return out
