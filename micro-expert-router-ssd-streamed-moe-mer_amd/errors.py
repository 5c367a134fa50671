"""Typed errors of the expert-execution boundary.

ExpertWeightsError mirrors the reference enum (inference.rs:1153-1188) and
GpuExpertDispatchError mirrors GpuExpertDispatchErrorKind
(backend/mod.rs:349-361 and :412-449).  Status codes come from the C ABI.
"""
from __future__ import annotations

import enum

from . import _lib


class ExpertWeightsError(Exception):
    """Base of the CPU-side error taxonomy (inference.rs:1153)."""

    status: int = -1

    def __init__(self, message: str, *, have=None, need=None, d_model=None, d_ff=None):
        super().__init__(message)
        self.have, self.need, self.d_model, self.d_ff = have, need, d_model, d_ff


class BufferTooSmall(ExpertWeightsError):
    status = _lib.Status.BUFFER_TOO_SMALL


class Misaligned(ExpertWeightsError):
    status = _lib.Status.MISALIGNED


class Candle(ExpertWeightsError):
    """The reference's Candle(String) variant: a compute-side failure."""

    status = _lib.Status.COMPUTE


class InvalidLayout(ExpertWeightsError):
    status = _lib.Status.INVALID_LAYOUT


class TruncatedPayload(ExpertWeightsError):
    status = _lib.Status.TRUNCATED_PAYLOAD


class GpuExpertDispatchErrorKind(enum.Enum):
    ResidencyMiss = _lib.Status.RESIDENCY_MISS
    PhysicalCapacity = _lib.Status.PHYSICAL_CAPACITY
    Upload = _lib.Status.UPLOAD
    ValidationDispatch = _lib.Status.VALIDATION_DISPATCH
    Submission = _lib.Status.SUBMISSION
    ReadbackChannel = _lib.Status.READBACK_CHANNEL
    ReadbackMap = _lib.Status.READBACK_MAP
    DeviceLost = _lib.Status.DEVICE_LOST
    RuntimeInvariant = _lib.Status.RUNTIME_INVARIANT

    def __str__(self) -> str:  # backend/mod.rs:412-425 display names
        return {
            "ResidencyMiss": "residency-miss", "PhysicalCapacity": "physical-capacity",
            "Upload": "upload", "ValidationDispatch": "validation-dispatch",
            "Submission": "submission", "ReadbackChannel": "readback-channel",
            "ReadbackMap": "readback-map", "DeviceLost": "device-lost",
            "RuntimeInvariant": "runtime-invariant",
        }[self.name]


class GpuExpertDispatchError(Exception):
    def __init__(self, kind: GpuExpertDispatchErrorKind, detail: str, layer: int = 0, expert_id: int = 0):
        super().__init__(f"GPU routed expert {expert_id} (layer {layer}) failed at {kind}: {detail}")
        self.kind, self.detail, self.layer, self.expert_id = kind, detail, layer, expert_id


class RoutedExpertGpuIncompatibility(Exception):
    """backend/mod.rs:4621-4650 (UnsupportedDtype / ShapeExceedsWorkspace)."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class LibraryStateError(RuntimeError):
    pass


_BY_STATUS = {cls.status: cls for cls in (BufferTooSmall, Misaligned, Candle, InvalidLayout, TruncatedPayload)}


def raise_for_status(rc: int, layer: int = 0, expert_id: int = 0) -> None:
    """Translate a non-zero C-ABI status into the typed Python error."""
    if rc == 0:
        return
    status, msg, info = _lib.last_error()
    if status != rc:
        msg = msg or f"status {rc}"
    if rc == _lib.Status.IO:  # the reference's io::Error
        raise OSError(msg)
    if rc in _BY_STATUS:
        raise _BY_STATUS[rc](msg, have=info.have, need=info.need, d_model=info.d_model, d_ff=info.d_ff)
    try:
        kind = GpuExpertDispatchErrorKind(rc)
    except ValueError:
        kind = None
    if kind is not None:
        raise GpuExpertDispatchError(kind, msg, layer, expert_id)
    if rc in (_lib.Status.UNSUPPORTED_DTYPE, _lib.Status.SHAPE_EXCEEDS_WORKSPACE):
        raise RoutedExpertGpuIncompatibility(rc, msg)
    raise LibraryStateError(f"{_lib.Status(rc).name if rc in _lib.Status._value2member_map_ else rc}: {msg}")
