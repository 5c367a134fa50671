"""MI355X-native routed-expert SwiGLU FFN for MER (Q4_0 / Q8_0 GGUF blocks).

Import as ``importlib.import_module("micro-expert-router-ssd-streamed-moe-mer_amd")``
(the directory name is not a Python identifier).  Compute lives in the
gfx950 library libmer_hip.so; this package is its host-side mirror of the
reference's expert-execution interface.
"""
from . import _lib
from .errors import (
    BufferTooSmall,
    Candle,
    ExpertWeightsError,
    GpuExpertDispatchError,
    GpuExpertDispatchErrorKind,
    InvalidLayout,
    LibraryStateError,
    Misaligned,
    RoutedExpertGpuIncompatibility,
    TruncatedPayload,
)
from .expert import (
    EXPERT_SIZE_TOLERANCE_BYTES,
    Q4_0_BLOCK_BYTES,
    Q4_0_BLOCK_ELEMS,
    Q4_0_LAYOUT_STANDARD_V1,
    Q8_0_BLOCK_BYTES,
    Q8_0_BLOCK_ELEMS,
    WeightDtype,
    dequantize_to_f32,
    dispatch_expert_forward,
    expert_forward_host,
    expert_matmul,
    expert_weight_bytes_for,
    fill_synthetic,
    forward_q8_0_direct_into,
    init,
    moe_forward,
    moe_forward_layers,
    moe_grouped,
    q4_0_forward,
    q4_0_qmm_forward,
    q4_0_matvec,
    routed_expert_gpu_compatibility,
    routed_expert_matmul_batch,
    set_swiglu_limit,
    stage_timing_enable,
    stage_timing_read,
    stream_release,
    summarise_output,
    swiglu_limit,
    take_device_status,
    validate_expert,
)
from .formats import (
    DEFAULT_BLOCK_ALIGN,
    GgufExperts,
    MoeLayer,
    ProjectionRange,
    StackedLayout,
    UthDtype,
    UthHeader,
    probe_uth,
    strip_uth,
    swiglu_expert_header,
)
from .slots import SlotCache, pinned_expert_buffer

__all__ = [n for n in dir() if not n.startswith("_")]
