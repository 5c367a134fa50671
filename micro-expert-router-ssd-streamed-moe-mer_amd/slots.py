"""VRAM expert-slot cache: the RAM -> VRAM tier in front of the routed forwards.

Host-side mirror of the GPU backend's physical VRAM registry
(backend/mod.rs:548-1047) with GpuExpertCache's generation keys
(expert_cache.rs:604-627, :1281-1340), over the mer_slot_cache_* C ABI.
A SlotCache can be passed wherever moe_forward / moe_forward_layers take an
expert table.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .errors import raise_for_status
from .expert import WeightDtype, _init_for, _stream


def pinned_expert_buffer(n_bytes: int) -> torch.Tensor:
    """Page-locked host bytes for one expert (the RAM tier's resident
    buffer, expert_cache.rs:55-253), so its H2D copy runs asynchronously."""
    return torch.empty(n_bytes, dtype=torch.uint8, pin_memory=True)


class SlotCache:
    """n_slots expert-sized VRAM slots, a device table of n_experts pointers
    and a copy stream of its own.

    prepare(ids, generations, host_blobs) makes the experts resident for the
    work enqueued next on the current stream (hits are LRU-touched, misses
    uploaded, the stream waits for the uploads by events); prefetch(...)
    starts uploads for predicted experts without making anything wait.
    Generations follow the registry's rule: equal = hit, a newer stored
    generation raises a residency miss, an older one is replaced.
    """

    def __init__(self, dtype: WeightDtype, d_model: int, d_ff: int, n_slots: int, n_experts: int,
                 device: int | None = None):
        dev = torch.cuda.current_device() if device is None else device
        _init_for(torch.empty(0, device=f"cuda:{dev}"))
        self.dtype, self.d_model, self.d_ff = dtype, d_model, d_ff
        self.n_slots, self.n_experts = n_slots, n_experts
        self.expert_bytes = _lib.lib().mer_expert_weight_bytes(int(dtype), d_model, d_ff)
        h = ctypes.c_void_p()
        rc = _lib.lib().mer_slot_cache_create(int(dtype), d_model, d_ff, n_slots, n_experts, ctypes.byref(h))
        if rc:
            raise_for_status(rc)
        self._h = h
        # Host buffers handed to an upload must outlive it: hold every one
        # until the cache is closed (they are the RAM tier's residents).
        self._host_refs: list[torch.Tensor] = []

    # expert-table protocol of moe_forward / moe_forward_layers
    @property
    def table_ptr(self) -> int:
        return int(_lib.lib().mer_slot_cache_table(self._h) or 0)

    @property
    def table_len(self) -> int:
        return self.n_experts

    def _args(self, ids, generations, host_blobs):
        ids = [int(i) for i in ids]
        n = len(ids)
        ids_arr = (ctypes.c_uint32 * max(n, 1))(*ids)
        gens_arr = None
        if generations is not None:
            if len(generations) != n:
                raise ValueError("generations must match ids")
            gens_arr = (ctypes.c_uint64 * max(n, 1))(*[int(g) for g in generations])
        blobs_arr = None
        if host_blobs is not None:
            if len(host_blobs) != n:
                raise ValueError("host_blobs must match ids")
            ptrs = []
            for b in host_blobs:
                if b is None:
                    ptrs.append(None)
                    continue
                if not isinstance(b, torch.Tensor) or b.is_cuda or b.dtype != torch.uint8 or not b.is_contiguous():
                    raise TypeError("host blobs must be contiguous uint8 host tensors")
                if b.numel() < self.expert_bytes:
                    raise ValueError(f"host blob has {b.numel()} bytes, an expert needs {self.expert_bytes}")
                self._host_refs.append(b)
                ptrs.append(b.data_ptr())
            blobs_arr = (ctypes.c_void_p * max(n, 1))(*ptrs)
        return ids_arr, gens_arr, blobs_arr, n

    def _call(self, name, ids, generations, host_blobs):
        if self._h is None:
            raise RuntimeError("slot cache is closed")
        ids_arr, gens_arr, blobs_arr, n = self._args(ids, generations, host_blobs)
        rc = getattr(_lib.lib(), name)(self._h, ids_arr, gens_arr, blobs_arr, n, _stream())
        if rc:
            raise_for_status(rc, expert_id=int(ids[0]) if len(ids) else 0)

    def prepare(self, ids, generations=None, host_blobs=None) -> None:
        self._call("mer_slot_cache_prepare", ids, generations, host_blobs)

    def prefetch(self, ids, generations=None, host_blobs=None) -> None:
        self._call("mer_slot_cache_prefetch", ids, generations, host_blobs)

    def release(self) -> None:
        rc = _lib.lib().mer_slot_cache_release(self._h, _stream())
        if rc:
            raise_for_status(rc)

    def stats(self) -> dict[str, int]:
        st = _lib.MerSlotStats()
        rc = _lib.lib().mer_slot_cache_stats(self._h, ctypes.byref(st))
        if rc:
            raise_for_status(rc)
        return {name: int(getattr(st, name)) for name, _ in _lib.MerSlotStats._fields_}

    def close(self) -> None:
        if self._h is not None:
            _lib.lib().mer_slot_cache_destroy(self._h)
            self._h = None
            self._host_refs.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
