"""LMCache torch-extension surface on the HIP library.

The reference builds a torch C++ extension (``csrc/kvcache/lmcache_kv_transfer_ext.cpp``, loaded
by ``musa_aiter/ops/lmcache_kv_transfer_ext.py:21-52``) exposing four tensor-level entry points:
``kv_buffer_to_paged_list2``, ``paged_to_kv_buffer_list2``, ``kv_buffer_to_paged_two_x_nl`` and
``paged_to_kv_buffer_two_x_nl`` (``lmcache_kv_transfer_ext.cpp:587-592``).  Here the loader
returns an object with the same four methods, the same argument checks and messages (raised as
``RuntimeError``, as ``TORCH_CHECK`` does) and the same return value, each one launch on the current stream: gathers through the library's
reference-named C entries, scatters through its generic row copy with claim tags from torch's
allocator (so that no call makes the library allocate device memory).  The reference's environment-selected
kernel variants (aten / coalesced / sorted / contiguous / torchmusa-style) all compute the same
bytes; one kernel serves them all here.  ``MUSA_AITER_LMCACHE_CPP_EXTENSION=0`` disables the
extension as in the reference; ``MUSA_AITER_LMCACHE_CPP_TIMING=1`` (or
``MUSA_AITER_LMCACHE_TIMING=1``) prints the reference's ``[musa_aiter_lmcache_timing]`` line for
the list2 calls (``lmcache_kv_transfer_ext.cpp:339-387``).
"""

from __future__ import annotations

import ctypes
import os
import sys
import time
from typing import Any

import torch

from musa_aiter.ops import _hip

_EXT_MODULE: "HipLMCacheKVTransferExtension | None" = None
_EXT_ATTEMPTED = False
_EXT_ERROR: Exception | None = None


def _extension_requested() -> bool:
    return os.environ.get("MUSA_AITER_LMCACHE_CPP_EXTENSION", "1") == "1"


def _timing_enabled() -> bool:
    value = os.environ.get("MUSA_AITER_LMCACHE_CPP_TIMING")
    if value is not None:
        return value[:1] == "1"
    return os.environ.get("MUSA_AITER_LMCACHE_TIMING", "")[:1] == "1"


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _on_gpu(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


def _check_common(memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor], slot_mapping: torch.Tensor,
                  block_size: int, num_heads: int, head_size: int) -> None:
    """check_common (lmcache_kv_transfer_ext.cpp:164-193)."""
    _check(len(kvcaches) == 2, "LMCache C++ extension currently expects exactly 2 layers")
    _check(_on_gpu(memory_tensor), "memory_tensor must be a ROCm GPU tensor")
    _check(_on_gpu(slot_mapping), "slot_mapping must be a ROCm GPU tensor")
    _check(memory_tensor.is_contiguous(), "memory_tensor must be contiguous")
    _check(slot_mapping.is_contiguous(), "slot_mapping must be contiguous")
    _check(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
    _check(memory_tensor.dtype in (torch.float16, torch.bfloat16), "memory_tensor must be float16 or bfloat16")
    _check(memory_tensor.dim() == 4, "memory_tensor must have shape [2, NL, T, hidden]")
    _check(memory_tensor.size(0) == 2, "memory_tensor first dim must be 2")
    _check(memory_tensor.size(1) == 2, "memory_tensor NL must be 2 for list2 extension path")
    _check(memory_tensor.size(3) == num_heads * head_size, "hidden dim mismatch")
    for kvcache in kvcaches:
        _check(_on_gpu(kvcache), "kvcache must be a ROCm GPU tensor")
        _check(kvcache.is_contiguous(), "kvcache must be contiguous")
        _check(kvcache.dtype == memory_tensor.dtype, "kvcache dtype must match memory_tensor dtype")
        _check(kvcache.dim() == 5, "kvcache must have shape [2, NB, BS, NH, HS]")
        _check(kvcache.size(0) == 2, "kvcache first dim must be 2")
        _check(kvcache.size(2) == block_size, "block_size mismatch")
        _check(kvcache.size(3) == num_heads, "num_heads mismatch")
        _check(kvcache.size(4) == head_size, "head_size mismatch")


def _check_two_x_nl(memory_tensor: torch.Tensor, kvcaches: list[list[torch.Tensor]], slot_mapping: torch.Tensor,
                    block_size: int, num_heads: int, head_size: int) -> None:
    """check_two_x_nl (lmcache_kv_transfer_ext.cpp:195-229)."""
    _check(len(kvcaches) == 2, "split cache must contain K and V groups")
    _check(_on_gpu(memory_tensor) and memory_tensor.is_contiguous(), "memory_tensor must be contiguous ROCm GPU")
    _check(memory_tensor.dim() == 4 and memory_tensor.size(0) == 2, "memory_tensor must be [2, NL, T, hidden]")
    num_layers = memory_tensor.size(1)
    memory_tokens = memory_tensor.size(2)
    hidden = num_heads * head_size
    _check(0 < num_layers <= 64, "split cache layer count must be in [1, 64]")
    _check(memory_tokens >= 0, "memory token count must be non-negative")
    _check(block_size > 0 and num_heads > 0 and head_size > 0,
           "block_size, num_heads, and head_size must be positive")
    _check(hidden % 4 == 0, "split cache hidden size must be divisible by 4")
    _check(memory_tensor.dtype in (torch.float16, torch.bfloat16), "memory_tensor must be float16 or bfloat16")
    _check(memory_tensor.size(3) == hidden, "hidden dim mismatch")
    _check(_on_gpu(slot_mapping) and slot_mapping.is_contiguous() and slot_mapping.dtype == torch.int64,
           "slot_mapping must be contiguous ROCm GPU int64")
    _check(slot_mapping.dim() == 1, "slot_mapping must be one-dimensional")
    _check(slot_mapping.device == memory_tensor.device, "slot_mapping and memory_tensor must share a device")
    num_blocks = -1
    for group in kvcaches:
        _check(len(group) == num_layers, "split cache layer count mismatch")
        for cache in group:
            _check(_on_gpu(cache) and cache.is_contiguous(), "split cache must be contiguous ROCm GPU")
            _check(cache.device == memory_tensor.device, "split cache and memory_tensor must share a device")
            _check(cache.dtype == memory_tensor.dtype, "split cache dtype mismatch")
            _check(cache.dim() == 4 and cache.size(1) == block_size and cache.size(2) == num_heads
                   and cache.size(3) == head_size, "split cache must be [NB, BS, NH, HS]")
            _check(cache.size(0) > 0, "split cache num_blocks must be positive")
            if num_blocks < 0:
                num_blocks = cache.size(0)
            _check(cache.size(0) == num_blocks, "split cache num_blocks mismatch")


class _Timing:
    """The reference's TimingScope (lmcache_kv_transfer_ext.cpp:339-387): host launch time, device
    time between two events on the stream, and the achieved rate, printed to stderr."""

    def __init__(self, op: str, tokens: int, hidden: int, nbytes: int, device: torch.device):
        self.enabled = _timing_enabled()
        if not self.enabled:
            return
        self.op, self.tokens, self.hidden, self.nbytes = op, tokens, hidden, nbytes
        self.stream = torch.cuda.current_stream(device)
        self.host_start = time.perf_counter()
        self.start = torch.cuda.Event(enable_timing=True)
        self.stop = torch.cuda.Event(enable_timing=True)
        self.start.record(self.stream)

    def finish_after_launch(self) -> None:
        if not self.enabled:
            return
        after_launch = time.perf_counter()
        self.stop.record(self.stream)
        self.stop.synchronize()
        device_ms = self.start.elapsed_time(self.stop)
        host_total = time.perf_counter()
        bandwidth = (self.nbytes / 1e9) / (device_ms / 1e3) if device_ms > 0 else 0.0
        print(f"[musa_aiter_lmcache_timing] op={self.op} impl={_hip.BACKEND} tokens={self.tokens} "
              f"hidden={self.hidden} bytes={self.nbytes} host_launch_us={(after_launch - self.host_start) * 1e6:.3f} "
              f"device_ms={device_ms:.6f} host_total_us={(host_total - self.host_start) * 1e6:.3f} "
              f"bandwidth_gbps={bandwidth:.3f}", file=sys.stderr, flush=True)


class HipLMCacheKVTransferExtension:
    """The four entry points of the reference's LMCache extension (lmcache_kv_transfer_ext.cpp:389-585)."""

    def kv_buffer_to_paged_list2(self, memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor],
                                 slot_mapping: torch.Tensor, skip_prefix_n_tokens: int, block_size: int,
                                 num_heads: int, head_size: int) -> bool:
        """memory [2, 2, T, hidden] rows skip_prefix_n_tokens + i -> both layers' [2, NB, BS, NH, HS] caches."""
        _check_common(memory_tensor, kvcaches, slot_mapping, block_size, num_heads, head_size)
        return self._list2(1, memory_tensor, kvcaches, slot_mapping, int(skip_prefix_n_tokens), block_size,
                           num_heads, head_size, "to_gpu_buffer_to_paged")

    def paged_to_kv_buffer_list2(self, kvcaches: list[torch.Tensor], memory_tensor: torch.Tensor,
                                 slot_mapping: torch.Tensor, block_size: int, num_heads: int,
                                 head_size: int) -> bool:
        """Both layers' caches -> memory rows [0, T); a skipped slot gives a zero row."""
        _check_common(memory_tensor, kvcaches, slot_mapping, block_size, num_heads, head_size)
        return self._list2(0, memory_tensor, kvcaches, slot_mapping, 0, block_size, num_heads, head_size,
                           "from_gpu_paged_to_buffer")

    def kv_buffer_to_paged_two_x_nl(self, memory_tensor: torch.Tensor, kvcaches: list[list[torch.Tensor]],
                                    slot_mapping: torch.Tensor, skip_prefix_n_tokens: int, block_size: int,
                                    num_heads: int, head_size: int) -> bool:
        """memory [2, NL, M, hidden] rows skip_prefix_n_tokens + i -> K/V layer caches [NB, BS, NH, HS]."""
        _check_two_x_nl(memory_tensor, kvcaches, slot_mapping, block_size, num_heads, head_size)
        skip = int(skip_prefix_n_tokens)
        _check(skip >= 0, "skip_prefix_n_tokens must be non-negative")
        _check(skip + slot_mapping.numel() <= memory_tensor.size(2),
               "transfer range exceeds memory_tensor token extent")
        caches = [cache for group in kvcaches for cache in group]
        nl = memory_tensor.size(1)
        self._scatter(memory_tensor, [(a, l) for a in range(2) for l in range(nl)], caches, slot_mapping, skip,
                      kvcaches[0][0].size(0) * block_size, num_heads * head_size, "kv_buffer_to_paged_two_x_nl")
        return True

    def paged_to_kv_buffer_two_x_nl(self, kvcaches: list[list[torch.Tensor]], memory_tensor: torch.Tensor,
                                    slot_mapping: torch.Tensor, block_size: int, num_heads: int,
                                    head_size: int) -> bool:
        """K/V layer caches -> memory rows [0, T); a skipped slot gives a zero row."""
        _check_two_x_nl(memory_tensor, kvcaches, slot_mapping, block_size, num_heads, head_size)
        ptrs = self._pointers(kvcaches)
        device = memory_tensor.device
        with torch.cuda.device(device):
            rc = _hip.fn("lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16")(
                _hip.ptr(memory_tensor), ptrs, _hip.ptr(slot_mapping), memory_tensor.size(1),
                memory_tensor.size(2), slot_mapping.numel(), kvcaches[0][0].size(0), block_size, num_heads,
                head_size, _hip.stream_ptr(device))
        _hip.check(rc, "paged_to_kv_buffer_two_x_nl")
        return True

    @staticmethod
    def _pointers(kvcaches: list[list[torch.Tensor]]) -> ctypes.Array:
        return _hip.u64_array([cache.data_ptr() for group in kvcaches for cache in group])

    @staticmethod
    def _scatter(memory_tensor: torch.Tensor, planes: list[tuple[int, int]], caches: list[int | torch.Tensor],
                 slot_mapping: torch.Tensor, skip: int, num_slots: int, hidden: int, op: str) -> None:
        """Rows skip + i of the memory planes (axis, layer) -> slot rows of the matching caches (a
        cache tensor or a plane address), the last token of a repeated slot winning."""
        row = hidden * memory_tensor.element_size()
        nl, m = memory_tensor.size(1), memory_tensor.size(2)
        base = memory_tensor.data_ptr()
        _hip.copy_rows(op=op, device=memory_tensor.device,
                       src_planes=[base + (a * nl + l) * m * row for a, l in planes],
                       dst_planes=[c.data_ptr() if isinstance(c, torch.Tensor) else int(c) for c in caches],
                       num_planes=len(planes), src_idx=None, dst_idx=slot_mapping,
                       num_tokens=slot_mapping.numel(), num_rows_out=slot_mapping.numel(), src_offset=skip,
                       src_rows=m, dst_rows=num_slots, row_bytes=row, src_stride=row, dst_stride=row,
                       zero_invalid=False)

    @staticmethod
    def _list2(scatter: int, memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor], slot_mapping: torch.Tensor,
               skip: int, block_size: int, num_heads: int, head_size: int, op: str) -> bool:
        device = memory_tensor.device
        hidden = num_heads * head_size
        nbytes = 2 * len(kvcaches) * slot_mapping.numel() * hidden * memory_tensor.element_size()
        with torch.cuda.device(device):
            timing = _Timing(op, slot_mapping.numel(), hidden, nbytes, device)
            if scatter:
                # Planes (axis, layer) of the memory, and of the caches: layer l's [2, NB, BS, NH, HS]
                # tensor holds its K plane, then its V plane.
                half = kvcaches[0][0].numel() * kvcaches[0].element_size()
                caches = [kvcaches[l].data_ptr() + a * half for a in range(2) for l in range(2)]
                HipLMCacheKVTransferExtension._scatter(
                    memory_tensor, [(a, l) for a in range(2) for l in range(2)], caches, slot_mapping, skip,
                    kvcaches[0].size(1) * block_size, hidden, op)
            else:
                rc = _hip.fn("lmcache_paged_to_kv_buffer_list2_u16")(
                    _hip.ptr(memory_tensor), _hip.ptr(kvcaches[0]), _hip.ptr(kvcaches[1]), _hip.ptr(slot_mapping),
                    memory_tensor.size(2), slot_mapping.numel(), skip, kvcaches[0].size(1), block_size, num_heads,
                    head_size, _hip.stream_ptr(device))
                _hip.check(rc, op)
            timing.finish_after_launch()
        return True


def load_lmcache_kv_transfer_ext() -> Any | None:
    """The extension object, or None when ``MUSA_AITER_LMCACHE_CPP_EXTENSION`` is not "1" or the HIP
    library cannot be loaded (the error is kept for :func:`lmcache_kv_transfer_ext_error`); the
    first outcome is remembered, as in the reference loader (lmcache_kv_transfer_ext.py:21-48)."""
    global _EXT_MODULE, _EXT_ATTEMPTED, _EXT_ERROR
    if not _extension_requested():
        return None
    if _EXT_MODULE is not None:
        return _EXT_MODULE
    if _EXT_ATTEMPTED:
        return None
    _EXT_ATTEMPTED = True
    try:
        _hip.library()
        _EXT_MODULE = HipLMCacheKVTransferExtension()
        return _EXT_MODULE
    except Exception as exc:  # noqa: BLE001 - the reference records any build/load failure
        _EXT_ERROR = exc
        return None


def lmcache_kv_transfer_ext_error() -> Exception | None:
    return _EXT_ERROR


__all__ = ["HipLMCacheKVTransferExtension", "load_lmcache_kv_transfer_ext", "lmcache_kv_transfer_ext_error"]
