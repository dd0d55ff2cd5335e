"""The host/device batch-copy extension object behind ``lmcache_musa_memcpy_batch_async``.

The reference builds an optional torch extension (``lmcache_musa_batch_copy_ext.py:19-43``)
whose module functions are ``abi_version``, ``runtime_version``, ``driver_version``,
``batch_memcpy_supported``, ``execute_batch_copy`` and ``execute_copy_loop``
(``lmcache_musa_batch_copy_ext.cpp:268-277``).  Here the same object is a thin Python layer over
``libmusa_aiter_kv_hip.so``: ``execute_batch_copy`` submits the whole batch through the
batch-copy kernel (pinned host memory; with ``prefer_overlap_with_compute`` on at most 16
workgroups instead of 64, so concurrent kernels keep the other compute units);
``execute_copy_loop`` issues one ``hipMemcpyAsync`` per range, as the reference's loop does
with ``musaMemcpyAsync``.  Both
check their arguments like the reference's ``prepare_copy`` (``:76-170``, ``RuntimeError``),
run on the current stream of the GPU endpoint's device and keep every tensor of a batch alive
until the stream has passed it, which is what the reference's allocator ``record_event`` /
``recordStream`` calls ensure.

The extension is opt-in exactly like the reference's: it is returned only when
``MUSA_AITER_LMCACHE_BATCH_COPY=1`` or ``LMCACHE_MUSA_DIRECT_COPY=1``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections import deque
from typing import Any, Sequence

import torch

from musa_aiter.ops import _hip

_ABI_VERSION = 1
_EXT: Any | None = None
_EXT_ERROR: Exception | None = None
_LOCK = threading.Lock()


def lmcache_musa_batch_copy_requested() -> bool:
    return (os.environ.get("MUSA_AITER_LMCACHE_BATCH_COPY", "0") == "1"
            or os.environ.get("LMCACHE_MUSA_DIRECT_COPY", "0") == "1")


def _gpu(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


class _InFlight:
    """Tensors of submitted batches, held until an event recorded after the batch has completed."""

    def __init__(self) -> None:
        self._pending: deque[tuple[torch.cuda.Event, tuple[torch.Tensor, ...]]] = deque()
        self._lock = threading.Lock()

    def add(self, stream: torch.cuda.Stream, tensors: tuple[torch.Tensor, ...]) -> None:
        event = torch.cuda.Event()
        event.record(stream)
        with self._lock:
            self._pending.append((event, tensors))
            self._release_done()

    def _release_done(self) -> None:
        kept = deque()
        while self._pending:
            event, tensors = self._pending.popleft()
            if not event.query():
                kept.append((event, tensors))
        self._pending = kept

    def __len__(self) -> int:
        with self._lock:
            self._release_done()
            return len(self._pending)


class HipBatchCopyExtension:
    """The reference extension's module functions over the HIP library."""

    def __init__(self) -> None:
        self.in_flight = _InFlight()

    def abi_version(self) -> int:
        return int(_hip.fn("musa_aiter_hip_batch_copy_abi_version")())

    def _versions(self) -> tuple[int, int]:
        runtime, driver = ctypes.c_int(0), ctypes.c_int(0)
        _hip.check(int(_hip.fn("musa_aiter_hip_runtime_versions")(ctypes.byref(runtime), ctypes.byref(driver))),
                   "runtime versions")
        return runtime.value, driver.value

    def runtime_version(self) -> int:
        return self._versions()[0]

    def driver_version(self) -> int:
        return self._versions()[1]

    def batch_memcpy_supported(self) -> bool:
        return True

    @staticmethod
    def _prepare(destinations: Sequence[torch.Tensor], sources: Sequence[torch.Tensor],
                 destination_offsets: Sequence[int], source_offsets: Sequence[int], sizes: Sequence[int]):
        """The reference's prepare_copy checks (lmcache_musa_batch_copy_ext.cpp:76-170)."""
        count = len(sizes)
        if len(destinations) != count or len(sources) != count:
            raise RuntimeError("destinations, sources, and sizes must have the same length")
        if len(destination_offsets) != count or len(source_offsets) != count:
            raise RuntimeError("offset vectors must have the same length as sizes")
        dsts, srcs, lens, gpu_tensors, host_tensors = [], [], [], [], []
        to_gpu = None
        device = None
        spans = []
        for i in range(count):
            dst, src = destinations[i], sources[i]
            if not dst.is_contiguous() or not src.is_contiguous():
                raise RuntimeError("batch-copy tensors must be contiguous")
            if _gpu(dst) == _gpu(src):
                raise RuntimeError("each entry must have exactly one GPU endpoint")
            if to_gpu is None:
                to_gpu = _gpu(dst)
            if _gpu(dst) != to_gpu:
                raise RuntimeError("one batch cannot mix h2d and d2h copies")
            gpu_t, host_t = (dst, src) if to_gpu else (src, dst)
            if host_t.device.type != "cpu":
                raise RuntimeError("the non-GPU endpoint must be a CPU tensor")
            if device is None:
                device = gpu_t.device
            if gpu_t.device != device:
                raise RuntimeError("all entries must use the same GPU device")
            d_off, s_off, size = int(destination_offsets[i]), int(source_offsets[i]), int(sizes[i])
            if d_off < 0:
                raise RuntimeError(f"destination_offsets[{i}] must be non-negative")
            if s_off < 0:
                raise RuntimeError(f"source_offsets[{i}] must be non-negative")
            if size <= 0:
                raise RuntimeError(f"copy_sizes[{i}] must be positive")
            if d_off + size > dst.numel() * dst.element_size():
                raise RuntimeError(f"destination range at index {i} exceeds tensor capacity")
            if s_off + size > src.numel() * src.element_size():
                raise RuntimeError(f"source range at index {i} exceeds tensor capacity")
            dsts.append(dst.data_ptr() + d_off)
            srcs.append(src.data_ptr() + s_off)
            lens.append(size)
            spans.append((dsts[-1], dsts[-1] + size))
            gpu_tensors.append(gpu_t)
            host_tensors.append(host_t)
        spans.sort()
        for (_, prev_end), (start, _) in zip(spans, spans[1:]):
            if start < prev_end:
                raise RuntimeError("overlapping destination ranges are invalid in an unordered batch")
        return dsts, srcs, lens, bool(to_gpu), device, gpu_tensors, host_tensors

    def _submit(self, destinations, sources, destination_offsets, source_offsets, sizes, mode: int) -> bool:
        dsts, srcs, lens, to_gpu, device, gpu_tensors, host_tensors = self._prepare(
            destinations, sources, destination_offsets, source_offsets, sizes)
        if not lens:
            return True
        n = len(lens)
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device)
            rc = _hip.fn("musa_aiter_hip_batch_copy")(
                (ctypes.c_void_p * n)(*dsts), (ctypes.c_void_p * n)(*srcs), (ctypes.c_uint64 * n)(*lens), n,
                0 if to_gpu else 1, int(mode), ctypes.c_void_p(stream.cuda_stream))
            _hip.check(int(rc), "lmcache_musa_memcpy_batch_async")
            for t in {id(t): t for t in gpu_tensors}.values():
                t.record_stream(stream)
            self.in_flight.add(stream, tuple({id(t): t for t in host_tensors + gpu_tensors}.values()))
        return True

    def execute_batch_copy(self, destinations, sources, destination_offsets, source_offsets, sizes,
                           prefer_overlap_with_compute: bool) -> bool:
        return self._submit(destinations, sources, destination_offsets, source_offsets, sizes,
                            mode=1 if prefer_overlap_with_compute else 0)

    def execute_copy_loop(self, destinations, sources, destination_offsets, source_offsets, sizes) -> bool:
        return self._submit(destinations, sources, destination_offsets, source_offsets, sizes, mode=2)


def load_lmcache_musa_batch_copy_ext() -> Any | None:
    """The extension object when the feature is requested and the HIP library loads, else None."""
    global _EXT, _EXT_ERROR
    if not lmcache_musa_batch_copy_requested():
        return None
    with _LOCK:
        if _EXT is None and _EXT_ERROR is None:
            try:
                _hip.library()
                _EXT = HipBatchCopyExtension()
            except (_hip.HipBackendError, OSError) as exc:
                _EXT_ERROR = exc
        return _EXT


def lmcache_musa_batch_copy_ext_error() -> Exception | None:
    return _EXT_ERROR
