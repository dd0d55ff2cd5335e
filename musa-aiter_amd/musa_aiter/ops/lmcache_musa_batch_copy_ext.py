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

import numpy as np
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
    def _prepare_entry(i: int, dst: torch.Tensor, src: torch.Tensor, d_off: int, s_off: int, size: int,
                       to_gpu: bool | None, device) -> None:
        """The reference's prepare_copy checks of entry ``i`` (lmcache_musa_batch_copy_ext.cpp:76-170), in its
        order; ``to_gpu`` / ``device`` are those of the first entry (None while checking the first)."""
        if not dst.is_contiguous() or not src.is_contiguous():
            raise RuntimeError("batch-copy tensors must be contiguous")
        if _gpu(dst) == _gpu(src):
            raise RuntimeError("each entry must have exactly one GPU endpoint")
        if to_gpu is not None and _gpu(dst) != to_gpu:
            raise RuntimeError("one batch cannot mix h2d and d2h copies")
        gpu_t, host_t = (dst, src) if _gpu(dst) else (src, dst)
        if host_t.device.type != "cpu":
            raise RuntimeError("the non-GPU endpoint must be a CPU tensor")
        if device is not None and gpu_t.device != device:
            raise RuntimeError("all entries must use the same GPU device")
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

    @classmethod
    def _prepare(cls, destinations: Sequence[torch.Tensor], sources: Sequence[torch.Tensor],
                 destination_offsets: Sequence[int], source_offsets: Sequence[int], sizes: Sequence[int]):
        """The reference's prepare_copy checks (lmcache_musa_batch_copy_ext.cpp:76-170) for a whole group.

        Each distinct tensor's facts (contiguity, device, address, byte size) are read once; the per-entry
        checks then run as int64 column operations, and the first entry that fails any of them is checked
        again on its own (``_prepare_entry``) to raise the reference's error for it."""
        count = len(sizes)
        if len(destinations) != count or len(sources) != count:
            raise RuntimeError("destinations, sources, and sizes must have the same length")
        if len(destination_offsets) != count or len(source_offsets) != count:
            raise RuntimeError("offset vectors must have the same length as sizes")
        if count == 0:
            return np.zeros(0, np.uint64), np.zeros(0, np.uint64), np.zeros(0, np.uint64), True, None, [], []
        # Distinct objects by identity: one sort of the entries' object ids, both sides together.
        both = (*destinations, *sources)
        ids = np.fromiter(map(id, both), dtype=np.uint64, count=2 * count)
        _, first, which = np.unique(ids, return_index=True, return_inverse=True)
        tensors = [both[i] for i in first.tolist()]
        try:
            d_off = np.fromiter(map(int, destination_offsets), dtype=np.int64, count=count)
            s_off = np.fromiter(map(int, source_offsets), dtype=np.int64, count=count)
            size = np.fromiter(map(int, sizes), dtype=np.int64, count=count)
        except OverflowError:
            d_off = s_off = size = None
        return cls._prepare_columns(
            tensors, which[:count], which[count:], d_off, s_off, size,
            lambda i: (destinations[i], sources[i], int(destination_offsets[i]), int(source_offsets[i]), int(sizes[i])))

    @classmethod
    def _prepare_columns(cls, tensors: Sequence[torch.Tensor], di: np.ndarray, si: np.ndarray,
                         d_off: np.ndarray | None, s_off: np.ndarray | None, size: np.ndarray | None, entry=None):
        """``_prepare`` for entries given as indices into distinct ``tensors`` and int64 columns (``None``
        columns: values beyond int64, checked entry by entry).  ``entry(i)`` gives entry i's
        (destination, source, destination offset, source offset, size) for the per-entry re-check."""
        count = int(di.shape[0])
        if entry is None:
            def entry(i: int):
                return tensors[di[i]], tensors[si[i]], int(d_off[i]), int(s_off[i]), int(size[i])
        contig = np.array([t.is_contiguous() for t in tensors])
        gpu = np.array([_gpu(t) for t in tensors])
        cpu = np.array([t.device.type == "cpu" for t in tensors])
        devices = [t.device for t in tensors]
        nbytes = np.array([t.numel() * t.element_size() for t in tensors], dtype=np.int64)
        big = d_off is None or any(int(a.max()) >= 1 << 61 for a in (d_off, s_off, size))
        first_gpu = bool(gpu[di[0]]) if gpu[di[0]] != gpu[si[0]] else None
        if big or first_gpu is None:
            bad_index = 0 if first_gpu is None else None
        else:
            gi = np.where(gpu[di], di, si)
            hi = np.where(gpu[di], si, di)
            device = devices[gi[0]]
            same_device = np.array([d == device for d in devices])
            bad = (~(contig[di] & contig[si]) | (gpu[di] == gpu[si]) | (gpu[di] != first_gpu) | ~cpu[hi]
                   | ~same_device[gi] | (d_off < 0) | (s_off < 0) | (size <= 0)
                   | (d_off + size > nbytes[di]) | (s_off + size > nbytes[si]))
            bad_index = int(np.argmax(bad)) if bad.any() else None
        if big or bad_index is not None:
            to_gpu = device = None
            for i in range(count if big else bad_index + 1):
                dst, src, d, s, n = entry(i)
                cls._prepare_entry(i, dst, src, d, s, n, to_gpu, device)
                if to_gpu is None:
                    to_gpu, device = _gpu(dst), (dst if _gpu(dst) else src).device
            if not big:
                raise AssertionError("a column check failed where the entry checks pass")
            raise RuntimeError("batch-copy offsets and sizes must stay below 2**61")
        ptr = np.array([t.data_ptr() for t in tensors], dtype=np.uint64)
        dsts = ptr[di] + d_off.astype(np.uint64)
        srcs = ptr[si] + s_off.astype(np.uint64)
        lens = size.astype(np.uint64)
        order = np.lexsort((dsts + lens, dsts))
        start, stop = dsts[order], (dsts + lens)[order]
        if np.any(start[1:] < stop[:-1]):
            raise RuntimeError("overlapping destination ranges are invalid in an unordered batch")
        used = np.zeros(len(tensors), dtype=bool)
        used[di] = used[si] = True
        gpu_tensors = [t for t, g, u in zip(tensors, gpu, used) if g and u]
        host_tensors = [t for t, g, u in zip(tensors, gpu, used) if u and not g]
        return dsts, srcs, lens, bool(first_gpu), device, gpu_tensors, host_tensors

    def _submit(self, destinations, sources, destination_offsets, source_offsets, sizes, mode: int) -> bool:
        return self._launch(self._prepare(destinations, sources, destination_offsets, source_offsets, sizes), mode)

    def _launch(self, prepared, mode: int) -> bool:
        dsts, srcs, lens, to_gpu, device, gpu_tensors, host_tensors = prepared
        n = int(lens.shape[0])
        if n == 0:
            return True
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device)
            rc = _hip.fn("musa_aiter_hip_batch_copy")(
                (ctypes.c_void_p * n).from_buffer_copy(dsts), (ctypes.c_void_p * n).from_buffer_copy(srcs),
                (ctypes.c_uint64 * n).from_buffer_copy(lens), n, 0 if to_gpu else 1, int(mode),
                ctypes.c_void_p(stream.cuda_stream))
            _hip.check(int(rc), "lmcache_musa_memcpy_batch_async")
            for t in gpu_tensors:
                t.record_stream(stream)
            self.in_flight.add(stream, tuple(host_tensors + gpu_tensors))
        return True

    def execute_batch_copy(self, destinations, sources, destination_offsets, source_offsets, sizes,
                           prefer_overlap_with_compute: bool) -> bool:
        return self._submit(destinations, sources, destination_offsets, source_offsets, sizes,
                            mode=1 if prefer_overlap_with_compute else 0)

    def execute_copy_loop(self, destinations, sources, destination_offsets, source_offsets, sizes) -> bool:
        return self._submit(destinations, sources, destination_offsets, source_offsets, sizes, mode=2)

    def execute_batch_copy_columns(self, tensors: Sequence[torch.Tensor], destination_index: np.ndarray,
                                   source_index: np.ndarray, destination_offsets: np.ndarray,
                                   source_offsets: np.ndarray, sizes: np.ndarray,
                                   prefer_overlap_with_compute: bool) -> bool:
        """``execute_batch_copy`` for a group given as int64 columns: entry i copies ``sizes[i]`` bytes from
        ``tensors[source_index[i]]`` to ``tensors[destination_index[i]]``.  Same checks, errors and
        submission; ``lmcache_musa_memcpy_batch_async`` uses it to hand its plan over without building
        per-entry lists (this build's addition: the reference extension takes lists only)."""
        if len(sizes) == 0:
            return True
        return self._launch(self._prepare_columns(tensors, destination_index, source_index, destination_offsets,
                                                  source_offsets, sizes), mode=1 if prefer_overlap_with_compute else 0)


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
