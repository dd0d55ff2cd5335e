"""Opt-in host/device byte-copy batches for LMCache on MI355X (ROCm HIP backend).

Contract (the reference's ``musa_aiter/ops/lmcache_musa_batch_copy.py``, 0.5.0; public names,
keyword arguments, defaults, return values, gate variables and messages, :1-263):

- ``lmcache_musa_memcpy_batch_async`` submits one unordered batch of byte copies, all host ->
  device or all device -> host, on the current stream of the GPU endpoints' device.  ``True``
  means submitted (or empty); ``False`` means the feature is not requested
  (``MUSA_AITER_LMCACHE_BATCH_COPY=1`` / ``LMCACHE_MUSA_DIRECT_COPY=1``), the backend is
  unavailable or an entry is not a host <-> GPU pair, so the caller keeps its own path;
- the batch is validated and split at host registration boundaries by
  ``lmcache_musa_batch_copy_plan`` and submitted in stream-ordered groups of at most
  ``max_batch_entries`` entries (default 1024, ``MUSA_AITER_LMCACHE_BATCH_MAX_ENTRIES``); a group
  that fails after an earlier one went out raises instead of falling back.

The host work is sized for batches of thousands of ranges: per-tensor facts are read once per
distinct tensor, and the plan is built and cut into groups as int64 columns (no per-range Python
objects on this path).

Each group becomes one ``execute_batch_copy`` call of the extension object
(``lmcache_musa_batch_copy_ext``), i.e. one ``musa_aiter_hip_batch_copy`` call of
``libmusa_aiter_kv_hip.so``: pinned host ranges move in one batch-copy kernel launch (the GPU
reads or writes the host memory over its mapping; ``prefer_overlap_with_compute=True`` keeps the
kernel to 16 workgroups), pageable ranges go through ``hipMemcpyAsync``.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Protocol, Sequence

import numpy as np
import torch

from . import _hip
from .kv_backend import KVBackendCapabilities, KVBackendDecision, select_kv_backend
from .kv_transfer_plan import KVTransferPlan
from .lmcache_musa_batch_copy_ext import HipBatchCopyExtension, lmcache_musa_batch_copy_requested
from .lmcache_musa_batch_copy_ext import load_lmcache_musa_batch_copy_ext
from .lmcache_musa_batch_copy_plan import build_batch_copy_plan as _build_batch_copy_plan
from .lmcache_musa_batch_copy_plan import chunk_batch_copy_plan as _chunk_batch_copy_plan
from .lmcache_musa_batch_copy_plan import plan_columns as _plan_columns

_ABI_VERSION = 1
_DEFAULT_MAX_BATCH_ENTRIES = 1024
_MAX_ENTRIES_ENV = "MUSA_AITER_LMCACHE_BATCH_MAX_ENTRIES"

# (source kind, destination kind) -> (direction, index of the host tensor in (source, destination)).
_ROUTES = {("cpu", "gpu"): ("h2d", 0), ("gpu", "cpu"): ("d2h", 1)}


class _BatchCopyExtension(Protocol):
    def abi_version(self) -> int: ...

    def runtime_version(self) -> int: ...

    def driver_version(self) -> int: ...

    def batch_memcpy_supported(self) -> bool: ...

    def execute_batch_copy(self, destinations: Sequence[torch.Tensor], sources: Sequence[torch.Tensor],
                           destination_offsets: Sequence[int], source_offsets: Sequence[int], sizes: Sequence[int],
                           prefer_overlap_with_compute: bool) -> bool: ...


def native_lmcache_musa_batch_copy_abi_version() -> int:
    return _ABI_VERSION


def _extension_if_requested(*, need_batch: bool) -> _BatchCopyExtension | None:
    """The extension object when the feature is requested and its ABI matches (and, with ``need_batch``,
    it supports batched copies); ``None`` otherwise.  Any error the extension raises counts as absent."""
    if not lmcache_musa_batch_copy_requested():
        return None
    extension = load_lmcache_musa_batch_copy_ext()
    if extension is None:
        return None
    try:
        usable = extension.abi_version() == _ABI_VERSION and (not need_batch or extension.batch_memcpy_supported())
    except Exception:
        return None
    return extension if usable else None


def native_lmcache_musa_batch_copy_runtime_versions() -> tuple[int, int] | None:
    """(HIP runtime, driver) versions reported by the extension, or ``None`` when the feature is off."""
    extension = _extension_if_requested(need_batch=False)
    if extension is None:
        return None
    try:
        return extension.runtime_version(), extension.driver_version()
    except Exception:
        return None


def is_native_lmcache_musa_batch_copy_available() -> bool:
    return _extension_if_requested(need_batch=True) is not None


def select_lmcache_batch_copy_backend(plan: KVTransferPlan, *, native_available: bool | None = None,
                                      require_native: bool = False) -> KVBackendDecision:
    """Backend decision for an LMCache transfer plan before any copy is submitted (the batch path counts
    as the direct-batch capability; the caller's own copies are the reference path)."""
    if native_available is None:
        native_available = is_native_lmcache_musa_batch_copy_available()
    capabilities = KVBackendCapabilities(direct_batch=bool(native_available), reference=True)
    return select_kv_backend(plan, capabilities=capabilities, require_native=require_native)


def _tensor_device_kind(tensor: torch.Tensor) -> str:
    """"cpu", "gpu" (a ROCm device: torch's "cuda" type) or "unsupported"."""
    return {"cpu": "cpu", "cuda": "gpu"}.get(tensor.device.type.lower(), "unsupported")


@dataclass(frozen=True)
class _Endpoints:
    """What a batch's tensors say about it: its direction and its one GPU device."""

    direction: str
    device: tuple[str, int | None]


def _classify(destinations: tuple, sources: tuple, pair_keys: np.ndarray,
              require_pinned_host: bool) -> _Endpoints | None:
    """Check every pair in order; ``None`` as soon as a pair is not host <-> GPU (not this backend's).

    A batch names the same few tensors many times (one staging buffer, one cache).  An entry whose
    (destination, source) pair of objects already appeared passes or fails exactly as its first
    appearance did, and the first failing entry is always a first appearance, so only the first
    appearance of each pair is checked, in entry order.  ``pair_keys[i]`` identifies entry i's pair
    of objects."""
    firsts = np.sort(np.unique(pair_keys, return_index=True)[1]).tolist()
    directions, devices = set(), set()
    for index in firsts:
        destination, source = destinations[index], sources[index]
        if not isinstance(destination, torch.Tensor) or not isinstance(source, torch.Tensor):
            raise TypeError("destinations and sources must contain torch.Tensor values")
        if not (destination.is_contiguous() and source.is_contiguous()):
            raise ValueError("batch-copy tensors must be contiguous")
        route = _ROUTES.get((_tensor_device_kind(source), _tensor_device_kind(destination)))
        if route is None:
            return None
        direction, host_side = route
        pair = (source, destination)
        if require_pinned_host and not pair[host_side].is_pinned():
            raise ValueError(f"host tensor at index {index} must use pinned memory")
        gpu = pair[1 - host_side]
        directions.add(direction)
        devices.add((gpu.device.type, gpu.device.index))
    if len(directions) != 1:
        raise ValueError("one batch cannot mix h2d and d2h copies")
    if len(devices) != 1:
        raise ValueError("all batch entries must use the same GPU device")
    return _Endpoints(directions.pop(), devices.pop())


def lmcache_musa_memcpy_batch_async(
    destinations: Sequence[torch.Tensor],
    sources: Sequence[torch.Tensor],
    sizes: Sequence[int],
    *,
    destination_offsets: Sequence[int] | None = None,
    source_offsets: Sequence[int] | None = None,
    host_registration_offsets: Sequence[int] | None = None,
    pin_chunk_size: int | None = None,
    require_pinned_host: bool = True,
    prefer_overlap_with_compute: bool = False,
    max_batch_entries: int | None = None,
) -> bool:
    """Submit an opt-in host/device byte-copy batch on the current stream.

    ``True`` means the batch was submitted (or was empty); ``False`` means the backend was not
    requested or is unavailable, so the caller uses its existing transfer path.  A plan longer than
    ``max_batch_entries`` goes out as ordered groups on the same current stream.
    """
    destinations, sources, sizes = tuple(destinations), tuple(sources), tuple(sizes)
    if not (destinations or sources or sizes):
        return True
    if not len(destinations) == len(sources) == len(sizes):
        raise ValueError("destinations, sources, and sizes must have the same length")
    # The batch's distinct objects (by identity) and each entry's index among them.  When the backend is
    # asked for, its host helper must load and numbers them; otherwise one sort of the object ids does.
    count = len(sizes)
    host = None
    if lmcache_musa_batch_copy_requested():
        try:
            host = _hip.host()
        except (_hip.HipBackendError, OSError, ImportError):
            host = None  # no helper module: the numpy numbering below serves, and the checks decide
    if host is not None:
        packed, tensors = host.object_index(destinations, sources)
        which = np.frombuffer(packed, dtype=np.int64)
    else:
        both = (*destinations, *sources)
        _, first, which = np.unique(np.fromiter(map(id, both), dtype=np.uint64, count=2 * count),
                                    return_index=True, return_inverse=True)
        tensors = [both[i] for i in first.tolist()]
    dst_index, src_index = which[:count], which[count:]
    endpoints = _classify(destinations, sources, dst_index * len(tensors) + src_index, require_pinned_host)
    if endpoints is None:
        return False
    capacity = np.array([t.numel() * t.element_size() for t in tensors], dtype=np.int64)
    # The columns go to the plan as int64 arrays made here or as tuples that it checks item by item (so
    # a caller's own array is rejected as the reference rejects it).  The host helper reads the
    # caller's lists of ints; a list it declines (an item that is not a plain int, or a large one)
    # stays a tuple.
    column = None if host is None else host.int64_column

    def own(values):
        packed = None if values is None or column is None else column(values)
        if packed is not None:
            return np.frombuffer(packed, dtype=np.int64)
        return None if values is None else tuple(values)

    sizes_in, offsets_in = own(sizes), [own(v) for v in (source_offsets, destination_offsets,
                                                         host_registration_offsets)]
    plan = _plan_columns(
        direction=endpoints.direction, sizes=sizes_in, source_capacities=capacity[src_index],
        destination_capacities=capacity[dst_index], source_offsets=offsets_in[0], destination_offsets=offsets_in[1],
        host_registration_offsets=offsets_in[2], pin_chunk_size=pin_chunk_size,
        destination_keys=dst_index.astype(np.int64), int64_arrays=True)
    extension = _extension_if_requested(need_batch=True)
    if extension is None:
        return False
    # Groups of max_batch_entries pieces in plan order, each one extension call.  This package's own
    # extension takes a group as columns; any other extension object gets the reference's lists.
    limit = _resolve_max_batch_entries(max_batch_entries)
    total = plan.input_index.shape[0]
    columns = isinstance(extension, HipBatchCopyExtension) and plan.size.dtype == np.int64
    for number, lo in enumerate(range(0, total, limit)):
        piece = slice(lo, lo + limit)
        if columns:
            index = plan.input_index[piece]
            ok = extension.execute_batch_copy_columns(tensors, dst_index[index], src_index[index],
                                                      plan.destination_offset[piece], plan.source_offset[piece],
                                                      plan.size[piece], prefer_overlap_with_compute)
        else:
            index = plan.input_index[piece].tolist()
            ok = extension.execute_batch_copy([destinations[i] for i in index], [sources[i] for i in index],
                                              plan.destination_offset[piece].tolist(),
                                              plan.source_offset[piece].tolist(), plan.size[piece].tolist(),
                                              prefer_overlap_with_compute)
        if ok:
            continue
        if number == 0:
            return False
        raise RuntimeError("batch-copy chunk failed after an earlier chunk was submitted")
    return True


def lmcache_musa_memcpy_batch_async_internal(
    destinations: Sequence[torch.Tensor],
    sources: Sequence[torch.Tensor],
    sizes: Sequence[int],
    *,
    host_registration_offsets: Sequence[int],
    pin_chunk_size: int,
    destination_offsets: Sequence[int] | None = None,
    source_offsets: Sequence[int] | None = None,
    require_pinned_host: bool = True,
    prefer_overlap_with_compute: bool = False,
    max_batch_entries: int | None = None,
) -> bool:
    """The LMCache entry: the same submission, with the host registration boundary mandatory."""
    if host_registration_offsets is None or pin_chunk_size is None:
        raise ValueError("LMCache internal API requires a host registration boundary")
    return lmcache_musa_memcpy_batch_async(
        destinations, sources, sizes, destination_offsets=destination_offsets, source_offsets=source_offsets,
        host_registration_offsets=host_registration_offsets, pin_chunk_size=pin_chunk_size,
        require_pinned_host=require_pinned_host, prefer_overlap_with_compute=prefer_overlap_with_compute,
        max_batch_entries=max_batch_entries)


def _resolve_max_batch_entries(value: int | None) -> int:
    """The explicit limit, else the environment's, else 1024."""
    if value is not None:
        if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
            raise ValueError("max_batch_entries must be a positive integer")
        return value
    text = os.environ.get(_MAX_ENTRIES_ENV)
    if text is None:
        return _DEFAULT_MAX_BATCH_ENTRIES
    try:
        limit = int(text)
    except ValueError as exc:
        raise ValueError(f"{_MAX_ENTRIES_ENV} must be an integer") from exc
    if limit <= 0:
        raise ValueError(f"{_MAX_ENTRIES_ENV} must be positive")
    return limit
