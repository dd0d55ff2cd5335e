"""Validation and splitting of one unordered host/device byte-copy batch (no torch dependency).

Interface and rules of the reference's ``musa_aiter/ops/lmcache_musa_batch_copy_plan.py``
(0.5.0): every entry copies ``size`` bytes from ``source_offset`` to ``destination_offset``;
offsets are non-negative, sizes positive, ranges inside their tensors, destination ranges of one
destination never overlap (the batch is unordered), and with ``pin_chunk_size`` an entry is cut
where its host-side offset crosses a multiple of ``pin_chunk_size`` (a host registration
boundary; :129-152).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Hashable, Sequence


@dataclass(frozen=True)
class BatchCopyEntry:
    input_index: int
    source_offset: int
    destination_offset: int
    size: int
    host_registration_offset: int


@dataclass(frozen=True)
class BatchCopyPlan:
    direction: str
    entries: tuple[BatchCopyEntry, ...]
    total_bytes: int
    input_entry_count: int


def _ints(name: str, values: Sequence[int], count: int) -> tuple[int, ...]:
    if len(values) != count:
        raise ValueError(f"{name} must have the same length as sizes")
    if any(isinstance(v, bool) or not isinstance(v, int) for v in values):
        raise ValueError(f"{name} must contain integers")
    return tuple(values)


def _hashables(name: str, values: Sequence[Hashable] | None, count: int) -> tuple[Hashable, ...]:
    keys = tuple(range(count)) if values is None else tuple(values)
    if len(keys) != count:
        raise ValueError(f"{name} must have the same length as sizes")
    for key in keys:
        try:
            hash(key)
        except TypeError as exc:
            raise ValueError(f"{name} must contain hashable values") from exc
    return keys


def _check_disjoint_destinations(offsets: Sequence[int], sizes: Sequence[int], keys: Sequence[Hashable]) -> None:
    by_key: dict[Hashable, list[tuple[int, int]]] = {}
    for off, size, key in zip(offsets, sizes, keys):
        by_key.setdefault(key, []).append((off, off + size))
    for spans in by_key.values():
        spans.sort()
        end = None
        for start, stop in spans:
            if end is not None and start < end:
                raise ValueError("overlapping destination ranges are invalid in an unordered batch")
            end = stop if end is None else max(end, stop)


def build_batch_copy_plan(
    *,
    direction: str,
    sizes: Sequence[int],
    source_capacities: Sequence[int],
    destination_capacities: Sequence[int],
    source_offsets: Sequence[int] | None = None,
    destination_offsets: Sequence[int] | None = None,
    host_registration_offsets: Sequence[int] | None = None,
    pin_chunk_size: int | None = None,
    destination_keys: Sequence[Hashable] | None = None,
) -> BatchCopyPlan:
    """Validate and split one unordered batch (reference :80-165)."""
    if direction not in ("h2d", "d2h"):
        raise ValueError("direction must be 'h2d' or 'd2h'")
    if pin_chunk_size is not None and (isinstance(pin_chunk_size, bool) or not isinstance(pin_chunk_size, int)
                                       or pin_chunk_size <= 0):
        raise ValueError("pin_chunk_size must be a positive integer")
    count = len(sizes)
    size_v = _ints("sizes", sizes, count)
    src_cap = _ints("source_capacities", source_capacities, count)
    dst_cap = _ints("destination_capacities", destination_capacities, count)
    src_off = _ints("source_offsets", [0] * count if source_offsets is None else source_offsets, count)
    dst_off = _ints("destination_offsets", [0] * count if destination_offsets is None else destination_offsets, count)
    # The host side's registration offsets default to the host-side copy offsets.
    host_default = src_off if direction == "h2d" else dst_off
    host_off = _ints("host_registration_offsets",
                     host_default if host_registration_offsets is None else host_registration_offsets, count)
    keys = _hashables("destination_keys", destination_keys, count)

    for i in range(count):
        if size_v[i] <= 0:
            raise ValueError(f"sizes[{i}] must be positive")
        if src_off[i] < 0 or dst_off[i] < 0 or host_off[i] < 0:
            raise ValueError("copy offsets must be non-negative")
        if dst_cap[i] < 0 or dst_off[i] + size_v[i] > dst_cap[i]:
            raise ValueError(f"destination range at index {i} exceeds tensor capacity")
        if src_cap[i] < 0 or src_off[i] + size_v[i] > src_cap[i]:
            raise ValueError(f"source range at index {i} exceeds tensor capacity")
    _check_disjoint_destinations(dst_off, size_v, keys)

    entries: list[BatchCopyEntry] = []
    for i in range(count):
        s, d, h, left = src_off[i], dst_off[i], host_off[i], size_v[i]
        while left:
            step = left if pin_chunk_size is None else min(left, pin_chunk_size - h % pin_chunk_size)
            entries.append(BatchCopyEntry(i, s, d, step, h))
            s, d, h, left = s + step, d + step, h + step, left - step
    return BatchCopyPlan(direction, tuple(entries), sum(size_v), count)


def chunk_batch_copy_plan(plan: BatchCopyPlan, max_batch_entries: int) -> tuple[tuple[BatchCopyEntry, ...], ...]:
    """Split a validated plan into stream-ordered submissions of at most ``max_batch_entries`` (reference :168-178)."""
    if isinstance(max_batch_entries, bool) or not isinstance(max_batch_entries, int) or max_batch_entries <= 0:
        raise ValueError("max_batch_entries must be a positive integer")
    entries = plan.entries
    return tuple(entries[i:i + max_batch_entries] for i in range(0, len(entries), max_batch_entries))
