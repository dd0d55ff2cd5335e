"""Validation and splitting of one unordered host/device byte-copy batch (no torch dependency).

Contract (the reference's ``musa_aiter/ops/lmcache_musa_batch_copy_plan.py``, 0.5.0; its
dataclasses, keyword arguments and ``ValueError`` messages are the public interface, :7-178):
every entry copies ``size`` bytes from ``source_offset`` to ``destination_offset``; sizes are
positive, offsets non-negative, both ranges inside their tensors, and the ranges written into one
destination never overlap, because the batch is unordered.  With ``pin_chunk_size`` an entry is
cut wherever its host-side offset reaches a multiple of ``pin_chunk_size`` (a host registration
boundary, :129-152), so no piece straddles two registrations.

Design: the six integer columns are normalised by one helper, the per-entry rules are a table of
(predicate, message) pairs evaluated in the reference's order, overlaps are found with one sort of
(destination group, start, end) triples, and an entry's pieces are the spans between its
boundary offsets.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import islice
from typing import Callable, Hashable, Iterator, Sequence


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


def _is_int(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _column(name: str, values: Sequence[int], count: int) -> tuple[int, ...]:
    column = tuple(values)
    if len(column) != count:
        raise ValueError(f"{name} must have the same length as sizes")
    if not all(_is_int(v) for v in column):
        raise ValueError(f"{name} must contain integers")
    return column


def _key_column(values: Sequence[Hashable] | None, count: int) -> tuple[Hashable, ...]:
    keys = tuple(range(count)) if values is None else tuple(values)
    if len(keys) != count:
        raise ValueError("destination_keys must have the same length as sizes")
    try:
        for key in keys:
            hash(key)
    except TypeError as exc:
        raise ValueError("destination_keys must contain hashable values") from exc
    return keys


# Per-entry rules, checked entry by entry in this order: (violated?, message).  The arguments are
# (index, size, source offset, destination offset, host offset, source capacity, destination capacity).
_Rule = Callable[[int, int, int, int, int, int, int], bool]
_ENTRY_RULES: tuple[tuple[_Rule, Callable[[int], str]], ...] = (
    (lambda i, n, so, do, ho, sc, dc: n <= 0,
     lambda i: f"sizes[{i}] must be positive"),
    (lambda i, n, so, do, ho, sc, dc: min(so, do, ho) < 0,
     lambda i: "copy offsets must be non-negative"),
    (lambda i, n, so, do, ho, sc, dc: dc < 0 or do + n > dc,
     lambda i: f"destination range at index {i} exceeds tensor capacity"),
    (lambda i, n, so, do, ho, sc, dc: sc < 0 or so + n > sc,
     lambda i: f"source range at index {i} exceeds tensor capacity"),
)


def _reject_overlaps(destination_offsets: Sequence[int], sizes: Sequence[int], keys: Sequence[Hashable]) -> None:
    """Any two overlapping ranges of one destination put an overlapping pair next to each other once the
    ranges are sorted by (destination, start), so one pass over the sorted triples finds them."""
    group: dict[Hashable, int] = {}
    spans = sorted((group.setdefault(k, len(group)), off, off + n) for k, off, n in zip(keys, destination_offsets, sizes))
    for (g0, _, end0), (g1, start1, _) in zip(spans, spans[1:]):
        if g0 == g1 and start1 < end0:
            raise ValueError("overlapping destination ranges are invalid in an unordered batch")


def _pieces(host_offset: int, size: int, pin_chunk_size: int | None) -> Iterator[tuple[int, int]]:
    """(start, length) of the pieces of one entry, relative to its first byte: cut where the host offset
    reaches a multiple of ``pin_chunk_size``."""
    if pin_chunk_size is None:
        yield 0, size
        return
    first_cut = pin_chunk_size - host_offset % pin_chunk_size
    bounds = [0, *range(first_cut, size, pin_chunk_size), size]
    for start, stop in zip(bounds, bounds[1:]):
        yield start, stop - start


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
    """Validate one unordered batch and split its entries at host registration boundaries."""
    if direction not in ("h2d", "d2h"):
        raise ValueError("direction must be 'h2d' or 'd2h'")
    if pin_chunk_size is not None and not (_is_int(pin_chunk_size) and pin_chunk_size > 0):
        raise ValueError("pin_chunk_size must be a positive integer")
    count = len(sizes)
    zeros = (0,) * count
    n = _column("sizes", sizes, count)
    src_cap = _column("source_capacities", source_capacities, count)
    dst_cap = _column("destination_capacities", destination_capacities, count)
    src_off = _column("source_offsets", zeros if source_offsets is None else source_offsets, count)
    dst_off = _column("destination_offsets", zeros if destination_offsets is None else destination_offsets, count)
    # The host side of the copy registers its memory: by default its registration offsets are its
    # copy offsets (the source of an h2d batch, the destination of a d2h one).
    host_off = _column("host_registration_offsets",
                       (src_off if direction == "h2d" else dst_off) if host_registration_offsets is None
                       else host_registration_offsets, count)
    keys = _key_column(destination_keys, count)

    for row in zip(range(count), n, src_off, dst_off, host_off, src_cap, dst_cap):
        for violated, message in _ENTRY_RULES:
            if violated(*row):
                raise ValueError(message(row[0]))
    _reject_overlaps(dst_off, n, keys)

    entries = tuple(
        BatchCopyEntry(input_index=i, source_offset=so + start, destination_offset=do + start, size=length,
                       host_registration_offset=ho + start)
        for i, so, do, ho, size in zip(range(count), src_off, dst_off, host_off, n)
        for start, length in _pieces(ho, size, pin_chunk_size))
    return BatchCopyPlan(direction=direction, entries=entries, total_bytes=sum(n), input_entry_count=count)


def chunk_batch_copy_plan(plan: BatchCopyPlan, max_batch_entries: int) -> tuple[tuple[BatchCopyEntry, ...], ...]:
    """The plan's entries in submission order, ``max_batch_entries`` at a time (the last group may be
    shorter); groups are submitted one after another on the same stream."""
    if not (_is_int(max_batch_entries) and max_batch_entries > 0):
        raise ValueError("max_batch_entries must be a positive integer")
    remaining = iter(plan.entries)
    return tuple(iter(lambda: tuple(islice(remaining, max_batch_entries)), ()))
