"""Validation and splitting of one unordered host/device byte-copy batch.

Contract (the reference's ``musa_aiter/ops/lmcache_musa_batch_copy_plan.py``, 0.5.0; its
dataclasses, keyword arguments and ``ValueError`` messages are the public interface, :7-178):
every entry copies ``size`` bytes from ``source_offset`` to ``destination_offset``; sizes are
positive, offsets non-negative, both ranges inside their tensors, and the ranges written into one
destination never overlap, because the batch is unordered.  With ``pin_chunk_size`` an entry is
cut wherever its host-side offset reaches a multiple of ``pin_chunk_size`` (a host registration
boundary, :129-152), so no piece straddles two registrations.

Design: a batch can hold thousands of ranges, so the checks and the split run column-wise on
int64 arrays.  The per-entry rules are a table of (predicate, message) pairs: all of them are
evaluated over whole columns, and only the first failing entry is re-checked rule by rule to
report the reference's message for it (entries in order, rules in order).  Overlaps are found with
one sort of (destination group, start) pairs; an entry's pieces are the spans between its
boundary offsets, computed for all entries at once.  Values too large for int64 arithmetic take
the same rules one entry at a time.  ``build_batch_copy_plan`` returns the reference's dataclasses;
the submission path reads the columns (``plan_columns``) and never builds per-entry objects.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import islice
from typing import Callable, Hashable, Iterator, NamedTuple, Sequence

import numpy as np


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


class PlanColumns(NamedTuple):
    """The plan's pieces in submission order, one int64 array per field."""

    direction: str
    input_index: np.ndarray
    source_offset: np.ndarray
    destination_offset: np.ndarray
    size: np.ndarray
    host_registration_offset: np.ndarray
    total_bytes: int
    input_entry_count: int


def _is_int(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _column(name: str, values: Sequence[int] | np.ndarray, count: int,
            arrays: bool = False) -> tuple[int, ...] | np.ndarray:
    # With ``arrays`` (the submission path) a column may come as a 1-D int64 array, taken as it is; the
    # reference's inputs are sequences of ints, and arrays elsewhere fail its integer check as there.
    if arrays and isinstance(values, np.ndarray) and values.dtype == np.int64 and values.ndim == 1:
        if values.shape[0] != count:
            raise ValueError(f"{name} must have the same length as sizes")
        return values
    column = tuple(values)
    if len(column) != count:
        raise ValueError(f"{name} must have the same length as sizes")
    # Plain ints pass in one C-level pass over the element types; anything else is checked one by one.
    if not set(map(type, column)) <= {int} and not all(_is_int(v) for v in column):
        raise ValueError(f"{name} must contain integers")
    return column


def _key_column(values: Sequence[Hashable] | np.ndarray | None, count: int,
                arrays: bool = False) -> tuple[Hashable, ...] | np.ndarray:
    if arrays and isinstance(values, np.ndarray) and values.dtype == np.int64 and values.ndim == 1:
        if values.shape[0] != count:
            raise ValueError("destination_keys must have the same length as sizes")
        return values
    keys = tuple(range(count)) if values is None else tuple(values)
    if len(keys) != count:
        raise ValueError("destination_keys must have the same length as sizes")
    if set(map(type, keys)) <= {int}:
        return keys
    try:
        for key in keys:
            hash(key)
    except TypeError as exc:
        raise ValueError("destination_keys must contain hashable values") from exc
    return keys


# Per-entry rules, checked entry by entry in this order: (violated?, message).  The arguments are
# (index, size, source offset, destination offset, host offset, source capacity, destination capacity);
# they hold for Python ints and, element-wise, for int64 arrays.
_Rule = Callable[..., object]
_ENTRY_RULES: tuple[tuple[_Rule, Callable[[int], str]], ...] = (
    (lambda i, n, so, do, ho, sc, dc: n <= 0,
     lambda i: f"sizes[{i}] must be positive"),
    (lambda i, n, so, do, ho, sc, dc: (so < 0) | (do < 0) | (ho < 0),
     lambda i: "copy offsets must be non-negative"),
    (lambda i, n, so, do, ho, sc, dc: (dc < 0) | (do + n > dc),
     lambda i: f"destination range at index {i} exceeds tensor capacity"),
    (lambda i, n, so, do, ho, sc, dc: (sc < 0) | (so + n > sc),
     lambda i: f"source range at index {i} exceeds tensor capacity"),
)

# Columns whose values all lie within +-2^61 cannot overflow int64 in the sums the rules and the
# split form (offset + size, offset + a piece start).
_LIMIT = 1 << 61


def _as_int64(columns: Sequence[tuple[int, ...] | np.ndarray]) -> list[np.ndarray] | None:
    arrays: list[np.ndarray] = []
    for column in columns:
        done = [a for c, a in zip(columns, arrays) if c is column]
        if done:  # the same column twice (host offsets defaulting to copy offsets)
            arrays.append(done[0])
            continue
        if isinstance(column, np.ndarray):
            array = column
        else:
            try:
                array = np.fromiter(column, dtype=np.int64, count=len(column))
            except OverflowError:
                return None
        if len(column) and (int(array.max()) >= _LIMIT or int(array.min()) <= -_LIMIT):
            return None
        arrays.append(array)
    return arrays


def _check_rules(columns: Sequence[tuple[int, ...]], arrays: list[np.ndarray] | None) -> None:
    """Raise the message of the first violated rule of the first entry that violates one."""
    count = len(columns[0])
    if arrays is not None:
        bad = np.zeros(count, dtype=bool)
        for violated, _ in _ENTRY_RULES:
            bad |= violated(None, *arrays)
        if not bad.any():
            return
        first = int(np.argmax(bad))
        rows = [(first, *(c[first] for c in columns))]
    else:
        rows = zip(range(count), *columns)
    for row in rows:
        for violated, message in _ENTRY_RULES:
            if violated(*row):
                raise ValueError(message(row[0]))


def _reject_overlaps(destination_offsets: np.ndarray, sizes: np.ndarray, keys: Sequence[Hashable]) -> None:
    """Sorted by (destination, start), any two overlapping ranges of one destination include an
    adjacent overlapping pair, so one comparison of neighbours finds them."""
    if isinstance(keys, np.ndarray):
        groups = keys  # int64 keys (tensor indices) group as they are
    elif set(map(type, keys)) <= {int} and (not keys or (max(keys) < 1 << 63 and min(keys) >= -(1 << 63))):
        groups = np.fromiter(keys, dtype=np.int64, count=len(keys))  # so do integer keys
    else:
        group: dict[Hashable, int] = {}
        groups = np.fromiter((group.setdefault(k, len(group)) for k in keys), dtype=np.int64, count=len(keys))
    order = np.lexsort((destination_offsets, groups))
    g, start, end = groups[order], destination_offsets[order], (destination_offsets + sizes)[order]
    if np.any((g[1:] == g[:-1]) & (start[1:] < end[:-1])):
        raise ValueError("overlapping destination ranges are invalid in an unordered batch")


def _reject_overlaps_scalar(destination_offsets: Sequence[int], sizes: Sequence[int],
                            keys: Sequence[Hashable]) -> None:
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


def _split(sizes: np.ndarray, host_offsets: np.ndarray, pin_chunk_size: int | None):
    """(entry index, start, length) of every piece, entries in order and pieces in order within each:
    piece 0 of an entry ends at its first boundary (``pin - host_offset % pin`` bytes in) or at its
    end, piece j > 0 starts j - 1 chunks after that boundary."""
    count = sizes.shape[0]
    if pin_chunk_size is None:
        return np.arange(count, dtype=np.int64), np.zeros(count, dtype=np.int64), sizes
    first_cut = pin_chunk_size - host_offsets % pin_chunk_size
    beyond = np.maximum(sizes - first_cut, 0)
    pieces = 1 + (beyond + pin_chunk_size - 1) // pin_chunk_size
    index = np.repeat(np.arange(count, dtype=np.int64), pieces)
    j = np.arange(index.shape[0], dtype=np.int64) - np.repeat(np.cumsum(pieces) - pieces, pieces)
    cut = first_cut[index]
    start = np.where(j == 0, 0, cut + (j - 1) * pin_chunk_size)
    stop = np.minimum(cut + j * pin_chunk_size, sizes[index])
    return index, start, stop - start


def plan_columns(
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
    int64_arrays: bool = False,
) -> PlanColumns:
    """``build_batch_copy_plan``'s checks and split, returned as int64 columns.  With ``int64_arrays``
    any column (and the keys) may also be a 1-D int64 array."""
    if direction not in ("h2d", "d2h"):
        raise ValueError("direction must be 'h2d' or 'd2h'")
    if pin_chunk_size is not None and not (_is_int(pin_chunk_size) and pin_chunk_size > 0):
        raise ValueError("pin_chunk_size must be a positive integer")
    count = len(sizes)
    zeros = np.zeros(count, dtype=np.int64) if int64_arrays else (0,) * count
    n = _column("sizes", sizes, count, int64_arrays)
    src_cap = _column("source_capacities", source_capacities, count, int64_arrays)
    dst_cap = _column("destination_capacities", destination_capacities, count, int64_arrays)
    src_off = _column("source_offsets", zeros if source_offsets is None else source_offsets, count, int64_arrays)
    dst_off = _column("destination_offsets", zeros if destination_offsets is None else destination_offsets, count,
                      int64_arrays)
    # The host side of the copy registers its memory: by default its registration offsets are its
    # copy offsets (the source of an h2d batch, the destination of a d2h one).
    host_off = _column("host_registration_offsets",
                       (src_off if direction == "h2d" else dst_off) if host_registration_offsets is None
                       else host_registration_offsets, count, int64_arrays)
    keys = _key_column(destination_keys, count, int64_arrays)
    total = sum(n.tolist() if isinstance(n, np.ndarray) else n)

    columns = (n, src_off, dst_off, host_off, src_cap, dst_cap)
    arrays = None if pin_chunk_size is not None and pin_chunk_size >= _LIMIT else _as_int64(columns)
    if arrays is None:
        n, src_off, dst_off, host_off, src_cap, dst_cap = columns = tuple(
            tuple(c.tolist()) if isinstance(c, np.ndarray) else c for c in columns)
    _check_rules(columns, arrays)
    if arrays is None:
        _reject_overlaps_scalar(dst_off, n, keys)
        pieces = [(i, start, length) for i, ho, size in zip(range(count), host_off, n)
                  for start, length in _pieces(ho, size, pin_chunk_size)]
        index = np.array([p[0] for p in pieces], dtype=np.int64)
        start = [p[1] for p in pieces]
        so_, do_, ho_ = ([c[i] + s for i, s in zip(index.tolist(), start)] for c in (src_off, dst_off, host_off))
        length = [p[2] for p in pieces]
        as_obj = (lambda v: np.array(v, dtype=object))
        return PlanColumns(direction, index, as_obj(so_), as_obj(do_), as_obj(length), as_obj(ho_), total, count)
    n_a, so_a, do_a, ho_a = arrays[:4]
    _reject_overlaps(do_a, n_a, keys)
    index, start, length = _split(n_a, ho_a, pin_chunk_size)
    return PlanColumns(direction, index, so_a[index] + start, do_a[index] + start, length, ho_a[index] + start,
                       total, count)


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
    c = plan_columns(direction=direction, sizes=sizes, source_capacities=source_capacities,
                     destination_capacities=destination_capacities, source_offsets=source_offsets,
                     destination_offsets=destination_offsets, host_registration_offsets=host_registration_offsets,
                     pin_chunk_size=pin_chunk_size, destination_keys=destination_keys)
    entries = tuple(
        BatchCopyEntry(input_index=i, source_offset=so, destination_offset=do, size=n, host_registration_offset=ho)
        for i, so, do, n, ho in zip(c.input_index.tolist(), c.source_offset.tolist(), c.destination_offset.tolist(),
                                    c.size.tolist(), c.host_registration_offset.tolist()))
    return BatchCopyPlan(direction=direction, entries=entries, total_bytes=c.total_bytes,
                         input_entry_count=c.input_entry_count)


def chunk_batch_copy_plan(plan: BatchCopyPlan, max_batch_entries: int) -> tuple[tuple[BatchCopyEntry, ...], ...]:
    """The plan's entries in submission order, ``max_batch_entries`` at a time (the last group may be
    shorter); groups are submitted one after another on the same stream."""
    if not (_is_int(max_batch_entries) and max_batch_entries > 0):
        raise ValueError("max_batch_entries must be a positive integer")
    remaining = iter(plan.entries)
    return tuple(iter(lambda: tuple(islice(remaining, max_batch_entries)), ()))
