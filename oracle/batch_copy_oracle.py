"""numpy restatement of the reference's LMCache host/device copy batches -- TEST INFRASTRUCTURE ONLY.

Follows musa_aiter 0.5.0 ``csrc/kvcache/lmcache_musa_batch_copy_ext.cpp`` (every entry copies
``size`` bytes from ``source + source_offset`` to ``destination + destination_offset``,
:80-170, submitted as one unordered batch, :173-222) and the splitting rule of
``musa_aiter/ops/lmcache_musa_batch_copy_plan.py:129-152``.  Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg use this module.
"""

from __future__ import annotations

import numpy as np


def apply_batch(destinations: list[np.ndarray], sources: list[np.ndarray], sizes: list[int],
                destination_offsets: list[int], source_offsets: list[int]) -> None:
    """Byte copies on flat uint8 views, in place.  The batch is unordered, so destination ranges
    of one call never overlap and the order of application does not matter."""
    for dst, src, size, d, s in zip(destinations, sources, sizes, destination_offsets, source_offsets):
        dst[d:d + size] = src[s:s + size]


def split_sizes(size: int, host_offset: int, pin_chunk_size: int | None) -> list[int]:
    """Sizes of the pieces an entry is cut into: a cut wherever the host-side byte offset reaches a
    multiple of ``pin_chunk_size`` (a host registration boundary), found byte by byte."""
    if pin_chunk_size is None:
        return [size]
    offsets = np.arange(host_offset, host_offset + size)
    cuts = np.flatnonzero(offsets % pin_chunk_size == 0)
    cuts = cuts[cuts > 0]
    edges = np.concatenate([[0], cuts, [size]])
    return [int(b - a) for a, b in zip(edges[:-1], edges[1:])]
