"""numpy restatement of the reference's SGLang HiCache transfers -- TEST INFRASTRUCTURE ONLY.

Every function follows one reference function of musa_aiter 0.5.0
(``musa_aiter/ops/hicache_transfer.py`` and ``csrc/kvcache/hicache_transfer.mu``,
cited as file:line).  Arrays are compared bit-for-bit, so callers pass raw bit
views (uint16 for bf16/fp16, uint32 for fp32).  Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg use this module.

Layouts (hicache_transfer.py:1-10, :96-116): ``layer_first`` tensors are
``[layers, pages, item]``, ``page_first`` tensors ``[pages, layers, item]``.
"""

from __future__ import annotations

import numpy as np


def _row(t: np.ndarray, layout: str, layer: int, page: int) -> np.ndarray:
    return t[layer, page] if layout == "layer_first" else t[page, layer]


def transfer(src_k: np.ndarray, dst_k: np.ndarray, src_v: np.ndarray | None, dst_v: np.ndarray | None,
             src_idx: np.ndarray, dst_idx: np.ndarray, *, src_layout: str, dst_layout: str, start_layer: int,
             num_layers: int) -> None:
    """The reference's torch path of _transfer (hicache_transfer.py:314-337), in place.

    Pairs run in table order and layers in ascending order; a pair with a
    negative index on either side is skipped, so a destination page named twice
    keeps the later pair.
    """
    for sp, dp in zip(np.asarray(src_idx, np.int64).tolist(), np.asarray(dst_idx, np.int64).tolist()):
        if sp < 0 or dp < 0:
            continue
        for layer in range(start_layer, start_layer + num_layers):
            _row(dst_k, dst_layout, layer, dp)[...] = _row(src_k, src_layout, layer, sp)
            if src_v is not None and dst_v is not None:
                _row(dst_v, dst_layout, layer, dp)[...] = _row(src_v, src_layout, layer, sp)


def layout_strides(shape: tuple[int, int, int], itemsize: int, layout: str) -> tuple[int, int]:
    """(page_stride, layer_stride) in bytes of a contiguous tensor (hicache_transfer.py:102-111)."""
    _, b, item = shape
    row = item * itemsize
    if layout == "layer_first":
        return row, b * row          # [layers, pages, item]
    return b * row, row              # [pages, layers, item]


def transfer_bytes(src_k: np.ndarray, dst_k: np.ndarray, src_v: np.ndarray | None, dst_v: np.ndarray | None,
                   src_idx: np.ndarray, dst_idx: np.ndarray, num_items: int, start_layer: int, num_layers: int,
                   item_size_bytes: int, src_page_stride: int, src_layer_stride: int, dst_page_stride: int,
                   dst_layer_stride: int) -> None:
    """The native kernel's byte-offset contract (hicache_transfer.mu:4-50) on flat uint8 buffers, in place.

    Every 64-bit word w < item_size_bytes // 8 of item i and layer l moves from
    src_page * src_page_stride + (start_layer + l) * src_layer_stride + 8 w to
    the matching destination offset; items with a negative page are skipped.
    """
    words = item_size_bytes // 8
    nbytes = words * 8
    for i in range(num_items):
        sp = int(src_idx[i])
        dp = int(dst_idx[i])
        if sp < 0 or dp < 0:
            continue
        for layer in range(num_layers):
            so = sp * src_page_stride + (start_layer + layer) * src_layer_stride
            do = dp * dst_page_stride + (start_layer + layer) * dst_layer_stride
            dst_k[do:do + nbytes] = src_k[so:so + nbytes]
            if src_v is not None and dst_v is not None:
                dst_v[do:do + nbytes] = src_v[so:so + nbytes]


def direct_runs(src_values: list[int], dst_values: list[int], page_size: int) -> list[tuple[int, int, int]]:
    """(src_start, dst_start, count) runs of _copy_direct_runs (hicache_transfer.py:560-583).

    A run starts with one page of tokens and then grows while both tables stay
    consecutive; it copies ``count`` rows from its first entries, whatever the
    entries inside its first page say.
    """
    runs = []
    start = 0
    n = len(src_values)
    while start < n:
        end = start + page_size
        while end < n:
            if src_values[end] != src_values[end - 1] + 1 or dst_values[end] != dst_values[end - 1] + 1:
                break
            end += 1
        runs.append((src_values[start], dst_values[start], end - start))
        start = end
    return runs


def direct(src_layers: list[np.ndarray], dst_layers: list[np.ndarray], src_idx: np.ndarray, dst_idx: np.ndarray,
           page_size: int) -> None:
    """hicache_transfer_kv_direct (hicache_transfer.py:586-599): each layer copies every run, in order."""
    runs = direct_runs(np.asarray(src_idx, np.int64).tolist(), np.asarray(dst_idx, np.int64).tolist(), page_size)
    for src, dst in zip(src_layers, dst_layers):
        for s0, d0, count in runs:
            if s0 + count > src.shape[0] or d0 + count > dst.shape[0]:
                raise ValueError("HiCache direct token range exceeds source or destination")
            dst[d0:d0 + count] = src[s0:s0 + count]


def per_layer_direct_pf_lf(src_planes: list[np.ndarray], dst_planes: list[np.ndarray], src_idx: np.ndarray,
                           dst_idx: np.ndarray, layer_id: int, page_size: int) -> None:
    """hicache_transfer_kv_per_layer_direct_pf_lf (hicache_transfer.py:602-634).

    Each page group g (entries g*page_size ...) copies the whole source page
    src_idx[g*page_size] // page_size of layer ``layer_id`` ([pages, layers,
    page, item]) to destination rows dst_idx[g*page_size] + [0, page_size) of
    a [tokens, item] plane; a one-row source page is broadcast (torch copy_).
    """
    src_values = np.asarray(src_idx, np.int64).tolist()
    dst_values = np.asarray(dst_idx, np.int64).tolist()
    for src, dst in zip(src_planes, dst_planes):
        for start in range(0, len(src_values), page_size):
            page = src_values[start] // page_size
            tok = dst_values[start]
            if page >= src.shape[0] or tok + page_size > dst.shape[0]:
                raise ValueError("HiCache direct page range exceeds source or destination")
            dst[tok:tok + page_size] = src[page, layer_id]


def all_layer_direct_lf_pf(src_planes: list[np.ndarray], dst_planes: list[np.ndarray], src_idx: np.ndarray,
                           dst_idx: np.ndarray, page_size: int) -> None:
    """hicache_transfer_kv_all_layer_direct_lf_pf (hicache_transfer.py:637-679).

    ``src_planes`` lists the K layers ([tokens, item]) then, for K/V, the V
    layers; page group g copies source rows src_idx[g*page_size] + [0,
    page_size) of every layer into destination page dst_idx[g*page_size] //
    page_size of the [pages, layers, page, item] plane(s).
    """
    mla = len(dst_planes) == 1
    num_layers = len(src_planes) if mla else len(src_planes) // 2
    src_values = np.asarray(src_idx, np.int64).tolist()
    dst_values = np.asarray(dst_idx, np.int64).tolist()
    for start in range(0, len(src_values), page_size):
        tok = src_values[start]
        page = dst_values[start] // page_size
        if page >= dst_planes[0].shape[0]:
            raise ValueError("HiCache direct destination page exceeds destination")
        for layer in range(num_layers):
            if tok + page_size > src_planes[layer].shape[0]:
                raise ValueError("HiCache direct source range exceeds source")
            dst_planes[0][page, layer] = src_planes[layer][tok:tok + page_size]
            if not mla:
                dst_planes[1][page, layer] = src_planes[layer + num_layers][tok:tok + page_size]
