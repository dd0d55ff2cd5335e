"""SGLang HiCache layer-first / page-first transfers on MI355X (ROCm HIP backend).

Public names, signatures, defaults, return values and exception messages
follow the reference module ``musa_aiter/ops/hicache_transfer.py`` (0.5.0):

- ``layer_first`` tensors are ``[layers, pages, item_elements]`` and
  ``page_first`` tensors ``[pages, layers, item_elements]`` (reference :1-10,
  :96-116); one (page, layer) item is ``item_elements * element_size`` bytes,
  a multiple of 8;
- two index tables pair source and destination pages; a pair with -1 on
  either side is skipped (:168-179, :317-319); a destination page named by
  several pairs keeps the last pair, as the reference's sequential loop does;
- the ``*_direct*`` functions copy token ranges for SGLang's direct HiCache
  path (:502-679), including its run coalescing.

Every transfer is one launch of the row kernel in ``libmusa_aiter_kv_hip.so``:
each (pair, layer, K/V plane) item is one row, all layers and both planes in
the same grid.  Validation runs before anything is launched and raises like
the reference; tensors must be on a ROCm device and there is no CPU path.
Source rows that the same call also writes read either their old or their new
contents (the reference's native kernel has the same unordered semantics).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import numpy as np
import torch

from musa_aiter.dispatch import DispatchRecord, emit, tensor_device_dtype, trace_enabled
from musa_aiter.ops import _hip
from musa_aiter.ops.kv_transfer import BuildResult, _require_rocm, build_native_kv_transfer

BACKEND = _hip.BACKEND
_ABI_VERSION = 1

LayoutName = Literal["layer_first", "page_first"]


# ---------------------------------------------------------------------------
# Build / availability probes (reference :37-82)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class NativeLibrary:
    """The loaded HIP library; ``handle`` is the ctypes handle, as in the reference's loader."""

    path: str
    handle: object


def build_native_hicache_transfer() -> BuildResult:
    return build_native_kv_transfer()


def load_native_hicache_transfer() -> NativeLibrary:
    result = build_native_hicache_transfer()
    if not result.ok or result.library_path is None:
        raise RuntimeError(result.message)
    return NativeLibrary(result.library_path, _hip.library())


def native_hicache_transfer_abi_version() -> int | None:
    try:
        return int(_hip.fn("musa_aiter_hicache_transfer_abi_version")())
    except (_hip.HipBackendError, OSError, AttributeError):
        return None


def is_native_hicache_transfer_available() -> bool:
    return native_hicache_transfer_abi_version() == _ABI_VERSION


# ---------------------------------------------------------------------------
# Layout-transfer validation (reference :96-193)
# ---------------------------------------------------------------------------


def _layout_geometry(tensor: torch.Tensor, layout: LayoutName) -> tuple[int, int, int, int, int]:
    """(layers, pages, item_elements, page_stride_bytes, layer_stride_bytes) of a contiguous tensor."""
    if not isinstance(tensor, torch.Tensor) or tensor.dim() != 3:
        raise ValueError("HiCache tensors must be rank-3 [layers/pages/item] or [pages/layers/item]")
    if not tensor.is_contiguous():
        raise ValueError("HiCache tensors must be contiguous")
    if layout == "layer_first":
        layers, pages, item_elements = map(int, tensor.shape)
        page_stride = item_elements * tensor.element_size()
        layer_stride = pages * page_stride
    elif layout == "page_first":
        pages, layers, item_elements = map(int, tensor.shape)
        layer_stride = item_elements * tensor.element_size()
        page_stride = layers * layer_stride
    else:
        raise ValueError(f"unsupported HiCache layout={layout!r}")
    if layers <= 0 or pages <= 0 or item_elements <= 0:
        raise ValueError("HiCache layer/page/item dimensions must be positive")
    return layers, pages, item_elements, page_stride, layer_stride


def _validate_inputs(
    src_k: torch.Tensor,
    dst_k: torch.Tensor,
    src_v: torch.Tensor | None,
    dst_v: torch.Tensor | None,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    src_layout: LayoutName,
    dst_layout: LayoutName,
    start_layer: int,
    num_layers: int,
    *,
    mla: bool,
) -> tuple[tuple[int, int, int, int, int], tuple[int, int, int, int, int], int]:
    if not isinstance(src_indices, torch.Tensor) or not isinstance(dst_indices, torch.Tensor):
        raise TypeError("HiCache index tables must be torch.Tensor values")
    if src_indices.dim() != 1 or dst_indices.dim() != 1:
        raise ValueError("HiCache index tables must be 1-D")
    if src_indices.numel() != dst_indices.numel():
        raise ValueError("source and destination index tables must have the same length")
    if src_indices.dtype not in (torch.int32, torch.int64) or dst_indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("HiCache index tables must use int32 or int64")
    if src_k.dtype != dst_k.dtype:
        raise ValueError("source and destination K tensors must have the same dtype")
    if src_k.device != dst_k.device:
        raise ValueError("source and destination K tensors must be on the same device")
    if src_v is not None or dst_v is not None:
        if mla:
            raise ValueError("MLA HiCache transfer does not accept a value plane")
        if src_v is None or dst_v is None:
            raise ValueError("source and destination value tensors must be provided together")
        if src_v.dtype != src_k.dtype or dst_v.dtype != dst_k.dtype:
            raise ValueError("K and V tensors must use the same dtype")
        if src_v.device != src_k.device or dst_v.device != dst_k.device:
            raise ValueError("K and V tensors must be on the same device")
    elif not mla:
        raise ValueError("non-MLA HiCache transfer requires K and V tensors")

    src_geometry = _layout_geometry(src_k, src_layout)
    dst_geometry = _layout_geometry(dst_k, dst_layout)
    if src_geometry[2] * src_k.element_size() != dst_geometry[2] * dst_k.element_size():
        raise ValueError("source and destination item byte sizes must match")
    if src_v is not None and _layout_geometry(src_v, src_layout) != src_geometry:
        raise ValueError("source K and V layouts must match")
    if dst_v is not None and _layout_geometry(dst_v, dst_layout) != dst_geometry:
        raise ValueError("destination K and V layouts must match")
    if start_layer < 0 or num_layers <= 0:
        raise ValueError("start_layer and num_layers must be non-negative/positive")
    if start_layer + num_layers > min(src_geometry[0], dst_geometry[0]):
        raise ValueError("requested layer range exceeds source or destination")
    item_size_bytes = src_geometry[2] * src_k.element_size()
    if item_size_bytes % 8 != 0:
        raise ValueError("HiCache item byte size must be divisible by 8")
    return src_geometry, dst_geometry, item_size_bytes


def _validate_page_indices(
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    src_pages: int,
    dst_pages: int,
    device: torch.device,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's per-pair checks (:182-193), evaluated on ``device`` with one host sync;
    returns both tables as contiguous int64 tensors on ``device``."""
    src = src_indices.to(device=device, dtype=torch.long).contiguous()
    dst = dst_indices.to(device=device, dtype=torch.long).contiguous()
    if src.numel() == 0:
        return src, dst
    # Common case in one host read: both tables' extremes inside [-1, pages).
    (s_lo, s_hi), (d_lo, d_hi) = torch.stack([torch.stack(torch.aminmax(src)), torch.stack(torch.aminmax(dst))]).tolist()
    if s_lo >= -1 and d_lo >= -1 and s_hi < src_pages and d_hi < dst_pages:
        return src, dst
    # Some pair is invalid: the first one in table order decides the message.
    negative = (src < -1) | (dst < -1)
    bad = negative | (src >= src_pages) | (dst >= dst_pages)
    first = int(bad.nonzero()[0, 0])
    if bool(negative[first]):
        raise ValueError("HiCache page indices must be -1 or non-negative")
    raise ValueError("HiCache page index is out of range")


def _transfer(
    src_k: torch.Tensor,
    dst_k: torch.Tensor,
    src_v: torch.Tensor | None,
    dst_v: torch.Tensor | None,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    *,
    src_layout: LayoutName,
    dst_layout: LayoutName,
    start_layer: int,
    num_layers: int,
    mla: bool,
) -> bool:
    """Reference :241-337: validate, then one row-kernel launch over every (pair, layer, plane)."""
    src_geometry, dst_geometry, item_size_bytes = _validate_inputs(
        src_k, dst_k, src_v, dst_v, src_indices, dst_indices, src_layout, dst_layout, start_layer, num_layers,
        mla=mla,
    )
    src_idx, dst_idx = _validate_page_indices(src_indices, dst_indices, src_geometry[1], dst_geometry[1],
                                              dst_k.device)
    planes = [(src_k, dst_k)] if src_v is None else [(src_k, dst_k), (src_v, dst_v)]
    _require_rocm("hicache_transfer", *(t for pair in planes for t in pair))
    layers = range(start_layer, start_layer + num_layers)
    bases = [(s.data_ptr(), d.data_ptr()) for s, d in planes]
    _hip.copy_rows_paged(
        op="hicache_transfer",
        device=dst_k.device,
        src_planes=[s + layer * src_geometry[4] for s, _ in bases for layer in layers],
        dst_planes=[d + layer * dst_geometry[4] for _, d in bases for layer in layers],
        src_idx=src_idx,
        dst_idx=dst_idx,
        src_rows=src_geometry[1],
        dst_rows=dst_geometry[1],
        row_bytes=item_size_bytes,
        src_stride=src_geometry[3],
        dst_stride=dst_geometry[3],
    )
    device, dtype = tensor_device_dtype(src_k)
    emit(DispatchRecord("hicache_transfer", BACKEND, device, dtype,
                        f"gfx950 byte-stride row copy ({src_layout}->{dst_layout}, {num_layers} layers)"))
    return True


# ---------------------------------------------------------------------------
# Layout transfers (reference :340-499)
# ---------------------------------------------------------------------------


def hicache_transfer_kv_per_layer(
    src_k: torch.Tensor,
    dst_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_v: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    *,
    layer_id: int = 0,
) -> bool:
    return _transfer(src_k, dst_k, src_v, dst_v, src_indices, dst_indices, src_layout="layer_first",
                     dst_layout="layer_first", start_layer=layer_id, num_layers=1, mla=False)


def hicache_transfer_kv_per_layer_pf_lf(
    src_k: torch.Tensor,
    dst_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_v: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    *,
    layer_id: int = 0,
) -> bool:
    return _transfer(src_k, dst_k, src_v, dst_v, src_indices, dst_indices, src_layout="page_first",
                     dst_layout="layer_first", start_layer=layer_id, num_layers=1, mla=False)


def hicache_transfer_kv_all_layer(
    src_k: torch.Tensor,
    dst_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_v: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
) -> bool:
    layers = int(src_k.shape[0])
    return _transfer(src_k, dst_k, src_v, dst_v, src_indices, dst_indices, src_layout="layer_first",
                     dst_layout="layer_first", start_layer=0, num_layers=layers, mla=False)


def hicache_transfer_kv_all_layer_lf_pf(
    src_k: torch.Tensor,
    dst_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_v: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
) -> bool:
    layers = int(src_k.shape[0])
    return _transfer(src_k, dst_k, src_v, dst_v, src_indices, dst_indices, src_layout="layer_first",
                     dst_layout="page_first", start_layer=0, num_layers=layers, mla=False)


def hicache_transfer_kv_per_layer_mla(
    src: torch.Tensor,
    dst: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    *,
    layer_id: int = 0,
    value: torch.Tensor | None = None,
) -> bool:
    if value is not None:
        raise ValueError("MLA HiCache transfer does not accept a value plane")
    return _transfer(src, dst, None, None, src_indices, dst_indices, src_layout="layer_first",
                     dst_layout="layer_first", start_layer=layer_id, num_layers=1, mla=True)


def hicache_transfer_kv_per_layer_mla_pf_lf(
    src: torch.Tensor,
    dst: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    *,
    layer_id: int = 0,
) -> bool:
    return _transfer(src, dst, None, None, src_indices, dst_indices, src_layout="page_first",
                     dst_layout="layer_first", start_layer=layer_id, num_layers=1, mla=True)


def hicache_transfer_kv_all_layer_mla(
    src: torch.Tensor,
    dst: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
) -> bool:
    layers = int(src.shape[0])
    return _transfer(src, dst, None, None, src_indices, dst_indices, src_layout="layer_first",
                     dst_layout="layer_first", start_layer=0, num_layers=layers, mla=True)


def hicache_transfer_kv_all_layer_mla_lf_pf(
    src: torch.Tensor,
    dst: torch.Tensor,
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
) -> bool:
    """Transfer all MLA layers from layer-first to page-first storage."""
    layers = int(src.shape[0])
    return _transfer(src, dst, None, None, src_indices, dst_indices, src_layout="layer_first",
                     dst_layout="page_first", start_layer=0, num_layers=layers, mla=True)


# ---------------------------------------------------------------------------
# Direct token-range transfers (reference :502-679)
# ---------------------------------------------------------------------------


def _validate_direct_indices(src_indices: torch.Tensor, dst_indices: torch.Tensor,
                             page_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Reference :502-523; returns both tables as host int64 arrays (the reference reads them on the host too)."""
    if not isinstance(src_indices, torch.Tensor) or not isinstance(dst_indices, torch.Tensor):
        raise TypeError("HiCache direct index tables must be torch.Tensor values")
    if src_indices.dim() != 1 or dst_indices.dim() != 1:
        raise ValueError("HiCache direct index tables must be 1-D")
    if src_indices.numel() != dst_indices.numel():
        raise ValueError("source and destination index tables must have the same length")
    if src_indices.dtype not in (torch.int32, torch.int64) or dst_indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("HiCache direct index tables must use int32 or int64")
    if page_size <= 0:
        raise ValueError("HiCache direct page_size must be positive")
    if src_indices.numel() % page_size != 0:
        raise ValueError("HiCache direct index count must be divisible by page_size")
    src_values = src_indices.detach().to(device="cpu", dtype=torch.long).numpy()
    dst_values = dst_indices.detach().to(device="cpu", dtype=torch.long).numpy()
    if (src_values < 0).any() or (dst_values < 0).any():
        raise ValueError("HiCache direct indices must be non-negative")
    return src_values, dst_values


def _validate_direct_tensor_lists(src_layers: list[torch.Tensor], dst_layers: list[torch.Tensor]) -> None:
    """Reference :526-544."""
    if not isinstance(src_layers, (list, tuple)) or not isinstance(dst_layers, (list, tuple)):
        raise TypeError("HiCache direct layers must be tensor lists")
    if not src_layers or len(src_layers) != len(dst_layers):
        raise ValueError("HiCache direct source and destination lists must have equal non-zero length")
    for src, dst in zip(src_layers, dst_layers):
        if not isinstance(src, torch.Tensor) or not isinstance(dst, torch.Tensor):
            raise TypeError("HiCache direct layer entries must be tensors")
        if src.dim() < 1 or dst.dim() < 1:
            raise ValueError("HiCache direct tensors must have at least one dimension")
        if tuple(src.shape[1:]) != tuple(dst.shape[1:]):
            raise ValueError("HiCache direct source and destination tails must match")
        if src.dtype != dst.dtype:
            raise ValueError("HiCache direct source and destination dtypes must match")
        if not src.is_contiguous() or not dst.is_contiguous():
            raise ValueError("HiCache direct tensors must be contiguous")


def _require_one_rocm_device(op: str, tensors) -> torch.device:
    """The one ROCm device every tensor of a direct transfer lives on (all layers and planes go in one
    launch there, so tensors on other devices are rejected instead of copied across devices)."""
    tensors = list(tensors)
    _require_rocm(op, *tensors)
    devices = {t.device for t in tensors}
    if len(devices) != 1:
        raise ValueError(f"{op}: all HiCache direct tensors must be on one device (got {sorted(map(str, devices))})")
    return tensors[0].device


def _emit_direct(operation: str, tensor: torch.Tensor, reason: str) -> None:
    if not trace_enabled():
        return
    device, dtype = tensor_device_dtype(tensor)
    emit(DispatchRecord(operation, BACKEND, device, dtype, reason))


@dataclass(frozen=True)
class _Side:
    """Row addressing of one side of a direct transfer: token t of a plane sits at byte
    (t // page_rows) * page_stride + (t % page_rows) * stride (page_rows 0: t * stride)."""

    stride: int
    page_rows: int = 0
    page_stride: int = 0


def _row_bytes(t: torch.Tensor, lead: int) -> int:
    return int(np.prod(t.shape[lead:], dtype=np.int64)) * t.element_size()


def _page_groups_regular(src_values: np.ndarray, dst_values: np.ndarray, page_size: int,
                         src_base: np.ndarray, dst_base: np.ndarray) -> bool:
    """True when every page group's entries already equal base + [0, page_size) on both sides."""
    j = np.tile(np.arange(page_size, dtype=np.int64), src_base.shape[0])
    return bool(np.array_equal(src_values, np.repeat(src_base, page_size) + j)
                and np.array_equal(dst_values, np.repeat(dst_base, page_size) + j))


def _token_tables(src_indices: torch.Tensor, dst_indices: torch.Tensor, src_tokens: np.ndarray | None,
                  dst_tokens: np.ndarray | None, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Device int64 tables of the tokens each row copies: the caller's own tables when they
    already name them (``*_tokens`` None), else the host-computed ones."""
    if src_tokens is None:
        return (src_indices.to(device=device, dtype=torch.long).contiguous(),
                dst_indices.to(device=device, dtype=torch.long).contiguous())
    return (torch.from_numpy(np.ascontiguousarray(src_tokens)).to(device),
            torch.from_numpy(np.ascontiguousarray(dst_tokens)).to(device))


def _launch_direct(op: str, device: torch.device, pairs: list[tuple[int, int, int, _Side, _Side, int, int]],
                   src_idx: torch.Tensor, dst_idx: torch.Tensor) -> None:
    """One launch per distinct (row bytes, addressing) group of (src base, dst base, row bytes,
    src side, dst side, src rows, dst rows) planes."""
    groups: dict[tuple, list[tuple[int, int, int, int]]] = {}
    for src_base, dst_base, row_bytes, src_side, dst_side, src_rows, dst_rows in pairs:
        groups.setdefault((row_bytes, src_side, dst_side), []).append((src_base, dst_base, src_rows, dst_rows))
    for (row_bytes, src_side, dst_side), members in groups.items():
        _hip.copy_rows_paged(
            op=op,
            device=device,
            src_planes=[m[0] for m in members],
            dst_planes=[m[1] for m in members],
            src_idx=src_idx,
            dst_idx=dst_idx,
            src_rows=min(m[2] for m in members),
            dst_rows=min(m[3] for m in members),
            row_bytes=row_bytes,
            src_stride=src_side.stride,
            dst_stride=dst_side.stride,
            src_page_rows=src_side.page_rows,
            src_page_stride=src_side.page_stride,
            dst_page_rows=dst_side.page_rows,
            dst_page_stride=dst_side.page_stride,
        )


def _direct_run_tokens(src_values: np.ndarray, dst_values: np.ndarray,
                       page_size: int) -> tuple[np.ndarray | None, np.ndarray | None, int, int]:
    """Tokens of the reference's run coalescing (:560-583) and the largest source / destination
    token they touch.

    A run starts with one page of entries and then grows while both tables
    stay consecutive, copying rows from its first entries on.  When every
    break between consecutive entries falls on a page boundary, runs start on
    page boundaries and the copied tokens are the tables themselves (None is
    returned for them); otherwise the runs are walked on the host.
    """
    n = src_values.shape[0]
    if n == 0:
        return None, None, -1, -1
    brk = np.flatnonzero((src_values[1:] != src_values[:-1] + 1) | (dst_values[1:] != dst_values[:-1] + 1)) + 1
    if not (brk % page_size).any():
        return None, None, int(src_values.max()), int(dst_values.max())
    starts, counts = [], []
    start = 0
    while start < n:
        k = int(np.searchsorted(brk, start + page_size))
        end = int(brk[k]) if k < brk.shape[0] else max(n, start + page_size)
        starts.append(start)
        counts.append(end - start)
        start = end
    starts_a = np.asarray(starts, dtype=np.int64)
    counts_a = np.asarray(counts, dtype=np.int64)
    offs = np.arange(int(counts_a.sum()), dtype=np.int64) - np.repeat(np.cumsum(counts_a) - counts_a, counts_a)
    src_tokens = np.repeat(src_values[starts_a], counts_a) + offs
    dst_tokens = np.repeat(dst_values[starts_a], counts_a) + offs
    return src_tokens, dst_tokens, int(src_tokens.max()), int(dst_tokens.max())


def hicache_transfer_kv_direct(
    src_layers: list[torch.Tensor],
    dst_layers: list[torch.Tensor],
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    page_size: int,
) -> bool:
    """Copy contiguous token ranges for SGLang's direct HiCache path (reference :586-599).

    Every layer copies the same runs; all layers go in one launch per distinct row size.
    """
    op = "hicache_transfer_direct"
    _validate_direct_tensor_lists(src_layers, dst_layers)
    page_size = int(page_size)
    src_values, dst_values = _validate_direct_indices(src_indices, dst_indices, page_size)
    src_tokens, dst_tokens, src_max, dst_max = _direct_run_tokens(src_values, dst_values, page_size)
    for src, dst in zip(src_layers, dst_layers):
        if src_max >= int(src.shape[0]) or dst_max >= int(dst.shape[0]):
            raise ValueError("HiCache direct token range exceeds source or destination")
    if src_values.shape[0] > 0:
        device = _require_one_rocm_device(op, [*dst_layers, *src_layers])
        src_idx, dst_idx = _token_tables(src_indices, dst_indices, src_tokens, dst_tokens, device)
        pairs = []
        for src, dst in zip(src_layers, dst_layers):
            row = _row_bytes(src, 1)
            pairs.append((src.data_ptr(), dst.data_ptr(), row, _Side(row), _Side(row), int(src.shape[0]),
                          int(dst.shape[0])))
        _launch_direct(op, device, pairs, src_idx, dst_idx)
    _emit_direct(op, dst_layers[0], "gfx950 token-run row copy")
    return True


def hicache_transfer_kv_per_layer_direct_pf_lf(
    src_ptrs: list[torch.Tensor],
    dst_ptrs: list[torch.Tensor],
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    layer_id: int,
    page_size: int,
) -> bool:
    """Copy page-first source pages into one layer-first destination layer (reference :602-634).

    Page group g copies source page src_indices[g * page_size] // page_size of
    layer ``layer_id`` to destination rows dst_indices[g * page_size] + [0,
    page_size); a one-row source page is broadcast over the group's rows.
    """
    op = "hicache_transfer_per_layer_direct_pf_lf"
    if layer_id < 0:
        raise ValueError("HiCache direct layer_id must be non-negative")
    if len(src_ptrs) not in (1, 2) or len(dst_ptrs) != len(src_ptrs):
        raise ValueError("HiCache per-layer direct expects one MLA plane or K/V plane pairs")
    page_size = int(page_size)
    src_values, dst_values = _validate_direct_indices(src_indices, dst_indices, page_size)
    starts = np.arange(0, src_values.shape[0], page_size)
    src_page = src_values[starts] // page_size
    dst_start = dst_values[starts]
    pairs = []
    for src, dst in zip(src_ptrs, dst_ptrs):
        if not isinstance(src, torch.Tensor) or not isinstance(dst, torch.Tensor):
            raise TypeError("HiCache direct layer entries must be tensors")
        if src.dim() != 4 or dst.dim() != 2:
            raise ValueError(
                "HiCache per-layer direct expects source [pages,layers,page,item] and destination [tokens,item]")
        if layer_id >= int(src.shape[1]):
            raise ValueError("HiCache direct layer_id exceeds source layers")
        if not src.is_contiguous() or not dst.is_contiguous():
            raise ValueError("HiCache direct tensors must be contiguous")
        if src.dtype != dst.dtype or tuple(src.shape[3:]) != tuple(dst.shape[1:]):
            raise ValueError("HiCache direct source and destination item shapes/dtypes must match")
        if starts.shape[0] > 0:
            if (src_page >= int(src.shape[0])).any() or (dst_start + page_size > int(dst.shape[0])).any():
                raise ValueError("HiCache direct page range exceeds source or destination")
        pages, layers, page_rows, _ = map(int, src.shape)
        if starts.shape[0] > 0 and page_rows not in (page_size, 1):
            raise RuntimeError(
                f"HiCache per-layer direct: a source page holds {page_rows} rows, which does not broadcast to "
                f"page_size={page_size}")
        row = _row_bytes(src, 3)
        # Token t of the source plane: page t // page_size, row t % page_size of layer `layer_id`
        # (stride 0 broadcasts a one-row page).
        src_side = _Side(row if page_rows == page_size else 0, page_size, layers * page_rows * row)
        pairs.append((src.data_ptr() + layer_id * page_rows * row, dst.data_ptr(), row, src_side, _Side(row),
                      pages * page_size, int(dst.shape[0])))
    if starts.shape[0] > 0:
        device = _require_one_rocm_device(op, [*dst_ptrs, *src_ptrs])
        if _page_groups_regular(src_values, dst_values, page_size, src_page * page_size, dst_start):
            src_tokens = dst_tokens = None
        else:
            j = np.tile(np.arange(page_size, dtype=np.int64), starts.shape[0])
            src_tokens = np.repeat(src_page * page_size, page_size) + j
            dst_tokens = np.repeat(dst_start, page_size) + j
        src_idx, dst_idx = _token_tables(src_indices, dst_indices, src_tokens, dst_tokens, device)
        _launch_direct(op, device, pairs, src_idx, dst_idx)
    _emit_direct(op, dst_ptrs[0], "gfx950 page-first page -> layer-first rows")
    return True


def hicache_transfer_kv_all_layer_direct_lf_pf(
    src_ptrs: list[torch.Tensor],
    dst_ptrs: list[torch.Tensor],
    src_indices: torch.Tensor,
    dst_indices: torch.Tensor,
    page_size: int,
) -> bool:
    """Copy layer-first source pages into an all-layer page-first destination (reference :637-679).

    ``src_ptrs`` lists the K layers ([tokens, item]) then, with two
    destination planes, the V layers.  Page group g copies source rows
    src_indices[g * page_size] + [0, page_size) of every layer into
    destination page dst_indices[g * page_size] // page_size.  All layers and
    planes go in one launch per distinct item size.
    """
    op = "hicache_transfer_all_layer_direct_lf_pf"
    if len(dst_ptrs) not in (1, 2):
        raise ValueError("HiCache all-layer direct expects one MLA plane or K/V plane pairs")
    is_mla = len(dst_ptrs) == 1
    if len(src_ptrs) == 0 or (not is_mla and len(src_ptrs) % 2 != 0):
        raise ValueError("HiCache all-layer direct source planes do not match destination planes")
    num_layers = len(src_ptrs) if is_mla else len(src_ptrs) // 2
    page_size = int(page_size)
    src_values, dst_values = _validate_direct_indices(src_indices, dst_indices, page_size)
    if not all(isinstance(tensor, torch.Tensor) for tensor in list(src_ptrs) + list(dst_ptrs)):
        raise TypeError("HiCache direct layer entries must be tensors")
    for tensor in src_ptrs:
        if tensor.dim() != 2 or not tensor.is_contiguous():
            raise ValueError("HiCache all-layer direct sources must be contiguous [tokens,item] tensors")
    for tensor in dst_ptrs:
        if tensor.dim() != 4 or not tensor.is_contiguous():
            raise ValueError(
                "HiCache all-layer direct destinations must be contiguous [pages,layers,page,item] tensors")
    for index in range(num_layers):
        if src_ptrs[index].dtype != dst_ptrs[0].dtype or tuple(src_ptrs[index].shape[1:]) != tuple(dst_ptrs[0].shape[3:]):
            raise ValueError("HiCache direct source and destination item shapes/dtypes must match")
    if not is_mla:
        # The reference compares the first V layer; later V layers would be converted or fail
        # inside torch's copy, so all of them are held to the same rule here.
        for index in range(num_layers, 2 * num_layers):
            if (src_ptrs[index].dtype != dst_ptrs[1].dtype
                    or tuple(src_ptrs[index].shape[1:]) != tuple(dst_ptrs[1].shape[3:])):
                raise ValueError("HiCache direct K/V item shapes/dtypes must match")

    starts = np.arange(0, src_values.shape[0], page_size)
    src_start = src_values[starts]
    dst_page = dst_values[starts] // page_size
    planes = [(0, 0)] if is_mla else [(0, 0), (1, num_layers)]
    if starts.shape[0] > 0:
        # Errors in the reference's order: group by group, the destination page, then each
        # layer's source range.
        src_short = np.zeros(starts.shape[0], dtype=bool)
        for tensor in src_ptrs:
            src_short |= src_start + page_size > int(tensor.shape[0])
        bad_page = dst_page >= int(dst_ptrs[0].shape[0])
        if not is_mla:
            bad_page_v = dst_page >= int(dst_ptrs[1].shape[0])
        else:
            bad_page_v = np.zeros_like(bad_page)
        bad = bad_page | src_short | bad_page_v
        if bad.any():
            g = int(np.flatnonzero(bad)[0])
            if bad_page[g]:
                raise ValueError("HiCache direct destination page exceeds destination")
            if src_short[g]:
                raise ValueError("HiCache direct source range exceeds source")
            raise IndexError("HiCache direct destination page exceeds the value destination")
        for dst in dst_ptrs:
            if num_layers > int(dst.shape[1]):
                raise IndexError("HiCache all-layer direct destination holds fewer layers than the source planes")
            page_rows = int(dst.shape[2])
            if page_rows != page_size and page_size != 1:
                raise RuntimeError(
                    f"HiCache all-layer direct: a destination page holds {page_rows} rows, which page_size="
                    f"{page_size} source rows do not broadcast to")

    if starts.shape[0] > 0:
        device = _require_one_rocm_device(op, [*dst_ptrs, *src_ptrs])
        page_rows = int(dst_ptrs[0].shape[2])
        if not is_mla and int(dst_ptrs[1].shape[2]) != page_rows:
            raise ValueError("HiCache all-layer direct K and V destinations must use one page size")
        if page_rows == page_size and _page_groups_regular(src_values, dst_values, page_size, src_start,
                                                           dst_page * page_size):
            src_tokens = dst_tokens = None
        else:
            # A page of page_rows destination rows per group; a one-token group broadcasts.
            j = np.tile(np.arange(page_rows, dtype=np.int64), starts.shape[0])
            src_tokens = np.repeat(src_start, page_rows) + (j if page_rows == page_size else 0)
            dst_tokens = np.repeat(dst_page * page_rows, page_rows) + j
        src_idx, dst_idx = _token_tables(src_indices, dst_indices, src_tokens, dst_tokens, device)
        pairs = []
        for plane, first in planes:
            dst = dst_ptrs[plane]
            _, dst_layers, _, _ = map(int, dst.shape)
            row = _row_bytes(dst, 3)
            dst_side = _Side(row, page_rows, dst_layers * page_rows * row)
            for layer in range(num_layers):
                src = src_ptrs[first + layer]
                pairs.append((src.data_ptr(), dst.data_ptr() + layer * page_rows * row, row, _Side(row), dst_side,
                              int(src.shape[0]), int(dst.shape[0]) * page_rows))
        _launch_direct(op, device, pairs, src_idx, dst_idx)
    _emit_direct(op, dst_ptrs[0], "gfx950 layer-first rows -> page-first pages")
    return True
