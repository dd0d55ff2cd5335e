"""Paged KV cache <-> linear buffer transfers on MI355X (ROCm HIP backend).

Public names, signatures, defaults, return conventions and exception types
follow the reference module ``musa_aiter/ops/kv_transfer.py`` (version 0.5.0),
so callers written against it run unchanged on ROCm tensors:

- single-layer paged caches ``[num_blocks, num_kv_heads, head_dim, block_size]``
  and stacked ``[num_layers, num_blocks, num_kv_heads, head_dim, block_size]``
  (reference :3-12);
- linear buffers ``[T, kv_heads, head_dim]`` / ``[L, T, kv_heads, head_dim]``,
  merged ``[T, 2, kv_heads, head_dim]`` / ``[L, T, 2, kv_heads, head_dim]``;
- ``slot = block * block_size + offset``; ``slot < 0`` is skipped: gathers
  write zeros there, scatters leave the cache untouched; duplicate scatter
  slots keep the last token in token order (reference :3321-3322).

Validation (shapes, dtypes, devices, slot bounds, FP8 scales) runs on the host
before the launch and raises ``ValueError`` like the reference.  The data
movement always runs in ``libmusa_aiter_kv_hip.so``; there is no CPU path, and
tensors that are not on a ROCm device are rejected with ``RuntimeError``.
"""

from __future__ import annotations

import threading
import time
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Literal

import torch

from musa_aiter.dispatch import DispatchRecord, emit, tensor_device_dtype, trace_enabled
from musa_aiter.ops import _hip
from musa_aiter.ops.kv_layout import KVLayoutSpec, KVScaleKind
from musa_aiter.ops.native_gate import native_requested

BACKEND = _hip.BACKEND

# Codec ids of the HIP library.
_CODEC_COPY, _CODEC_E4M3, _CODEC_E5M2 = 0, 1, 2
# Linear dtype ids of the HIP library's FP8 paths.
_LIN_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_ELT = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}
_FP8_CACHE_DTYPES = ("torch.float8_e4m3fn", "torch.float8_e5m2")


# ---------------------------------------------------------------------------
# Build / availability probes (reference :52-205)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class BuildResult:
    ok: bool
    library_path: str | None
    message: str


def _build_result() -> BuildResult:
    if _hip.LIB_PATH.exists():
        return BuildResult(True, str(_hip.LIB_PATH), "prebuilt gfx950 library")
    return BuildResult(False, None, f"{_hip.LIB_NAME} not built; run python musa-aiter_amd/build.py")


def build_native_kv_transfer() -> BuildResult:
    return _build_result()


def build_native_fp8_kv_cache() -> BuildResult:
    return _build_result()


def is_native_kv_transfer_available() -> bool:
    return _hip.is_available()


def is_native_fp8_kv_cache_available(fp8_format: str = "e4m3") -> bool:
    _normalize_fp8_format(fp8_format)
    return _hip.is_available()


def is_native_fp8_kv_vectorized_available() -> bool:
    return _hip.is_available()


def native_kv_transfer_abi_version() -> int | None:
    return int(_hip.fn("musa_aiter_kv_transfer_abi_version")()) if _hip.is_available() else None


def native_fp8_kv_cache_abi_version() -> int | None:
    return int(_hip.fn("musa_aiter_fp8_kv_cache_abi_version")()) if _hip.is_available() else None


# ---------------------------------------------------------------------------
# Shared validation (reference :2987-3044)
# ---------------------------------------------------------------------------


def _require_rocm(op: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{op}: the {BACKEND} backend moves KV data with gfx950 kernels and needs tensors on a ROCm "
                f"GPU device (got {t.device})"
            )


def _validate_paged_shapes(key_cache: torch.Tensor, value_cache: torch.Tensor, *, name: str) -> tuple[int, int, int, int]:
    if key_cache.dim() != 4 or value_cache.dim() != 4:
        raise ValueError(f"{name}: caches must be 4-D [blocks, kv_heads, head_dim, block_size]")
    if key_cache.shape != value_cache.shape:
        raise ValueError(f"{name}: key_cache and value_cache shapes must match")
    nb, nh, hd, bs = map(int, key_cache.shape)
    if nb <= 0 or nh <= 0 or hd <= 0 or bs <= 0:
        raise ValueError(f"{name}: all cache extents must be positive")
    return nb, nh, hd, bs


def _validate_stacked_paged_shapes(key_cache: torch.Tensor, value_cache: torch.Tensor, *,
                                   name: str) -> tuple[int, int, int, int, int]:
    if key_cache.dim() != 5 or value_cache.dim() != 5:
        raise ValueError(f"{name}: caches must be 5-D [layers, blocks, kv_heads, head_dim, block_size]")
    if key_cache.shape != value_cache.shape:
        raise ValueError(f"{name}: key_cache and value_cache shapes must match")
    nl, nb, nh, hd, bs = map(int, key_cache.shape)
    if nl <= 0 or nb <= 0 or nh <= 0 or hd <= 0 or bs <= 0:
        raise ValueError(f"{name}: all cache extents must be positive")
    return nl, nb, nh, hd, bs


def _ensure_slotmapping_vector(slot_mapping: torch.Tensor, *, expected_len: int, name: str) -> torch.Tensor:
    if slot_mapping.dim() != 1:
        raise ValueError(f"{name}: slot_mapping must be a 1-D tensor")
    if slot_mapping.numel() != expected_len:
        raise ValueError(
            f"{name}: slot_mapping length {slot_mapping.numel()} does not match num_tokens={expected_len}",
        )
    if slot_mapping.dtype not in (torch.int32, torch.int64, torch.int16):
        raise ValueError(f"{name}: slot_mapping must be integer-valued (int16/int32/int64)")
    return slot_mapping.to(torch.long).contiguous()


def _check_slots_in_bounds(slots_long: torch.Tensor, nb: int, bs: int, name: str) -> None:
    """Raise if a non-negative slot is >= nb*bs; one device->host sync per call."""
    if slots_long.numel() == 0:
        return
    if slots_long.is_cuda and slots_long.dtype == torch.int64 and slots_long.is_contiguous() and _hip.is_available():
        max_slot = _hip.index_max(slots_long)
    else:
        max_slot = int(slots_long.max().item())
    if max_slot >= nb * bs:
        raise ValueError(f"{name}: slot index {max_slot} out of bounds for caches (max {nb * bs - 1})")


def _float_elt(name: str, *tensors: torch.Tensor) -> int:
    dtype = tensors[0].dtype
    for t in tensors:
        if t.dtype not in _ELT:
            raise ValueError(f"{name}: the {BACKEND} backend moves float32, float16 and bfloat16 KV data, got {t.dtype}")
        if t.dtype != dtype:
            raise ValueError(f"{name}: all KV tensors must share one dtype (got {dtype} and {t.dtype})")
    return _ELT[dtype]


def _emit(op: str, tensor: torch.Tensor, reason: str) -> None:
    if not trace_enabled():
        return
    device, dtype = tensor_device_dtype(tensor)
    emit(DispatchRecord(op, BACKEND, device, dtype, reason))


def _rows_compatible(x: torch.Tensor, inner: int) -> bool:
    """True when the trailing ``inner`` elements of every token row are contiguous."""
    if x.dim() < 2:
        return x.is_contiguous()
    if inner == 1:
        return True
    # [.., H, D] with D contiguous and H packed right after it.
    if x.stride(-1) != 1 and x.shape[-1] != 1:
        return False
    if x.dim() >= 2 and x.shape[-2] != 1 and x.stride(-2) != x.shape[-1]:
        return False
    return True


def _token_strides(x: torch.Tensor, token_dim: int, row: int) -> tuple[int, int]:
    """(token stride, layer stride) in elements of a linear tensor laid out [.., T, rows]."""
    tok = x.stride(token_dim) if x.shape[token_dim] > 1 else row
    layer = x.stride(token_dim - 1) if token_dim >= 1 and x.shape[token_dim - 1] > 1 else 0
    return tok, layer


class _LinearPair:
    """K/V linear operands sharing token and layer strides (copied through temporaries otherwise)."""

    def __init__(self, k: torch.Tensor, v: torch.Tensor, *, token_dim: int, row: int, writable: bool):
        self.user = (k, v)
        inner = row
        ok = _rows_compatible(k, inner) and _rows_compatible(v, inner)
        if ok:
            sk = _token_strides(k, token_dim, row)
            sv = _token_strides(v, token_dim, row)
            ok = sk == sv
        if ok:
            self.k, self.v = k, v
            self.copy_back = False
            self.tok_stride, self.layer_stride = sk
        else:
            self.k = k.contiguous() if not writable else torch.empty(k.shape, dtype=k.dtype, device=k.device)
            self.v = v.contiguous() if not writable else torch.empty(v.shape, dtype=v.dtype, device=v.device)
            if writable:
                self.k.copy_(k)
                self.v.copy_(v)
            self.copy_back = writable
            self.tok_stride, self.layer_stride = _token_strides(self.k, token_dim, row)
        if self.layer_stride == 0:
            self.layer_stride = self.tok_stride * int(k.shape[token_dim])

    def finish(self) -> None:
        if self.copy_back:
            self.user[0].copy_(self.k)
            self.user[1].copy_(self.v)


class _CachePair:
    """Paged caches as contiguous buffers; writes go back when a copy was needed."""

    def __init__(self, k: torch.Tensor, v: torch.Tensor, *, writable: bool):
        self.user = (k, v)
        self.k = k if k.is_contiguous() else k.contiguous()
        self.v = v if v.is_contiguous() else v.contiguous()
        self.copy_back = writable and (self.k is not k or self.v is not v)

    def finish(self) -> None:
        if self.copy_back:
            if self.k is not self.user[0]:
                self.user[0].copy_(self.k)
            if self.v is not self.user[1]:
                self.user[1].copy_(self.v)


# ---------------------------------------------------------------------------
# Paged <-> linear (reference :3115-3457)
# ---------------------------------------------------------------------------


def _check_gather_out(out: torch.Tensor | None, shape: tuple[int, ...], dtype: torch.dtype, device: torch.device,
                      name: str) -> None:
    if out is None:
        return
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"{name}: out buffer shape mismatch {tuple(out.shape)}")
    if out.dtype != dtype:
        raise ValueError(f"{name}: out buffer dtype mismatch")
    if out.device != device:
        raise ValueError(f"{name}: out buffer device mismatch")


def _fill_mode(fill_skipped: str, out_k: torch.Tensor | None, out_v: torch.Tensor | None, name: str) -> bool:
    """Return True when skipped rows are zero filled; mirrors the reference's _finalize (:3069-3087)."""
    if fill_skipped == "preserve":
        if out_k is None or out_v is None:
            raise ValueError(f"{name}: fill_skipped=preserve requires out_k/out_v buffers")
        return False
    if fill_skipped != "zeros" and (out_k is not None or out_v is not None):
        raise AssertionError(f"{name}: fill_skipped must be 'zeros' or 'preserve'")
    return True


def _paged_gather(op: str, key_cache: torch.Tensor, value_cache: torch.Tensor, slots: torch.Tensor, *, nl: int,
                  tcount: int, nb: int, nh: int, hd: int, bs: int, out_k: torch.Tensor, out_v: torch.Tensor,
                  token_dim: int, fill_zeros: bool) -> None:
    caches = _CachePair(key_cache, value_cache, writable=False)
    lin = _LinearPair(out_k, out_v, token_dim=token_dim, row=nh * hd, writable=True)
    elt = _ELT[key_cache.dtype]
    _hip.paged_tiles(
        op=op, scatter=False, codec=_CODEC_COPY, cache_elt=elt, lin_elt=elt, lin_dtype=0,
        key_cache=caches.k, value_cache=caches.v, key_linear=lin.k, value_linear=lin.v, slots=slots,
        num_layers=nl, num_tokens=tcount, num_blocks=nb, num_heads=nh, head_dim=hd, block_size=bs,
        lin_token_stride=lin.tok_stride, lin_layer_stride=lin.layer_stride, fill_zeros=fill_zeros,
    )
    lin.finish()


def _paged_scatter(op: str, key_linear: torch.Tensor, value_linear: torch.Tensor, key_cache: torch.Tensor,
                   value_cache: torch.Tensor, slots: torch.Tensor, *, nl: int, tcount: int, nb: int, nh: int, hd: int,
                   bs: int, token_dim: int) -> None:
    if key_linear.dtype != key_cache.dtype:
        key_linear = key_linear.to(key_cache.dtype)
    if value_linear.dtype != value_cache.dtype:
        value_linear = value_linear.to(value_cache.dtype)
    caches = _CachePair(key_cache, value_cache, writable=True)
    lin = _LinearPair(key_linear, value_linear, token_dim=token_dim, row=nh * hd, writable=False)
    elt = _ELT[key_cache.dtype]
    _hip.paged_tiles(
        op=op, scatter=True, codec=_CODEC_COPY, cache_elt=elt, lin_elt=elt, lin_dtype=0,
        key_cache=caches.k, value_cache=caches.v, key_linear=lin.k, value_linear=lin.v, slots=slots,
        num_layers=nl, num_tokens=tcount, num_blocks=nb, num_heads=nh, head_dim=hd, block_size=bs,
        lin_token_stride=lin.tok_stride, lin_layer_stride=lin.layer_stride, fill_zeros=False,
    )
    caches.finish()


def kv_paged_to_linear(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    fill_skipped: Literal["zeros", "preserve"] = "zeros",
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather ``cache[block, :, :, offset]`` for every token into ``[T, kv_heads, head_dim]``.

    Reference: ``kv_paged_to_linear`` (kv_transfer.py:3115-3206), compute
    ``_kv_paged_to_linear_compute`` (:3047-3089).
    """
    op = "kv_paged_to_linear"
    nb, nh, hd, bs = _validate_paged_shapes(key_cache, value_cache, name=op)
    tcount = slot_mapping.numel()
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if key_cache.device != value_cache.device or slots.device != key_cache.device:
        raise ValueError("kv_paged_to_linear: all tensors must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    _check_gather_out(out_k, (tcount, nh, hd), key_cache.dtype, key_cache.device, op)
    _check_gather_out(out_v, (tcount, nh, hd), value_cache.dtype, value_cache.device, op)
    fill_zeros = _fill_mode(fill_skipped, out_k, out_v, op)
    _require_rocm(op, key_cache)
    ok = out_k if out_k is not None else torch.empty((tcount, nh, hd), dtype=key_cache.dtype, device=key_cache.device)
    ov = out_v if out_v is not None else torch.empty((tcount, nh, hd), dtype=value_cache.dtype, device=value_cache.device)
    _paged_gather(op, key_cache, value_cache, slots, nl=1, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, out_k=ok,
                  out_v=ov, token_dim=0, fill_zeros=fill_zeros)
    _emit(op, key_cache, "gfx950 paged->linear tile gather")
    return ok, ov


def kv_paged_to_linear_multi_layer(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    fill_skipped: Literal["zeros", "preserve"] = "zeros",
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather stacked caches ``[L, NB, H, D, BS]`` into ``[L, T, H, D]`` in one launch (reference :3209-3309)."""
    op = "kv_paged_to_linear_multi_layer"
    nl, nb, nh, hd, bs = _validate_stacked_paged_shapes(key_cache, value_cache, name=op)
    tcount = slot_mapping.numel()
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if value_cache.device != key_cache.device or slots.device != key_cache.device:
        raise ValueError("kv_paged_to_linear_multi_layer: all tensors must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    if out_k is not None and tuple(out_k.shape) != (nl, tcount, nh, hd):
        raise ValueError(
            f"kv_paged_to_linear_multi_layer: out_k must be [num_layers, T, kv_heads, head_dim], got {tuple(out_k.shape)}")
    if out_v is not None and tuple(out_v.shape) != (nl, tcount, nh, hd):
        raise ValueError(
            f"kv_paged_to_linear_multi_layer: out_v must be [num_layers, T, kv_heads, head_dim], got {tuple(out_v.shape)}")
    if fill_skipped == "preserve" and (out_k is None or out_v is None):
        raise ValueError("kv_paged_to_linear_multi_layer: fill_skipped=preserve requires out_k and out_v")
    _float_elt(op, key_cache, value_cache)
    _check_gather_out(out_k, (nl, tcount, nh, hd), key_cache.dtype, key_cache.device, op)
    _check_gather_out(out_v, (nl, tcount, nh, hd), value_cache.dtype, value_cache.device, op)
    fill_zeros = _fill_mode(fill_skipped, out_k, out_v, op)
    _require_rocm(op, key_cache)
    shape = (nl, tcount, nh, hd)
    ok = out_k if out_k is not None else torch.empty(shape, dtype=key_cache.dtype, device=key_cache.device)
    ov = out_v if out_v is not None else torch.empty(shape, dtype=value_cache.dtype, device=value_cache.device)
    _paged_gather(op, key_cache, value_cache, slots, nl=nl, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, out_k=ok,
                  out_v=ov, token_dim=1, fill_zeros=fill_zeros)
    _emit(op, key_cache, f"gfx950 paged->linear tile gather ({nl} layers, one launch)")
    return ok, ov


def kv_linear_to_paged(
    key_linear: torch.Tensor,
    value_linear: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter ``[T, H, D]`` rows into the paged caches in place (reference :3312-3379).

    Skipped tokens leave the cache untouched; duplicated slots keep the last
    token in token order.
    """
    op = "kv_linear_to_paged"
    if key_linear.shape != value_linear.shape or key_linear.dim() != 3:
        raise ValueError("kv_linear_to_paged: key_linear/value_linear must be 3-D and match shapes")
    tcount = key_linear.shape[0]
    nb, nh, hd, bs = _validate_paged_shapes(key_cache, value_cache, name=op)
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if key_linear.shape[1:] != (nh, hd):
        raise ValueError(
            "kv_linear_to_paged: last dims must match caches [num_kv_heads, head_dim] "
            f"got tail {tuple(key_linear.shape[1:])} vs {(nh, hd)}",
        )
    dev = key_cache.device
    if any(x.device != dev for x in (key_linear, value_linear, key_cache, value_cache, slots)):
        raise ValueError("kv_linear_to_paged: all tensors must be on same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    _require_rocm(op, key_cache)
    _paged_scatter(op, key_linear, value_linear, key_cache, value_cache, slots, nl=1, tcount=int(tcount), nb=nb,
                   nh=nh, hd=hd, bs=bs, token_dim=0)
    _emit(op, key_linear, "gfx950 linear->paged tile scatter")


def kv_linear_to_paged_multi_layer(
    key_linear: torch.Tensor,
    value_linear: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter ``[L, T, H, D]`` into stacked caches in one launch (reference :3382-3457)."""
    op = "kv_linear_to_paged_multi_layer"
    if key_linear.shape != value_linear.shape or key_linear.dim() != 4:
        raise ValueError(
            "kv_linear_to_paged_multi_layer: key_linear/value_linear must be 4-D "
            "[num_layers, num_tokens, num_kv_heads, head_dim] and match",
        )
    nl, tcount, nh_lin, hd_lin = map(int, key_linear.shape)
    nb, nh, hd, bs = _validate_stacked_paged_shapes(key_cache, value_cache, name=op)[1:]
    if nh_lin != nh or hd_lin != hd:
        raise ValueError(
            f"kv_linear_to_paged_multi_layer: linear tail dims must match caches got {(nh_lin, hd_lin)} vs cache {(nh, hd)}",
        )
    if key_cache.shape[0] != nl:
        raise ValueError(
            f"kv_linear_to_paged_multi_layer: layer count mismatch linear L={nl} vs cache L={key_cache.shape[0]}",
        )
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    dev = key_cache.device
    if any(x.device != dev for x in (key_linear, value_linear, key_cache, value_cache, slots)):
        raise ValueError("kv_linear_to_paged_multi_layer: all tensors must be on same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    _require_rocm(op, key_cache)
    _paged_scatter(op, key_linear, value_linear, key_cache, value_cache, slots, nl=nl, tcount=tcount, nb=nb, nh=nh,
                   hd=hd, bs=bs, token_dim=1)
    _emit(op, key_linear, f"gfx950 linear->paged tile scatter ({nl} layers, one launch)")


# ---------------------------------------------------------------------------
# Merged linear layouts (reference :3556-3766)
# ---------------------------------------------------------------------------


def kv_paged_to_merged_linear(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    fill_skipped: Literal["zeros", "preserve"] = "zeros",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Gather into merged ``[T, 2, kv_heads, head_dim]`` (axis 1 = key, value) (reference :3556-3618)."""
    op = "kv_paged_to_merged_linear"
    nb, nh, hd, bs = _validate_paged_shapes(key_cache, value_cache, name=op)
    tcount = slot_mapping.numel()
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if value_cache.device != key_cache.device or slots.device != key_cache.device:
        raise ValueError("kv_paged_to_merged_linear: all tensors must be on the same device")
    if out is not None:
        if tuple(out.shape) != (tcount, 2, nh, hd):
            raise ValueError("kv_paged_to_merged_linear: out must be [T, 2, kv_heads, head_dim]")
        if out.device != key_cache.device or out.dtype != key_cache.dtype:
            raise ValueError("kv_paged_to_merged_linear: out dtype/device must match caches")
    if fill_skipped == "preserve" and out is None:
        raise ValueError("kv_paged_to_merged_linear: fill_skipped=preserve requires out")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    fill_zeros = fill_skipped != "preserve"
    _require_rocm(op, key_cache)
    res = out if out is not None else torch.empty((tcount, 2, nh, hd), dtype=key_cache.dtype, device=key_cache.device)
    _paged_gather(op, key_cache, value_cache, slots, nl=1, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs,
                  out_k=res[:, 0], out_v=res[:, 1], token_dim=0, fill_zeros=fill_zeros)
    _emit(op, key_cache, "gfx950 paged->merged-linear tile gather")
    return res


def kv_merged_linear_to_paged(
    merged_linear: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter merged ``[T, 2, kv_heads, head_dim]`` into separate caches (reference :3621-3654)."""
    op = "kv_merged_linear_to_paged"
    if merged_linear.dim() != 4 or merged_linear.shape[1] != 2:
        raise ValueError("kv_merged_linear_to_paged: merged_linear must be [T, 2, kv_heads, head_dim]")
    tcount = int(merged_linear.shape[0])
    nb, nh, hd, bs = _validate_paged_shapes(key_cache, value_cache, name=op)
    if tuple(merged_linear.shape[2:]) != (nh, hd):
        raise ValueError("kv_merged_linear_to_paged: merged tail dims must match caches")
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if any(x.device != key_cache.device for x in (merged_linear, key_cache, value_cache, slots)):
        raise ValueError("kv_merged_linear_to_paged: all tensors must be on same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    _require_rocm(op, key_cache)
    _paged_scatter(op, merged_linear[:, 0], merged_linear[:, 1], key_cache, value_cache, slots, nl=1, tcount=tcount,
                   nb=nb, nh=nh, hd=hd, bs=bs, token_dim=0)
    _emit(op, merged_linear, "gfx950 merged-linear->paged tile scatter")


def kv_paged_to_merged_linear_multi_layer(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    fill_skipped: Literal["zeros", "preserve"] = "zeros",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Gather stacked caches into merged ``[L, T, 2, kv_heads, head_dim]`` (reference :3657-3724)."""
    op = "kv_paged_to_merged_linear_multi_layer"
    nl, nb, nh, hd, bs = _validate_stacked_paged_shapes(key_cache, value_cache, name=op)
    tcount = slot_mapping.numel()
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if value_cache.device != key_cache.device or slots.device != key_cache.device:
        raise ValueError("kv_paged_to_merged_linear_multi_layer: all tensors must be on the same device")
    if out is not None:
        if tuple(out.shape) != (nl, tcount, 2, nh, hd):
            raise ValueError("kv_paged_to_merged_linear_multi_layer: out must be [L, T, 2, kv_heads, head_dim]")
        if out.device != key_cache.device or out.dtype != key_cache.dtype:
            raise ValueError("kv_paged_to_merged_linear_multi_layer: out dtype/device must match caches")
    if fill_skipped == "preserve" and out is None:
        raise ValueError("kv_paged_to_merged_linear_multi_layer: fill_skipped=preserve requires out")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    fill_zeros = fill_skipped != "preserve"
    _require_rocm(op, key_cache)
    res = out if out is not None else torch.empty((nl, tcount, 2, nh, hd), dtype=key_cache.dtype,
                                                  device=key_cache.device)
    _paged_gather(op, key_cache, value_cache, slots, nl=nl, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs,
                  out_k=res[:, :, 0], out_v=res[:, :, 1], token_dim=1, fill_zeros=fill_zeros)
    _emit(op, key_cache, f"gfx950 paged->merged-linear tile gather ({nl} layers, one launch)")
    return res


def kv_merged_linear_to_paged_multi_layer(
    merged_linear: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter merged ``[L, T, 2, kv_heads, head_dim]`` into stacked caches (reference :3727-3766)."""
    op = "kv_merged_linear_to_paged_multi_layer"
    if merged_linear.dim() != 5 or merged_linear.shape[2] != 2:
        raise ValueError(
            "kv_merged_linear_to_paged_multi_layer: merged_linear must be [L, T, 2, kv_heads, head_dim]",
        )
    nl, tcount, _, nh_lin, hd_lin = map(int, merged_linear.shape)
    nb, nh, hd, bs = _validate_stacked_paged_shapes(key_cache, value_cache, name=op)[1:]
    if nh_lin != nh or hd_lin != hd or key_cache.shape[0] != nl:
        raise ValueError("kv_merged_linear_to_paged_multi_layer: merged dims must match caches")
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if any(x.device != key_cache.device for x in (merged_linear, key_cache, value_cache, slots)):
        raise ValueError("kv_merged_linear_to_paged_multi_layer: all tensors must be on same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    _float_elt(op, key_cache, value_cache)
    _require_rocm(op, key_cache)
    _paged_scatter(op, merged_linear[:, :, 0], merged_linear[:, :, 1], key_cache, value_cache, slots, nl=nl,
                   tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, token_dim=1)
    _emit(op, merged_linear, f"gfx950 merged-linear->paged tile scatter ({nl} layers, one launch)")


# ---------------------------------------------------------------------------
# FP8 KV cache (reference :2094-2400, :3460-3553)
# ---------------------------------------------------------------------------


def _normalize_fp8_format(fp8_format: str) -> str:
    normalized = fp8_format.lower().replace("-", "_")
    if normalized in ("fp8", "fp8_e4m3", "fp8_e4m3fn", "e4m3", "e4m3fn"):
        return "e4m3"
    if normalized in ("fp8_e5m2", "e5m2"):
        return "e5m2"
    raise ValueError(f"unsupported FP8 KV cache format: {fp8_format}")


def _fp8_format_params(fp8_format: str) -> tuple[int, int, int, int]:
    """(exponent bits, mantissa bits, bias, max unbiased exponent) of the FP8 format."""
    if _normalize_fp8_format(fp8_format) == "e4m3":
        return 4, 3, 7, 8
    return 5, 2, 15, 16


def _codec(fp8_format: str) -> int:
    return _CODEC_E4M3 if _normalize_fp8_format(fp8_format) == "e4m3" else _CODEC_E5M2


def _ensure_fp8_scale(scale: torch.Tensor | float, *, device: torch.device, name: str, num_heads: int,
                      num_layers: int | None = None) -> torch.Tensor:
    scale_tensor = torch.as_tensor(scale, dtype=torch.float32, device=device)
    if scale_tensor.numel() == 0 or not bool(((scale_tensor > 0) & torch.isfinite(scale_tensor)).all()):
        raise ValueError(f"{name}: FP8 scale must be positive and finite")
    if scale_tensor.numel() == 1:
        return scale_tensor.reshape(()).contiguous()
    if scale_tensor.dim() == 1 and int(scale_tensor.shape[0]) == num_heads:
        return scale_tensor.reshape(num_heads).contiguous()
    if num_layers is not None and scale_tensor.dim() == 2 and tuple(scale_tensor.shape) == (num_layers, num_heads):
        return scale_tensor.reshape(num_layers, num_heads).contiguous()
    expected = "scalar or [kv_heads]" if num_layers is None else "scalar, [kv_heads], or [layers, kv_heads]"
    raise ValueError(f"{name}: FP8 scale must be {expected}")


def _scale_pair(k: torch.Tensor, v: torch.Tensor, nh: int) -> tuple[torch.Tensor, torch.Tensor, int]:
    """Bring K and V scales to one scale mode (0 scalar, 1 [H], 2 [L, H])."""
    mode = max(k.dim(), v.dim())
    if k.dim() != v.dim():
        if mode == 1:
            k = k.reshape(-1).expand(nh).contiguous() if k.dim() == 0 else k
            v = v.reshape(-1).expand(nh).contiguous() if v.dim() == 0 else v
        else:
            nl = (k if k.dim() == 2 else v).shape[0]
            k = k.reshape(1, -1).expand(nl, nh).contiguous() if k.dim() < 2 else k
            v = v.reshape(1, -1).expand(nl, nh).contiguous() if v.dim() < 2 else v
    return k, v, mode


def _validate_fp8_cache_tensor(tensor: torch.Tensor, *, name: str) -> None:
    if tensor.dtype is torch.uint8 or str(tensor.dtype) in _FP8_CACHE_DTYPES:
        return
    raise ValueError(f"{name}: FP8 cache storage must be torch.uint8 or a supported torch.float8 dtype")


def _fp8_bytes(cache: torch.Tensor) -> torch.Tensor:
    return cache if cache.dtype is torch.uint8 else cache.view(torch.uint8)


def _fp8_linear_input(x: torch.Tensor) -> torch.Tensor:
    # float64 and other float inputs are first rounded to float32, exactly as
    # the reference's ``tensor.to(torch.float32) / scale`` (:2163).
    return x if x.dtype in _LIN_DTYPE else x.to(torch.float32)


def _fp8_scatter(op: str, key_linear: torch.Tensor, value_linear: torch.Tensor, key_cache: torch.Tensor,
                 value_cache: torch.Tensor, slots: torch.Tensor, k_scale: torch.Tensor, v_scale: torch.Tensor, *,
                 fp8_format: str, nl: int, tcount: int, nb: int, nh: int, hd: int, bs: int, token_dim: int) -> None:
    key_linear = _fp8_linear_input(key_linear)
    value_linear = _fp8_linear_input(value_linear)
    if value_linear.dtype != key_linear.dtype:
        value_linear = value_linear.to(key_linear.dtype)
    k_scale, v_scale, mode = _scale_pair(k_scale, v_scale, nh)
    caches = _CachePair(_fp8_bytes(key_cache), _fp8_bytes(value_cache), writable=True)
    lin = _LinearPair(key_linear, value_linear, token_dim=token_dim, row=nh * hd, writable=False)
    _hip.paged_tiles(
        op=op, scatter=True, codec=_codec(fp8_format), cache_elt=1, lin_elt=_ELT[key_linear.dtype],
        lin_dtype=_LIN_DTYPE[key_linear.dtype], key_cache=caches.k, value_cache=caches.v, key_linear=lin.k,
        value_linear=lin.v, slots=slots, num_layers=nl, num_tokens=tcount, num_blocks=nb, num_heads=nh,
        head_dim=hd, block_size=bs, lin_token_stride=lin.tok_stride, lin_layer_stride=lin.layer_stride,
        k_scale=k_scale, v_scale=v_scale, scale_mode=mode, fill_zeros=False,
    )
    caches.finish()


def _fp8_gather(op: str, key_cache: torch.Tensor, value_cache: torch.Tensor, slots: torch.Tensor,
                k_scale: torch.Tensor, v_scale: torch.Tensor, *, fp8_format: str, out_dtype: torch.dtype,
                out_k: torch.Tensor, out_v: torch.Tensor, nl: int, tcount: int, nb: int, nh: int, hd: int, bs: int,
                token_dim: int) -> None:
    k_scale, v_scale, mode = _scale_pair(k_scale, v_scale, nh)
    work_dtype = out_dtype if out_dtype in _LIN_DTYPE else torch.float32
    if work_dtype is out_dtype:
        tk, tv = out_k, out_v
    else:
        tk = torch.empty(out_k.shape, dtype=work_dtype, device=out_k.device)
        tv = torch.empty(out_v.shape, dtype=work_dtype, device=out_v.device)
    caches = _CachePair(_fp8_bytes(key_cache), _fp8_bytes(value_cache), writable=False)
    lin = _LinearPair(tk, tv, token_dim=token_dim, row=nh * hd, writable=True)
    _hip.paged_tiles(
        op=op, scatter=False, codec=_codec(fp8_format), cache_elt=1, lin_elt=_ELT[work_dtype],
        lin_dtype=_LIN_DTYPE[work_dtype], key_cache=caches.k, value_cache=caches.v, key_linear=lin.k,
        value_linear=lin.v, slots=slots, num_layers=nl, num_tokens=tcount, num_blocks=nb, num_heads=nh,
        head_dim=hd, block_size=bs, lin_token_stride=lin.tok_stride, lin_layer_stride=lin.layer_stride,
        k_scale=k_scale, v_scale=v_scale, scale_mode=mode, fill_zeros=True,
    )
    lin.finish()
    if tk is not out_k:
        out_k.copy_(tk)
        out_v.copy_(tv)


def kv_linear_to_paged_fp8(
    key_linear: torch.Tensor,
    value_linear: torch.Tensor,
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
) -> None:
    """Quantize ``[T, H, D]`` rows to FP8 and scatter them into uint8/float8 paged caches (reference :2203-2247).

    Each element is encoded from ``x.float() / scale`` with the reference
    encoder's rules (clamp to the format maximum, flush below the smallest
    normal, round half to even); scales are scalar or per kv-head.
    """
    op = "kv_linear_to_paged_fp8"
    fp8_format = _normalize_fp8_format(fp8_format)
    _validate_fp8_cache_tensor(key_cache_fp8, name="kv_linear_to_paged_fp8 key_cache_fp8")
    _validate_fp8_cache_tensor(value_cache_fp8, name="kv_linear_to_paged_fp8 value_cache_fp8")
    nb, nh, hd, bs = _validate_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    if key_linear.shape != value_linear.shape or key_linear.dim() != 3:
        raise ValueError("kv_linear_to_paged_fp8: key_linear and value_linear must be [tokens, kv_heads, head_dim]")
    tcount = int(key_linear.shape[0])
    if tuple(key_linear.shape[1:]) != (nh, hd):
        raise ValueError("kv_linear_to_paged_fp8: linear shape does not match FP8 cache shape")
    if (key_linear.device != value_linear.device or key_cache_fp8.device != key_linear.device
            or value_cache_fp8.device != key_linear.device):
        raise ValueError("kv_linear_to_paged_fp8: all tensors must be on the same device")
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if slots.device != key_linear.device:
        raise ValueError("kv_linear_to_paged_fp8: slot_mapping must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    ks = _ensure_fp8_scale(k_scale, device=key_linear.device, name="k_scale", num_heads=nh)
    vs = _ensure_fp8_scale(v_scale, device=value_linear.device, name="v_scale", num_heads=nh)
    _require_rocm(op, key_linear)
    _fp8_scatter(op, key_linear, value_linear, key_cache_fp8, value_cache_fp8, slots, ks, vs, fp8_format=fp8_format,
                 nl=1, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, token_dim=0)
    _emit(op, key_linear, f"gfx950 fused {fp8_format.upper()} quantize scatter")


def kv_paged_fp8_to_linear(
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather FP8 cache slots, decode ``code * scale`` in fp32 and round to ``out_dtype`` (reference :2250-2301)."""
    op = "kv_paged_fp8_to_linear"
    fp8_format = _normalize_fp8_format(fp8_format)
    _validate_fp8_cache_tensor(key_cache_fp8, name="kv_paged_fp8_to_linear key_cache_fp8")
    _validate_fp8_cache_tensor(value_cache_fp8, name="kv_paged_fp8_to_linear value_cache_fp8")
    nb, nh, hd, bs = _validate_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    tcount = int(slot_mapping.numel())
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if slots.device != key_cache_fp8.device:
        raise ValueError("kv_paged_fp8_to_linear: slot_mapping must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    ks = _ensure_fp8_scale(k_scale, device=key_cache_fp8.device, name="k_scale", num_heads=nh)
    vs = _ensure_fp8_scale(v_scale, device=value_cache_fp8.device, name="v_scale", num_heads=nh)
    ok = out_k if out_k is not None else torch.empty(tcount, nh, hd, dtype=out_dtype, device=key_cache_fp8.device)
    ov = out_v if out_v is not None else torch.empty(tcount, nh, hd, dtype=out_dtype, device=value_cache_fp8.device)
    if ok.shape != (tcount, nh, hd) or ov.shape != (tcount, nh, hd):
        raise ValueError("kv_paged_fp8_to_linear: output shape mismatch")
    if ok.dtype is not out_dtype or ov.dtype is not out_dtype:
        raise ValueError("kv_paged_fp8_to_linear: output dtype mismatch")
    _require_rocm(op, key_cache_fp8)
    _fp8_gather(op, key_cache_fp8, value_cache_fp8, slots, ks, vs, fp8_format=fp8_format, out_dtype=out_dtype,
                out_k=ok, out_v=ov, nl=1, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, token_dim=0)
    _emit(op, key_cache_fp8, f"gfx950 fused {fp8_format.upper()} dequantize gather")
    return ok, ov


def kv_linear_to_paged_fp8_multi_layer(
    key_linear: torch.Tensor,
    value_linear: torch.Tensor,
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
) -> None:
    """Multi-layer FP8 quantize scatter; scales scalar, ``[H]`` or ``[L, H]`` (reference :2304-2347)."""
    op = "kv_linear_to_paged_fp8_multi_layer"
    fp8_format = _normalize_fp8_format(fp8_format)
    _validate_fp8_cache_tensor(key_cache_fp8, name="kv_linear_to_paged_fp8_multi_layer key_cache_fp8")
    _validate_fp8_cache_tensor(value_cache_fp8, name="kv_linear_to_paged_fp8_multi_layer value_cache_fp8")
    nl, nb, nh, hd, bs = _validate_stacked_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    if key_linear.shape != value_linear.shape or key_linear.dim() != 4:
        raise ValueError(
            "kv_linear_to_paged_fp8_multi_layer: key_linear and value_linear must be [layers, tokens, kv_heads, head_dim]")
    if key_linear.shape[0] != nl or tuple(key_linear.shape[2:]) != (nh, hd):
        raise ValueError("kv_linear_to_paged_fp8_multi_layer: linear shape does not match FP8 cache shape")
    if (key_linear.device != value_linear.device or key_cache_fp8.device != key_linear.device
            or value_cache_fp8.device != key_linear.device):
        raise ValueError("kv_linear_to_paged_fp8_multi_layer: all tensors must be on the same device")
    tcount = int(key_linear.shape[1])
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if slots.device != key_linear.device:
        raise ValueError("kv_linear_to_paged_fp8_multi_layer: slot_mapping must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    ks = _ensure_fp8_scale(k_scale, device=key_linear.device, name="k_scale", num_heads=nh, num_layers=nl)
    vs = _ensure_fp8_scale(v_scale, device=value_linear.device, name="v_scale", num_heads=nh, num_layers=nl)
    _require_rocm(op, key_linear)
    _fp8_scatter(op, key_linear, value_linear, key_cache_fp8, value_cache_fp8, slots, ks, vs, fp8_format=fp8_format,
                 nl=nl, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, token_dim=1)
    _emit(op, key_linear, f"gfx950 fused {fp8_format.upper()} quantize scatter ({nl} layers)")


def kv_paged_fp8_to_linear_multi_layer(
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Multi-layer FP8 dequantize gather into ``[L, T, H, D]`` (reference :2350-2398)."""
    op = "kv_paged_fp8_to_linear_multi_layer"
    fp8_format = _normalize_fp8_format(fp8_format)
    _validate_fp8_cache_tensor(key_cache_fp8, name="kv_paged_fp8_to_linear_multi_layer key_cache_fp8")
    _validate_fp8_cache_tensor(value_cache_fp8, name="kv_paged_fp8_to_linear_multi_layer value_cache_fp8")
    nl, nb, nh, hd, bs = _validate_stacked_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    tcount = int(slot_mapping.numel())
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if slots.device != key_cache_fp8.device:
        raise ValueError("kv_paged_fp8_to_linear_multi_layer: slot_mapping must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    ks = _ensure_fp8_scale(k_scale, device=key_cache_fp8.device, name="k_scale", num_heads=nh, num_layers=nl)
    vs = _ensure_fp8_scale(v_scale, device=value_cache_fp8.device, name="v_scale", num_heads=nh, num_layers=nl)
    shape = (nl, tcount, nh, hd)
    ok = out_k if out_k is not None else torch.empty(shape, dtype=out_dtype, device=key_cache_fp8.device)
    ov = out_v if out_v is not None else torch.empty(shape, dtype=out_dtype, device=value_cache_fp8.device)
    if ok.shape != shape or ov.shape != shape:
        raise ValueError("kv_paged_fp8_to_linear_multi_layer: output shape mismatch")
    if ok.dtype is not out_dtype or ov.dtype is not out_dtype:
        raise ValueError("kv_paged_fp8_to_linear_multi_layer: output dtype mismatch")
    _require_rocm(op, key_cache_fp8)
    _fp8_gather(op, key_cache_fp8, value_cache_fp8, slots, ks, vs, fp8_format=fp8_format, out_dtype=out_dtype,
                out_k=ok, out_v=ov, nl=nl, tcount=tcount, nb=nb, nh=nh, hd=hd, bs=bs, token_dim=1)
    _emit(op, key_cache_fp8, f"gfx950 fused {fp8_format.upper()} dequantize gather ({nl} layers)")
    return ok, ov


def kv_paged_fp8_to_merged_linear(
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """FP8 dequantize gather into merged ``[T, 2, H, D]`` (reference :3460-3486)."""
    op = "kv_paged_fp8_to_merged_linear"
    _, nh, hd, _ = _validate_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    tcount = int(slot_mapping.numel())
    if out is not None:
        if tuple(out.shape) != (tcount, 2, nh, hd):
            raise ValueError("kv_paged_fp8_to_merged_linear: out must be [T, 2, kv_heads, head_dim]")
        if out.device != key_cache_fp8.device or out.dtype is not out_dtype:
            raise ValueError("kv_paged_fp8_to_merged_linear: out dtype/device mismatch")
    res = out if out is not None else torch.empty(tcount, 2, nh, hd, dtype=out_dtype, device=key_cache_fp8.device)
    kv_paged_fp8_to_linear(key_cache_fp8, value_cache_fp8, slot_mapping, k_scale, v_scale, out_dtype=out_dtype,
                           fp8_format=fp8_format, out_k=res[:, 0], out_v=res[:, 1])
    _emit(op, key_cache_fp8, f"merged FP8 {_normalize_fp8_format(fp8_format)} dequantize gather")
    return res


def kv_merged_linear_to_paged_fp8(
    merged_linear: torch.Tensor,
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
) -> None:
    """FP8 quantize scatter from merged ``[T, 2, H, D]`` (reference :3489-3505)."""
    op = "kv_merged_linear_to_paged_fp8"
    if merged_linear.dim() != 4 or merged_linear.shape[1] != 2:
        raise ValueError("kv_merged_linear_to_paged_fp8: merged_linear must be [T, 2, kv_heads, head_dim]")
    kv_linear_to_paged_fp8(merged_linear[:, 0], merged_linear[:, 1], key_cache_fp8, value_cache_fp8, slot_mapping,
                           k_scale, v_scale, fp8_format=fp8_format)
    _emit(op, merged_linear, f"merged FP8 {_normalize_fp8_format(fp8_format)} quantize scatter")


def kv_paged_fp8_to_merged_linear_multi_layer(
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Multi-layer FP8 dequantize gather into merged ``[L, T, 2, H, D]`` (reference :3508-3534)."""
    op = "kv_paged_fp8_to_merged_linear_multi_layer"
    nl, _, nh, hd, _ = _validate_stacked_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    tcount = int(slot_mapping.numel())
    if out is not None:
        if tuple(out.shape) != (nl, tcount, 2, nh, hd):
            raise ValueError("kv_paged_fp8_to_merged_linear_multi_layer: out must be [L, T, 2, kv_heads, head_dim]")
        if out.device != key_cache_fp8.device or out.dtype is not out_dtype:
            raise ValueError("kv_paged_fp8_to_merged_linear_multi_layer: out dtype/device mismatch")
    res = out if out is not None else torch.empty(nl, tcount, 2, nh, hd, dtype=out_dtype, device=key_cache_fp8.device)
    kv_paged_fp8_to_linear_multi_layer(key_cache_fp8, value_cache_fp8, slot_mapping, k_scale, v_scale,
                                       out_dtype=out_dtype, fp8_format=fp8_format, out_k=res[:, :, 0],
                                       out_v=res[:, :, 1])
    _emit(op, key_cache_fp8, f"merged multi-layer FP8 {_normalize_fp8_format(fp8_format)} dequantize gather")
    return res


def kv_merged_linear_to_paged_fp8_multi_layer(
    merged_linear: torch.Tensor,
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
) -> None:
    """Multi-layer FP8 quantize scatter from merged ``[L, T, 2, H, D]`` (reference :3537-3553)."""
    op = "kv_merged_linear_to_paged_fp8_multi_layer"
    if merged_linear.dim() != 5 or merged_linear.shape[2] != 2:
        raise ValueError(
            "kv_merged_linear_to_paged_fp8_multi_layer: merged_linear must be [L, T, 2, kv_heads, head_dim]")
    kv_linear_to_paged_fp8_multi_layer(merged_linear[:, :, 0], merged_linear[:, :, 1], key_cache_fp8,
                                       value_cache_fp8, slot_mapping, k_scale, v_scale, fp8_format=fp8_format)
    _emit(op, merged_linear, f"merged multi-layer FP8 {_normalize_fp8_format(fp8_format)} quantize scatter")


# ---------------------------------------------------------------------------
# Dense preload for attention (reference :1220-1795)
# ---------------------------------------------------------------------------

_INDEX_DTYPES = (torch.int16, torch.int32, torch.int64)


def _first_bad_block(block_tables_cpu: torch.Tensor, seq_lens_cpu: torch.Tensor, bs: int,
                     nb: int) -> tuple[int, int] | None:
    """(batch index, block id) of the first block id outside [0, nb) that a sequence uses, in the
    (batch, logical block) order of the reference's loops (:1578-1585, :1670-1676), or None."""
    batch, max_blocks = block_tables_cpu.shape
    if batch == 0 or max_blocks == 0:
        return None
    needed = (seq_lens_cpu.clamp(min=0) + bs - 1) // bs
    used = torch.arange(max_blocks).unsqueeze(0) < needed.unsqueeze(1)
    bad = used & ((block_tables_cpu < 0) | (block_tables_cpu >= nb))
    if not bool(bad.any()):
        return None
    first = int(bad.reshape(-1).nonzero()[0].item())
    return first // max_blocks, int(block_tables_cpu.reshape(-1)[first].item())


def _flash_dense_len(op: str, cache: torch.Tensor, value_cache: torch.Tensor, block_tables: torch.Tensor,
                     seq_lens: torch.Tensor, max_seq_len: int | None, bs: int, *,
                     joint_dtype_message: bool) -> tuple[int, torch.Tensor, torch.Tensor]:
    """Shared block_tables / seq_lens validation of the Flash-style loads, in the reference's order
    (:1541-1564 and :1741-1763, whose dtype messages differ); returns (dense_len, seq_lens, tables) on the CPU."""
    if block_tables.dim() != 2:
        raise ValueError(f"{op}: block_tables must be [batch, max_blocks]")
    if seq_lens.dim() != 1 or seq_lens.shape[0] != block_tables.shape[0]:
        raise ValueError(f"{op}: seq_lens must be [batch]")
    if (cache.device != value_cache.device or block_tables.device != cache.device
            or seq_lens.device != cache.device):
        raise ValueError(f"{op}: all tensors must be on the same device")
    if joint_dtype_message:
        if block_tables.dtype not in _INDEX_DTYPES or seq_lens.dtype not in _INDEX_DTYPES:
            raise ValueError(f"{op}: block_tables and seq_lens must be integer tensors")
    else:
        if block_tables.dtype not in _INDEX_DTYPES:
            raise ValueError(f"{op}: block_tables must use an integer dtype")
        if seq_lens.dtype not in _INDEX_DTYPES:
            raise ValueError(f"{op}: seq_lens must use an integer dtype")
    seq_lens_cpu = seq_lens.to(device="cpu", dtype=torch.long)
    if seq_lens_cpu.numel() > 0 and int(seq_lens_cpu.min().item()) < 0:
        raise ValueError(f"{op}: seq_lens must be non-negative")
    inferred_max = int(seq_lens_cpu.max().item()) if seq_lens_cpu.numel() > 0 else 0
    dense_len = inferred_max if max_seq_len is None else int(max_seq_len)
    if dense_len < inferred_max:
        raise ValueError(f"{op}: max_seq_len is smaller than seq_lens max")
    if (dense_len + bs - 1) // bs > int(block_tables.shape[1]):
        raise ValueError(f"{op}: block_tables does not contain enough columns")
    return dense_len, seq_lens_cpu, block_tables.to(device="cpu", dtype=torch.long)


def _dense_out(op: str, out: torch.Tensor | None, which: str, shape: tuple[int, ...], dtype: torch.dtype,
               device: torch.device, *, exact_dtype: bool = False) -> torch.Tensor:
    if out is None:
        # Every dense position is written by the kernel (zeros past seq_lens), so no clearing pass.
        return torch.empty(shape, dtype=dtype, device=device)
    dtype_bad = (out.dtype is not dtype) if exact_dtype else (out.dtype != dtype)
    if tuple(out.shape) != tuple(shape) or dtype_bad or out.device != device:
        raise ValueError(f"{op}: {which} must match [B, S, kv_heads, head_dim] dtype/device")
    return out


def _dense_work(out: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The tensor the kernel writes: ``out`` itself when it is contiguous and of ``dtype``."""
    if out.is_contiguous() and out.dtype is dtype:
        return out
    return torch.empty(out.shape, dtype=dtype, device=out.device)


def _index_tensor(t: torch.Tensor) -> torch.Tensor:
    return t.to(dtype=torch.long).contiguous()


def kv_triton_indexed_to_dense(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    *,
    max_seq_len: int,
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Load SGLang Triton-decode CSR-indexed KV rows into dense ``[B, S, kv_heads, head_dim]`` tensors
    (reference :1291-1366).

    Sequence b copies ``min(max(end - start, 0), max_seq_len)`` rows
    ``cache[kv_indices[kv_indptr[b] + i]]``; the rest of its dense rows are zeros.
    Indices are read on the device (nothing is synchronised, so the call can be
    captured in a graph); an offset past ``kv_indices`` or a row outside the cache
    yields a zero row, as in the reference's native kernel
    (kv_transfer_float.mu:114-128).
    """
    op = "kv_triton_indexed_to_dense"
    if key_cache.dim() != 3 or value_cache.dim() != 3:
        raise ValueError(f"{op}: key/value cache must be [tokens, kv_heads, head_dim]")
    if key_cache.shape != value_cache.shape or key_cache.dtype != value_cache.dtype or key_cache.device != value_cache.device:
        raise ValueError(f"{op}: key/value cache shape, dtype, and device must match")
    if kv_indptr.dim() != 1 or kv_indptr.numel() < 2:
        raise ValueError(f"{op}: kv_indptr must be [batch + 1]")
    if kv_indices.dim() != 1:
        raise ValueError(f"{op}: kv_indices must be 1-D")
    if kv_indptr.device != key_cache.device or kv_indices.device != key_cache.device:
        raise ValueError(f"{op}: all tensors must be on the same device")
    if kv_indptr.dtype not in _INDEX_DTYPES or kv_indices.dtype not in _INDEX_DTYPES:
        raise ValueError(f"{op}: indices must use integer dtype")
    batch = int(kv_indptr.shape[0] - 1)
    dense_len = int(max_seq_len)
    if dense_len < 0:
        raise ValueError(f"{op}: max_seq_len must be non-negative")
    ntok, nh, hd = map(int, key_cache.shape)
    shape = (batch, dense_len, nh, hd)
    for name, out, cache in (("out_k", out_k, key_cache), ("out_v", out_v, value_cache)):
        if out is not None and (tuple(out.shape) != shape or out.dtype != cache.dtype or out.device != cache.device
                                or not out.is_contiguous()):
            raise ValueError(f"{op}: {name} must match [B, S, kv_heads, head_dim] dtype/device and be contiguous")
    _require_rocm(op, key_cache)
    if out_k is None:
        out_k = torch.empty(shape, dtype=key_cache.dtype, device=key_cache.device)
    if out_v is None:
        out_v = torch.empty(shape, dtype=value_cache.dtype, device=value_cache.device)
    _hip.csr_dense_rows(
        op=op, key_cache=key_cache.contiguous(), value_cache=value_cache.contiguous(),
        kv_indptr=_index_tensor(kv_indptr), kv_indices=_index_tensor(kv_indices), out_k=out_k, out_v=out_v,
        batch=batch, dense_len=dense_len, num_tokens=ntok, row_bytes=nh * hd * key_cache.element_size(),
    )
    _emit(op, key_cache, "gfx950 CSR-indexed dense KV preload")
    return out_k, out_v


def kv_load_and_reshape_flash(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    max_seq_len: int | None = None,
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Load paged KV blocks into dense Flash-style ``[B, S, kv_heads, head_dim]`` tensors (reference :1527-1622).

    Dense position ``pos`` of sequence ``b`` holds cache slot
    ``block_tables[b, pos // block_size] * block_size + pos % block_size`` for
    ``pos < seq_lens[b]`` and zeros after it.  One launch moves both caches.
    """
    op = "kv_load_and_reshape_flash"
    nb, nh, hd, bs = _validate_paged_shapes(key_cache, value_cache, name=op)
    dense_len, seq_lens_cpu, tables_cpu = _flash_dense_len(op, key_cache, value_cache, block_tables, seq_lens,
                                                           max_seq_len, bs, joint_dtype_message=False)
    batch = int(block_tables.shape[0])
    shape = (batch, dense_len, nh, hd)
    out_k = _dense_out(op, out_k, "out_k", shape, key_cache.dtype, key_cache.device)
    out_v = _dense_out(op, out_v, "out_v", shape, value_cache.dtype, value_cache.device)
    bad = _first_bad_block(tables_cpu, seq_lens_cpu, bs, nb)
    if bad is not None:
        raise ValueError(f"{op}: invalid block id {bad[1]}")
    elt = _float_elt(op, key_cache, value_cache)
    _require_rocm(op, key_cache)
    caches = _CachePair(key_cache, value_cache, writable=False)
    wk, wv = _dense_work(out_k, key_cache.dtype), _dense_work(out_v, value_cache.dtype)
    _hip.paged_dense_tiles(
        op=op, scatter=False, codec=_CODEC_COPY, cache_elt=elt, lin_elt=elt, lin_dtype=0,
        key_cache=caches.k, value_cache=caches.v, dense_k=wk, dense_v=wv,
        block_tables=_index_tensor(block_tables), seq_lens=_index_tensor(seq_lens), batch=batch,
        dense_len=dense_len, max_blocks=int(block_tables.shape[1]), num_blocks=nb, num_heads=nh, head_dim=hd,
        block_size=bs, dense_token_stride=nh * hd, fill_zeros=True,
    )
    if wk is not out_k:
        out_k.copy_(wk)
    if wv is not out_v:
        out_v.copy_(wv)
    _emit(op, key_cache, "gfx950 block-table dense preload")
    return out_k, out_v


def kv_reshape_and_cache_back_flash(
    dense_k: torch.Tensor,
    dense_v: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
) -> bool:
    """Scatter dense Flash-style KV tensors back into paged cache blocks (reference :1625-1726).

    Positions ``pos < seq_lens[b]`` are written; blocks shared by several
    sequences keep the last (batch, position) in row-major order, as the
    reference's batch loop does.  Returns True.
    """
    op = "kv_reshape_and_cache_back_flash"
    if dense_k.dim() != 4 or dense_v.dim() != 4:
        raise ValueError("dense Flash KV tensors must be [batch, seq, heads, head_dim]")
    if dense_k.shape != dense_v.shape or dense_k.dtype != dense_v.dtype:
        raise ValueError("dense K and V tensors must have matching shape and dtype")
    if dense_k.device != dense_v.device:
        raise ValueError("dense K and V tensors must be on the same device")
    nb, nh, hd, bs = _validate_paged_shapes(key_cache, value_cache, name=op)
    if key_cache.dtype != dense_k.dtype or value_cache.dtype != dense_v.dtype:
        raise ValueError("dense and paged KV tensors must have matching dtypes")
    if key_cache.device != dense_k.device or value_cache.device != dense_k.device:
        raise ValueError("dense and paged KV tensors must be on the same device")
    if tuple(dense_k.shape[2:]) != (nh, hd):
        raise ValueError("dense KV head shape does not match paged cache")
    if block_tables.dim() != 2:
        raise ValueError(f"{op}: block_tables must be [batch, max_blocks]")
    if seq_lens.dim() != 1 or seq_lens.shape[0] != block_tables.shape[0]:
        raise ValueError(f"{op}: seq_lens must be [batch]")
    if dense_k.shape[0] != block_tables.shape[0]:
        raise ValueError(f"{op}: dense batch does not match block_tables")
    if block_tables.device != dense_k.device or seq_lens.device != dense_k.device:
        raise ValueError(f"{op}: all tensors must be on the same device")
    if block_tables.dtype not in _INDEX_DTYPES:
        raise ValueError(f"{op}: block_tables must use an integer dtype")
    if seq_lens.dtype not in _INDEX_DTYPES:
        raise ValueError(f"{op}: seq_lens must use an integer dtype")
    seq_lens_cpu = seq_lens.to(device="cpu", dtype=torch.long)
    tables_cpu = block_tables.to(device="cpu", dtype=torch.long)
    batch, dense_len = int(dense_k.shape[0]), int(dense_k.shape[1])
    max_blocks = int(block_tables.shape[1])
    # The reference checks each sequence in turn (:1660-1676): length, table width, block ids.
    bad_len = (seq_lens_cpu < 0) | (seq_lens_cpu > dense_len)
    bad_width = (seq_lens_cpu.clamp(min=0) + bs - 1) // bs > max_blocks
    bad_block = _first_bad_block(tables_cpu, torch.where(bad_len | bad_width, 0, seq_lens_cpu), bs, nb)
    first = [int(bad_len.nonzero()[0].item()) if bool(bad_len.any()) else batch,
             int(bad_width.nonzero()[0].item()) if bool(bad_width.any()) else batch,
             bad_block[0] if bad_block is not None else batch]
    b = min(first)
    if b < batch:
        if first[0] == b:
            raise ValueError(f"{op}: seq_lens exceeds dense sequence length")
        if first[1] == b:
            raise ValueError(f"{op}: block_tables does not contain enough columns")
        raise ValueError(f"{op}: invalid block id {bad_block[1]}")
    elt = _float_elt(op, dense_k, key_cache)
    _require_rocm(op, dense_k)
    caches = _CachePair(key_cache, value_cache, writable=True)
    _hip.paged_dense_tiles(
        op=op, scatter=True, codec=_CODEC_COPY, cache_elt=elt, lin_elt=elt, lin_dtype=0,
        key_cache=caches.k, value_cache=caches.v, dense_k=dense_k.contiguous(), dense_v=dense_v.contiguous(),
        block_tables=_index_tensor(block_tables), seq_lens=_index_tensor(seq_lens), batch=batch,
        dense_len=dense_len, max_blocks=max_blocks, num_blocks=nb, num_heads=nh, head_dim=hd, block_size=bs,
        dense_token_stride=nh * hd, fill_zeros=False,
    )
    caches.finish()
    _emit(op, dense_k, "gfx950 block-table dense write-back")
    return True


def kv_load_and_dequantize_fp8_flash(
    key_cache_fp8: torch.Tensor,
    value_cache_fp8: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    k_scale: torch.Tensor | float,
    v_scale: torch.Tensor | float,
    *,
    max_seq_len: int | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    fp8_format: Literal["e4m3", "e5m2"] = "e4m3",
    out_k: torch.Tensor | None = None,
    out_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Load paged FP8 blocks into dense dequantized ``[B, S, kv_heads, head_dim]`` tensors (reference :1729-1781).

    Each dense position decodes like kv_paged_fp8_to_linear over the
    sequence's slots (``code * scale`` in fp32, rounded to ``out_dtype``);
    positions past ``seq_lens[b]`` are zeros.  One launch covers the batch.
    """
    op = "kv_load_and_dequantize_fp8_flash"
    nb, nh, hd, bs = _validate_paged_shapes(key_cache_fp8, value_cache_fp8, name=op)
    dense_len, seq_lens_cpu, tables_cpu = _flash_dense_len(op, key_cache_fp8, value_cache_fp8, block_tables,
                                                           seq_lens, max_seq_len, bs, joint_dtype_message=True)
    batch = int(block_tables.shape[0])
    shape = (batch, dense_len, nh, hd)
    out_k = _dense_out(op, out_k, "out_k", shape, out_dtype, key_cache_fp8.device, exact_dtype=True)
    out_v = _dense_out(op, out_v, "out_v", shape, out_dtype, value_cache_fp8.device, exact_dtype=True)
    bad = _first_bad_block(tables_cpu, seq_lens_cpu, bs, nb)
    if bad is not None:
        raise ValueError(f"{op}: invalid block id {bad[1]}")
    if batch == 0:
        return out_k, out_v
    # The reference decodes through kv_paged_fp8_to_linear, whose checks and messages apply.
    fp8_format = _normalize_fp8_format(fp8_format)
    _validate_fp8_cache_tensor(key_cache_fp8, name="kv_paged_fp8_to_linear key_cache_fp8")
    _validate_fp8_cache_tensor(value_cache_fp8, name="kv_paged_fp8_to_linear value_cache_fp8")
    ks = _ensure_fp8_scale(k_scale, device=key_cache_fp8.device, name="k_scale", num_heads=nh)
    vs = _ensure_fp8_scale(v_scale, device=value_cache_fp8.device, name="v_scale", num_heads=nh)
    _require_rocm(op, key_cache_fp8)
    ks, vs, mode = _scale_pair(ks, vs, nh)
    work_dtype = out_dtype if out_dtype in _LIN_DTYPE else torch.float32
    caches = _CachePair(_fp8_bytes(key_cache_fp8), _fp8_bytes(value_cache_fp8), writable=False)
    wk, wv = _dense_work(out_k, work_dtype), _dense_work(out_v, work_dtype)
    _hip.paged_dense_tiles(
        op=op, scatter=False, codec=_codec(fp8_format), cache_elt=1, lin_elt=_ELT[work_dtype],
        lin_dtype=_LIN_DTYPE[work_dtype], key_cache=caches.k, value_cache=caches.v, dense_k=wk, dense_v=wv,
        block_tables=_index_tensor(block_tables), seq_lens=_index_tensor(seq_lens), batch=batch,
        dense_len=dense_len, max_blocks=int(block_tables.shape[1]), num_blocks=nb, num_heads=nh, head_dim=hd,
        block_size=bs, dense_token_stride=nh * hd, k_scale=ks, v_scale=vs, scale_mode=mode, fill_zeros=True,
    )
    if wk is not out_k:
        out_k.copy_(wk)
    if wv is not out_v:
        out_v.copy_(wv)
    _emit(op, key_cache_fp8, f"gfx950 block-table {fp8_format.upper()} dequantize preload")
    return out_k, out_v


# ---------------------------------------------------------------------------
# Paged block copies (reference :1798-2091)
# ---------------------------------------------------------------------------


def _validate_block_copy_shapes(src_key_cache: torch.Tensor, src_value_cache: torch.Tensor,
                                dst_key_cache: torch.Tensor, dst_value_cache: torch.Tensor, *,
                                name: str) -> tuple[int, int, bool]:
    if src_key_cache.shape != src_value_cache.shape:
        raise ValueError(f"{name}: source key/value cache shapes must match")
    if dst_key_cache.shape != dst_value_cache.shape:
        raise ValueError(f"{name}: destination key/value cache shapes must match")
    if src_key_cache.dim() not in (4, 5) or dst_key_cache.dim() != src_key_cache.dim():
        raise ValueError(f"{name}: caches must be 4-D single-layer or 5-D multi-layer paged tensors")
    if src_key_cache.dtype != src_value_cache.dtype or dst_key_cache.dtype != dst_value_cache.dtype:
        raise ValueError(f"{name}: key/value dtype pairs must match")
    if src_key_cache.dtype != dst_key_cache.dtype:
        raise ValueError(f"{name}: source and destination dtypes must match")
    if src_key_cache.dim() == 4:
        if src_key_cache.shape[1:] != dst_key_cache.shape[1:]:
            raise ValueError(f"{name}: single-layer cache tails must match")
        return int(src_key_cache.shape[0]), int(dst_key_cache.shape[0]), False
    if src_key_cache.shape[0] != dst_key_cache.shape[0] or src_key_cache.shape[2:] != dst_key_cache.shape[2:]:
        raise ValueError(f"{name}: multi-layer cache layer count and tails must match")
    return int(src_key_cache.shape[1]), int(dst_key_cache.shape[1]), True


def _ensure_block_mapping_pairs(block_mapping: torch.Tensor, *, src_blocks: int, dst_blocks: int,
                                name: str) -> torch.Tensor:
    if block_mapping.dim() != 2 or block_mapping.shape[1] != 2:
        raise ValueError(f"{name}: block_mapping must be [num_pairs, 2] with source and destination block ids")
    if block_mapping.dtype not in _INDEX_DTYPES:
        raise ValueError(f"{name}: block_mapping must use an integer dtype")
    pairs = block_mapping.to(device="cpu", dtype=torch.long)
    if pairs.numel() == 0:
        return pairs
    valid = (pairs[:, 0] >= 0) & (pairs[:, 1] >= 0)
    if not bool(valid.any()):
        return pairs
    src_max = int(pairs[valid, 0].max().item())
    dst_max = int(pairs[valid, 1].max().item())
    if src_max >= src_blocks:
        raise ValueError(f"{name}: source block index {src_max} out of bounds for {src_blocks} blocks")
    if dst_max >= dst_blocks:
        raise ValueError(f"{name}: destination block index {dst_max} out of bounds for {dst_blocks} blocks")
    return pairs


def _copy_blocks(op: str, src_k: torch.Tensor, src_v: torch.Tensor, dst_k: torch.Tensor, dst_v: torch.Tensor,
                 pairs: torch.Tensor, *, src_blocks: int, dst_blocks: int, multi_layer: bool) -> int:
    count = int(((pairs[:, 0] >= 0) & (pairs[:, 1] >= 0)).sum().item()) if pairs.numel() else 0
    if count == 0:
        return 0
    _require_rocm(op, src_k, dst_k)
    if src_k.device != dst_k.device:
        raise NotImplementedError(f"{op}: source and destination caches must be on one device")
    dst = _CachePair(dst_k, dst_v, writable=True)
    nl = int(src_k.shape[0]) if multi_layer else 1
    tail = src_k.shape[2:] if multi_layer else src_k.shape[1:]
    block_bytes = src_k.element_size()
    for extent in tail:
        block_bytes *= int(extent)
    _hip.copy_blocks(
        op=op, src_k=src_k.contiguous(), src_v=src_v.contiguous(), dst_k=dst.k, dst_v=dst.v,
        block_mapping=pairs.to(device=dst_k.device).contiguous(), num_layers=nl, src_blocks=src_blocks,
        dst_blocks=dst_blocks, block_bytes=block_bytes,
    )
    dst.finish()
    return count


def kv_copy_paged_blocks(
    src_key_cache: torch.Tensor,
    src_value_cache: torch.Tensor,
    dst_key_cache: torch.Tensor,
    dst_value_cache: torch.Tensor,
    block_mapping: torch.Tensor,
) -> int:
    """Copy selected paged KV cache blocks between same-layout caches (reference :2035-2091).

    ``block_mapping`` is ``[num_pairs, 2]`` (source, destination) block ids;
    pairs with a negative id are skipped and the number of copied pairs is
    returned.  A destination named twice keeps the last pair.  Source and
    destination blocks of one call must not overlap: all pairs copy at once.
    """
    op = "kv_copy_paged_blocks"
    src_blocks, dst_blocks, multi_layer = _validate_block_copy_shapes(
        src_key_cache, src_value_cache, dst_key_cache, dst_value_cache, name=op)
    pairs = _ensure_block_mapping_pairs(block_mapping, src_blocks=src_blocks, dst_blocks=dst_blocks, name=op)
    copied = _copy_blocks(op, src_key_cache, src_value_cache, dst_key_cache, dst_value_cache, pairs,
                          src_blocks=src_blocks, dst_blocks=dst_blocks, multi_layer=multi_layer)
    _emit(op, dst_key_cache, "gfx950 whole-block copy")
    return copied


def kv_copy_paged_blocks_fp8(
    src_key_cache_fp8: torch.Tensor,
    src_value_cache_fp8: torch.Tensor,
    dst_key_cache_fp8: torch.Tensor,
    dst_value_cache_fp8: torch.Tensor,
    block_mapping: torch.Tensor,
) -> int:
    """Raw FP8 paged block copy between same-layout caches (reference :1871-1906); see kv_copy_paged_blocks."""
    op = "kv_copy_paged_blocks_fp8"
    src_blocks, dst_blocks, multi_layer = _validate_block_copy_shapes(
        src_key_cache_fp8, src_value_cache_fp8, dst_key_cache_fp8, dst_value_cache_fp8, name=op)
    for tensor in (src_key_cache_fp8, src_value_cache_fp8, dst_key_cache_fp8, dst_value_cache_fp8):
        _validate_fp8_cache_tensor(tensor, name=op)
    pairs = _ensure_block_mapping_pairs(block_mapping, src_blocks=src_blocks, dst_blocks=dst_blocks, name=op)
    copied = _copy_blocks(op, src_key_cache_fp8, src_value_cache_fp8, dst_key_cache_fp8, dst_value_cache_fp8, pairs,
                          src_blocks=src_blocks, dst_blocks=dst_blocks, multi_layer=multi_layer)
    _emit(op, dst_key_cache_fp8, "gfx950 raw FP8 whole-block copy")
    return copied


# ---------------------------------------------------------------------------
# CacheGen-style uniform-bin codec (reference :1048-1215)
# ---------------------------------------------------------------------------

_CACHEGEN_INPUT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}


def _cachegen_native_rounding(tensor: torch.Tensor) -> bool:
    """The reference rounds bins with its native kernel only for float32 input and only when
    ``MUSA_AITER_NATIVE_KV_TRANSFER=1`` (reference :208-209, :1054); otherwise with torch ops."""
    return tensor.dtype == torch.float32 and native_requested("MUSA_AITER_NATIVE_KV_TRANSFER")


def kv_cachegen_encode(
    tensor: torch.Tensor,
    *,
    num_bins: int = 256,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Encode a KV tensor into uint8 bins plus a dequant codebook and the bins' empirical CDF
    (reference :1111-1172).

    Bins are uniform over the tensor's own [min, max] in float32: ``rint((x - min) * scale)``
    clamped to [0, num_bins - 1] with ``scale = (1 / (max - min)) * (num_bins - 1)``, or, for
    float32 input with ``MUSA_AITER_NATIVE_KV_TRANSFER=1``, the reference kernel's
    ``trunc((x - min) * scale + 0.5)`` with the scale computed in double.  The codebook is
    ``torch.linspace(min, max, num_bins)`` (all ``min`` for a constant tensor) and the CDF is
    ``[0, cumsum(counts) / numel]``, as float32.  Range, bins, histogram, codebook and CDF are
    computed on the device in three launches without a host synchronisation (the reference
    reads min and max back to the host and counts the bins on the CPU).
    """
    op = "kv_cachegen_encode"
    if num_bins < 2 or num_bins > 256:
        raise ValueError("kv_cachegen_encode: num_bins must be in [2, 256]")
    if not tensor.is_floating_point():
        raise ValueError("kv_cachegen_encode: tensor must use a floating dtype")
    if tensor.numel() == 0:
        codebook = torch.zeros(num_bins, dtype=torch.float32, device=tensor.device)
        cdf = torch.zeros(num_bins + 1, dtype=torch.float32, device=tensor.device)
        return torch.empty_like(tensor, dtype=torch.uint8), codebook, cdf
    _require_rocm(op, tensor)
    native = _cachegen_native_rounding(tensor)
    input_code = _CACHEGEN_INPUT.get(tensor.dtype)
    work = tensor if input_code is not None else tensor.float()  # float8 inputs: widened first, as the reference
    work = work.contiguous()
    encoded = torch.empty(tensor.shape, dtype=torch.uint8, device=tensor.device)
    codebook = torch.empty(num_bins, dtype=torch.float32, device=tensor.device)
    cdf = torch.empty(num_bins + 1, dtype=torch.float32, device=tensor.device)
    _hip.cachegen_encode(op=op, x=work, input_dtype=input_code if input_code is not None else 0,
                         num_bins=num_bins, native_rounding=native, encoded=encoded, codebook=codebook, cdf=cdf)
    _emit(op, tensor, "gfx950 CacheGen encode: range, bins and histogram on device" +
          (" (native-kernel rounding)" if native else ""))
    return encoded, codebook, cdf


def kv_cachegen_decode(
    encoded: torch.Tensor,
    codebook: torch.Tensor,
    *,
    dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Decode uint8 CacheGen-style bins through a dequant codebook: ``codebook[encoded]``, cast to
    ``dtype`` when given (reference :1175-1215).

    The gather runs through the (cast) codebook staged in LDS.  A bin past the end of a codebook
    of fewer than 256 entries raises ``ValueError`` as in the reference; it is detected by the
    decode launch itself, which costs one synchronisation for such codebooks and none for
    256-entry ones.
    """
    op = "kv_cachegen_decode"
    if encoded.dtype != torch.uint8:
        raise ValueError("kv_cachegen_decode: encoded must be uint8")
    if codebook.dim() != 1 or codebook.numel() < 2 or codebook.numel() > 256:
        raise ValueError("kv_cachegen_decode: codebook must be 1-D with 2..256 bins")
    if codebook.device != encoded.device:
        raise ValueError("kv_cachegen_decode: encoded and codebook must be on same device")
    if not codebook.is_floating_point():
        raise ValueError("kv_cachegen_decode: codebook must use a floating dtype")
    out_dtype = codebook.dtype if dtype is None else dtype
    if encoded.numel() == 0:
        return torch.empty(encoded.shape, dtype=out_dtype, device=encoded.device)
    _require_rocm(op, encoded)
    table = (codebook if out_dtype == codebook.dtype else codebook.to(out_dtype)).contiguous()
    codes = encoded.contiguous()
    out = torch.empty(encoded.shape, dtype=out_dtype, device=encoded.device)
    max_code = torch.zeros(1, dtype=torch.int32, device=encoded.device) if table.numel() < 256 else None
    _hip.cachegen_decode(op=op, codes=codes, table=table, out=out, max_code=max_code)
    if max_code is not None and int(max_code.item()) >= table.numel():
        raise ValueError("kv_cachegen_decode: encoded bin exceeds codebook size")
    _emit(op, encoded, "gfx950 CacheGen decode: LDS codebook gather")
    return out


# ---------------------------------------------------------------------------
# MLA / DSA flat caches [NB, BS, D] (reference :3769-4118)
# ---------------------------------------------------------------------------


def _validate_flat_paged_shapes(first_cache: torch.Tensor, second_cache: torch.Tensor, *,
                                name: str) -> tuple[int, int, int, int]:
    if first_cache.dim() != 3 or second_cache.dim() != 3:
        raise ValueError(f"{name}: caches must be 3-D [blocks, block_size, hidden_dim]")
    if first_cache.shape[:2] != second_cache.shape[:2]:
        raise ValueError(f"{name}: caches must share [blocks, block_size]")
    nb, bs, first_dim = map(int, first_cache.shape)
    second_dim = int(second_cache.shape[2])
    if nb <= 0 or bs <= 0 or first_dim <= 0 or second_dim <= 0:
        raise ValueError(f"{name}: all cache extents must be positive")
    return nb, bs, first_dim, second_dim


def _validate_stacked_mla_shapes(kv_cache: torch.Tensor, k_pe_cache: torch.Tensor, *,
                                 name: str) -> tuple[int, int, int, int, int]:
    if kv_cache.dim() != 4 or k_pe_cache.dim() != 4:
        raise ValueError(f"{name}: caches must be [layers, blocks, block_size, hidden_dim]")
    if tuple(kv_cache.shape[:3]) != tuple(k_pe_cache.shape[:3]):
        raise ValueError(f"{name}: caches must share [layers, blocks, block_size]")
    nl, nb, bs, kv_dim = map(int, kv_cache.shape)
    pe_dim = int(k_pe_cache.shape[3])
    if nl <= 0 or nb <= 0 or bs <= 0 or kv_dim <= 0 or pe_dim <= 0:
        raise ValueError(f"{name}: all cache extents must be positive")
    return nl, nb, bs, kv_dim, pe_dim


def _elt_any(name: str, t: torch.Tensor) -> int:
    if t.dtype not in _ELT:
        raise ValueError(f"{name}: the {BACKEND} backend moves float32, float16 and bfloat16 KV data, got {t.dtype}")
    return _ELT[t.dtype]


def _row_view(x: torch.Tensor, dim: int) -> tuple[torch.Tensor, int, bool]:
    """(tensor, row stride elements, copied) for a tensor whose last dim is a contiguous row."""
    if x.stride(-1) == 1 or x.shape[-1] == 1:
        stride = x.stride(dim) if x.shape[dim] > 1 else x.shape[-1]
        return x, stride, False
    return x.contiguous(), x.shape[-1], True


def _flat_rows(op: str, *, gather: bool, caches: Sequence[torch.Tensor], lins: Sequence[torch.Tensor],
               slots: torch.Tensor, nl: int, tcount: int, nb: int, bs: int) -> None:
    """Row copies between flat caches [L?, NB, BS, D] and linear [L?, T, D], one launch per (cache, linear) pair."""
    for cache, lin in zip(caches, lins):
        elt = _elt_any(op, cache)
        if lin.dtype != cache.dtype:
            if gather:
                raise ValueError(f"{op}: output dtype must match cache dtype")
            lin = lin.to(cache.dtype)
        d = int(cache.shape[-1])
        row = d * elt
        cache_c = cache if cache.is_contiguous() else cache.contiguous()
        lin_w, lstride, copied = _row_view(lin, lin.dim() - 2)
        if copied and gather:
            lin_w = torch.empty(lin.shape, dtype=lin.dtype, device=lin.device)
            lstride = d
        layer_stride_l = lin_w.stride(0) if nl > 1 else 0
        cache_planes = [cache_c.data_ptr() + layer * nb * bs * row for layer in range(nl)]
        lin_planes = [lin_w.data_ptr() + layer * layer_stride_l * elt for layer in range(nl)]
        if gather:
            _hip.copy_rows(op=op, device=cache.device, src_planes=cache_planes, dst_planes=lin_planes,
                           num_planes=nl, src_idx=slots, dst_idx=None, num_tokens=tcount, num_rows_out=tcount,
                           src_rows=nb * bs, dst_rows=tcount, row_bytes=row, src_stride=row,
                           dst_stride=lstride * elt, zero_invalid=True)
            if lin_w is not lin:
                lin.copy_(lin_w)
        else:
            _hip.copy_rows(op=op, device=cache.device, src_planes=lin_planes, dst_planes=cache_planes,
                           num_planes=nl, src_idx=None, dst_idx=slots, num_tokens=tcount, num_rows_out=tcount,
                           src_rows=tcount, dst_rows=nb * bs, row_bytes=row, src_stride=lstride * elt,
                           dst_stride=row, zero_invalid=False)
            if cache_c is not cache:
                cache.copy_(cache_c)


def kv_paged_to_mla_linear(
    kv_cache: torch.Tensor,
    k_pe_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    out_kv: torch.Tensor | None = None,
    out_k_pe: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather MLA flat caches ``[NB, BS, D]`` into ``[T, kv_dim]`` and ``[T, pe_dim]`` (reference :3841-3903)."""
    op = "kv_paged_to_mla_linear"
    nb, bs, kv_dim, pe_dim = _validate_flat_paged_shapes(kv_cache, k_pe_cache, name=op)
    tcount = slot_mapping.numel()
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if k_pe_cache.device != kv_cache.device or slots.device != kv_cache.device:
        raise ValueError("kv_paged_to_mla_linear: all tensors must be on the same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    if out_kv is not None and tuple(out_kv.shape) != (tcount, kv_dim):
        raise ValueError(f"{op}: first_out shape mismatch {tuple(out_kv.shape)}")
    if out_k_pe is not None and tuple(out_k_pe.shape) != (tcount, pe_dim):
        raise ValueError(f"{op}: second_out shape mismatch {tuple(out_k_pe.shape)}")
    _require_rocm(op, kv_cache)
    okv = out_kv if out_kv is not None else torch.empty((tcount, kv_dim), dtype=kv_cache.dtype, device=kv_cache.device)
    ope = out_k_pe if out_k_pe is not None else torch.empty((tcount, pe_dim), dtype=k_pe_cache.dtype,
                                                            device=k_pe_cache.device)
    _flat_rows(op, gather=True, caches=(kv_cache, k_pe_cache), lins=(okv, ope), slots=slots, nl=1, tcount=tcount,
               nb=nb, bs=bs)
    _emit(op, kv_cache, "gfx950 MLA flat-row gather")
    return okv, ope


def kv_mla_linear_to_paged(
    kv_linear: torch.Tensor,
    k_pe_linear: torch.Tensor,
    kv_cache: torch.Tensor,
    k_pe_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter ``[T, kv_dim]`` / ``[T, pe_dim]`` rows into MLA flat caches (reference :3906-3962)."""
    op = "kv_mla_linear_to_paged"
    if kv_linear.dim() != 2 or k_pe_linear.dim() != 2:
        raise ValueError("kv_mla_linear_to_paged: linear buffers must be [T, hidden_dim]")
    if kv_linear.shape[0] != k_pe_linear.shape[0]:
        raise ValueError("kv_mla_linear_to_paged: linear buffers must share token count")
    tcount = int(kv_linear.shape[0])
    nb, bs, kv_dim, pe_dim = _validate_flat_paged_shapes(kv_cache, k_pe_cache, name=op)
    if tuple(kv_linear.shape[1:]) != (kv_dim,) or tuple(k_pe_linear.shape[1:]) != (pe_dim,):
        raise ValueError("kv_mla_linear_to_paged: linear hidden dims must match caches")
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name=op)
    if any(x.device != kv_cache.device for x in (kv_linear, k_pe_linear, kv_cache, k_pe_cache, slots)):
        raise ValueError("kv_mla_linear_to_paged: all tensors must be on same device")
    _check_slots_in_bounds(slots, nb, bs, op)
    _require_rocm(op, kv_cache)
    _flat_rows(op, gather=False, caches=(kv_cache, k_pe_cache), lins=(kv_linear, k_pe_linear), slots=slots, nl=1,
               tcount=tcount, nb=nb, bs=bs)
    _emit(op, kv_linear, "gfx950 MLA flat-row scatter")


def kv_paged_to_mla_linear_multi_layer(
    kv_cache: torch.Tensor,
    k_pe_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather stacked MLA caches ``[L, NB, BS, D]`` into ``[L, T, D]`` (reference :3982-4050)."""
    op = "kv_paged_to_mla_linear_multi_layer"
    nl, nb, bs, kv_dim, pe_dim = _validate_stacked_mla_shapes(kv_cache, k_pe_cache, name=op)
    if k_pe_cache.dtype != kv_cache.dtype or k_pe_cache.device != kv_cache.device:
        raise ValueError("kv_paged_to_mla_linear_multi_layer: caches must share dtype and device")
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=int(slot_mapping.numel()), name=op)
    if slots.device != kv_cache.device:
        raise ValueError("kv_paged_to_mla_linear_multi_layer: slot_mapping must share device")
    tcount = int(slots.numel())
    _check_slots_in_bounds(slots, nb, bs, "kv_paged_to_mla_linear")
    _require_rocm(op, kv_cache)
    kv_out = torch.empty((nl, tcount, kv_dim), dtype=kv_cache.dtype, device=kv_cache.device)
    pe_out = torch.empty((nl, tcount, pe_dim), dtype=k_pe_cache.dtype, device=k_pe_cache.device)
    _flat_rows(op, gather=True, caches=(kv_cache, k_pe_cache), lins=(kv_out, pe_out), slots=slots, nl=nl,
               tcount=tcount, nb=nb, bs=bs)
    _emit(op, kv_cache, f"gfx950 MLA flat-row gather ({nl} layers)")
    return kv_out, pe_out


def kv_mla_linear_to_paged_multi_layer(
    kv_linear: torch.Tensor,
    k_pe_linear: torch.Tensor,
    kv_cache: torch.Tensor,
    k_pe_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> bool:
    """Scatter ``[L, T, D]`` rows into stacked MLA caches; returns True (reference :4053-4118)."""
    op = "kv_mla_linear_to_paged_multi_layer"
    nl, nb, bs, kv_dim, pe_dim = _validate_stacked_mla_shapes(kv_cache, k_pe_cache, name=op)
    if kv_linear.dim() != 3 or k_pe_linear.dim() != 3:
        raise ValueError("kv_mla_linear_to_paged_multi_layer: linear buffers must be [layers, tokens, hidden]")
    if kv_linear.shape[0] != nl or k_pe_linear.shape[0] != nl:
        raise ValueError("kv_mla_linear_to_paged_multi_layer: layer counts must match caches")
    if kv_linear.shape[1] != k_pe_linear.shape[1]:
        raise ValueError("kv_mla_linear_to_paged_multi_layer: token counts must match")
    if tuple(kv_linear.shape[2:]) != (kv_dim,) or tuple(k_pe_linear.shape[2:]) != (pe_dim,):
        raise ValueError("kv_mla_linear_to_paged_multi_layer: hidden dims must match caches")
    if kv_linear.dtype != kv_cache.dtype or k_pe_linear.dtype != k_pe_cache.dtype:
        raise ValueError("kv_mla_linear_to_paged_multi_layer: dtypes must match caches")
    if any(t.device != kv_cache.device for t in (kv_linear, k_pe_linear, kv_cache, k_pe_cache, slot_mapping)):
        raise ValueError("kv_mla_linear_to_paged_multi_layer: all tensors must share device")
    tcount = int(kv_linear.shape[1])
    slots = _ensure_slotmapping_vector(slot_mapping, expected_len=tcount, name="kv_mla_linear_to_paged")
    _check_slots_in_bounds(slots, nb, bs, "kv_mla_linear_to_paged")
    _require_rocm(op, kv_cache)
    _flat_rows(op, gather=False, caches=(kv_cache, k_pe_cache), lins=(kv_linear, k_pe_linear), slots=slots, nl=nl,
               tcount=tcount, nb=nb, bs=bs)
    _emit(op, kv_linear, f"gfx950 MLA flat-row scatter ({nl} layers)")
    return True


# ---------------------------------------------------------------------------
# DSV4 opaque byte rows (reference :4164-4736)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class InterleavedFp8Layout:
    """Descriptor of DSV4 interleaved FP8 block-scale page rows ``[value region][scale region]`` (reference :4411-4452)."""

    value_bytes: int
    scale_bytes: int
    scale_granularity: int

    def __post_init__(self) -> None:
        if self.value_bytes <= 0 or self.scale_bytes <= 0:
            raise ValueError("InterleavedFp8Layout: value_bytes and scale_bytes must be positive")
        if self.scale_granularity <= 0:
            raise ValueError("InterleavedFp8Layout: scale_granularity must be positive")

    @property
    def item_bytes(self) -> int:
        return self.value_bytes + self.scale_bytes

    def as_kv_layout_spec(self, *, num_layers: int, num_blocks: int, block_size: int,
                          dtype_name: str = "uint8") -> KVLayoutSpec:
        return KVLayoutSpec.dsv4(
            num_layers=num_layers,
            num_blocks=num_blocks,
            block_size=block_size,
            row_bytes=self.item_bytes,
            block_stride_bytes=self.item_bytes * block_size,
            dtype_name=dtype_name,
            scale_kind=KVScaleKind.BLOCKED,
            value_bytes=self.value_bytes,
            scale_bytes=self.scale_bytes,
        )


@dataclass
class PoolSpec:
    """One pool of the DSV4 shared-index multi-pool copy (reference :4455-4464)."""

    src_ptrs: list
    dst_ptrs: list
    item_bytes: int


def _is_integer_indices(indices: torch.Tensor) -> bool:
    return isinstance(indices, torch.Tensor) and indices.dim() == 1 and indices.dtype in (
        torch.int16, torch.int32, torch.int64)


def _check_row_indices(indices: torch.Tensor, num_rows: int, name: str) -> None:
    # Host-resident indices are checked eagerly; device indices are bounds
    # checked in the kernel (out-of-range rows are skipped), avoiding a sync.
    if indices.numel() == 0 or indices.device.type != "cpu":
        return
    idx = indices.to(dtype=torch.long)
    lo = int(idx.min().item())
    hi = int(idx.max().item())
    if lo < 0:
        raise IndexError(f"{name} row index {lo} is negative")
    if hi >= num_rows:
        raise IndexError(f"{name} row index {hi} out of bounds for {num_rows} rows")


def _validate_kv_copy_paged_rows_args(src, dst, src_indices, dst_indices, *, name: str) -> tuple[int, int, int]:
    if not isinstance(src, torch.Tensor) or not isinstance(dst, torch.Tensor):
        raise TypeError(f"{name}: src and dst must be torch.Tensor")
    if src.dtype is not torch.uint8 or dst.dtype is not torch.uint8:
        raise ValueError(f"{name}: src and dst must be uint8 byte rows, got src={src.dtype}, dst={dst.dtype}")
    if src.dim() != 2 or dst.dim() != 2:
        raise ValueError(f"{name}: src and dst must be [rows, item_bytes]")
    item_bytes = int(src.shape[1])
    if int(dst.shape[1]) != item_bytes:
        raise ValueError(f"{name}: src and dst item_bytes must match, got src={item_bytes}, dst={int(dst.shape[1])}")
    if item_bytes <= 0:
        raise ValueError(f"{name}: item_bytes must be positive")
    if not _is_integer_indices(src_indices) or not _is_integer_indices(dst_indices):
        raise ValueError(f"{name}: indices must use an integer dtype")
    if src_indices.numel() != dst_indices.numel():
        raise ValueError(f"{name}: src_indices and dst_indices must have the same length")
    _check_row_indices(src_indices, int(src.shape[0]), f"{name}: src")
    _check_row_indices(dst_indices, int(dst.shape[0]), f"{name}: dst")
    return item_bytes, int(src.shape[0]), int(dst.shape[0])


def _validate_layer_table(src_ptrs, dst_ptrs, src_indices, dst_indices, *, name: str) -> int:
    if not isinstance(src_ptrs, (list, tuple)) or not isinstance(dst_ptrs, (list, tuple)):
        raise TypeError(f"{name}: src_ptrs and dst_ptrs must be lists of tensors")
    if len(src_ptrs) == 0 or len(dst_ptrs) == 0:
        raise ValueError(f"{name}: ptr-tables must be non-empty")
    if len(src_ptrs) != len(dst_ptrs):
        raise ValueError(f"{name}: src/dst layer counts must match, got {len(src_ptrs)} vs {len(dst_ptrs)}")
    item_bytes = int(src_ptrs[0].shape[1])
    for layer, (src, dst) in enumerate(zip(src_ptrs, dst_ptrs)):
        _validate_kv_copy_paged_rows_args(src, dst, src_indices, dst_indices, name=f"{name}[layer{layer}]")
        if int(dst.shape[1]) != item_bytes:
            raise ValueError(f"{name}: layer {layer} item_bytes mismatch, expected {item_bytes}, got {int(dst.shape[1])}")
    return item_bytes


def _byte_row_indices(indices: torch.Tensor, device: torch.device) -> torch.Tensor:
    return indices.to(device=device, dtype=torch.long).contiguous()


def _copy_byte_rows(op: str, srcs: Sequence[torch.Tensor], dsts: Sequence[torch.Tensor], src_indices: torch.Tensor,
                    dst_indices: torch.Tensor, item_bytes: int) -> None:
    device = dsts[0].device
    for t in list(srcs) + list(dsts):
        if t.device != device:
            raise NotImplementedError(
                f"{op}: host<->device byte-row staging is not part of the {BACKEND} backend; "
                "place src and dst on the same ROCm device")
        if not t.is_contiguous():
            raise ValueError(f"{op}: byte-row tensors must be contiguous")
    _require_rocm(op, dsts[0])
    n = int(src_indices.numel())
    if n == 0:
        return
    start = time.perf_counter_ns()
    _hip.copy_rows(op=op, device=device, src_planes=[t.data_ptr() for t in srcs],
                   dst_planes=[t.data_ptr() for t in dsts], num_planes=len(srcs),
                   src_idx=_byte_row_indices(src_indices, device), dst_idx=_byte_row_indices(dst_indices, device),
                   num_tokens=n, num_rows_out=n, src_rows=int(srcs[0].shape[0]), dst_rows=int(dsts[0].shape[0]),
                   row_bytes=item_bytes, src_stride=item_bytes, dst_stride=item_bytes, zero_invalid=False)
    _record_copy_stats(n * item_bytes * len(srcs), time.perf_counter_ns() - start)


def kv_copy_paged_rows(src: torch.Tensor, dst: torch.Tensor, src_indices: torch.Tensor, dst_indices: torch.Tensor, *,
                       layout: InterleavedFp8Layout | None = None) -> None:
    """Copy ``src[src_indices[i]] -> dst[dst_indices[i]]`` for uint8 rows (reference :4518-4557).

    Repeated destination rows keep the last source in index order, like the
    reference's ``index_copy_``.  ``layout`` only pins the row width.
    """
    op = "kv_copy_paged_rows"
    item_bytes, _, _ = _validate_kv_copy_paged_rows_args(src, dst, src_indices, dst_indices, name=op)
    if layout is not None and layout.item_bytes != item_bytes:
        raise ValueError(
            f"kv_copy_paged_rows: layout.item_bytes={layout.item_bytes} != tensor row width {item_bytes}")
    _copy_byte_rows(op, [src], [dst], src_indices, dst_indices, item_bytes)
    _emit(op, src, "gfx950 opaque byte-row copy (per layer)")


def kv_copy_paged_rows_layer_table(src_ptrs, dst_ptrs, src_indices: torch.Tensor, dst_indices: torch.Tensor) -> None:
    """Copy the same rows of every layer of a layer table in one launch (reference :4588-4616)."""
    op = "kv_copy_paged_rows_layer_table"
    item_bytes = _validate_layer_table(src_ptrs, dst_ptrs, src_indices, dst_indices, name=op)
    shapes = {(int(s.shape[0]), int(d.shape[0])) for s, d in zip(src_ptrs, dst_ptrs)}
    if len(shapes) == 1:
        _copy_byte_rows(op, list(src_ptrs), list(dst_ptrs), src_indices, dst_indices, item_bytes)
    else:
        for s, d in zip(src_ptrs, dst_ptrs):
            _copy_byte_rows(op, [s], [d], src_indices, dst_indices, item_bytes)
    _emit(op, src_ptrs[0], f"gfx950 opaque byte-row copy ({len(src_ptrs)} layers, item_bytes={item_bytes})")


def kv_copy_paged_rows_multi_pool(pools: list[PoolSpec], indices: torch.Tensor, *,
                                  direction: Literal["H2D", "D2H"]) -> None:
    """Copy rows of several pools that share one index set (reference :4619-4660)."""
    op = "kv_copy_paged_rows_multi_pool"
    if direction not in ("H2D", "D2H"):
        raise ValueError(f"kv_copy_paged_rows_multi_pool: direction must be 'H2D' or 'D2H', got {direction!r}")
    if not isinstance(pools, (list, tuple)) or len(pools) == 0:
        raise ValueError("kv_copy_paged_rows_multi_pool: pools must be a non-empty list of PoolSpec")
    for pool_idx, pool in enumerate(pools):
        if not isinstance(pool, PoolSpec):
            raise TypeError(f"kv_copy_paged_rows_multi_pool: pools[{pool_idx}] must be PoolSpec")
        item_bytes = _validate_layer_table(pool.src_ptrs, pool.dst_ptrs, indices, indices,
                                           name=f"kv_copy_paged_rows_multi_pool[pool{pool_idx}]")
        if pool.item_bytes != item_bytes:
            raise ValueError(
                f"kv_copy_paged_rows_multi_pool: pools[{pool_idx}].item_bytes={pool.item_bytes} "
                f"!= tensor row width {item_bytes}")
    for pool in pools:
        shapes = {(int(s.shape[0]), int(d.shape[0])) for s, d in zip(pool.src_ptrs, pool.dst_ptrs)}
        if len(shapes) == 1:
            _copy_byte_rows(op, list(pool.src_ptrs), list(pool.dst_ptrs), indices, indices, pool.item_bytes)
        else:
            for s, d in zip(pool.src_ptrs, pool.dst_ptrs):
                _copy_byte_rows(op, [s], [d], indices, indices, pool.item_bytes)
    _emit(op, pools[0].dst_ptrs[0], f"gfx950 multi-pool byte-row copy ({len(pools)} pools, direction={direction})")


def clear_dsv4_ptr_table_cache() -> None:
    """The HIP backend passes plane pointers by value per launch; nothing is cached."""


# ---------------------------------------------------------------------------
# Transfer telemetry (reference :4663-4736)
# ---------------------------------------------------------------------------

_stats_lock = threading.Lock()
_stats: dict = {
    "pinned_calls": 0,
    "unpinned_calls": 0,
    "pinned_bytes": 0,
    "unpinned_bytes": 0,
    "pinned_ns_total": 0,
    "unpinned_ns_total": 0,
}


def kv_transfer_stats() -> dict:
    """Snapshot of byte-row copy telemetry: call counts, bytes and host-side ns."""
    with _stats_lock:
        return dict(_stats)


def reset_kv_transfer_stats() -> None:
    with _stats_lock:
        for key in _stats:
            _stats[key] = 0


def _record_copy_stats(moved: int, elapsed_ns: int) -> None:
    # Device-resident copies count as pinned (no pageable host side).
    with _stats_lock:
        _stats["pinned_calls"] += 1
        _stats["pinned_bytes"] += moved
        _stats["pinned_ns_total"] += elapsed_ns


__all__ = [
    "BuildResult",
    "build_native_kv_transfer",
    "build_native_fp8_kv_cache",
    "is_native_kv_transfer_available",
    "is_native_fp8_kv_cache_available",
    "is_native_fp8_kv_vectorized_available",
    "native_kv_transfer_abi_version",
    "native_fp8_kv_cache_abi_version",
    "kv_paged_to_linear",
    "kv_paged_fp8_to_linear",
    "kv_paged_fp8_to_linear_multi_layer",
    "kv_paged_fp8_to_merged_linear",
    "kv_paged_fp8_to_merged_linear_multi_layer",
    "kv_paged_to_linear_multi_layer",
    "kv_linear_to_paged",
    "kv_linear_to_paged_fp8",
    "kv_linear_to_paged_fp8_multi_layer",
    "kv_merged_linear_to_paged_fp8",
    "kv_merged_linear_to_paged_fp8_multi_layer",
    "kv_linear_to_paged_multi_layer",
    "kv_paged_to_merged_linear",
    "kv_paged_to_merged_linear_multi_layer",
    "kv_merged_linear_to_paged",
    "kv_merged_linear_to_paged_multi_layer",
    "kv_paged_to_mla_linear",
    "kv_mla_linear_to_paged",
    "kv_paged_to_mla_linear_multi_layer",
    "kv_mla_linear_to_paged_multi_layer",
    "kv_copy_paged_rows",
    "kv_copy_paged_rows_layer_table",
    "kv_copy_paged_rows_multi_pool",
    "kv_load_and_reshape_flash",
    "kv_reshape_and_cache_back_flash",
    "kv_load_and_dequantize_fp8_flash",
    "kv_triton_indexed_to_dense",
    "kv_copy_paged_blocks",
    "kv_copy_paged_blocks_fp8",
    "kv_cachegen_encode",
    "kv_cachegen_decode",
    "InterleavedFp8Layout",
    "PoolSpec",
    "clear_dsv4_ptr_table_cache",
    "kv_transfer_stats",
    "reset_kv_transfer_stats",
]
