"""LMCache / SGLang-MP KV converters on MI355X (ROCm HIP backend).

Entry points, argument orders, validation messages and the ``True`` return
value follow the reference module ``musa_aiter/ops/lmcache_kv_transfer.py``
(0.5.0).  Supported cache layouts:

- SGLang-MP split caches ``[[K_0..K_{NL-1}], [V_0..V_{NL-1}]]``, each
  ``[NB, BS, NH, HS]`` <-> LMCache ``[2, NL, T, NH*HS]`` (reference :176-269);
- LMCache per-layer lists of ``[2, NB, BS, NH, HS]`` (:416-460);
- the legacy 6-D cache ``[NL, 2, NB, BS, NH, HS]`` (:51-115);
- MLA caches ``[NL, NB, BS, HS]`` <-> ``[NL, T, HS]`` (:118-151) and MLA
  per-layer lists ``[NB, BS, HS]`` <-> ``[1, NL, T, HS]`` (:272-502).

Gathers overwrite the whole buffer: rows of skipped tokens (slot < 0) and
rows past the slot count are zero.  Scatters read ``memory[:, :, skip +
t]`` and leave caches untouched for skipped tokens; duplicate slots keep the
last token.  Every call is one (or, past 128 planes, a few) HIP launches on
the current stream; non-contiguous LMCache buffers are addressed through
their strides.  Slot bounds are only checked for host-resident slot
tensors, like the reference; device slots outside the cache are skipped by
the kernel, which avoids a device-to-host sync per chunk.
"""

from __future__ import annotations

import ctypes
import os
import sys
import time
from array import array
from typing import Any

import torch

from musa_aiter.dispatch import DispatchRecord, emit, env_bytes, trace_enabled
from musa_aiter.ops import _hip
from musa_aiter.ops.native_gate import native_requested

_LMCACHE_KV_TRANSFER_ABI_VERSION = 1
_ELT = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}
BACKEND = _hip.BACKEND


def native_lmcache_kv_transfer_abi_version() -> int:
    return _LMCACHE_KV_TRANSFER_ABI_VERSION


def clear_native_lmcache_kv_transfer_cache() -> None:
    """Symbols are bound once per process by the HIP loader; nothing to clear."""


def is_native_lmcache_kv_transfer_available() -> bool:
    return _hip.is_available()


def is_native_lmcache_two_x_nl_kv_transfer_available() -> bool:
    return _hip.is_available()


def _native_requested() -> bool:
    return native_requested("MUSA_AITER_NATIVE_LMCACHE_KV_TRANSFER", "LMCACHE_MUSA_NATIVE_KV_TRANSFER",
                            "MUSA_AITER_NATIVE_KV_TRANSFER")


_UNSET = b"\0"  # no environment value can hold a NUL byte


def _timing_enabled() -> bool:
    value = env_bytes(b"MUSA_AITER_LMCACHE_PY_TIMING", _UNSET)
    if value == _UNSET:
        value = env_bytes(b"MUSA_AITER_LMCACHE_TIMING", b"0")
    return value == b"1"


def _log_timing(op: str, elapsed_us: float, **fields: Any) -> None:
    if not _timing_enabled():
        return
    suffix = " ".join(f"{key}={value}" for key, value in fields.items())
    print(f"[musa_aiter_lmcache_py_timing] op={op} elapsed_us={elapsed_us:.3f} {suffix}", file=sys.stderr)


def _emit(op: str, tensor: torch.Tensor, reason: str) -> None:
    if not trace_enabled():
        return
    emit(DispatchRecord(op, BACKEND, str(tensor.device), str(tensor.dtype), reason))


# ---------------------------------------------------------------------------
# Contracts (reference :297-545)
# ---------------------------------------------------------------------------


def _slot_values(slot_mapping: torch.Tensor) -> list[int]:
    return [int(v) for v in slot_mapping.detach().cpu().reshape(-1).tolist()]


def _validate_slots(slot_mapping: torch.Tensor, *, num_tokens: int, num_blocks: int, block_size: int) -> None:
    if slot_mapping.dim() != 1:
        raise ValueError("LMCache slot_mapping rank must be 1")
    if int(slot_mapping.numel()) != num_tokens:
        raise ValueError("LMCache slot_mapping length must equal num_tokens")
    if slot_mapping.device.type != "cpu":
        return
    max_slot = num_blocks * block_size
    if slot_mapping.numel() and int(slot_mapping.max()) >= max_slot:
        bad = next(s for s in _slot_values(slot_mapping) if s >= max_slot)
        raise ValueError(f"LMCache slot_mapping value out of range: slot={bad} max={max_slot - 1}")


def _validate_non_mla_contract(kv_buffer: torch.Tensor, paged_kv_cache: torch.Tensor,
                               slot_mapping: torch.Tensor) -> None:
    if kv_buffer.dim() != 4:
        raise ValueError("LMCache non-MLA kv_buffer rank must be 4: [2, NL, T, NH*HS]")
    if paged_kv_cache.dim() != 6:
        raise ValueError("LMCache non-MLA paged_kv_cache rank must be 6: [NL, 2, NB, BS, NH, HS]")
    if int(kv_buffer.shape[0]) != 2 or int(paged_kv_cache.shape[1]) != 2:
        raise ValueError("LMCache non-MLA layout requires K/V axis size 2")
    _, num_layers, num_tokens, hidden = map(int, kv_buffer.shape)
    cache_layers, _, num_blocks, block_size, num_heads, head_size = map(int, paged_kv_cache.shape)
    if num_layers != cache_layers:
        raise ValueError("LMCache non-MLA layer count mismatch")
    if hidden != num_heads * head_size:
        raise ValueError("LMCache non-MLA hidden size must equal num_heads * head_size")
    _validate_slots(slot_mapping, num_tokens=num_tokens, num_blocks=num_blocks, block_size=block_size)


def _validate_mla_contract(kv_buffer: torch.Tensor, paged_kv_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    if kv_buffer.dim() != 3:
        raise ValueError("LMCache MLA kv_buffer rank must be 3: [NL, T, HS]")
    if paged_kv_cache.dim() != 4:
        raise ValueError("LMCache MLA paged_kv_cache rank must be 4: [NL, NB, BS, HS]")
    num_layers, num_tokens, hidden = map(int, kv_buffer.shape)
    cache_layers, num_blocks, block_size, cache_hidden = map(int, paged_kv_cache.shape)
    if num_layers != cache_layers:
        raise ValueError("LMCache MLA layer count mismatch")
    if hidden != cache_hidden:
        raise ValueError("LMCache MLA hidden size mismatch")
    _validate_slots(slot_mapping, num_tokens=num_tokens, num_blocks=num_blocks, block_size=block_size)


def _contains_nested_cache_list(kvcaches: list[Any]) -> bool:
    return any(isinstance(axis_or_tensor, list) for axis_or_tensor in kvcaches)


def _validate_two_x_nl_contract(memory_tensor: torch.Tensor, kvcaches: list[list[torch.Tensor]],
                                slot_mapping: torch.Tensor, skip_prefix_n_tokens: int, block_size: int,
                                num_heads: int, head_size: int) -> tuple[int, bytes]:
    """The reference's 2 x NL contract (lmcache_kv_transfer.py:323-413).  Returns, for the caches in
    [K layers, V layers] order, the index of the first non-contiguous one (-1 if none) and their
    addresses packed as uint64, from one pass of the host module over the 2 x NL tensors."""
    name = "LMCache TWO_X_NL_X_NB_BS_NH_HS"
    if memory_tensor.dim() != 4 or int(memory_tensor.shape[0]) != 2:
        raise ValueError(f"{name} memory_tensor must be [2, NL, T, NH*HS]")
    if len(kvcaches) != 2 or not all(isinstance(axis, list) for axis in kvcaches):
        raise ValueError(f"{name} cache must be [K_layers, V_layers]")
    if not kvcaches[0] or len(kvcaches[0]) != len(kvcaches[1]):
        raise ValueError(f"{name} K/V layer lists must be non-empty and have equal length")
    num_layers = len(kvcaches[0])
    if int(memory_tensor.shape[1]) != num_layers:
        raise ValueError(f"{name} layer count mismatch")
    if min(block_size, num_heads, head_size) <= 0:
        raise ValueError(f"{name} block_size, num_heads, and head_size must be positive")
    if int(memory_tensor.shape[3]) != num_heads * head_size:
        raise ValueError(f"{name} hidden size must equal num_heads * head_size")
    if memory_tensor.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"{name} supports float16, bfloat16, and float32")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} slot_mapping must be int32 or int64")
    if skip_prefix_n_tokens < 0:
        raise ValueError(f"{name} skip_prefix_n_tokens must be non-negative")
    if skip_prefix_n_tokens + int(slot_mapping.numel()) > int(memory_tensor.shape[2]):
        raise ValueError(f"{name} transfer range exceeds memory_tensor token extent")
    first = kvcaches[0][0]
    if not isinstance(first, torch.Tensor) or first.dim() != 4:
        raise ValueError(f"{name} each cache tensor must be [NB, BS, NH, HS]")
    num_blocks = int(first.shape[0])
    expected = (num_blocks, block_size, num_heads, head_size)
    if num_blocks <= 0:
        raise ValueError(f"{name} num_blocks must be positive")
    # Per cache, in [K layers, V layers] order: type and shape, then dtype, then device.
    h = _hip.host()
    status, index, noncontig, packed = h.check_tensors(kvcaches[0] + kvcaches[1], expected, memory_tensor)
    if status != h.OK:
        kv_axis, layer = divmod(index, num_layers)
        if status == h.SHAPE:
            raise ValueError(f"{name} cache[{kv_axis}][{layer}] must have shape {expected}")
        if status == h.DTYPE:
            raise ValueError(f"{name} cache dtype must match memory_tensor")
        raise ValueError(f"{name} caches and memory_tensor must share a device")
    if slot_mapping.device != memory_tensor.device:
        raise ValueError(f"{name} slot_mapping and data tensors must share a device")
    _validate_slots(slot_mapping, num_tokens=int(slot_mapping.numel()), num_blocks=num_blocks, block_size=block_size)
    return noncontig, packed


def _fast_cache_list(kvcaches: list[torch.Tensor], rank: int, nb_dim: int, shape_of, memory_tensor: torch.Tensor):
    """Packed addresses of a per-layer cache list when every cache has the list's shape
    (``shape_of(num_blocks)``), memory_tensor's dtype and device and is contiguous, from one pass of
    the host module; None otherwise, and the caller runs its per-cache checks, which raise the
    reference's error for the first offending cache."""
    if not isinstance(kvcaches, list) or not kvcaches:
        return None
    first = kvcaches[0]
    if not isinstance(first, torch.Tensor) or first.dim() != rank:
        return None
    h = _hip.host()
    status, _, noncontig, packed = h.check_tensors(kvcaches, shape_of(int(first.shape[nb_dim])), memory_tensor)
    return packed if status == h.OK and noncontig < 0 else None


def _validate_non_mla_list_contract(memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor],
                                    slot_mapping: torch.Tensor, block_size: int, num_heads: int,
                                    head_size: int, *, per_cache: bool = True) -> None:
    if memory_tensor.dim() != 4 or int(memory_tensor.shape[0]) != 2:
        raise ValueError("LMCache list non-MLA memory_tensor rank must be 4: [2, NL, T, NH*HS]")
    if len(kvcaches) != int(memory_tensor.shape[1]):
        raise ValueError("LMCache list non-MLA layer count mismatch")
    if int(memory_tensor.shape[3]) != num_heads * head_size:
        raise ValueError("LMCache list non-MLA hidden size must equal num_heads * head_size")
    if not kvcaches:
        raise ValueError("LMCache list non-MLA kvcaches must not be empty")
    num_blocks = int(kvcaches[0].shape[1])
    for kvcache in (kvcaches if per_cache else ()):
        if (kvcache.dim() != 5 or int(kvcache.shape[0]) != 2 or int(kvcache.shape[2]) != block_size
                or int(kvcache.shape[3]) != num_heads or int(kvcache.shape[4]) != head_size):
            raise ValueError("LMCache list non-MLA kvcache rank must be 5: [2, NB, BS, NH, HS]")
        if int(kvcache.shape[1]) != num_blocks:
            raise ValueError("LMCache list non-MLA num_blocks mismatch")
    _validate_slots(slot_mapping, num_tokens=int(slot_mapping.numel()), num_blocks=num_blocks, block_size=block_size)


def _validate_mla_list_contract(memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor], slot_mapping: torch.Tensor,
                                block_size: int, head_size: int, *, per_cache: bool = True) -> None:
    if memory_tensor.dim() != 4 or int(memory_tensor.shape[0]) != 1:
        raise ValueError("LMCache list MLA memory_tensor rank must be 4: [1, NL, T, HS]")
    if len(kvcaches) != int(memory_tensor.shape[1]):
        raise ValueError("LMCache list MLA layer count mismatch")
    if not kvcaches:
        raise ValueError("LMCache list MLA kvcaches must not be empty")
    num_blocks = int(kvcaches[0].shape[0])
    for kvcache in (kvcaches if per_cache else ()):
        if kvcache.dim() != 3 or int(kvcache.shape[1]) != block_size or int(kvcache.shape[2]) != head_size:
            raise ValueError("LMCache list MLA kvcache rank must be 3: [NB, BS, HS]")
        if int(kvcache.shape[0]) != num_blocks:
            raise ValueError("LMCache list MLA num_blocks mismatch")
    _validate_slots(slot_mapping, num_tokens=int(slot_mapping.numel()), num_blocks=num_blocks, block_size=block_size)


# ---------------------------------------------------------------------------
# Launch helpers
# ---------------------------------------------------------------------------


def _elt(op: str, *tensors: torch.Tensor) -> int:
    dtype = tensors[0].dtype
    for t in tensors:
        if t.dtype not in _ELT:
            raise ValueError(f"{op}: the {BACKEND} backend moves float32, float16 and bfloat16 KV data, got {t.dtype}")
        if t.dtype != dtype:
            raise ValueError(f"{op}: cache dtype must match memory_tensor")
    return _ELT[dtype]


def _same_device(op: str, device: torch.device, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device != device:
            raise ValueError(f"{op}: caches, memory_tensor and slot_mapping must share a device")
    if device.type != "cuda":
        raise RuntimeError(
            f"{op}: the {BACKEND} backend moves KV data with gfx950 kernels and needs tensors on a ROCm GPU device "
            f"(got {device})")


def _device_slots(slot_mapping: torch.Tensor, device: torch.device) -> torch.Tensor:
    return slot_mapping.to(device=device, dtype=torch.long).contiguous()


class _Buffer:
    """An LMCache buffer [A, L, M, H] addressed by plane (axis, layer) with a token stride.

    The innermost (hidden) dimension must be contiguous; otherwise the kernel
    runs on a contiguous copy that is written back after a gather.
    """

    def __init__(self, t: torch.Tensor, *, writable: bool, initialise: bool):
        self.user = t
        if t.stride(-1) == 1 or t.shape[-1] == 1:
            self.work = t
        elif writable:
            self.work = torch.empty(t.shape, dtype=t.dtype, device=t.device)
            if initialise:
                self.work.copy_(t)
        else:
            self.work = t.contiguous()
        self.elt = t.element_size()
        # Read once: plane() runs for every (axis, layer) of every call.
        w = self.work
        self._base = w.data_ptr()
        self._axis_bytes = w.stride(0) * self.elt
        self._layer_bytes = w.stride(1) * self.elt

    def plane(self, axis: int, layer: int) -> int:
        return self._base + axis * self._axis_bytes + layer * self._layer_bytes

    def all_planes(self, axes: int, layers: int):
        """Every (axis, layer) plane in row-major order, as a ctypes uint64 array."""
        return _hip.u64_packed(_hip.host().strided_table(self._base, self._axis_bytes, axes, self._layer_bytes,
                                                           layers))

    @property
    def token_stride_bytes(self) -> int:
        w = self.work
        return (w.stride(2) if w.shape[2] > 1 else w.shape[3]) * self.elt

    def finish(self) -> None:
        if self.work is not self.user:
            self.user.copy_(self.work)


def _buf_planes(buf: _Buffer, buf_planes):
    """Plane addresses of ``buf``: a list of (axis, layer) pairs, or a ready ctypes array."""
    if isinstance(buf_planes, list):
        return [buf.plane(a, l) for a, l in buf_planes]
    return buf_planes


def _rows_gather(op: str, *, device: torch.device, cache_planes, buf: _Buffer,
                 buf_planes, slots: torch.Tensor, num_tokens: int, memory_tokens: int,
                 slot_rows: int, row_bytes: int, cache_stride: int) -> None:
    _hip.copy_rows(op=op, device=device, src_planes=cache_planes, dst_planes=_buf_planes(buf, buf_planes),
                   num_planes=len(cache_planes), src_idx=slots, dst_idx=None, num_tokens=num_tokens,
                   num_rows_out=memory_tokens, src_rows=slot_rows, dst_rows=memory_tokens, row_bytes=row_bytes,
                   src_stride=cache_stride, dst_stride=buf.token_stride_bytes, zero_invalid=True)


def _rows_scatter(op: str, *, device: torch.device, cache_planes, buf: _Buffer,
                  buf_planes, slots: torch.Tensor, num_tokens: int, memory_tokens: int,
                  skip: int, slot_rows: int, row_bytes: int, cache_stride: int) -> None:
    _hip.copy_rows(op=op, device=device, src_planes=_buf_planes(buf, buf_planes), dst_planes=cache_planes,
                   num_planes=len(cache_planes), src_idx=None, dst_idx=slots, num_tokens=num_tokens,
                   num_rows_out=num_tokens, src_offset=skip, src_rows=memory_tokens, dst_rows=slot_rows,
                   row_bytes=row_bytes, src_stride=buf.token_stride_bytes, dst_stride=cache_stride,
                   zero_invalid=False)


def _contig_cache(op: str, cache: torch.Tensor) -> torch.Tensor:
    if not cache.is_contiguous():
        raise ValueError(f"{op}: paged caches must be contiguous tensors")
    return cache


# ---------------------------------------------------------------------------
# SGLang MP 2 x NL (reference :176-269)
# ---------------------------------------------------------------------------


_COPY_ROWS_ENTRY: list[int] = []


def _two_x_nl_fast(op: str, kvcaches, memory_tensor, slot_mapping, skip: int, block_size: int, num_heads: int,
                   head_size: int, scatter: bool) -> bool:
    """One 2 x NL call checked and launched by the host module in one C++ pass (about half the host time
    of the checks below, which matters for back-to-back 256-token chunks).  False, with nothing launched,
    when the arguments are not all ones that path takes as they are: the caller then runs the reference's
    checks, which raise its errors."""
    if not (type(memory_tensor) is torch.Tensor and memory_tensor.is_cuda and type(kvcaches) is list
            and len(kvcaches) == 2 and type(kvcaches[0]) is list and kvcaches[0]
            and type(kvcaches[0][0]) is torch.Tensor and kvcaches[0][0].dim() == 4):
        return False
    h = _hip.host()
    if not _COPY_ROWS_ENTRY:
        _COPY_ROWS_ENTRY.append(ctypes.cast(_hip.fn("musa_aiter_hip_copy_rows_packed"), ctypes.c_void_p).value)
    index = torch._C._cuda_getDevice()
    stream = torch._C._cuda_getCurrentRawStream(index)
    claims, keep = 0, None
    if scatter:
        if memory_tensor.device.index != index:
            return False
        claims, keep = _hip.claims_for(memory_tensor.device, ctypes.c_void_p(stream),
                                       int(kvcaches[0][0].shape[0]) * int(block_size))
    rc = h.two_x_nl_rows(kvcaches, memory_tensor, slot_mapping, int(skip), int(block_size), int(num_heads),
                         int(head_size), bool(scatter), _COPY_ROWS_ENTRY[0], claims, stream, index)
    del keep
    if rc < 0:
        return False
    _hip.check(rc, op)
    return True


def lmcache_kv_buffer_to_paged_two_x_nl(memory_tensor: torch.Tensor, kvcaches: list[list[torch.Tensor]],
                                        slot_mapping: torch.Tensor, skip_prefix_n_tokens: int, block_size: int,
                                        num_heads: int, head_size: int) -> bool:
    """Scatter ``memory[:, :, skip:skip+T]`` into SGLang-MP ``2 x NL x [NB, BS, NH, HS]`` caches, one launch."""
    op = "lmcache_kv_buffer_to_paged_two_x_nl"
    start = time.perf_counter()
    if _two_x_nl_fast(op, kvcaches, memory_tensor, slot_mapping, skip_prefix_n_tokens, block_size, num_heads,
                      head_size, True):
        _emit(op, memory_tensor, f"gfx950 row scatter, {2 * len(kvcaches[0])} planes in one launch")
        _log_timing(op, (time.perf_counter() - start) * 1e6, tokens=int(slot_mapping.numel()),
                    layers=len(kvcaches[0]))
        return True
    noncontig, packed = _validate_two_x_nl_contract(memory_tensor, kvcaches, slot_mapping, skip_prefix_n_tokens,
                                                    block_size, num_heads, head_size)
    start = time.perf_counter()
    device = memory_tensor.device
    # The contract has checked every cache's dtype and device against memory_tensor.
    _same_device(op, device, slot_mapping)
    num_layers = len(kvcaches[0])
    num_tokens = int(slot_mapping.numel())
    elt = _elt(op, memory_tensor)
    row = num_heads * head_size * elt
    buf = _Buffer(memory_tensor, writable=False, initialise=False)
    if noncontig >= 0:
        raise ValueError(f"{op}: paged caches must be contiguous tensors")
    _rows_scatter(op, device=device, cache_planes=_hip.u64_packed(packed), buf=buf,
                  buf_planes=buf.all_planes(2, num_layers), slots=_device_slots(slot_mapping, device),
                  num_tokens=num_tokens, memory_tokens=int(memory_tensor.shape[2]), skip=int(skip_prefix_n_tokens),
                  slot_rows=int(kvcaches[0][0].shape[0]) * block_size, row_bytes=row, cache_stride=row)
    _emit(op, memory_tensor, f"gfx950 row scatter, {2 * num_layers} planes in one launch")
    _log_timing(op, (time.perf_counter() - start) * 1e6, tokens=num_tokens, layers=num_layers)
    return True


def lmcache_kv_paged_to_buffer_two_x_nl(kvcaches: list[list[torch.Tensor]], memory_tensor: torch.Tensor,
                                        slot_mapping: torch.Tensor, block_size: int, num_heads: int,
                                        head_size: int) -> bool:
    """Gather SGLang-MP caches into ``[2, NL, T, NH*HS]``; the whole buffer is overwritten (zeros where skipped)."""
    op = "lmcache_kv_paged_to_buffer_two_x_nl"
    start = time.perf_counter()
    if _two_x_nl_fast(op, kvcaches, memory_tensor, slot_mapping, 0, block_size, num_heads, head_size, False):
        _emit(op, memory_tensor, f"gfx950 row gather, {2 * len(kvcaches[0])} planes in one launch")
        _log_timing(op, (time.perf_counter() - start) * 1e6, tokens=int(slot_mapping.numel()),
                    layers=len(kvcaches[0]))
        return True
    noncontig, packed = _validate_two_x_nl_contract(memory_tensor, kvcaches, slot_mapping, 0, block_size, num_heads,
                                                    head_size)
    start = time.perf_counter()
    device = memory_tensor.device
    # The contract has checked every cache's dtype and device against memory_tensor.
    _same_device(op, device, slot_mapping)
    num_layers = len(kvcaches[0])
    num_tokens = int(slot_mapping.numel())
    elt = _elt(op, memory_tensor)
    row = num_heads * head_size * elt
    buf = _Buffer(memory_tensor, writable=True, initialise=False)
    if noncontig >= 0:
        raise ValueError(f"{op}: paged caches must be contiguous tensors")
    _rows_gather(op, device=device, cache_planes=_hip.u64_packed(packed), buf=buf,
                 buf_planes=buf.all_planes(2, num_layers), slots=_device_slots(slot_mapping, device),
                 num_tokens=num_tokens, memory_tokens=int(memory_tensor.shape[2]),
                 slot_rows=int(kvcaches[0][0].shape[0]) * block_size, row_bytes=row, cache_stride=row)
    buf.finish()
    _emit(op, memory_tensor, f"gfx950 row gather, {2 * num_layers} planes in one launch")
    _log_timing(op, (time.perf_counter() - start) * 1e6, tokens=num_tokens, layers=num_layers)
    return True


# ---------------------------------------------------------------------------
# Per-layer list caches [2, NB, BS, NH, HS] (reference :416-460)
# ---------------------------------------------------------------------------


def _list_planes(kvcaches: list[torch.Tensor], op: str) -> tuple[list[int], list[tuple[int, int]]]:
    cache_planes, buf_planes = [], []
    for axis in range(2):
        for layer, kvcache in enumerate(kvcaches):
            c = _contig_cache(op, kvcache)
            cache_planes.append(c[axis].data_ptr())
            buf_planes.append((axis, layer))
    return cache_planes, buf_planes


def _list_cache_planes(op: str, kvcaches: list[torch.Tensor], packed, memory_tensor: torch.Tensor,
                       slot_mapping: torch.Tensor, buf: "_Buffer"):
    """(cache planes, buffer planes, element bytes) of a [2, NB, BS, NH, HS] cache list: K planes of
    every layer, then V planes.  With ``packed`` (every cache already checked by the host module)
    the planes come from the packed addresses; otherwise the reference's device, dtype and
    contiguity checks run cache by cache."""
    device = memory_tensor.device
    if packed is None:
        _same_device(op, device, slot_mapping, *kvcaches)
        elt = _elt(op, memory_tensor, *kvcaches)
        cache_planes, buf_planes = _list_planes(kvcaches, op)
        return cache_planes, buf_planes, elt
    _same_device(op, device, slot_mapping)
    elt = _elt(op, memory_tensor)
    plane_bytes = kvcaches[0][0].numel() * elt
    ptrs = array("Q", packed)
    planes = array("Q", ptrs)
    planes.extend(p + plane_bytes for p in ptrs)
    return _hip.u64_packed(planes.tobytes()), buf.all_planes(2, len(kvcaches)), elt


def _lmcache_kv_buffer_to_paged_list(memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor],
                                     slot_mapping: torch.Tensor, skip_prefix_n_tokens: int, block_size: int,
                                     num_heads: int, head_size: int) -> bool:
    op = "lmcache_kv_buffer_to_paged"
    packed = _fast_cache_list(kvcaches, 5, 1, lambda nb: (2, nb, block_size, num_heads, head_size), memory_tensor)
    _validate_non_mla_list_contract(memory_tensor, kvcaches, slot_mapping, block_size, num_heads, head_size,
                                    per_cache=packed is None)
    device = memory_tensor.device
    buf = _Buffer(memory_tensor, writable=False, initialise=False)
    cache_planes, buf_planes, elt = _list_cache_planes(op, kvcaches, packed, memory_tensor, slot_mapping, buf)
    row = num_heads * head_size * elt
    _rows_scatter(op, device=device, cache_planes=cache_planes, buf=buf, buf_planes=buf_planes,
                  slots=_device_slots(slot_mapping, device), num_tokens=int(slot_mapping.numel()),
                  memory_tokens=int(memory_tensor.shape[2]), skip=int(skip_prefix_n_tokens),
                  slot_rows=int(kvcaches[0].shape[1]) * block_size, row_bytes=row, cache_stride=row)
    _emit(op, memory_tensor, f"gfx950 list-cache row scatter ({len(kvcaches)} layers)")
    return True


def _lmcache_kv_paged_to_buffer_list(kvcaches: list[torch.Tensor], memory_tensor: torch.Tensor,
                                     slot_mapping: torch.Tensor, block_size: int, num_heads: int,
                                     head_size: int) -> bool:
    op = "lmcache_kv_paged_to_buffer"
    packed = _fast_cache_list(kvcaches, 5, 1, lambda nb: (2, nb, block_size, num_heads, head_size), memory_tensor)
    _validate_non_mla_list_contract(memory_tensor, kvcaches, slot_mapping, block_size, num_heads, head_size,
                                    per_cache=packed is None)
    device = memory_tensor.device
    buf = _Buffer(memory_tensor, writable=True, initialise=False)
    cache_planes, buf_planes, elt = _list_cache_planes(op, kvcaches, packed, memory_tensor, slot_mapping, buf)
    row = num_heads * head_size * elt
    _rows_gather(op, device=device, cache_planes=cache_planes, buf=buf, buf_planes=buf_planes,
                 slots=_device_slots(slot_mapping, device), num_tokens=int(slot_mapping.numel()),
                 memory_tokens=int(memory_tensor.shape[2]), slot_rows=int(kvcaches[0].shape[1]) * block_size,
                 row_bytes=row, cache_stride=row)
    buf.finish()
    _emit(op, memory_tensor, f"gfx950 list-cache row gather ({len(kvcaches)} layers)")
    return True


# ---------------------------------------------------------------------------
# Dispatching entry points (reference :51-173)
# ---------------------------------------------------------------------------


def lmcache_kv_buffer_to_paged(kv_buffer: torch.Tensor,
                               paged_kv_cache: torch.Tensor | list[torch.Tensor] | list[list[torch.Tensor]],
                               slot_mapping: torch.Tensor, *args: Any) -> bool:
    """Scatter an LMCache non-MLA chunk into a legacy 6-D, list or SGLang-MP nested-list cache."""
    if isinstance(paged_kv_cache, list):
        if len(args) != 4:
            raise TypeError(
                "LMCache list-cache buffer_to_paged expects skip_prefix_n_tokens, block_size, num_heads, head_size")
        skip_prefix_n_tokens, block_size, num_heads, head_size = map(int, args)
        if _contains_nested_cache_list(paged_kv_cache):
            return lmcache_kv_buffer_to_paged_two_x_nl(kv_buffer, paged_kv_cache, slot_mapping, skip_prefix_n_tokens,
                                                       block_size, num_heads, head_size)
        return _lmcache_kv_buffer_to_paged_list(kv_buffer, paged_kv_cache, slot_mapping, skip_prefix_n_tokens,
                                                block_size, num_heads, head_size)
    op = "lmcache_kv_buffer_to_paged"
    _validate_non_mla_contract(kv_buffer, paged_kv_cache, slot_mapping)
    device = kv_buffer.device
    _same_device(op, device, paged_kv_cache, slot_mapping)
    elt = _elt(op, kv_buffer, paged_kv_cache)
    num_layers, _, num_blocks, block_size, num_heads, head_size = map(int, paged_kv_cache.shape)
    row = num_heads * head_size * elt
    cache = _contig_cache(op, paged_kv_cache)
    cache_planes = [cache[l, a].data_ptr() for a in range(2) for l in range(num_layers)]
    buf_planes = [(a, l) for a in range(2) for l in range(num_layers)]
    buf = _Buffer(kv_buffer, writable=False, initialise=False)
    _rows_scatter(op, device=device, cache_planes=cache_planes, buf=buf, buf_planes=buf_planes,
                  slots=_device_slots(slot_mapping, device), num_tokens=int(slot_mapping.numel()),
                  memory_tokens=int(kv_buffer.shape[2]), skip=0, slot_rows=num_blocks * block_size, row_bytes=row,
                  cache_stride=row)
    _emit(op, kv_buffer, "gfx950 6-D cache row scatter")
    return True


def lmcache_paged_to_kv_buffer(paged_kv_cache: torch.Tensor, kv_buffer: torch.Tensor,
                               slot_mapping: torch.Tensor) -> bool:
    """Gather a legacy 6-D ``[NL, 2, NB, BS, NH, HS]`` cache into ``[2, NL, T, NH*HS]`` (zeros where skipped)."""
    op = "lmcache_paged_to_kv_buffer"
    _validate_non_mla_contract(kv_buffer, paged_kv_cache, slot_mapping)
    device = kv_buffer.device
    _same_device(op, device, paged_kv_cache, slot_mapping)
    elt = _elt(op, kv_buffer, paged_kv_cache)
    num_layers, _, num_blocks, block_size, num_heads, head_size = map(int, paged_kv_cache.shape)
    row = num_heads * head_size * elt
    cache = paged_kv_cache if paged_kv_cache.is_contiguous() else paged_kv_cache.contiguous()
    cache_planes = [cache[l, a].data_ptr() for a in range(2) for l in range(num_layers)]
    buf_planes = [(a, l) for a in range(2) for l in range(num_layers)]
    buf = _Buffer(kv_buffer, writable=True, initialise=False)
    _rows_gather(op, device=device, cache_planes=cache_planes, buf=buf, buf_planes=buf_planes,
                 slots=_device_slots(slot_mapping, device), num_tokens=int(slot_mapping.numel()),
                 memory_tokens=int(kv_buffer.shape[2]), slot_rows=num_blocks * block_size, row_bytes=row,
                 cache_stride=row)
    buf.finish()
    _emit(op, kv_buffer, "gfx950 6-D cache row gather")
    return True


def lmcache_kv_paged_to_buffer(kvcaches: list[torch.Tensor] | list[list[torch.Tensor]], memory_tensor: torch.Tensor,
                               slot_mapping: torch.Tensor, block_size: int, num_heads: int, head_size: int) -> bool:
    """Gather LMCache list or SGLang-MP nested-list caches into a contiguous buffer."""
    if _contains_nested_cache_list(kvcaches):
        return lmcache_kv_paged_to_buffer_two_x_nl(kvcaches, memory_tensor, slot_mapping, block_size, num_heads,
                                                   head_size)
    return _lmcache_kv_paged_to_buffer_list(kvcaches, memory_tensor, slot_mapping, block_size, num_heads, head_size)


# ---------------------------------------------------------------------------
# MLA (reference :118-151, :272-294, :463-502)
# ---------------------------------------------------------------------------


def _mla_planes(cache: torch.Tensor, buf: _Buffer, num_layers: int) -> tuple[list[int], list[tuple[int, int]]]:
    return [cache[l].data_ptr() for l in range(num_layers)], [(0, l) for l in range(num_layers)]


class _Buffer3D(_Buffer):
    """An MLA buffer [L, T, D] viewed as [1, L, T, D]."""

    def __init__(self, t: torch.Tensor, *, writable: bool):
        super().__init__(t.unsqueeze(0), writable=writable, initialise=False)
        self.user3 = t

    def finish(self) -> None:
        if self.work is not self.user:
            self.user3.copy_(self.work[0])


def lmcache_kv_buffer_to_paged_mla(kv_buffer: torch.Tensor, paged_kv_cache: torch.Tensor,
                                   slot_mapping: torch.Tensor) -> bool:
    """Scatter ``[NL, T, HS]`` MLA rows into an ``[NL, NB, BS, HS]`` cache."""
    op = "lmcache_kv_buffer_to_paged_mla"
    _validate_mla_contract(kv_buffer, paged_kv_cache, slot_mapping)
    device = kv_buffer.device
    _same_device(op, device, paged_kv_cache, slot_mapping)
    elt = _elt(op, kv_buffer, paged_kv_cache)
    num_layers, num_blocks, block_size, hidden = map(int, paged_kv_cache.shape)
    row = hidden * elt
    cache = _contig_cache(op, paged_kv_cache)
    buf = _Buffer3D(kv_buffer, writable=False)
    cache_planes, buf_planes = _mla_planes(cache, buf, num_layers)
    _rows_scatter(op, device=device, cache_planes=cache_planes, buf=buf, buf_planes=buf_planes,
                  slots=_device_slots(slot_mapping, device), num_tokens=int(slot_mapping.numel()),
                  memory_tokens=int(kv_buffer.shape[1]), skip=0, slot_rows=num_blocks * block_size, row_bytes=row,
                  cache_stride=row)
    _emit(op, kv_buffer, f"gfx950 MLA row scatter ({num_layers} layers)")
    return True


def lmcache_paged_to_kv_buffer_mla(paged_kv_cache: torch.Tensor, kv_buffer: torch.Tensor,
                                   slot_mapping: torch.Tensor) -> bool:
    """Gather an ``[NL, NB, BS, HS]`` MLA cache into ``[NL, T, HS]`` (zeros where skipped)."""
    op = "lmcache_paged_to_kv_buffer_mla"
    _validate_mla_contract(kv_buffer, paged_kv_cache, slot_mapping)
    device = kv_buffer.device
    _same_device(op, device, paged_kv_cache, slot_mapping)
    elt = _elt(op, kv_buffer, paged_kv_cache)
    num_layers, num_blocks, block_size, hidden = map(int, paged_kv_cache.shape)
    row = hidden * elt
    cache = paged_kv_cache if paged_kv_cache.is_contiguous() else paged_kv_cache.contiguous()
    buf = _Buffer3D(kv_buffer, writable=True)
    cache_planes, buf_planes = _mla_planes(cache, buf, num_layers)
    _rows_gather(op, device=device, cache_planes=cache_planes, buf=buf, buf_planes=buf_planes,
                 slots=_device_slots(slot_mapping, device), num_tokens=int(slot_mapping.numel()),
                 memory_tokens=int(kv_buffer.shape[1]), slot_rows=num_blocks * block_size, row_bytes=row,
                 cache_stride=row)
    buf.finish()
    _emit(op, kv_buffer, f"gfx950 MLA row gather ({num_layers} layers)")
    return True


def _lmcache_mla_buffer_to_paged_list(memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor],
                                      slot_mapping: torch.Tensor, skip_prefix_n_tokens: int, block_size: int,
                                      head_size: int) -> bool:
    op = "lmcache_mla_buffer_to_paged"
    packed = _fast_cache_list(kvcaches, 3, 0, lambda nb: (nb, block_size, head_size), memory_tensor)
    _validate_mla_list_contract(memory_tensor, kvcaches, slot_mapping, block_size, head_size,
                                per_cache=packed is None)
    device = memory_tensor.device
    buf = _Buffer(memory_tensor, writable=False, initialise=False)
    if packed is None:
        _same_device(op, device, slot_mapping, *kvcaches)
        elt = _elt(op, memory_tensor, *kvcaches)
        cache_planes = [_contig_cache(op, c).data_ptr() for c in kvcaches]
        buf_planes = [(0, l) for l in range(len(kvcaches))]
    else:
        _same_device(op, device, slot_mapping)
        elt = _elt(op, memory_tensor)
        cache_planes, buf_planes = _hip.u64_packed(packed), buf.all_planes(1, len(kvcaches))
    row = head_size * elt
    _rows_scatter(op, device=device, cache_planes=cache_planes, buf=buf,
                  buf_planes=buf_planes, slots=_device_slots(slot_mapping, device),
                  num_tokens=int(slot_mapping.numel()), memory_tokens=int(memory_tensor.shape[2]),
                  skip=int(skip_prefix_n_tokens), slot_rows=int(kvcaches[0].shape[0]) * block_size, row_bytes=row,
                  cache_stride=row)
    _emit(op, memory_tensor, f"gfx950 MLA list row scatter ({len(kvcaches)} layers)")
    return True


def _lmcache_mla_paged_to_buffer_list(kvcaches: list[torch.Tensor], memory_tensor: torch.Tensor,
                                      slot_mapping: torch.Tensor, block_size: int, head_size: int) -> bool:
    op = "lmcache_mla_paged_to_buffer"
    packed = _fast_cache_list(kvcaches, 3, 0, lambda nb: (nb, block_size, head_size), memory_tensor)
    _validate_mla_list_contract(memory_tensor, kvcaches, slot_mapping, block_size, head_size,
                                per_cache=packed is None)
    device = memory_tensor.device
    buf = _Buffer(memory_tensor, writable=True, initialise=False)
    caches = kvcaches  # keeps contiguous copies alive until the launch
    if packed is None:
        _same_device(op, device, slot_mapping, *kvcaches)
        elt = _elt(op, memory_tensor, *kvcaches)
        caches = [c if c.is_contiguous() else c.contiguous() for c in kvcaches]
        cache_planes = [c.data_ptr() for c in caches]
        buf_planes = [(0, l) for l in range(len(kvcaches))]
    else:
        _same_device(op, device, slot_mapping)
        elt = _elt(op, memory_tensor)
        cache_planes, buf_planes = _hip.u64_packed(packed), buf.all_planes(1, len(kvcaches))
    row = head_size * elt
    _rows_gather(op, device=device, cache_planes=cache_planes, buf=buf,
                 buf_planes=buf_planes, slots=_device_slots(slot_mapping, device),
                 num_tokens=int(slot_mapping.numel()), memory_tokens=int(memory_tensor.shape[2]),
                 slot_rows=int(kvcaches[0].shape[0]) * block_size, row_bytes=row, cache_stride=row)
    buf.finish()
    _emit(op, memory_tensor, f"gfx950 MLA list row gather ({len(kvcaches)} layers)")
    return True


def lmcache_mla_buffer_to_paged(memory_tensor: torch.Tensor, kvcaches: list[torch.Tensor], slot_mapping: torch.Tensor,
                                skip_prefix_n_tokens: int, block_size: int, head_size: int) -> bool:
    """Scatter an LMCache ``[1, NL, T, HS]`` MLA buffer into per-layer ``[NB, BS, HS]`` caches."""
    return _lmcache_mla_buffer_to_paged_list(memory_tensor, kvcaches, slot_mapping, skip_prefix_n_tokens, block_size,
                                             head_size)


def lmcache_mla_paged_to_buffer(kvcaches: list[torch.Tensor], memory_tensor: torch.Tensor, slot_mapping: torch.Tensor,
                                block_size: int, head_size: int) -> bool:
    """Gather per-layer ``[NB, BS, HS]`` MLA caches into an LMCache ``[1, NL, T, HS]`` buffer."""
    return _lmcache_mla_paged_to_buffer_list(kvcaches, memory_tensor, slot_mapping, block_size, head_size)


# ---------------------------------------------------------------------------
# DSV4 strided block transfer (reference :1294-1403; semantics from the kernel text
# csrc/kvcache/kv_transfer_float.mu:3281-3358 since there is no Python reference)
# ---------------------------------------------------------------------------


def lmcache_kv_strided_block_transfer(
    staging: "torch.Tensor | int",
    paged_ptrs: list[int],
    block_ids: torch.Tensor,
    direction: int,
    num_layers: int,
    idx_start: int,
    n_valid: int,
    offset_in_object: int,
    staging_tokens: int,
    block_size: int,
    row_bytes: int,
    paged_block_stride: int,
    mode: int,
    value_bytes: int = 0,
    scale_bytes: int = 0,
) -> bool:
    """Move whole blocks between staging ``[NL, staging_tokens, row_bytes]`` and per-layer pages.

    ``direction`` 0 writes pages from staging, 1 reads pages into staging.
    ``mode`` 0 pages hold plain rows; mode 1 pages hold all value parts then all
    scale parts of a block.  Returns False (nothing launched) for arguments the
    kernel does not accept, like the reference.
    """
    if num_layers <= 0 or num_layers > 128:
        return False
    if n_valid <= 0 or block_size <= 0 or staging_tokens <= 0:
        return False
    if row_bytes <= 0 or row_bytes % 4 != 0:
        return False
    if mode not in (0, 1) or int(direction) not in (0, 1):
        return False
    if mode == 1 and (value_bytes <= 0 or scale_bytes <= 0 or value_bytes % 4 != 0 or scale_bytes % 4 != 0
                      or value_bytes + scale_bytes != row_bytes):
        return False
    if paged_block_stride <= 0:
        return False
    if not isinstance(paged_ptrs, (list, tuple)) or len(paged_ptrs) != num_layers:
        return False
    if not isinstance(block_ids, torch.Tensor):
        return False
    if block_ids.dtype is not torch.int64 or block_ids.device.type != "cuda" or not block_ids.is_contiguous():
        return False
    if idx_start < 0 or idx_start + n_valid > int(block_ids.numel()):
        return False
    staging_ptr = int(staging.data_ptr()) if isinstance(staging, torch.Tensor) else int(staging)
    if staging_ptr <= 0:
        return False
    device = block_ids.device
    ptrs = _hip.u64_array(paged_ptrs)
    with torch.cuda.device(device):
        rc = _hip.fn("lmcache_kv_strided_block_transfer")(
            _hip.ctypes.c_void_p(staging_ptr), ptrs, _hip.ptr(block_ids), int(direction), int(num_layers),
            int(idx_start), int(n_valid), int(offset_in_object), int(staging_tokens), int(block_size),
            int(row_bytes), int(paged_block_stride), int(mode), int(value_bytes), int(scale_bytes),
            _hip.stream_ptr(device))
    _hip.check(rc, "lmcache_kv_strided_block_transfer")
    emit(DispatchRecord("lmcache_kv_strided_block_transfer", BACKEND, str(device), "uint8",
                        f"gfx950 strided block transfer mode={mode} direction={direction}"))
    return True


__all__ = [
    "native_lmcache_kv_transfer_abi_version",
    "clear_native_lmcache_kv_transfer_cache",
    "is_native_lmcache_kv_transfer_available",
    "is_native_lmcache_two_x_nl_kv_transfer_available",
    "lmcache_kv_buffer_to_paged",
    "lmcache_paged_to_kv_buffer",
    "lmcache_kv_buffer_to_paged_mla",
    "lmcache_paged_to_kv_buffer_mla",
    "lmcache_kv_paged_to_buffer",
    "lmcache_kv_buffer_to_paged_two_x_nl",
    "lmcache_kv_paged_to_buffer_two_x_nl",
    "lmcache_mla_buffer_to_paged",
    "lmcache_mla_paged_to_buffer",
    "lmcache_kv_strided_block_transfer",
]
