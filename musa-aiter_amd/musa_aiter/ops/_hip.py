"""ctypes boundary to ``libmusa_aiter_kv_hip.so`` (the gfx950 HIP kernels).

The library is built in-tree by ``musa-aiter_amd/build.py`` into
``musa_aiter/_lib``.  There is no fallback: if the library is missing or a
launch fails, the calling op raises.  torch is imported before the library is
opened so both share torch's HIP runtime (same ``libamdhip64.so.7`` soname),
which keeps torch's stream handles and allocations valid in the kernels.
"""

from __future__ import annotations

import contextlib
import ctypes
import importlib.util
import struct
import sysconfig
import threading
from pathlib import Path

import torch

LIB_NAME = "libmusa_aiter_kv_hip.so"
LIB_PATH = Path(__file__).resolve().parent.parent / "_lib" / LIB_NAME
HOST_PATH = LIB_PATH.parent / ("_kv_host" + sysconfig.get_config_var("EXT_SUFFIX"))
BACKEND = "rocm-hip"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_u64p = ctypes.POINTER(ctypes.c_uint64)

# Generic entry points used by the host layer: name -> argtypes.
_SIGNATURES: dict[str, list] = {
    "musa_aiter_hip_paged_tiles": [
        _i32, _i32, _i32, _i32, _i32,            # scatter, codec, cache_elt, lin_elt, lin_dtype
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # key_cache, value_cache, key_linear, value_linear
        _c_void_p,                               # slot_mapping
        _i64, _i64, _i64, _i64, _i64, _i64,      # layers, tokens, blocks, heads, head_dim, block_size
        _i64, _i64,                              # linear token / layer stride (elements)
        _c_void_p, _c_void_p, _i32,              # k_scale, v_scale, scale_mode
        _i32, _i32, _c_void_p, _c_void_p,        # fill_zeros, dedupe, claims, stream
    ],
    # musa_aiter_hip_paged_tiles without the claims argument (allocation-free entry; tests only).
    "musa_aiter_hip_paged_tiles_noalloc": [
        _i32, _i32, _i32, _i32, _i32,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_void_p,
        _i64, _i64, _i64, _i64, _i64, _i64,
        _i64, _i64,
        _c_void_p, _c_void_p, _i32,
        _i32, _i32, _c_void_p,
    ],
    "musa_aiter_hip_paged_dense_tiles": [
        _i32, _i32, _i32, _i32, _i32,            # scatter, codec, cache_elt, lin_elt, lin_dtype
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # key_cache, value_cache, dense_k, dense_v
        _c_void_p, _c_void_p,                    # block_tables, seq_lens
        _i64, _i64, _i64, _i64,                  # batch, dense_len, max_blocks, blocks
        _i64, _i64, _i64, _i64,                  # heads, head_dim, block_size, dense token stride (elements)
        _c_void_p, _c_void_p, _i32,              # k_scale, v_scale, scale_mode
        _i32, _i32, _c_void_p, _c_void_p,        # fill_zeros, dedupe, claims, stream
    ],
    "musa_aiter_hip_copy_rows": [
        _u64p, _u64p, _c_void_p, _c_void_p, _i64,  # host planes, device tables, planes
        _c_void_p, _c_void_p,                    # src_idx, dst_idx
        _i64, _i64, _i64, _i64, _i64, _i64,      # tokens, rows_out, src_off, dst_off, src_rows, dst_rows
        _i64, _i64, _i64,                        # row_bytes, src_stride, dst_stride
        _i32, _i32, _c_void_p, _c_void_p,        # zero_invalid, dedupe, claims, stream
    ],
    "musa_aiter_hip_copy_rows_packed": [ctypes.c_char_p, _c_void_p],  # musa_aiter_hip_copy_rows_call, stream
    "musa_aiter_hip_copy_rows_paged": [
        _u64p, _u64p, _i64,                      # host planes, planes
        _c_void_p, _c_void_p, _i64,              # src_idx, dst_idx, tokens
        _i64, _i64, _i64, _i64, _i64,            # src_rows, dst_rows, row_bytes, src_stride, dst_stride
        _i64, _i64, _i64, _i64,                  # src page rows / stride, dst page rows / stride
        _i32, _c_void_p, _c_void_p,              # dedupe, claims, stream
    ],
    # (src_k, src_v, dst_k, dst_v, block_mapping, pairs, layers, src_blocks, dst_blocks, block_bytes, claims, stream)
    "musa_aiter_hip_copy_blocks": [_c_void_p] * 5 + [_i64] * 5 + [_c_void_p, _c_void_p],
    # (src_k, dst_k, src_v, dst_v, src_indices, dst_indices, items, start_layer, layers, item_bytes,
    #  src_page_stride, src_layer_stride, dst_page_stride, dst_layer_stride, stream)
    "musa_aiter_hicache_transfer_bytes": [_c_void_p] * 6 + [_i64] * 8 + [_c_void_p],
    "lmcache_kv_strided_block_transfer": [
        _c_void_p, _u64p, _c_void_p,
        _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _c_void_p,
    ],
    # (key, value, kv_indptr, kv_indices, out_k, out_v, batch, dense_len, index_count, num_tokens,
    #  row_bytes, stream)
    "musa_aiter_hip_csr_dense_rows": [_c_void_p] * 6 + [_i64] * 5 + [_c_void_p],
    # (src_k, src_v, dst_k, dst_v, block_mapping, pairs, layers, src_blocks, dst_blocks, heads,
    #  head_dim, block_size, stream); the "_fp8_vec8" entry copies one-byte elements.
    "musa_aiter_kv_copy_paged_blocks_fp8_vec8": [_c_void_p] * 5 + [_i64] * 7 + [_c_void_p],
    "musa_aiter_hip_error_string": [_i32],
    "musa_aiter_hip_backend_name": [],
    "musa_aiter_hip_graph_claim_arrays": [],
    "musa_aiter_hip_allocated_bytes": [],
    "musa_aiter_hip_index_max": [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p],  # idx, n, partial, parts, stamp, stream
    "musa_aiter_kv_transfer_abi_version": [],
    "native_lmcache_kv_transfer_abi_version": [],
    "musa_aiter_fp8_kv_cache_abi_version": [],
    "musa_aiter_dsv4_kv_copy_abi_version": [],
    "musa_aiter_hicache_transfer_abi_version": [],
    # (dsts, srcs, sizes, count, direction 0 h2d / 1 d2h, mode 0 kernel / 1 kernel on 32 groups / 2 memcpy, stream)
    "musa_aiter_hip_batch_copy": [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p), _u64p, _i64,
                                  _i32, _i32, _c_void_p],
    "musa_aiter_hip_batch_copy_abi_version": [],
    "musa_aiter_hip_runtime_versions": [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)],
    # LMCache extension entries (memory, [kvcache0, kvcache1 | host cache pointer array], slots, sizes..., stream)
    "lmcache_kv_buffer_to_paged_list2_u16": [_c_void_p] * 4 + [_i64] * 7 + [_c_void_p],
    "lmcache_paged_to_kv_buffer_list2_u16": [_c_void_p] * 4 + [_i64] * 7 + [_c_void_p],
    "lmcache_kv_buffer_to_paged_two_x_nl_coalesced_u16": [_c_void_p, _u64p, _c_void_p] + [_i64] * 8 + [_c_void_p],
    "lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16": [_c_void_p, _u64p, _c_void_p] + [_i64] * 7 + [_c_void_p],
    # CacheGen codec.  Reference entries: (input, encoded, min_val, scale, numel, num_bins, stream) and
    # (encoded, codebook, output, numel, stream).
    "musa_aiter_kv_cachegen_encode_float": [_c_void_p, _c_void_p, ctypes.c_float, ctypes.c_float, _i64, _i64,
                                            _c_void_p],
    "musa_aiter_kv_cachegen_decode_float": [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p],
    "musa_aiter_hip_cachegen_workspace_bytes": [],
    # (input, input_dtype, numel, num_bins, native_rounding, encoded, codebook, cdf, workspace,
    #  workspace_bytes, stream)
    "musa_aiter_hip_cachegen_encode": [_c_void_p, _i32, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p,
                                       _c_void_p, _i64, _c_void_p],
    # (encoded, numel, table, table_len, elem_bytes, output, max_code, stream)
    "musa_aiter_hip_cachegen_decode": [_c_void_p, _i64, _c_void_p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p],
}

_RESTYPES = {
    "musa_aiter_hip_error_string": ctypes.c_char_p,
    "musa_aiter_hip_backend_name": ctypes.c_char_p,
    "musa_aiter_hip_cachegen_workspace_bytes": ctypes.c_int64,
    "musa_aiter_hip_graph_claim_arrays": ctypes.c_int64,
    "musa_aiter_hip_allocated_bytes": ctypes.c_int64,
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_fns: dict[str, object] = {}
_host = None


class HipBackendError(RuntimeError):
    """Raised when the HIP library is missing or a launch reports an error."""


def library() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise HipBackendError(
                    f"{LIB_NAME} is not built (expected at {LIB_PATH}); "
                    "run `python musa-aiter_amd/build.py` to compile the gfx950 kernels"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, argtypes in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
                _fns[name] = fn
            _lib = lib
    return _lib


def fn(name: str):
    library()
    return _fns[name]


def host():
    """The ``_kv_host`` helper module (tensor-list checks and address tables); raise if not built."""
    global _host
    if _host is not None:
        return _host
    with _lock:
        if _host is None:
            if not HOST_PATH.exists():
                raise HipBackendError(
                    f"{HOST_PATH.name} is not built (expected at {HOST_PATH}); "
                    "run `python musa-aiter_amd/build.py`"
                )
            spec = importlib.util.spec_from_file_location("_kv_host", HOST_PATH)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            _host = mod
    return _host


def u64_packed(packed: bytes) -> ctypes.Array:
    """A ctypes uint64 array over addresses packed by the host module."""
    n = len(packed) // 8
    if n == 0:
        return (ctypes.c_uint64 * 1)()
    return (ctypes.c_uint64 * n).from_buffer_copy(packed)


def is_available() -> bool:
    try:
        library()
    except (HipBackendError, OSError):
        return False
    return True


def check(rc: int, op: str) -> None:
    if rc != 0:
        msg = fn("musa_aiter_hip_error_string")(int(rc))
        text = msg.decode() if isinstance(msg, bytes) else str(msg)
        raise HipBackendError(f"{op}: HIP launch failed with error {rc} ({text})")


_SAME_DEVICE = contextlib.nullcontext()


def on_device(device: torch.device):
    """Context making ``device`` the current device; a no-op (no device exchange) when it already is."""
    if device.index is None or device.index == torch._C._cuda_getDevice():
        return _SAME_DEVICE
    return torch.cuda.device(device)


def stream_ptr(device: torch.device) -> ctypes.c_void_p:
    # The raw accessor returns the same handle as current_stream(device).cuda_stream
    # without building a Stream object (about 2 us less per call).
    index = device.index if device.index is not None else torch.cuda.current_device()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(index))


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


# musa_aiter_hip_copy_rows_call: four plane pointers, num_planes, two index pointers, nine int64
# sizes and strides, two int32 flags, the claims pointer (144 bytes, no padding).
_COPY_ROWS_CALL = struct.Struct("<4Qq2Q9q2iQ")


class _Claims(ctypes.Structure):
    """musa_aiter_hip_claims: caller-owned duplicate-slot claim tags of one scatter call."""
    _fields_ = [("tags", ctypes.c_void_p), ("capacity", ctypes.c_int64), ("epoch", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32)]


_EPOCH_LAST = 0xFFFFFFFF
_MIN_CLAIM_TAGS = 1 << 16
# (device index, stream handle) -> (tag tensor, its _Claims).  The tags come from torch's caching
# allocator on the stream that uses them, so the library allocates nothing for these scatters.
_claim_sets: dict[tuple[int, int], tuple[torch.Tensor, _Claims]] = {}


def claims_for(device: torch.device, stream: ctypes.c_void_p, rows: int):
    """The claims of one scatter with ``rows`` destination rows on ``stream``: returns the address of a
    musa_aiter_hip_claims to pass and the objects to keep alive until the call has returned.

    Eager calls share one tag array per (device, stream), zeroed when allocated, with an epoch that
    advances per call (no clearing pass; the array is re-zeroed when the 32-bit epoch runs out).
    A call being captured into a graph gets a fresh array from the graph's memory pool and epoch 0,
    so that the library clears the tags it claims on every replay."""
    rows = max(int(rows), 1)
    if torch.cuda.is_current_stream_capturing():
        tags = torch.empty(rows, dtype=torch.int64, device=device)
        c = _Claims(tags.data_ptr(), rows, 0, 0)
        return ctypes.addressof(c), (tags, c)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.value or 0)
    entry = _claim_sets.get(key)
    if entry is None or entry[1].capacity < rows:
        have = entry[1].capacity if entry is not None else 0
        cap = max(rows, 2 * have, _MIN_CLAIM_TAGS)
        tags = torch.zeros(cap, dtype=torch.int64, device=device)
        entry = (tags, _Claims(tags.data_ptr(), cap, 0, 0))
        _claim_sets[key] = entry
    tags, c = entry
    if c.epoch == _EPOCH_LAST:
        tags.zero_()
        c.epoch = 0
    c.epoch += 1
    return ctypes.addressof(c), entry


_INDEX_MAX_PARTS = 64
_index_max_lock = threading.Lock()
_index_max_bufs: dict[int, list] = {}


def index_max(idx: torch.Tensor) -> int:
    """Largest entry of a non-empty contiguous int64 device vector, read on the host.

    One small reduction kernel writes per-workgroup maxima, each followed by a stamp, into a pinned host
    tensor of this module (from torch's host allocator, one per device); the C entry returns when the
    stamps have arrived.  The same value as ``int(idx.max().item())``, the reference's read."""
    n = idx.numel()
    device = idx.device
    index = device.index if device.index is not None else torch.cuda.current_device()
    parts = max(1, min(_INDEX_MAX_PARTS, (n + 4095) // 4096))
    with on_device(device), _index_max_lock:
        entry = _index_max_bufs.get(index)
        if entry is None:
            entry = [torch.zeros(2 * _INDEX_MAX_PARTS, dtype=torch.int64, pin_memory=True), 0]
            _index_max_bufs[index] = entry
        buf = entry[0]
        entry[1] += 1  # the stamp of this call (nonzero, never repeated)
        check(fn("musa_aiter_hip_index_max")(ptr(idx), n, ptr(buf), parts, entry[1], stream_ptr(device)),
              "index_max")
        return int(buf.numpy()[:parts].max())


def allocated_bytes() -> int:
    """Device and pinned host bytes the HIP library has allocated itself (musa_aiter_hip_allocated_bytes)."""
    return int(fn("musa_aiter_hip_allocated_bytes")())


def _address(arr: ctypes.Array | None) -> int:
    return 0 if arr is None else ctypes.addressof(arr)


def _data(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.data_ptr()


def u64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_uint64 * max(1, len(vals)))(*vals)


def _as_u64(values) -> ctypes.Array | None:
    """Addresses as a ctypes uint64 array: None, a ready array, or a sequence of ints."""
    if values is None or isinstance(values, ctypes.Array):
        return values
    return u64_array(values)


def paged_tiles(
    *,
    op: str,
    scatter: bool,
    codec: int,
    cache_elt: int,
    lin_elt: int,
    lin_dtype: int,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    key_linear: torch.Tensor,
    value_linear: torch.Tensor,
    slots: torch.Tensor,
    num_layers: int,
    num_tokens: int,
    num_blocks: int,
    num_heads: int,
    head_dim: int,
    block_size: int,
    lin_token_stride: int,
    lin_layer_stride: int,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    scale_mode: int = 0,
    fill_zeros: bool = True,
    dedupe: bool = True,
) -> None:
    if num_tokens <= 0 or num_layers <= 0:
        return
    device = key_cache.device
    with on_device(device):
        stream = stream_ptr(device)
        claims, keep = (claims_for(device, stream, num_blocks * block_size) if scatter and dedupe
                        else (None, None))
        rc = fn("musa_aiter_hip_paged_tiles")(
            int(scatter), int(codec), int(cache_elt), int(lin_elt), int(lin_dtype),
            ptr(key_cache), ptr(value_cache), ptr(key_linear), ptr(value_linear), ptr(slots),
            int(num_layers), int(num_tokens), int(num_blocks), int(num_heads), int(head_dim), int(block_size),
            int(lin_token_stride), int(lin_layer_stride),
            ptr(k_scale), ptr(v_scale), int(scale_mode),
            int(bool(fill_zeros)), int(bool(dedupe)), claims, stream,
        )
        del keep
    check(rc, op)


def copy_rows(
    *,
    op: str,
    device: torch.device,
    src_planes=None,
    dst_planes=None,
    src_table: torch.Tensor | None = None,
    dst_table: torch.Tensor | None = None,
    num_planes: int,
    src_idx: torch.Tensor | None,
    dst_idx: torch.Tensor | None,
    num_tokens: int,
    num_rows_out: int,
    src_offset: int = 0,
    dst_offset: int = 0,
    src_rows: int,
    dst_rows: int,
    row_bytes: int,
    src_stride: int,
    dst_stride: int,
    zero_invalid: bool,
    dedupe: bool = True,
) -> None:
    if num_rows_out <= 0 or num_planes <= 0 or row_bytes <= 0:
        return
    src_arr = _as_u64(src_planes)
    dst_arr = _as_u64(dst_planes)
    with on_device(device):
        stream = stream_ptr(device)
        claims, keep = (claims_for(device, stream, dst_rows) if dedupe and dst_idx is not None
                        else (0, None))
        # One struct (musa_aiter_hip_copy_rows_call) instead of 19 converted ctypes arguments; the plane
        # arrays stay referenced by src_arr / dst_arr until the call returns.
        call = _COPY_ROWS_CALL.pack(
            _address(src_arr), _address(dst_arr), _data(src_table), _data(dst_table), num_planes,
            _data(src_idx), _data(dst_idx), num_tokens, num_rows_out, src_offset, dst_offset, src_rows, dst_rows,
            row_bytes, src_stride, dst_stride, bool(zero_invalid), bool(dedupe), claims)
        rc = fn("musa_aiter_hip_copy_rows_packed")(call, stream)
        del keep
    check(rc, op)


def paged_dense_tiles(
    *,
    op: str,
    scatter: bool,
    codec: int,
    cache_elt: int,
    lin_elt: int,
    lin_dtype: int,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    dense_k: torch.Tensor,
    dense_v: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    batch: int,
    dense_len: int,
    max_blocks: int,
    num_blocks: int,
    num_heads: int,
    head_dim: int,
    block_size: int,
    dense_token_stride: int,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    scale_mode: int = 0,
    fill_zeros: bool = True,
    dedupe: bool = True,
) -> None:
    """Paged-A caches <-> dense [batch, dense_len, heads, head_dim] through int64 block tables."""
    if batch <= 0 or dense_len <= 0:
        return
    device = key_cache.device
    with on_device(device):
        stream = stream_ptr(device)
        claims, keep = (claims_for(device, stream, num_blocks * block_size) if scatter and dedupe
                        else (None, None))
        rc = fn("musa_aiter_hip_paged_dense_tiles")(
            int(scatter), int(codec), int(cache_elt), int(lin_elt), int(lin_dtype),
            ptr(key_cache), ptr(value_cache), ptr(dense_k), ptr(dense_v), ptr(block_tables), ptr(seq_lens),
            int(batch), int(dense_len), int(max_blocks), int(num_blocks), int(num_heads), int(head_dim),
            int(block_size), int(dense_token_stride), ptr(k_scale), ptr(v_scale), int(scale_mode),
            int(bool(fill_zeros)), int(bool(dedupe)), claims, stream,
        )
        del keep
    check(rc, op)


def csr_dense_rows(
    *,
    op: str,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    out_k: torch.Tensor,
    out_v: torch.Tensor,
    batch: int,
    dense_len: int,
    num_tokens: int,
    row_bytes: int,
) -> None:
    """Dense rows gathered from token-major caches through int64 CSR indices (any element type)."""
    if batch <= 0 or dense_len <= 0 or row_bytes <= 0:
        return
    device = key_cache.device
    with on_device(device):
        rc = fn("musa_aiter_hip_csr_dense_rows")(
            ptr(key_cache), ptr(value_cache), ptr(kv_indptr), ptr(kv_indices), ptr(out_k), ptr(out_v),
            int(batch), int(dense_len), int(kv_indices.numel()), int(num_tokens), int(row_bytes),
            stream_ptr(device),
        )
    check(rc, op)


def copy_rows_paged(
    *,
    op: str,
    device: torch.device,
    src_planes,
    dst_planes,
    src_idx: torch.Tensor,
    dst_idx: torch.Tensor,
    src_rows: int,
    dst_rows: int,
    row_bytes: int,
    src_stride: int,
    dst_stride: int,
    src_page_rows: int = 0,
    src_page_stride: int = 0,
    dst_page_rows: int = 0,
    dst_page_stride: int = 0,
    dedupe: bool = True,
) -> None:
    """Rows between two index-addressed plane sets; `src_idx` / `dst_idx` are contiguous int64
    device tensors of one length, the plane lists hold device base addresses."""
    tokens = int(src_idx.numel())
    planes = len(src_planes)
    if tokens <= 0 or planes <= 0 or row_bytes <= 0:
        return
    if len(dst_planes) != planes:
        raise ValueError(f"{op}: source and destination plane lists differ in length")
    with on_device(device):
        stream = stream_ptr(device)
        claims, keep = claims_for(device, stream, dst_rows) if dedupe else (None, None)
        rc = fn("musa_aiter_hip_copy_rows_paged")(
            u64_array(src_planes), u64_array(dst_planes), planes, ptr(src_idx), ptr(dst_idx), tokens,
            int(src_rows), int(dst_rows), int(row_bytes), int(src_stride), int(dst_stride),
            int(src_page_rows), int(src_page_stride), int(dst_page_rows), int(dst_page_stride),
            int(bool(dedupe)), claims, stream,
        )
        del keep
    check(rc, op)


def copy_blocks(
    *,
    op: str,
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    block_mapping: torch.Tensor,
    num_layers: int,
    src_blocks: int,
    dst_blocks: int,
    block_bytes: int,
) -> None:
    """Whole-block byte copies; `block_mapping` is a contiguous int64 [pairs, 2] device tensor.

    Blocks are opaque bytes, so every element type goes through the byte entry
    musa_aiter_hip_copy_blocks (the form of musa_aiter_kv_copy_paged_blocks_*
    that takes caller-owned claims).
    """
    pairs = int(block_mapping.shape[0])
    if pairs <= 0 or num_layers <= 0:
        return
    device = dst_k.device
    with on_device(device):
        stream = stream_ptr(device)
        claims, keep = claims_for(device, stream, dst_blocks)
        rc = fn("musa_aiter_hip_copy_blocks")(
            ptr(src_k), ptr(src_v), ptr(dst_k), ptr(dst_v), ptr(block_mapping), pairs, int(num_layers),
            int(src_blocks), int(dst_blocks), int(block_bytes), claims, stream,
        )
        del keep
    check(rc, op)


def cachegen_encode(*, op: str, x: torch.Tensor, input_dtype: int, num_bins: int, native_rounding: bool,
                    encoded: torch.Tensor, codebook: torch.Tensor, cdf: torch.Tensor) -> None:
    """Bins, codebook and CDF of contiguous ``x`` in three launches on the current stream."""
    device = x.device
    ws_bytes = int(fn("musa_aiter_hip_cachegen_workspace_bytes")())
    with on_device(device):
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
        rc = fn("musa_aiter_hip_cachegen_encode")(
            ptr(x), int(input_dtype), int(x.numel()), int(num_bins), int(bool(native_rounding)),
            ptr(encoded), ptr(codebook), ptr(cdf), ptr(workspace), ws_bytes, stream_ptr(device),
        )
    check(rc, op)


def cachegen_decode(*, op: str, codes: torch.Tensor, table: torch.Tensor, out: torch.Tensor,
                    max_code: torch.Tensor | None) -> None:
    """out[i] = table[codes[i]] for contiguous ``codes`` / ``out`` and a contiguous table."""
    device = codes.device
    with on_device(device):
        rc = fn("musa_aiter_hip_cachegen_decode")(
            ptr(codes), int(codes.numel()), ptr(table), int(table.numel()), int(table.element_size()),
            ptr(out), ptr(max_code), stream_ptr(device),
        )
    check(rc, op)
