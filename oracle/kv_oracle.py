"""numpy restatement of the reference KV-movement algorithms -- TEST INFRASTRUCTURE ONLY.

Every function follows one reference function (cited as file:line of
musa_aiter 0.5.0).  Copies operate on arrays of any dtype and are compared
bit-for-bit; callers pass raw bit views (uint16 for bf16/fp16, uint32 for
fp32, uint8 for FP8 caches).  Only tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg use this module.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Slot helpers (kv_transfer.py:12-14, :3062-3064)
# ---------------------------------------------------------------------------


def split_slots(slots: np.ndarray, block_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(valid, block, offset) with ``slot = block * block_size + offset``; slot < 0 is skipped."""
    slots = np.asarray(slots, dtype=np.int64)
    valid = slots >= 0
    safe = np.where(valid, slots, 0)
    block = safe // block_size
    return valid, block, safe - block * block_size


def last_writer_mask(idx: np.ndarray) -> np.ndarray:
    """Tokens whose (non-negative) destination is not written again later in token order.

    The reference scatters in a Python token loop (kv_transfer.py:3104-3112),
    so for duplicated destinations the last token wins.
    """
    idx = np.asarray(idx, dtype=np.int64)
    n = idx.shape[0]
    mask = np.zeros(n, dtype=bool)
    if n == 0:
        return mask
    order = np.argsort(idx, kind="stable")
    ordered = idx[order]
    last = np.ones(n, dtype=bool)
    last[:-1] = ordered[1:] != ordered[:-1]
    mask[order[last]] = True
    return mask & (idx >= 0)


# ---------------------------------------------------------------------------
# Paged [NB, NH, HD, BS] <-> linear [T, NH, HD]  (kv_transfer.py:3047-3112)
# ---------------------------------------------------------------------------


def paged_to_linear(cache: np.ndarray, slots: np.ndarray, *, fill_skipped: str = "zeros",
                    out: np.ndarray | None = None) -> np.ndarray:
    """_kv_paged_to_linear_compute (kv_transfer.py:3047-3089) for one cache."""
    bs = cache.shape[3]
    valid, block, offset = split_slots(slots, bs)
    gathered = cache[block, :, :, offset]  # advanced indices first: [T, NH, HD]
    if out is None:
        res = np.zeros_like(gathered)
        res[valid] = gathered[valid]
        return res
    if fill_skipped == "zeros":
        out[...] = 0
    out[valid] = gathered[valid]
    return out


def linear_to_paged_loop(lin: np.ndarray, cache: np.ndarray, slots: np.ndarray) -> None:
    """Literal token loop of _kv_linear_to_paged_scatter (kv_transfer.py:3092-3112)."""
    bs = cache.shape[3]
    for t, s in enumerate(np.asarray(slots, dtype=np.int64).tolist()):
        if s < 0:
            continue
        b, o = divmod(s, bs)
        cache[b, :, :, o] = lin[t]


def linear_to_paged(lin: np.ndarray, cache: np.ndarray, slots: np.ndarray) -> None:
    """Vectorised _kv_linear_to_paged_scatter with last-writer-wins (kv_transfer.py:3092-3112)."""
    bs = cache.shape[3]
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    cache[block[keep], :, :, offset[keep]] = lin[keep]


def paged_to_linear_multi_layer(cache: np.ndarray, slots: np.ndarray, *, fill_skipped: str = "zeros",
                                out: np.ndarray | None = None) -> np.ndarray:
    """kv_paged_to_linear_multi_layer's per-layer loop (kv_transfer.py:3288-3309)."""
    layers = [paged_to_linear(cache[layer], slots, fill_skipped=fill_skipped,
                              out=None if out is None else out[layer]) for layer in range(cache.shape[0])]
    return out if out is not None else np.stack(layers, axis=0)


def linear_to_paged_multi_layer(lin: np.ndarray, cache: np.ndarray, slots: np.ndarray) -> None:
    """kv_linear_to_paged_multi_layer's per-layer loop (kv_transfer.py:3445-3457)."""
    for layer in range(cache.shape[0]):
        linear_to_paged(lin[layer], cache[layer], slots)


def paged_to_merged_linear(key_cache: np.ndarray, value_cache: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """kv_paged_to_merged_linear (kv_transfer.py:3617-3618): stack K, V on axis 1."""
    return np.stack((paged_to_linear(key_cache, slots), paged_to_linear(value_cache, slots)), axis=1)


def merged_linear_to_paged(merged: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                           slots: np.ndarray) -> None:
    """kv_merged_linear_to_paged (kv_transfer.py:3654)."""
    linear_to_paged(merged[:, 0], key_cache, slots)
    linear_to_paged(merged[:, 1], value_cache, slots)


# ---------------------------------------------------------------------------
# FP8 codec (kv_transfer.py:2094-2200)
# ---------------------------------------------------------------------------

# (exponent bits, mantissa bits, bias, max unbiased exponent) -- _fp8_format_params (:2103-2107)
FP8_FORMATS = {"e4m3": (4, 3, 7, 8), "e5m2": (5, 2, 15, 16)}


def fp8_quantize(x: np.ndarray, scale: np.ndarray | float, fmt: str) -> np.ndarray:
    """_fp8_quantize_to_uint8 (kv_transfer.py:2161-2183), step for step, in float32 numpy.

    ``x`` must already be float32 (the reference's ``tensor.to(torch.float32)``).
    """
    _, mant, bias, emax = FP8_FORMATS[fmt]
    x = np.asarray(x, dtype=np.float32)
    scale = np.asarray(scale, dtype=np.float32)
    with np.errstate(all="ignore"):
        work = (x / scale).astype(np.float32)
        sign = work < 0
        a = np.abs(work)
        a = np.where(np.isfinite(a), a, np.float32(0))
        max_value = np.float32((2.0 - 2.0 ** (-mant)) * (2.0 ** emax))
        min_normal = np.float32(2.0 ** (1 - bias))
        clipped = np.minimum(a, max_value)
        nonzero = clipped >= min_normal
        safe = np.where(nonzero, clipped, np.float32(1)).astype(np.float32)
        exponent = np.floor(np.log2(safe)).astype(np.int32)
        exponent = np.clip(exponent, 1 - bias, emax)
        base = np.power(np.float32(2.0), exponent.astype(np.float32)).astype(np.float32)
        frac = ((safe / base).astype(np.float32) - np.float32(1.0)) * np.float32(2 ** mant)
        mantissa = np.round(frac.astype(np.float32)).astype(np.int32)  # round half to even
        overflow = mantissa == 2 ** mant
        exponent = np.minimum(np.where(overflow, exponent + 1, exponent), emax)
        mantissa = np.clip(np.where(overflow, 0, mantissa), 0, 2 ** mant - 1)
        exponent_field = np.where(nonzero, exponent + bias, 0)
        mantissa = np.where(nonzero, mantissa, 0)
        bits = (sign.astype(np.int32) << 7) | (exponent_field << mant) | mantissa
    return bits.astype(np.uint8)


def fp8_dequantize_f32(encoded: np.ndarray, scale: np.ndarray | float, fmt: str) -> np.ndarray:
    """_fp8_dequantize_from_uint8 (kv_transfer.py:2186-2200) up to ``value * scale`` in float32."""
    _, mant, bias, _ = FP8_FORMATS[fmt]
    bits = np.asarray(encoded).astype(np.int32)
    sign = ((bits >> 7) & 1).astype(np.float32)
    exponent_field = (bits >> mant) & ((1 << (7 - mant)) - 1)
    mantissa = bits & ((1 << mant) - 1)
    nonzero = exponent_field != 0
    exponent = exponent_field.astype(np.float32) - np.float32(bias)
    with np.errstate(all="ignore"):
        value = (np.float32(1.0) + mantissa.astype(np.float32) / np.float32(2 ** mant)) * np.power(
            np.float32(2.0), exponent).astype(np.float32)
        value = np.where(nonzero, value, np.float32(0.0)).astype(np.float32)
        value = np.where(sign > 0, -value, value).astype(np.float32)
        return (value * np.asarray(scale, dtype=np.float32)).astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even; NaN -> 0x7FC0 (torch's c10::BFloat16 rule)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), rounded).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_storage(x_f32: np.ndarray, dtype: str) -> np.ndarray:
    """``.to(out_dtype)`` of a float32 array, returned as raw storage bits (uint16 / uint32)."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x_f32)
    if dtype == "float16":
        with np.errstate(all="ignore"):
            return np.asarray(x_f32, dtype=np.float32).astype(np.float16).view(np.uint16)
    if dtype == "float32":
        return np.asarray(x_f32, dtype=np.float32).view(np.uint32)
    raise ValueError(dtype)


def from_storage(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Raw storage bits -> float32 values (exact widening)."""
    if dtype == "bfloat16":
        return bf16_bits_to_f32(bits)
    if dtype == "float16":
        return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
    if dtype == "float32":
        return np.asarray(bits, dtype=np.uint32).view(np.float32)
    raise ValueError(dtype)


def _head_scale(scale: np.ndarray, head_dim: int, layer: int | None = None) -> np.ndarray:
    """_fp8_scale_for_head / _fp8_scale_for_layer_head (kv_transfer.py:2124-2135)."""
    scale = np.asarray(scale, dtype=np.float32)
    if scale.ndim == 0:
        return scale
    if scale.ndim == 2:
        scale = scale[layer]
    return np.broadcast_to(scale.reshape(-1, 1), (scale.shape[-1], head_dim))


def linear_to_paged_fp8(lin_f32: np.ndarray, cache_u8: np.ndarray, slots: np.ndarray, scale: np.ndarray, fmt: str,
                        layer: int | None = None) -> None:
    """kv_linear_to_paged_fp8's token loop (kv_transfer.py:2239-2247) for one cache (K or V)."""
    nb, nh, hd, bs = cache_u8.shape
    sc = _head_scale(scale, hd, layer)
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    encoded = fp8_quantize(lin_f32[keep], sc, fmt)  # scale broadcasts over [T, NH, HD]
    cache_u8[block[keep], :, :, offset[keep]] = encoded


def paged_fp8_to_linear(cache_u8: np.ndarray, slots: np.ndarray, scale: np.ndarray, fmt: str, out_dtype: str,
                        layer: int | None = None) -> np.ndarray:
    """kv_paged_fp8_to_linear's token loop (kv_transfer.py:2283-2301): zeros for skipped tokens."""
    nb, nh, hd, bs = cache_u8.shape
    sc = _head_scale(scale, hd, layer)
    valid, block, offset = split_slots(slots, bs)
    values = fp8_dequantize_f32(cache_u8[block, :, :, offset], sc, fmt)
    out = to_storage(values, out_dtype)
    out[~valid] = 0
    return out


# ---------------------------------------------------------------------------
# Dense preload for attention (kv_transfer.py:1291-1781)
# ---------------------------------------------------------------------------


def _logical_blocks(seq_len: int, bs: int, max_blocks: int, num_blocks: int, table_row: np.ndarray):
    """(start, end, block_id) of every logical block of one sequence (kv_transfer.py:1609-1622).

    The reference's Python path raises on a block id outside [0, num_blocks)
    (:1581-1585); its native kernels, which C-ABI callers reach, skip such a
    block and any logical block at or past ``max_blocks``
    (kv_transfer_float.mu:1006-1030).  Both are expressed by skipping here.
    """
    for lb in range((max(seq_len, 0) + bs - 1) // bs):
        if lb >= max_blocks:
            break
        blk = int(table_row[lb])
        if blk < 0 or blk >= num_blocks:
            continue
        start = lb * bs
        yield start, min(start + bs, seq_len), blk


def load_and_reshape_flash(cache: np.ndarray, block_tables: np.ndarray, seq_lens: np.ndarray,
                           dense_len: int) -> np.ndarray:
    """kv_load_and_reshape_flash (kv_transfer.py:1599-1622) for one cache: dense [B, S, NH, HD].

    Positions at or past ``seq_lens[b]`` stay zero (``out.zero_()``, :1565-1576).
    """
    nb, nh, hd, bs = cache.shape
    block_tables = np.asarray(block_tables, dtype=np.int64)
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    batch, max_blocks = block_tables.shape
    out = np.zeros((batch, dense_len, nh, hd), dtype=cache.dtype)
    for b in range(batch):
        for start, end, blk in _logical_blocks(int(seq_lens[b]), bs, max_blocks, nb, block_tables[b]):
            end = min(end, dense_len)
            if end > start:
                out[b, start:end] = cache[blk, :, :, :end - start].transpose(2, 0, 1)
    return out


def reshape_and_cache_back_flash(dense: np.ndarray, cache: np.ndarray, block_tables: np.ndarray,
                                 seq_lens: np.ndarray) -> None:
    """kv_reshape_and_cache_back_flash's loop (kv_transfer.py:1700-1715) for one cache, in place.

    Later (batch, position) pairs overwrite earlier ones on shared blocks, as
    the reference's batch-major loop does.
    """
    nb, nh, hd, bs = cache.shape
    block_tables = np.asarray(block_tables, dtype=np.int64)
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    batch, max_blocks = block_tables.shape
    dense_len = dense.shape[1]
    for b in range(batch):
        for start, end, blk in _logical_blocks(int(seq_lens[b]), bs, max_blocks, nb, block_tables[b]):
            end = min(end, dense_len)
            if end > start:
                cache[blk, :, :, :end - start] = dense[b, start:end].transpose(1, 2, 0)


def flash_dense_slots(block_tables: np.ndarray, seq_lens: np.ndarray, dense_len: int, block_size: int,
                      num_blocks: int) -> np.ndarray:
    """Per-sequence slot vectors of kv_load_and_dequantize_fp8_flash (kv_transfer.py:1766-1776): [B, S]."""
    block_tables = np.asarray(block_tables, dtype=np.int64)
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    batch, max_blocks = block_tables.shape
    slots = np.full((batch, dense_len), -1, dtype=np.int64)
    for b in range(batch):
        for start, end, blk in _logical_blocks(int(seq_lens[b]), block_size, max_blocks, num_blocks,
                                               block_tables[b]):
            end = min(end, dense_len)
            slots[b, start:end] = blk * block_size + np.arange(end - start)
    return slots


def load_and_dequantize_fp8_flash(cache_u8: np.ndarray, block_tables: np.ndarray, seq_lens: np.ndarray,
                                  scale: np.ndarray, fmt: str, out_dtype: str, dense_len: int) -> np.ndarray:
    """kv_load_and_dequantize_fp8_flash (kv_transfer.py:1764-1781) for one cache: one
    kv_paged_fp8_to_linear per sequence over its slot vector."""
    nb, nh, hd, bs = cache_u8.shape
    slots = flash_dense_slots(block_tables, seq_lens, dense_len, bs, nb)
    rows = [paged_fp8_to_linear(cache_u8, slots[b], scale, fmt, out_dtype) for b in range(slots.shape[0])]
    if not rows:
        return np.zeros((0, dense_len, nh, hd), dtype=np.uint16 if out_dtype != "float32" else np.uint32)
    return np.stack(rows)


def triton_indexed_to_dense(cache: np.ndarray, kv_indptr: np.ndarray, kv_indices: np.ndarray,
                            dense_len: int) -> np.ndarray:
    """kv_triton_indexed_to_dense (kv_transfer.py:1355-1366) for one token-major cache [N, NH, HD].

    Sequence b copies ``min(max(end - start, 0), dense_len)`` rows
    ``cache[kv_indices[start + i]]``.  Where the reference's Python path would
    fail (an offset past ``kv_indices``, a row outside the cache, a negative
    ``start``) its native kernel writes zeros (kv_transfer_float.mu:114-128);
    so does this function.
    """
    kv_indptr = np.asarray(kv_indptr, dtype=np.int64)
    kv_indices = np.asarray(kv_indices, dtype=np.int64)
    n = cache.shape[0]
    batch = kv_indptr.shape[0] - 1
    out = np.zeros((batch, dense_len) + cache.shape[1:], dtype=cache.dtype)
    for b in range(batch):
        start, end = int(kv_indptr[b]), int(kv_indptr[b + 1])
        if start < 0:
            continue
        copy_len = min(max(end - start, 0), dense_len)
        for i in range(copy_len):
            off = start + i
            if off >= kv_indices.shape[0]:
                break
            row = int(kv_indices[off])
            if 0 <= row < n:
                out[b, i] = cache[row]
    return out


def copy_paged_blocks(src: np.ndarray, dst: np.ndarray, pairs: np.ndarray, *, multi_layer: bool) -> int:
    """kv_copy_paged_blocks's pair loop (kv_transfer.py:2078-2091) for one cache, in place.

    Pairs with a negative id are skipped; later pairs overwrite earlier ones.
    The reference's native kernel (kv_transfer_float.mu:934-937) also skips ids
    past either cache, which the Python layer rejects beforehand.
    """
    copied = 0
    for s_blk, d_blk in np.asarray(pairs, dtype=np.int64).reshape(-1, 2).tolist():
        nsrc = src.shape[1] if multi_layer else src.shape[0]
        ndst = dst.shape[1] if multi_layer else dst.shape[0]
        if s_blk < 0 or d_blk < 0 or s_blk >= nsrc or d_blk >= ndst:
            continue
        if multi_layer:
            dst[:, d_blk] = src[:, s_blk]
        else:
            dst[d_blk] = src[s_blk]
        copied += 1
    return copied


# ---------------------------------------------------------------------------
# Token-major flat caches [NB, BS, D] (kv_transfer.py:3786-3838)
# ---------------------------------------------------------------------------


def flat_paged_to_linear(cache: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """_flat_paged_to_linear_compute (kv_transfer.py:3786-3815) for one cache."""
    bs = cache.shape[1]
    valid, block, offset = split_slots(slots, bs)
    rows = cache[block, offset]
    rows = np.where(valid.reshape((-1,) + (1,) * (rows.ndim - 1)), rows, np.zeros_like(rows))
    return rows


def flat_linear_to_paged(lin: np.ndarray, cache: np.ndarray, slots: np.ndarray) -> None:
    """_flat_linear_to_paged_scatter (kv_transfer.py:3818-3838) with last-writer-wins."""
    bs = cache.shape[1]
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    cache[block[keep], offset[keep]] = lin[keep]


# ---------------------------------------------------------------------------
# LMCache converters (lmcache_kv_transfer.py)
# ---------------------------------------------------------------------------


def two_x_nl_to_buffer(caches: list[list[np.ndarray]], memory: np.ndarray, slots: np.ndarray) -> None:
    """lmcache_kv_paged_to_buffer_two_x_nl reference path (lmcache_kv_transfer.py:258-269).

    The whole memory tensor is zeroed first, then valid tokens are filled.
    """
    memory[...] = 0
    nb, bs = caches[0][0].shape[:2]
    valid, block, offset = split_slots(slots, bs)
    t_idx = np.nonzero(valid)[0]
    for axis in range(2):
        for layer, cache in enumerate(caches[axis]):
            memory[axis, layer, t_idx] = cache[block[t_idx], offset[t_idx]].reshape(len(t_idx), -1)


def buffer_to_two_x_nl(memory: np.ndarray, caches: list[list[np.ndarray]], slots: np.ndarray, skip: int) -> None:
    """lmcache_kv_buffer_to_paged_two_x_nl reference path (lmcache_kv_transfer.py:212-226)."""
    nb, bs, nh, hs = caches[0][0].shape
    n = len(slots)
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    for axis in range(2):
        for layer, cache in enumerate(caches[axis]):
            values = memory[axis, layer, skip:skip + n].reshape(n, nh, hs)
            cache[block[keep], offset[keep]] = values[keep]


def native_gather_rows(cache_rows: np.ndarray, slots: np.ndarray, out_rows: np.ndarray, skip: int = 0) -> None:
    """The reference's native token-row gathers for one buffer plane (kv_transfer_float.mu:2233-2308,
    :2518-2560): row ``skip + i`` (when inside the plane) gets slot row ``slots[i]``, or zeros for a
    negative slot; the plane's other rows are untouched.  ``cache_rows`` is the cache as
    [num_slots, row]; callers map slots past the cache to -1, as the kernels skip them."""
    for i, s in enumerate(np.asarray(slots, dtype=np.int64).tolist()):
        if 0 <= skip + i < out_rows.shape[0]:
            out_rows[skip + i] = cache_rows[s] if s >= 0 else 0


def native_scatter_rows(in_rows: np.ndarray, slots: np.ndarray, cache_rows: np.ndarray, skip: int = 0) -> None:
    """The native token-row scatters for one plane: slot row ``slots[i]`` gets buffer row
    ``skip + i``; negative slots are skipped and a repeated slot keeps the last token."""
    slots = np.asarray(slots, dtype=np.int64)
    keep = last_writer_mask(slots)
    for i in np.nonzero(keep)[0]:
        cache_rows[slots[i]] = in_rows[skip + i]


def list_to_buffer(kvcaches: list[np.ndarray], memory: np.ndarray, slots: np.ndarray) -> None:
    """_lmcache_kv_paged_to_buffer_list reference path (lmcache_kv_transfer.py:451-460)."""
    memory[...] = 0
    bs = kvcaches[0].shape[2]
    valid, block, offset = split_slots(slots, bs)
    t_idx = np.nonzero(valid)[0]
    for layer, kvcache in enumerate(kvcaches):
        for axis in range(2):
            memory[axis, layer, t_idx] = kvcache[axis, block[t_idx], offset[t_idx]].reshape(len(t_idx), -1)


def buffer_to_list(memory: np.ndarray, kvcaches: list[np.ndarray], slots: np.ndarray, skip: int) -> None:
    """_lmcache_kv_buffer_to_paged_list reference path (lmcache_kv_transfer.py:428-437)."""
    _, nb, bs, nh, hs = kvcaches[0].shape
    n = len(slots)
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    for layer, kvcache in enumerate(kvcaches):
        for axis in range(2):
            values = memory[axis, layer, skip:skip + n].reshape(n, nh, hs)
            kvcache[axis, block[keep], offset[keep]] = values[keep]


def six_d_to_buffer(paged: np.ndarray, kv_buffer: np.ndarray, slots: np.ndarray) -> None:
    """lmcache_paged_to_kv_buffer reference path (lmcache_kv_transfer.py:105-115), cache [NL, 2, NB, BS, NH, HS]."""
    kv_buffer[...] = 0
    bs = paged.shape[3]
    valid, block, offset = split_slots(slots, bs)
    t_idx = np.nonzero(valid)[0]
    for layer in range(paged.shape[0]):
        for axis in range(2):
            kv_buffer[axis, layer, t_idx] = paged[layer, axis, block[t_idx], offset[t_idx]].reshape(len(t_idx), -1)


def buffer_to_six_d(kv_buffer: np.ndarray, paged: np.ndarray, slots: np.ndarray) -> None:
    """lmcache_kv_buffer_to_paged reference path (lmcache_kv_transfer.py:87-96)."""
    nl, _, nb, bs, nh, hs = paged.shape
    n = len(slots)
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    for layer in range(nl):
        for axis in range(2):
            values = kv_buffer[axis, layer, :n].reshape(n, nh, hs)
            paged[layer, axis, block[keep], offset[keep]] = values[keep]


def mla_to_buffer(paged: np.ndarray, kv_buffer: np.ndarray, slots: np.ndarray) -> None:
    """lmcache_paged_to_kv_buffer_mla reference path (lmcache_kv_transfer.py:144-151), cache [NL, NB, BS, HS]."""
    kv_buffer[...] = 0
    bs = paged.shape[2]
    valid, block, offset = split_slots(slots, bs)
    t_idx = np.nonzero(valid)[0]
    for layer in range(paged.shape[0]):
        kv_buffer[layer, t_idx] = paged[layer, block[t_idx], offset[t_idx]]


def buffer_to_mla(kv_buffer: np.ndarray, paged: np.ndarray, slots: np.ndarray) -> None:
    """lmcache_kv_buffer_to_paged_mla reference path (lmcache_kv_transfer.py:129-135)."""
    bs = paged.shape[2]
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    for layer in range(paged.shape[0]):
        paged[layer, block[keep], offset[keep]] = kv_buffer[layer, :len(slots)][keep]


def mla_list_to_buffer(kvcaches: list[np.ndarray], memory: np.ndarray, slots: np.ndarray) -> None:
    """_lmcache_mla_paged_to_buffer_list reference path (lmcache_kv_transfer.py:494-502), memory [1, NL, M, HS]."""
    memory[...] = 0
    bs = kvcaches[0].shape[1]
    valid, block, offset = split_slots(slots, bs)
    t_idx = np.nonzero(valid)[0]
    for layer, kvcache in enumerate(kvcaches):
        memory[0, layer, t_idx] = kvcache[block[t_idx], offset[t_idx]]


def buffer_to_mla_list(memory: np.ndarray, kvcaches: list[np.ndarray], slots: np.ndarray, skip: int) -> None:
    """_lmcache_mla_buffer_to_paged_list reference path (lmcache_kv_transfer.py:474-481)."""
    bs = kvcaches[0].shape[1]
    n = len(slots)
    keep = last_writer_mask(slots)
    _, block, offset = split_slots(slots, bs)
    for layer, kvcache in enumerate(kvcaches):
        values = memory[0, layer, skip:skip + n]
        kvcache[block[keep], offset[keep]] = values[keep]


# ---------------------------------------------------------------------------
# Opaque byte rows (kv_transfer.py:4728-4736) and strided blocks
# ---------------------------------------------------------------------------


def copy_rows(src: np.ndarray, dst: np.ndarray, src_idx: np.ndarray, dst_idx: np.ndarray) -> None:
    """``dst.index_copy_(0, dst_rows, src.index_select(0, src_rows))`` in index order (last wins)."""
    for s, d in zip(np.asarray(src_idx).tolist(), np.asarray(dst_idx).tolist()):
        dst[d] = src[s]


def strided_block_transfer(staging: np.ndarray, pages: list[np.ndarray], block_ids: np.ndarray, *, direction: int,
                           idx_start: int, n_valid: int, offset_in_object: int, staging_tokens: int, block_size: int,
                           row_bytes: int, paged_block_stride: int, mode: int, value_bytes: int = 0,
                           scale_bytes: int = 0) -> None:
    """Byte semantics of lmcache_kv_strided_block_transfer (kernel text kv_transfer_float.mu:3302-3358).

    ``staging`` is a flat uint8 array of NL * staging_tokens * row_bytes bytes;
    ``pages`` are flat uint8 arrays, one per layer.
    """
    for layer, page in enumerate(pages):
        for p in range(n_valid):
            blk = int(block_ids[idx_start + p])
            for t in range(block_size):
                srow = ((layer * staging_tokens) + offset_in_object + p * block_size + t) * row_bytes
                if mode == 0:
                    spans = [(srow, blk * paged_block_stride + t * row_bytes, row_bytes)]
                else:
                    spans = [(srow, blk * paged_block_stride + t * value_bytes, value_bytes),
                             (srow + value_bytes, blk * paged_block_stride + block_size * value_bytes + t * scale_bytes,
                              scale_bytes)]
                for s_off, p_off, n in spans:
                    if direction == 0:
                        page[p_off:p_off + n] = staging[s_off:s_off + n]
                    else:
                        staging[s_off:s_off + n] = page[p_off:p_off + n]
