"""Pins the copy functions of the oracle against independent implementations (CPU only).

Each vectorised oracle function is compared with (a) a brute-force
per-element Python loop written from the layout definitions, and/or (b)
torch's own indexing ops (advanced indexing, index_put_, index_copy_), on
small random inputs with skipped and duplicated slots.  A transposed axis, a
wrong block/offset split or a lost last-writer rule fails here.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as ko
from tests.kvgen import make_slots


def _rand(rng, shape):
    return rng.integers(0, 2 ** 16, size=shape, dtype=np.uint16)


@pytest.mark.parametrize("kind", ["sequences", "random", "skips", "duplicates"])
@pytest.mark.parametrize("bs", [4, 16])
def test_paged_to_linear_brute_force_and_torch(kind, bs):
    rng = np.random.default_rng(1)
    nh, hd, t = 3, 5, 37
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=t)
    cache = _rand(rng, (nb, nh, hd, bs))
    got = ko.paged_to_linear(cache, slots)
    brute = np.zeros((t, nh, hd), np.uint16)
    for i, s in enumerate(slots):
        if s < 0:
            continue
        for h in range(nh):
            for d in range(hd):
                brute[i, h, d] = cache.reshape(-1)[((s // bs * nh + h) * hd + d) * bs + s % bs]
    assert np.array_equal(got, brute)
    tc = torch.from_numpy(cache.astype(np.int32))
    st = torch.from_numpy(slots)
    valid = st >= 0
    safe = torch.where(valid, st, 0)
    theirs = tc[safe // bs, :, :, safe % bs] * valid.view(-1, 1, 1)
    assert np.array_equal(got.astype(np.int32), theirs.numpy())


@pytest.mark.parametrize("kind", ["sequences", "skips", "duplicates"])
def test_linear_to_paged_vectorised_equals_token_loop(kind):
    rng = np.random.default_rng(2)
    nh, hd, bs, t = 2, 3, 4, 60
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=t)
    lin = _rand(rng, (t, nh, hd))
    base = _rand(rng, (nb, nh, hd, bs))
    a, b = base.copy(), base.copy()
    ko.linear_to_paged(lin, a, slots)
    ko.linear_to_paged_loop(lin, b, slots)
    assert np.array_equal(a, b)
    # torch's index_put_ with accumulate=False is not ordered for duplicates; compare on unique keeps only.
    keep = ko.last_writer_mask(slots)
    tc = torch.from_numpy(base.astype(np.int32))
    st = torch.from_numpy(slots[keep])
    tc[st // bs, :, :, st % bs] = torch.from_numpy(lin[keep].astype(np.int32))
    assert np.array_equal(a.astype(np.int32), tc.numpy())


def test_last_writer_mask_definition():
    idx = np.array([3, -1, 3, 5, 7, 5, 5, -1, 0], np.int64)
    assert ko.last_writer_mask(idx).tolist() == [False, False, True, False, True, False, True, False, True]


def test_multi_layer_and_merged_compose_single_layer():
    rng = np.random.default_rng(3)
    nl, nh, hd, bs, t = 3, 2, 4, 8, 40
    slots, nb = make_slots("skips", rng, block_size=bs, tokens=t)
    cache = _rand(rng, (nl, nb, nh, hd, bs))
    ml = ko.paged_to_linear_multi_layer(cache, slots)
    for layer in range(nl):
        assert np.array_equal(ml[layer], ko.paged_to_linear(cache[layer], slots))
    merged = ko.paged_to_merged_linear(cache[0], cache[1], slots)
    assert np.array_equal(merged[:, 0], ml[0]) and np.array_equal(merged[:, 1], ml[1])
    out = _rand(rng, (t, nh, hd))
    kept = ko.paged_to_linear(cache[0], slots, fill_skipped="preserve", out=out.copy())
    valid = slots >= 0
    assert np.array_equal(kept[valid], ml[0][valid]) and np.array_equal(kept[~valid], out[~valid])


def test_fp8_cache_functions_equal_token_loop():
    rng = np.random.default_rng(4)
    nh, hd, bs, t = 2, 8, 4, 30
    slots, nb = make_slots("duplicates", rng, block_size=bs, tokens=t)
    x = (rng.standard_normal((t, nh, hd)) * 3).astype(np.float32)
    scale = np.array([0.02, 0.5], np.float32)
    cache = np.zeros((nb, nh, hd, bs), np.uint8)
    ko.linear_to_paged_fp8(x, cache, slots, scale, "e4m3")
    loop = np.zeros_like(cache)
    for i, s in enumerate(slots):
        if s < 0:
            continue
        loop[s // bs, :, :, s % bs] = ko.fp8_quantize(x[i], scale.reshape(-1, 1), "e4m3")
    assert np.array_equal(cache, loop)
    out = ko.paged_fp8_to_linear(cache, slots, scale, "e4m3", "float32")
    for i, s in enumerate(slots):
        want = np.zeros((nh, hd), np.float32) if s < 0 else ko.fp8_dequantize_f32(
            cache[s // bs, :, :, s % bs], scale.reshape(-1, 1), "e4m3")
        assert np.array_equal(out[i], want.view(np.uint32))


def test_lmcache_two_x_nl_and_list_brute_force():
    rng = np.random.default_rng(5)
    nl, bs, nh, hs, t, m, skip = 2, 4, 2, 3, 13, 17, 2
    slots, nb = make_slots("duplicates", rng, block_size=bs, tokens=t)
    caches = [[_rand(rng, (nb, bs, nh, hs)) for _ in range(nl)] for _ in range(2)]
    mem = _rand(rng, (2, nl, m, nh * hs))
    got = mem.copy()
    ko.two_x_nl_to_buffer(caches, got, slots)
    brute = np.zeros_like(mem)
    for i, s in enumerate(slots):
        if s >= 0:
            for a in range(2):
                for layer in range(nl):
                    brute[a, layer, i] = caches[a][layer].reshape(-1, nh * hs)[s]
    assert np.array_equal(got, brute)
    dst = [[c.copy() for c in axis] for axis in caches]
    ko.buffer_to_two_x_nl(mem, dst, slots, skip)
    ref = [[c.copy().reshape(-1, nh * hs) for c in axis] for axis in caches]
    for i, s in enumerate(slots):  # token order: later tokens overwrite earlier ones
        if s >= 0:
            for a in range(2):
                for layer in range(nl):
                    ref[a][layer][s] = mem[a, layer, skip + i]
    for a in range(2):
        for layer in range(nl):
            assert np.array_equal(dst[a][layer].reshape(-1, nh * hs), ref[a][layer])
    lists = [np.stack([caches[0][layer], caches[1][layer]]) for layer in range(nl)]
    got_l = mem.copy()
    ko.list_to_buffer(lists, got_l, slots)
    assert np.array_equal(got_l, brute)


def test_six_d_and_mla_brute_force():
    rng = np.random.default_rng(6)
    nl, bs, nh, hs, t = 2, 4, 2, 3, 11
    slots, nb = make_slots("skips", rng, block_size=bs, tokens=t)
    paged = _rand(rng, (nl, 2, nb, bs, nh, hs))
    buf = _rand(rng, (2, nl, t, nh * hs))
    ko.six_d_to_buffer(paged, buf, slots)
    for i, s in enumerate(slots):
        for a in range(2):
            for layer in range(nl):
                want = paged[layer, a].reshape(-1, nh * hs)[s] if s >= 0 else 0
                assert np.array_equal(buf[a, layer, i], np.broadcast_to(want, (nh * hs,)))
    mla = _rand(rng, (nl, nb, bs, 5))
    mbuf = _rand(rng, (nl, t, 5))
    ko.mla_to_buffer(mla, mbuf, slots)
    tm = torch.from_numpy(mla.astype(np.int32)).reshape(nl, -1, 5)
    st = torch.from_numpy(slots)
    ref = torch.where((st >= 0).view(1, -1, 1), tm[:, st.clamp(min=0)], 0)
    assert np.array_equal(mbuf.astype(np.int32), ref.numpy())


def test_flat_mla_split_matches_torch_indexing():
    rng = np.random.default_rng(7)
    bs, t = 8, 25
    slots, nb = make_slots("skips", rng, block_size=bs, tokens=t)
    cache = _rand(rng, (nb, bs, 6))
    got = ko.flat_paged_to_linear(cache, slots)
    tc = torch.from_numpy(cache.astype(np.int32)).reshape(-1, 6)
    st = torch.from_numpy(slots)
    ref = torch.where((st >= 0).view(-1, 1), tc[st.clamp(min=0)], 0)
    assert np.array_equal(got.astype(np.int32), ref.numpy())


def test_copy_rows_equals_torch_index_copy():
    rng = np.random.default_rng(8)
    src = rng.integers(0, 256, size=(9, 37), dtype=np.uint8)
    dst = rng.integers(0, 256, size=(6, 37), dtype=np.uint8)
    si = np.array([0, 3, 8, 1, 2], np.int64)
    di = np.array([5, 0, 5, 2, 0], np.int64)
    got = dst.copy()
    ko.copy_rows(src, got, si, di)
    ref = torch.from_numpy(dst.copy())
    ref.index_copy_(0, torch.from_numpy(di), torch.from_numpy(src).index_select(0, torch.from_numpy(si)))
    assert np.array_equal(got, ref.numpy())


def test_strided_blocks_closed_forms():
    rng = np.random.default_rng(9)
    nl, bs, row, stride, nb = 2, 4, 12, 4 * 12 + 8, 5
    staging_tokens, offset = 3 * bs + 2, 1
    pages = [rng.integers(0, 256, size=nb * stride, dtype=np.uint8) for _ in range(nl)]
    staging = rng.integers(0, 256, size=nl * staging_tokens * row, dtype=np.uint8)
    ids = np.array([3, 0, 4], np.int64)
    # mode 0 gather: block p of layer l is the contiguous [bs * row] page span.
    st = staging.copy()
    ko.strided_block_transfer(st, [p.copy() for p in pages], ids, direction=1, idx_start=0, n_valid=3,
                              offset_in_object=offset, staging_tokens=staging_tokens, block_size=bs, row_bytes=row,
                              paged_block_stride=stride, mode=0)
    for layer in range(nl):
        for p, blk in enumerate(ids):
            s0 = (layer * staging_tokens + offset + p * bs) * row
            assert np.array_equal(st[s0:s0 + bs * row], pages[layer][blk * stride:blk * stride + bs * row])
    # mode 1: scatter then gather is the identity on the staged rows, values and scales land in their planes.
    pg = [p.copy() for p in pages]
    ko.strided_block_transfer(staging, pg, ids, direction=0, idx_start=0, n_valid=3, offset_in_object=offset,
                              staging_tokens=staging_tokens, block_size=bs, row_bytes=row, paged_block_stride=stride,
                              mode=1, value_bytes=8, scale_bytes=4)
    blk = ids[1]
    s0 = (0 * staging_tokens + offset + 1 * bs + 2) * row
    assert np.array_equal(pg[0][blk * stride + 2 * 8: blk * stride + 3 * 8], staging[s0:s0 + 8])
    assert np.array_equal(pg[0][blk * stride + bs * 8 + 2 * 4: blk * stride + bs * 8 + 3 * 4], staging[s0 + 8:s0 + 12])
    back = np.zeros_like(staging)
    ko.strided_block_transfer(back, pg, ids, direction=1, idx_start=0, n_valid=3, offset_in_object=offset,
                              staging_tokens=staging_tokens, block_size=bs, row_bytes=row, paged_block_stride=stride,
                              mode=1, value_bytes=8, scale_bytes=4)
    for layer in range(nl):
        s0 = (layer * staging_tokens + offset) * row
        assert np.array_equal(back[s0:s0 + 3 * bs * row], staging[s0:s0 + 3 * bs * row])


@pytest.mark.parametrize("kind", ["skips", "duplicates"])
def test_native_row_functions_agree_with_the_python_paths(kind):
    """With no prefix skip and a buffer of exactly T rows, the native row gather / scatter equal the
    reference's Python-path restatements (which zero the whole buffer first); with a skip, rows
    outside [skip, skip + T) stay untouched and row skip + i is token i."""
    rng = np.random.default_rng(3)
    nl, bs, nh, hs, t = 2, 4, 2, 3, 29
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=t)
    caches = [[_rand(rng, (nb, bs, nh, hs)) for _ in range(nl)] for _ in range(2)]
    want = np.empty((2, nl, t, nh * hs), np.uint16)
    ko.two_x_nl_to_buffer(caches, want, slots)
    got = _rand(rng, (2, nl, t, nh * hs))
    for a in range(2):
        for layer in range(nl):
            ko.native_gather_rows(caches[a][layer].reshape(nb * bs, -1), slots, got[a, layer])
    assert np.array_equal(got, want)
    mem = _rand(rng, (2, nl, t + 5, nh * hs))
    want_c = [[c.copy() for c in g] for g in caches]
    ko.buffer_to_two_x_nl(mem, want_c, slots, 5)
    got_c = [[c.copy() for c in g] for g in caches]
    for a in range(2):
        for layer in range(nl):
            ko.native_scatter_rows(mem[a, layer], slots, got_c[a][layer].reshape(nb * bs, -1), 5)
            assert np.array_equal(got_c[a][layer], want_c[a][layer])
    # prefix skip: only rows [skip, skip + T) of the plane change, clipped at the plane's end
    plane = _rand(rng, (t + 3, nh * hs))
    before = plane.copy()
    rows = caches[0][0].reshape(nb * bs, -1)
    ko.native_gather_rows(rows, slots, plane, 6)
    assert np.array_equal(plane[:6], before[:6])
    for i in range(t + 3 - 6):
        assert np.array_equal(plane[6 + i], rows[slots[i]] if slots[i] >= 0 else np.zeros(nh * hs, np.uint16))
