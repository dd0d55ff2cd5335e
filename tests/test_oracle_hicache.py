"""Pins oracle/hicache_oracle.py: the reference's own HiCache test expectations, two independent
formulations of the layout transfer, round trips and brute-force token copies.

- Known answers: every assertion of the reference's op_tests/test_hicache_transfer.py
  (:27-247), restated on numpy arrays.
- ``transfer`` (tensor indexing, the reference's torch path) and ``transfer_bytes`` (byte
  offsets, the native kernel's contract) must agree for every layout pair, layer window and
  item width; a wrong stride, layer offset or skip rule in either one fails here.
- The direct functions equal per-token copies whenever page groups are consecutive, and the
  run coalescing matches hand-worked cases where they are not.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from oracle import hicache_oracle as ho


def _kv_layer_first(layers=2, pages=4, item=8):
    key = np.arange(layers * pages * item, dtype=np.float32).reshape(layers, pages, item)
    return key, key + 10000


# ----- known answers from the reference's tests ------------------------------------------------


def test_kat_per_layer_layer_first_two_index_tables():
    src_k, src_v = _kv_layer_first()
    dst_k, dst_v = np.zeros_like(src_k), np.zeros_like(src_v)
    ho.transfer(src_k, dst_k, src_v, dst_v, np.array([3, 1]), np.array([0, 2]), src_layout="layer_first",
                dst_layout="layer_first", start_layer=1, num_layers=1)
    assert np.array_equal(dst_k[1, 0], src_k[1, 3])
    assert np.array_equal(dst_k[1, 2], src_k[1, 1])
    assert np.count_nonzero(dst_k[0]) == 0
    assert np.array_equal(dst_v[1, 0], src_v[1, 3])


def test_kat_per_layer_page_first_to_layer_first():
    layers, pages, item = 2, 4, 8
    src_k = np.arange(pages * layers * item, dtype=np.float32).reshape(pages, layers, item)
    src_v = src_k + 5000
    dst_k = np.zeros((layers, pages, item), np.float32)
    dst_v = np.zeros_like(dst_k)
    ho.transfer(src_k, dst_k, src_v, dst_v, np.array([2, 0]), np.array([1, 3]), src_layout="page_first",
                dst_layout="layer_first", start_layer=0, num_layers=1)
    assert np.array_equal(dst_k[0, 1], src_k[2, 0])
    assert np.array_equal(dst_k[0, 3], src_k[0, 0])
    assert np.count_nonzero(dst_k[1]) == 0
    assert np.array_equal(dst_v[0, 1], src_v[2, 0])


def test_kat_all_layer_layer_first_to_page_first():
    src_k, src_v = _kv_layer_first()
    dst_k = np.zeros((4, 2, 8), np.float32)
    dst_v = np.zeros_like(dst_k)
    ho.transfer(src_k, dst_k, src_v, dst_v, np.array([0, 2]), np.array([1, 3]), src_layout="layer_first",
                dst_layout="page_first", start_layer=0, num_layers=2)
    assert np.array_equal(dst_k[1, 0], src_k[0, 0])
    assert np.array_equal(dst_k[1, 1], src_k[1, 0])
    assert np.array_equal(dst_k[3, 0], src_k[0, 2])
    assert np.array_equal(dst_k[3, 1], src_k[1, 2])


def test_kat_all_layer_negative_index_skip():
    src_k, src_v = _kv_layer_first()
    dst_k, dst_v = np.full_like(src_k, -1), np.full_like(src_v, -1)
    ho.transfer(src_k, dst_k, src_v, dst_v, np.array([-1, 1]), np.array([0, 2]), src_layout="layer_first",
                dst_layout="layer_first", start_layer=0, num_layers=2)
    assert np.array_equal(dst_k[:, 2], src_k[:, 1])
    assert np.array_equal(dst_v[:, 2], src_v[:, 1])
    assert np.all(dst_k[:, 0] == -1)


def test_kat_mla_page_first_to_layer_first_and_all_layers():
    layers, pages, item = 2, 3, 6
    src = np.arange(pages * layers * item, dtype=np.float32).reshape(pages, layers, item)
    dst = np.zeros((layers, pages, item), np.float32)
    ho.transfer(src, dst, None, None, np.array([1]), np.array([2]), src_layout="page_first",
                dst_layout="layer_first", start_layer=1, num_layers=1)
    assert np.array_equal(dst[1, 2], src[1, 1])
    assert np.count_nonzero(dst[0]) == 0

    layers, pages = 2, 4
    src = np.arange(layers * pages * item, dtype=np.float32).reshape(layers, pages, item)
    dst = np.zeros((pages, layers, item), np.float32)
    ho.transfer(src, dst, None, None, np.array([-1, 1, 3]), np.array([0, 2, 1]), src_layout="layer_first",
                dst_layout="page_first", start_layer=0, num_layers=2)
    assert np.array_equal(dst[2], src[:, 1])
    assert np.array_equal(dst[1], src[:, 3])
    assert np.all(dst[0] == 0)


def test_kat_direct_coalesces_token_ranges():
    layers, tokens, item = 2, 8, 4
    src_k = np.arange(layers * tokens * item, dtype=np.float32).reshape(layers, tokens, item)
    src_v = src_k + 1000
    dst_k, dst_v = np.zeros_like(src_k), np.zeros_like(src_v)
    ho.direct([src_k[0], src_k[1], src_v[0], src_v[1]], [dst_k[0], dst_k[1], dst_v[0], dst_v[1]],
              np.array([0, 1, 4, 5]), np.array([2, 3, 0, 1]), 2)
    assert np.array_equal(dst_k[:, 2:4], src_k[:, 0:2])
    assert np.array_equal(dst_k[:, 0:2], src_k[:, 4:6])
    assert np.array_equal(dst_v[:, 2:4], src_v[:, 0:2])


def test_kat_direct_per_layer_page_first_to_layer_first():
    pages, layers, page_size, item = 3, 2, 2, 4
    src_k = np.arange(pages * layers * page_size * item, dtype=np.float32).reshape(pages, layers, page_size, item)
    src_v = src_k + 5000
    dst_k = np.zeros((layers, pages * page_size, item), np.float32)
    dst_v = np.zeros_like(dst_k)
    ho.per_layer_direct_pf_lf([src_k, src_v], [dst_k[1], dst_v[1]], np.array([0, 1, 4, 5]), np.array([2, 3, 0, 1]),
                              1, 2)
    assert np.array_equal(dst_k[1, 2:4], src_k[0, 1])
    assert np.array_equal(dst_k[1, 0:2], src_k[2, 1])
    assert np.array_equal(dst_v[1, 2:4], src_v[0, 1])
    assert np.count_nonzero(dst_k[0]) == 0

    dst = np.zeros((layers, pages * page_size, item), np.float32)
    ho.per_layer_direct_pf_lf([src_k], [dst[0]], np.array([2, 3]), np.array([4, 5]), 0, 2)
    assert np.array_equal(dst[0, 4:6], src_k[1, 0])


def test_kat_direct_all_layer_layer_first_to_page_first():
    layers, tokens, pages, page_size, item = 2, 6, 3, 2, 4
    src_k = np.arange(layers * tokens * item, dtype=np.float32).reshape(layers, tokens, item)
    src_v = src_k + 7000
    dst_k = np.zeros((pages, layers, page_size, item), np.float32)
    dst_v = np.zeros_like(dst_k)
    ho.all_layer_direct_lf_pf([src_k[0], src_k[1], src_v[0], src_v[1]], [dst_k, dst_v], np.array([0, 1, 4, 5]),
                              np.array([2, 3, 0, 1]), 2)
    assert np.array_equal(dst_k[1], src_k[:, 0:2])
    assert np.array_equal(dst_k[0], src_k[:, 4:6])
    assert np.array_equal(dst_v[1], src_v[:, 0:2])

    dst_mla = np.zeros((pages, layers, page_size, item), np.float32)
    ho.all_layer_direct_lf_pf([src_k[0], src_k[1]], [dst_mla], np.array([0, 1]), np.array([2, 3]), 2)
    assert np.array_equal(dst_mla[1], src_k[:, 0:2])


# ----- two formulations of the layout transfer ------------------------------------------------


def _random_pairs(rng, n, src_pages, dst_pages, *, skips=True, duplicates=False):
    src = rng.integers(0, src_pages, size=n)
    dst = rng.permutation(dst_pages)[:n] if not duplicates else rng.integers(0, dst_pages, size=n)
    if skips:
        src[rng.random(n) < 0.2] = -1
        dst[rng.random(n) < 0.1] = -1
    return src.astype(np.int64), dst.astype(np.int64)


def _shape(layout, layers, pages, item):
    return (layers, pages, item) if layout == "layer_first" else (pages, layers, item)


@pytest.mark.parametrize("src_layout,dst_layout", list(itertools.product(["layer_first", "page_first"], repeat=2)))
@pytest.mark.parametrize("item,dtype", [(4, np.uint16), (6, np.uint32), (24, np.uint8)])
@pytest.mark.parametrize("window", [(0, 5), (2, 1), (1, 3)])
@pytest.mark.parametrize("mla", [False, True])
def test_tensor_path_equals_byte_offset_contract(src_layout, dst_layout, item, dtype, window, mla):
    rng = np.random.default_rng(7)
    layers, src_pages, dst_pages, n = 5, 11, 9, 8
    start, count = window
    duplicates = src_layout == dst_layout
    src_idx, dst_idx = _random_pairs(rng, n, src_pages, dst_pages, duplicates=duplicates)
    info = np.iinfo(dtype)
    mk = lambda shape: rng.integers(0, info.max, size=shape, dtype=dtype, endpoint=True)  # noqa: E731
    src_k, src_v = mk(_shape(src_layout, layers, src_pages, item)), mk(_shape(src_layout, layers, src_pages, item))
    dst_k, dst_v = mk(_shape(dst_layout, layers, dst_pages, item)), mk(_shape(dst_layout, layers, dst_pages, item))
    want_k, want_v = dst_k.copy(), dst_v.copy()
    ho.transfer(src_k, want_k, None if mla else src_v, None if mla else want_v, src_idx, dst_idx,
                src_layout=src_layout, dst_layout=dst_layout, start_layer=start, num_layers=count)
    got_k, got_v = dst_k.copy(), dst_v.copy()
    sps, sls = ho.layout_strides(src_k.shape, src_k.itemsize, src_layout)
    dps, dls = ho.layout_strides(dst_k.shape, dst_k.itemsize, dst_layout)
    flat = lambda a: a.reshape(-1).view(np.uint8)  # noqa: E731
    ho.transfer_bytes(flat(src_k), flat(got_k), None if mla else flat(src_v), None if mla else flat(got_v),
                      src_idx, dst_idx, n, start, count, item * src_k.itemsize, sps, sls, dps, dls)
    assert np.array_equal(got_k, want_k)
    assert np.array_equal(got_v, want_v)
    if mla:
        assert np.array_equal(got_v, dst_v)


def test_layout_strides_closed_form():
    # [layers=3, pages=5, item=4] of 2-byte elements: a page is one 8-byte item, a layer 5 items.
    assert ho.layout_strides((3, 5, 4), 2, "layer_first") == (8, 40)
    # [pages=5, layers=3, item=4]: a layer is one item, a page three.
    assert ho.layout_strides((5, 3, 4), 2, "page_first") == (24, 8)


def test_byte_contract_copies_whole_words_only():
    src = np.arange(64, dtype=np.uint8)
    dst = np.zeros(64, np.uint8)
    # 12-byte items copy one 8-byte word (the kernel's item_size_bytes / 8 words).
    ho.transfer_bytes(src, dst, None, None, np.array([1]), np.array([2]), 1, 0, 1, 12, 16, 0, 16, 0)
    assert np.array_equal(dst[32:40], src[16:24])
    assert np.count_nonzero(dst) == 8


def test_layer_first_page_first_round_trip():
    rng = np.random.default_rng(3)
    layers, pages, item = 4, 10, 6
    src_k = rng.integers(1, 60000, size=(layers, pages, item), dtype=np.uint16)
    src_v = rng.integers(1, 60000, size=(layers, pages, item), dtype=np.uint16)
    host_k = np.zeros((pages, layers, item), np.uint16)
    host_v = np.zeros_like(host_k)
    sel, slots = np.array([7, 2, 5]), np.array([0, 9, 4])
    ho.transfer(src_k, host_k, src_v, host_v, sel, slots, src_layout="layer_first", dst_layout="page_first",
                start_layer=0, num_layers=layers)
    back_k, back_v = np.zeros_like(src_k), np.zeros_like(src_v)
    for layer in range(layers):
        ho.transfer(host_k, back_k, host_v, back_v, slots, sel, src_layout="page_first", dst_layout="layer_first",
                    start_layer=layer, num_layers=1)
    assert np.array_equal(back_k[:, sel], src_k[:, sel])
    assert np.array_equal(back_v[:, sel], src_v[:, sel])
    others = np.setdiff1d(np.arange(pages), sel)
    assert np.count_nonzero(back_k[:, others]) == 0


def test_duplicate_destination_keeps_the_last_pair():
    src = np.arange(1, 1 + 2 * 3 * 2, dtype=np.uint32).reshape(2, 3, 2)
    dst = np.zeros_like(src)
    ho.transfer(src, dst, None, None, np.array([0, 2, 1]), np.array([1, 1, -1]), src_layout="layer_first",
                dst_layout="layer_first", start_layer=0, num_layers=2)
    assert np.array_equal(dst[:, 1], src[:, 2])


# ----- direct token ranges -------------------------------------------------------------------


def test_direct_runs_hand_worked():
    # Regular: every break on a page boundary, runs merge across consecutive pages.
    assert ho.direct_runs([0, 1, 2, 3, 8, 9], [4, 5, 6, 7, 0, 1], 2) == [(0, 4, 4), (8, 0, 2)]
    # A page whose entries are not consecutive still copies page_size rows from its first entry.
    assert ho.direct_runs([0, 5], [0, 1], 2) == [(0, 0, 2)]
    # A break inside a run's first page is ignored; the next run starts mid-page and may reach
    # past the end of the tables.
    assert ho.direct_runs([0, 1, 2, 9], [0, 1, 2, 3], 2) == [(0, 0, 3), (9, 3, 2)]


def _regular_token_tables(rng, groups, page_size, src_pages, dst_pages, *, src_aligned=True, dst_aligned=True):
    sp = rng.choice(src_pages, size=groups, replace=False) * page_size
    dp = rng.choice(dst_pages, size=groups, replace=False) * page_size
    if not src_aligned:
        sp = sp + rng.integers(0, 3, size=groups)
    if not dst_aligned:
        dp = dp + rng.integers(0, 3, size=groups)
    j = np.tile(np.arange(page_size), groups)
    return np.repeat(sp, page_size) + j, np.repeat(dp, page_size) + j


@pytest.mark.parametrize("page_size", [1, 4, 16])
def test_direct_equals_per_token_copy_for_consecutive_pages(page_size):
    rng = np.random.default_rng(page_size)
    groups, pages, item = 6, 12, 5
    src_t, dst_t = _regular_token_tables(rng, groups, page_size, pages, pages, src_aligned=False, dst_aligned=False)
    src = [rng.integers(0, 2**31, size=(pages * page_size + 3, item), dtype=np.uint32) for _ in range(3)]
    dst = [np.zeros_like(s) for s in src]
    ho.direct(src, dst, src_t, dst_t, page_size)
    for s, d in zip(src, dst):
        want = np.zeros_like(s)
        for a, b in zip(src_t, dst_t):
            want[b] = s[a]
        assert np.array_equal(d, want)


@pytest.mark.parametrize("page_size", [1, 2, 8])
def test_per_layer_direct_equals_per_token_copy(page_size):
    rng = np.random.default_rng(11 + page_size)
    groups, pages, layers, item, layer = 5, 9, 3, 6, 2
    src_t, dst_t = _regular_token_tables(rng, groups, page_size, pages, pages, dst_aligned=False)
    src = rng.integers(0, 2**15, size=(pages, layers, page_size, item), dtype=np.uint16)
    dst = np.zeros((pages * page_size + 2, item), np.uint16)
    ho.per_layer_direct_pf_lf([src], [dst], src_t, dst_t, layer, page_size)
    want = np.zeros_like(dst)
    for a, b in zip(src_t, dst_t):
        want[b] = src[a // page_size, layer, a % page_size]
    assert np.array_equal(dst, want)


@pytest.mark.parametrize("page_size", [1, 2, 8])
def test_all_layer_direct_equals_per_token_copy(page_size):
    rng = np.random.default_rng(21 + page_size)
    groups, pages, layers, item = 5, 9, 3, 6
    src_t, dst_t = _regular_token_tables(rng, groups, page_size, pages, pages, src_aligned=False)
    src = [rng.integers(0, 2**15, size=(pages * page_size + 2, item), dtype=np.uint16) for _ in range(2 * layers)]
    dst = [np.zeros((pages, layers, page_size, item), np.uint16) for _ in range(2)]
    ho.all_layer_direct_lf_pf(src, dst, src_t, dst_t, page_size)
    for plane in range(2):
        want = np.zeros_like(dst[plane])
        for layer in range(layers):
            for a, b in zip(src_t, dst_t):
                want[b // page_size, layer, b % page_size] = src[plane * layers + layer][a]
        assert np.array_equal(dst[plane], want)
