"""The reference test suite's known-answer scenarios, replayed against the oracle (CPU only).

Each test names the reference test it restates (op_tests/*.py:line) and uses
its shapes, slot mappings and assertions, so the oracle is held to the same
behavioural contract the reference's own CI checks.
"""

from __future__ import annotations

import numpy as np

from oracle import kv_oracle as ko


def _randn(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def test_kv_linear_to_paged_then_paged_to_linear_matches():
    # op_tests/test_kv_transfer.py:28-43
    rng = np.random.default_rng(42)
    nb, kvh, d, blk, t = 2, 3, 8, 4, 5
    k_lin, v_lin = _randn(rng, (t, kvh, d)), _randn(rng, (t, kvh, d))
    kc, vc = np.zeros((nb, kvh, d, blk), np.float32), np.zeros((nb, kvh, d, blk), np.float32)
    slots = np.array([0, 2, 5, 6, 7])
    ko.linear_to_paged(k_lin, kc, slots)
    ko.linear_to_paged(v_lin, vc, slots)
    assert np.array_equal(ko.paged_to_linear(kc, slots), k_lin)
    assert np.array_equal(ko.paged_to_linear(vc, slots), v_lin)


def test_copy_to_kv_cache_layout_agrees():
    # op_tests/test_kv_transfer.py:46-58 (copy_to_kv_cache writes cache[b, :, :, off] = k[t], ops/cache.py:105-144)
    rng = np.random.default_rng(1)
    nb, kvh, d, blk, t = 4, 2, 6, 4, 3
    k_tok = _randn(rng, (t, kvh, d))
    kc = np.zeros((nb, kvh, d, blk), np.float32)
    slots = np.array([1, blk + 3, blk * 2 + 2])
    for i, s in enumerate(slots):
        kc[s // blk, :, :, s % blk] = k_tok[i]
    assert np.array_equal(ko.paged_to_linear(kc, slots), k_tok)


def test_negative_slot_zeros_gather_and_skip_scatter():
    # op_tests/test_kv_transfer.py:61-84
    rng = np.random.default_rng(2)
    nb, kvh, d, blk, t = 3, 2, 4, 8, 4
    slots = np.array([-1, 14, -1, 19])
    kr = ko.paged_to_linear(_randn(rng, (nb, kvh, d, blk)), slots)
    assert np.abs(kr[0]).max() == 0 and np.abs(kr[2]).max() == 0
    k_lin = _randn(rng, (t, kvh, d))
    kz = np.zeros((nb, kvh, d, blk), np.float32)
    ko.linear_to_paged(k_lin, kz, slots)
    kr2 = ko.paged_to_linear(kz, slots)
    assert np.array_equal(kr2[1], k_lin[1]) and np.array_equal(kr2[3], k_lin[3])
    assert np.abs(kr2[0]).max() == 0 and np.count_nonzero(kz) == 2 * kvh * d


def test_multi_layer_roundtrip_matches_single_layer_loop():
    # op_tests/test_kv_transfer.py:86-111
    rng = np.random.default_rng(3)
    L, nb, kvh, d, blk, t = 3, 2, 2, 5, 4, 5
    k_lin = _randn(rng, (L, t, kvh, d))
    kc = np.zeros((L, nb, kvh, d, blk), np.float32)
    slots = np.array([0, 2, blk + 2, blk + 1, nb * blk - 1])
    ko.linear_to_paged_multi_layer(k_lin, kc, slots)
    assert np.array_equal(ko.paged_to_linear_multi_layer(kc, slots), k_lin)
    for layer in range(L):
        kc1 = np.zeros((nb, kvh, d, blk), np.float32)
        ko.linear_to_paged(k_lin[layer], kc1, slots)
        assert np.array_equal(kc[layer], kc1)


def test_merged_roundtrip_and_mla_asymmetric():
    # op_tests/test_kv_transfer.py:139-160, :181-201
    rng = np.random.default_rng(4)
    nb, kvh, d, blk, t = 2, 2, 4, 4, 4
    merged = _randn(rng, (t, 2, kvh, d))
    slots = np.array([0, 3, -1, 7])
    kc, vc = np.zeros((nb, kvh, d, blk), np.float32), np.zeros((nb, kvh, d, blk), np.float32)
    ko.merged_linear_to_paged(merged, kc, vc, slots)
    rec = ko.paged_to_merged_linear(kc, vc, slots)
    assert np.array_equal(rec[[0, 1, 3]], merged[[0, 1, 3]]) and np.abs(rec[2]).max() == 0
    kv_lin, pe_lin = _randn(rng, (t, 6)), _randn(rng, (t, 3))
    kv_c, pe_c = np.zeros((nb, blk, 6), np.float32), np.zeros((nb, blk, 3), np.float32)
    ko.flat_linear_to_paged(kv_lin, kv_c, slots)
    ko.flat_linear_to_paged(pe_lin, pe_c, slots)
    r_kv, r_pe = ko.flat_paged_to_linear(kv_c, slots), ko.flat_paged_to_linear(pe_c, slots)
    assert np.array_equal(r_kv[[0, 1, 3]], kv_lin[[0, 1, 3]]) and np.abs(r_kv[2]).max() == 0
    assert np.array_equal(r_pe[[0, 1, 3]], pe_lin[[0, 1, 3]]) and np.abs(r_pe[2]).max() == 0


def test_large_edge_sparse_and_duplicate_last_writer():
    # op_tests/test_kv_transfer.py:262-279 and :281-303
    rng = np.random.default_rng(5)
    L, nb, kvh, d, blk = 5, 17, 3, 7, 8
    slots = np.array([0, 3, -1, 15, 16, 31, -1, 63, 64, 95, 127, 135])
    k_lin = _randn(rng, (L, len(slots), kvh, d))
    kc = np.zeros((L, nb, kvh, d, blk), np.float32)
    ko.linear_to_paged_multi_layer(k_lin, kc, slots)
    rec = ko.paged_to_linear_multi_layer(kc, slots)
    valid = slots >= 0
    assert np.array_equal(rec[:, valid], k_lin[:, valid]) and np.abs(rec[:, ~valid]).max() == 0
    dup = np.array([0, 1, 0, -1, 7, 7, 11])
    lin = _randn(rng, (len(dup), 2, 5))
    cache = np.zeros((3, 2, 5, 4), np.float32)
    ko.linear_to_paged(lin, cache, dup)
    rec = ko.paged_to_linear(cache, dup)
    for got, want in ((0, 2), (2, 2), (4, 5), (5, 5)):
        assert np.array_equal(rec[got], lin[want])
    assert np.abs(rec[3]).max() == 0


def test_fp8_reference_roundtrip_tolerances():
    # op_tests/test_kv_transfer.py:402-488 (tolerance roundtrips are the reference's only FP8 pins)
    t, kvh, d = 5, 2, 8
    k_lin = np.linspace(-1.5, 1.5, t * kvh * d, dtype=np.float32).reshape(t, kvh, d)
    slots = np.array([0, 7, -1, 5, 9])
    cache = np.zeros((3, kvh, d, 4), np.uint8)
    ko.linear_to_paged_fp8(k_lin, cache, slots, np.float32(0.125), "e4m3")
    rk = ko.from_storage(ko.paged_fp8_to_linear(cache, slots, np.float32(0.125), "e4m3", "float32"), "float32")
    valid = slots >= 0
    assert np.all(np.abs(rk[valid] - k_lin[valid]) <= 0.065 + 0.08 * np.abs(k_lin[valid]))
    assert np.abs(rk[~valid]).max() == 0
    k5 = np.linspace(-8.0, 8.0, 2 * 4 * kvh * d, dtype=np.float32).reshape(2, 4, kvh, d)
    s5 = np.array([0, 4, -1, 11])
    for layer in range(2):
        c5 = np.zeros((3, kvh, d, 4), np.uint8)
        ko.linear_to_paged_fp8(k5[layer], c5, s5, np.float32(0.25), "e5m2")
        r5 = ko.from_storage(ko.paged_fp8_to_linear(c5, s5, np.float32(0.25), "e5m2", "float32"), "float32")
        v5 = s5 >= 0
        assert np.all(np.abs(r5[v5] - k5[layer][v5]) <= 0.55 + 0.16 * np.abs(k5[layer][v5]))


def test_lmcache_two_x_nl_roundtrip_and_prefix_skip():
    # op_tests/test_lmcache_kv_transfer.py:90-140
    nl, nb, bs, nh, hs = 3, 2, 4, 2, 3
    hidden = nh * hs
    slots = np.array([0, 3, 5, -1, 7])
    source = [[np.arange(nb * bs * nh * hs, dtype=np.float32).reshape(nb, bs, nh, hs) + a * 10_000 + layer * 1_000
               for layer in range(nl)] for a in range(2)]
    dest = [[np.full_like(source[a][layer], -7.0) for layer in range(nl)] for a in range(2)]
    memory = np.empty((2, nl, len(slots), hidden), np.float32)
    ko.two_x_nl_to_buffer(source, memory, slots)
    ko.buffer_to_two_x_nl(memory, dest, slots, 0)
    vs = slots[slots >= 0]
    for a in range(2):
        for layer in range(nl):
            assert np.array_equal(dest[a][layer].reshape(-1, hidden)[vs], source[a][layer].reshape(-1, hidden)[vs])
    assert np.abs(memory[:, :, 3]).max() == 0
    nl, nb, bs, nh, hs = 2, 2, 2, 1, 2
    slots = np.array([0, 3])
    memory = np.arange(2 * nl * 4 * nh * hs, dtype=np.float32).reshape(2, nl, 4, nh * hs)
    dest = [[np.full((nb, bs, nh, hs), -1.0, np.float32) for _ in range(nl)] for _ in range(2)]
    ko.buffer_to_two_x_nl(memory, dest, slots, 2)
    for a in range(2):
        for layer in range(nl):
            flat = dest[a][layer].reshape(-1, nh * hs)
            assert np.array_equal(flat[0], memory[a, layer, 2]) and np.array_equal(flat[3], memory[a, layer, 3])
            assert np.array_equal(flat[1], np.full(2, -1.0, np.float32))


def test_lmcache_non_mla_and_mla_roundtrips():
    # op_tests/test_lmcache_kv_transfer.py:243-296
    nl, nb, bs, nh, hs = 3, 2, 4, 2, 3
    slots = np.array([0, 3, 5, -1, 7])
    t = len(slots)
    kv_buffer = np.arange(2 * nl * t * nh * hs, dtype=np.float32).reshape(2, nl, t, nh * hs)
    paged = np.zeros((nl, 2, nb, bs, nh, hs), np.float32)
    ko.buffer_to_six_d(kv_buffer, paged, slots)
    rec = np.empty_like(kv_buffer)
    ko.six_d_to_buffer(paged, rec, slots)
    for i in (0, 1, 2, 4):
        assert np.array_equal(rec[:, :, i], kv_buffer[:, :, i])
    assert np.abs(rec[:, :, 3]).max() == 0
    one = np.ones((2, 1, 2, 2), np.float32)
    paged1 = np.full((1, 2, 1, 4, 1, 2), 7.0, np.float32)
    ko.buffer_to_six_d(one, paged1, np.array([-1, 2]))
    assert np.array_equal(paged1[:, :, 0, 0], np.full((1, 2, 1, 2), 7.0)) and np.array_equal(
        paged1[:, :, 0, 2], np.ones((1, 2, 1, 2)))
    nl, nb, bs, hs = 2, 2, 4, 5
    slots = np.array([0, 4, -1, 7])
    kvb = np.arange(nl * len(slots) * hs, dtype=np.float32).reshape(nl, len(slots), hs)
    pm = np.zeros((nl, nb, bs, hs), np.float32)
    ko.buffer_to_mla(kvb, pm, slots)
    rec = np.empty_like(kvb)
    ko.mla_to_buffer(pm, rec, slots)
    assert np.array_equal(rec[:, [0, 1, 3]], kvb[:, [0, 1, 3]]) and np.abs(rec[:, 2]).max() == 0


def test_mla_list_roundtrip():
    # op_tests/test_lmcache_kv_transfer.py:226-240
    nl, nb, bs, hs = 2, 2, 4, 5
    slots = np.array([0, 4, -1, 7])
    source = [np.arange(nb * bs * hs, dtype=np.float32).reshape(nb, bs, hs) + layer * 1000 for layer in range(nl)]
    dest = [np.zeros_like(s) for s in source]
    memory = np.empty((1, nl, len(slots), hs), np.float32)
    ko.mla_list_to_buffer(source, memory, slots)
    ko.buffer_to_mla_list(memory, dest, slots, 0)
    vs = slots[slots >= 0]
    for s, d in zip(source, dest):
        assert np.array_equal(d.reshape(-1, hs)[vs], s.reshape(-1, hs)[vs])


def test_copy_rows_duplicate_destination_last_wins():
    # op_tests/test_kv_copy_paged_rows_correctness.py:82-96
    src = np.arange(8 * 256, dtype=np.uint32).astype(np.uint8).reshape(8, 256)
    dst = np.zeros((4, 256), np.uint8)
    ko.copy_rows(src, dst, np.arange(8), np.array([1, 1, 2, 2, 3, 3, 0, 0]))
    assert np.array_equal(dst[[1, 2, 3, 0]], src[[1, 3, 5, 7]])
