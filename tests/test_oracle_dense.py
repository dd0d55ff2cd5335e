"""Oracle checks for the dense-preload family and whole-block copies (CPU only).

Each oracle function is pinned three ways, none of which retypes its loop:
the reference tests' known-answer scenarios (cited as op_tests/*.py:line),
a per-element restatement of the reference's native kernel index formulas
(csrc/kvcache/kv_transfer_float.mu) on random inputs with skipped and invalid
entries, and composition with already-pinned oracle functions (the block-table
load equals a slot-vector gather over the slots the block table implies).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kv_oracle as ko


# ----- known answers from the reference's tests ----------------------------------------------


def test_load_and_reshape_flash_known_answer():
    # op_tests/test_kv_transfer.py:305-332 (and test_phase5_musa.py:421-445)
    nb, kvh, d, blk = 4, 2, 3, 4
    kc = np.arange(nb * kvh * d * blk, dtype=np.float32).reshape(nb, kvh, d, blk)
    vc = kc + 1000
    tables = np.array([[1, 3], [0, 2]])
    seq_lens = np.array([6, 3])
    k = ko.load_and_reshape_flash(kc, tables, seq_lens, 7)
    v = ko.load_and_reshape_flash(vc, tables, seq_lens, 7)
    assert k.shape == (2, 7, kvh, d)
    expected0 = np.concatenate((kc[1].transpose(2, 0, 1), kc[3].transpose(2, 0, 1)), axis=0)[:6]
    expected1 = kc[0].transpose(2, 0, 1)[:3]
    assert np.array_equal(k[0, :6], expected0) and np.array_equal(v[0, :6], expected0 + 1000)
    assert np.array_equal(k[1, :3], expected1) and np.array_equal(v[1, :3], expected1 + 1000)
    assert np.abs(k[0, 6]).max() == 0 and np.abs(k[1, 3:]).max() == 0 and np.abs(v[1, 3:]).max() == 0


def test_reshape_and_cache_back_round_trip_known_answer():
    # op_tests/test_kv_flash_reverse.py:12-42: partial pages written, then read back
    nb, kvh, hd, blk = 4, 2, 3, 4
    dense_k = np.arange(2 * 7 * kvh * hd, dtype=np.float32).reshape(2, 7, kvh, hd)
    dense_v = dense_k + 1000
    kc = np.zeros((nb, kvh, hd, blk), np.float32)
    vc = np.zeros_like(kc)
    tables = np.array([[1, 3], [0, 2]])
    seq_lens = np.array([6, 3])
    ko.reshape_and_cache_back_flash(dense_k, kc, tables, seq_lens)
    ko.reshape_and_cache_back_flash(dense_v, vc, tables, seq_lens)
    rk = ko.load_and_reshape_flash(kc, tables, seq_lens, 7)
    rv = ko.load_and_reshape_flash(vc, tables, seq_lens, 7)
    assert np.array_equal(rk[0, :6], dense_k[0, :6]) and np.array_equal(rv[0, :6], dense_v[0, :6])
    assert np.array_equal(rk[1, :3], dense_k[1, :3]) and np.array_equal(rv[1, :3], dense_v[1, :3])
    assert np.abs(rk[0, 6]).max() == 0 and np.abs(rk[1, 3:]).max() == 0
    # Only the written positions changed: block 3 holds positions 4..5 of sequence 0, block 2 nothing.
    assert np.count_nonzero(kc[3, :, :, 2:]) == 0 and np.count_nonzero(kc[2]) == 0


def test_triton_indexed_to_dense_known_answer():
    # op_tests/test_sglang_kv_integration.py:650-697
    key = np.arange(8 * 2 * 4, dtype=np.float32).reshape(8, 2, 4)
    value = key + 100
    indptr = np.array([0, 3, 7])
    indices = np.array([0, 2, 4, 1, 3, 5, 7])
    k = ko.triton_indexed_to_dense(key, indptr, indices, 4)
    v = ko.triton_indexed_to_dense(value, indptr, indices, 4)
    assert k.shape == (2, 4, 2, 4)
    assert np.array_equal(k[0, :3], key[[0, 2, 4]]) and np.abs(k[0, 3]).max() == 0
    assert np.array_equal(k[1], key[[1, 3, 5, 7]]) and np.array_equal(v[1], value[[1, 3, 5, 7]])


def test_fp8_flash_known_answer():
    # op_tests/test_phase5_musa.py:826-858: merged FP8 store, then a Flash-style dequantized load
    nb, kvh, d, blk, t = 3, 2, 8, 4, 8
    merged = np.linspace(-2.0, 2.0, t * 2 * kvh * d, dtype=np.float32).reshape(t, 2, kvh, d)
    merged = ko.bf16_bits_to_f32(ko.f32_to_bf16_bits(merged))
    kc = np.zeros((nb, kvh, d, blk), np.uint8)
    vc = np.zeros_like(kc)
    slots = np.arange(t)
    k_scale = np.array([0.125, 0.25], np.float32)
    v_scale = np.array([0.25, 0.125], np.float32)
    ko.linear_to_paged_fp8(merged[:, 0], kc, slots, k_scale, "e4m3")
    ko.linear_to_paged_fp8(merged[:, 1], vc, slots, v_scale, "e4m3")
    tables = np.array([[0, 1], [0, 1]])
    seq_lens = np.array([6, 3])
    dk = ko.bf16_bits_to_f32(ko.load_and_dequantize_fp8_flash(kc, tables, seq_lens, k_scale, "e4m3", "bfloat16", 7))
    dv = ko.bf16_bits_to_f32(ko.load_and_dequantize_fp8_flash(vc, tables, seq_lens, v_scale, "e4m3", "bfloat16", 7))
    np.testing.assert_allclose(dk[0, :6], merged[:6, 0], atol=0.13, rtol=0.12)
    np.testing.assert_allclose(dv[1, :3], merged[:3, 1], atol=0.13, rtol=0.12)
    assert np.abs(dk[0, 6:]).max() == 0 and np.abs(dv[1, 3:]).max() == 0


def test_copy_paged_blocks_known_answers():
    # op_tests/test_kv_transfer.py:349-384
    src_k = np.arange(3 * 2 * 4 * 5, dtype=np.float32).reshape(3, 2, 4, 5)
    dst_k = np.zeros((4, 2, 4, 5), np.float32)
    assert ko.copy_paged_blocks(src_k, dst_k, np.array([[0, 2], [2, 0], [-1, 1]]), multi_layer=False) == 2
    assert np.array_equal(dst_k[2], src_k[0]) and np.array_equal(dst_k[0], src_k[2])
    assert np.abs(dst_k[1]).max() == 0
    src_m = np.arange(2 * 3 * 2 * 4 * 5, dtype=np.float32).reshape(2, 3, 2, 4, 5)
    dst_m = np.zeros((2, 4, 2, 4, 5), np.float32)
    assert ko.copy_paged_blocks(src_m, dst_m, np.array([[1, 3], [2, 0]]), multi_layer=True) == 2
    assert np.array_equal(dst_m[:, 3], src_m[:, 1]) and np.array_equal(dst_m[:, 0], src_m[:, 2])
    assert np.abs(dst_m[:, 1]).max() == 0


# ----- the native kernels' per-element formulas ------------------------------------------------


def _random_tables(rng, batch, max_blocks, nb, *, invalid: bool):
    tables = rng.integers(0, nb, size=(batch, max_blocks))
    if invalid:
        mask = rng.random((batch, max_blocks)) < 0.15
        tables[mask] = rng.choice([-1, -7, nb, nb + 3], size=int(mask.sum()))
    return tables


def _kernel_load(cache, tables, seq_lens, dense_len):
    # musa_aiter_kv_load_and_reshape_flash_float_kernel (kv_transfer_float.mu:985-1037), element by element
    nb, nh, hd, bs = cache.shape
    batch, max_blocks = tables.shape
    flat = cache.reshape(-1)
    out = np.empty(batch * dense_len * nh * hd, cache.dtype)
    for idx in range(out.size):
        dim = idx % hd
        tmp = idx // hd
        head = tmp % nh
        tmp //= nh
        seq_pos = tmp % dense_len
        b = tmp // dense_len
        out[idx] = 0
        if seq_pos >= seq_lens[b]:
            continue
        lb, off = divmod(seq_pos, bs)
        if lb >= max_blocks:
            continue
        blk = tables[b, lb]
        if blk < 0 or blk >= nb:
            continue
        out[idx] = flat[((blk * nh + head) * hd + dim) * bs + off]
    return out.reshape(batch, dense_len, nh, hd)


@pytest.mark.parametrize("bs", [1, 4, 16])
def test_load_and_reshape_flash_equals_kernel_formula(bs):
    rng = np.random.default_rng(bs)
    nb, nh, hd, batch, max_blocks = 6, 2, 3, 4, 5
    cache = rng.standard_normal((nb, nh, hd, bs)).astype(np.float32)
    tables = _random_tables(rng, batch, max_blocks, nb, invalid=True)
    dense_len = min(max_blocks * bs, 3 * bs + 1)
    seq_lens = rng.integers(0, dense_len + 1, size=batch)
    seq_lens[0] = dense_len
    got = ko.load_and_reshape_flash(cache, tables, seq_lens, dense_len)
    assert np.array_equal(got, _kernel_load(cache, tables, seq_lens, dense_len))


def test_reshape_and_cache_back_equals_kernel_formula_without_collisions():
    # musa_aiter_kv_reshape_and_cache_back_flash_float_kernel (kv_transfer_float.mu:1078-1125)
    rng = np.random.default_rng(5)
    nb, nh, hd, bs, batch, max_blocks, dense_len = 12, 2, 3, 4, 3, 3, 10
    perm = rng.permutation(nb)[:batch * max_blocks].reshape(batch, max_blocks)  # distinct blocks
    perm[1, 2] = -1
    seq_lens = np.array([10, 9, 5])
    dense = rng.standard_normal((batch, dense_len, nh, hd)).astype(np.float32)
    cache = rng.standard_normal((nb, nh, hd, bs)).astype(np.float32)
    want = cache.copy().reshape(-1)
    for idx in range(dense.size):
        dim = idx % hd
        tmp = idx // hd
        head = tmp % nh
        tmp //= nh
        seq_pos = tmp % dense_len
        b = tmp // dense_len
        if seq_pos >= seq_lens[b]:
            continue
        lb, off = divmod(seq_pos, bs)
        blk = perm[b, lb] if lb < max_blocks else -1
        if blk < 0 or blk >= nb:
            continue
        want[((blk * nh + head) * hd + dim) * bs + off] = dense.reshape(-1)[idx]
    ko.reshape_and_cache_back_flash(dense, cache, perm, seq_lens)
    assert np.array_equal(cache.reshape(-1), want)


def test_reshape_and_cache_back_shared_block_last_sequence_wins():
    nb, nh, hd, bs = 2, 1, 2, 4
    cache = np.zeros((nb, nh, hd, bs), np.float32)
    dense = np.stack([np.full((4, nh, hd), 1.0, np.float32), np.full((4, nh, hd), 2.0, np.float32)])
    ko.reshape_and_cache_back_flash(dense, cache, np.array([[1], [1]]), np.array([4, 2]))
    assert np.all(cache[1, :, :, :2] == 2.0) and np.all(cache[1, :, :, 2:] == 1.0) and np.all(cache[0] == 0)


def test_triton_indexed_to_dense_equals_kernel_formula():
    # musa_aiter_kv_triton_indexed_to_dense_float_kernel (kv_transfer_float.mu:88-133)
    rng = np.random.default_rng(9)
    ntok, nh, hd, batch, dense_len = 20, 2, 3, 5, 6
    cache = rng.standard_normal((ntok, nh, hd)).astype(np.float32)
    indices = rng.integers(-2, ntok + 3, size=17)
    indptr = np.array([0, 4, 4, 11, 9, 19])  # empty, long, decreasing and past-the-end sequences
    got = ko.triton_indexed_to_dense(cache, indptr, indices, dense_len)
    flat = cache.reshape(-1)
    want = np.empty(batch * dense_len * nh * hd, np.float32)
    for idx in range(want.size):
        dim = idx % hd
        tmp = idx // hd
        head = tmp % nh
        tmp //= nh
        seq_pos = tmp % dense_len
        b = tmp // dense_len
        start, end = indptr[b], indptr[b + 1]
        offset = start + seq_pos
        want[idx] = 0
        if start < 0 or end < start or offset >= end or offset < 0 or offset >= indices.size:
            continue
        token = indices[offset]
        if token < 0 or token >= ntok:
            continue
        want[idx] = flat[(token * nh + head) * hd + dim]
    assert np.array_equal(got, want.reshape(batch, dense_len, nh, hd))


def test_copy_paged_blocks_equals_kernel_formula():
    # musa_aiter_kv_copy_paged_blocks_float_kernel (kv_transfer_float.mu:907-946), distinct destinations
    rng = np.random.default_rng(3)
    nl, sb, db, nh, hd, bs = 2, 5, 6, 2, 3, 4
    src = rng.standard_normal((nl, sb, nh, hd, bs)).astype(np.float32)
    dst = rng.standard_normal((nl, db, nh, hd, bs)).astype(np.float32)
    pairs = np.array([[4, 0], [-1, 1], [0, 5], [2, -3], [7, 2], [1, 3]])
    want = dst.copy().reshape(-1)
    per_pair = nl * nh * hd * bs
    for idx in range(pairs.shape[0] * per_pair):
        inner, pair = idx % per_pair, idx // per_pair
        off = inner % bs
        inner //= bs
        dim = inner % hd
        inner //= hd
        head = inner % nh
        layer = inner // nh
        s_blk, d_blk = pairs[pair]
        if s_blk < 0 or d_blk < 0 or s_blk >= sb or d_blk >= db:
            continue
        want[((((layer * db + d_blk) * nh + head) * hd + dim) * bs + off)] = \
            src.reshape(-1)[((((layer * sb + s_blk) * nh + head) * hd + dim) * bs + off)]
    assert ko.copy_paged_blocks(src, dst, pairs, multi_layer=True) == 3
    assert np.array_equal(dst.reshape(-1), want)


# ----- composition with the pinned slot-vector functions ----------------------------------------


def test_flash_loads_equal_slot_vector_gathers():
    rng = np.random.default_rng(21)
    nb, nh, hd, bs, batch, max_blocks = 9, 2, 8, 4, 3, 4
    tables = _random_tables(rng, batch, max_blocks, nb, invalid=False)
    seq_lens = np.array([13, 0, 7])
    dense_len = 15
    slots = ko.flash_dense_slots(tables, seq_lens, dense_len, bs, nb)
    cache = rng.standard_normal((nb, nh, hd, bs)).astype(np.float32)
    want = ko.paged_to_linear(cache, slots.reshape(-1)).reshape(batch, dense_len, nh, hd)
    assert np.array_equal(ko.load_and_reshape_flash(cache, tables, seq_lens, dense_len), want)
    lin = rng.standard_normal((30, nh, hd)).astype(np.float32) * 3
    cache8 = np.zeros((nb, nh, hd, bs), np.uint8)
    ko.linear_to_paged_fp8(lin, cache8, rng.permutation(nb * bs)[:30], np.float32(0.5), "e5m2")
    got = ko.load_and_dequantize_fp8_flash(cache8, tables, seq_lens, np.float32(0.5), "e5m2", "float16", dense_len)
    want8 = ko.paged_fp8_to_linear(cache8, slots.reshape(-1), np.float32(0.5), "e5m2", "float16")
    assert np.array_equal(got.reshape(want8.shape), want8)
