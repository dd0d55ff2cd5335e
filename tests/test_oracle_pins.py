"""Pins for the oracle's scatter functions and small helpers (CPU only).

Every scatter here is checked against a literal per-token loop written from the
reference's own loop structure (a Python ``for token_index, slot in
enumerate(slots)`` with ``divmod(slot, block_size)`` and one row assignment per
layer/axis), never against the oracle's vectorised formula.  Inputs are chosen
so that a plausible mistake fails: at least two layers with values that differ
per (axis, layer), so a transposed axis/layer fails; a non-zero skip prefix with
buffer rows that differ from the ones after it, so a dropped or doubled skip
fails; repeated slots, so first-writer-wins fails; negative slots, so a
``slot % block_size`` on -1 (which lands in the last block) fails.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import batch_copy_oracle as bo
from oracle import cachegen_oracle as co
from oracle import kv_oracle as ko


def _distinct(shape, base=0):
    """Values that are unique over the whole array (no accidental equalities)."""
    return (np.arange(int(np.prod(shape)), dtype=np.float32) + base).reshape(shape)


def _dup_slots(num_slots: int, n: int, rng) -> np.ndarray:
    """n slots with repeats and skips: half drawn from a small pool so repeats are certain."""
    pool = rng.choice(num_slots, size=max(2, n // 3), replace=False)
    slots = np.where(rng.random(n) < 0.5, rng.choice(pool, size=n), rng.integers(0, num_slots, size=n))
    slots[rng.random(n) < 0.2] = -1
    slots[1] = slots[0] = pool[0]       # a repeat at the very start
    slots[-1] = -1                      # and a skip at the very end
    return slots.astype(np.int64)


# ----- the list LMCache scatter --------------------------------------------------------------


def test_buffer_to_list_reference_alias_roundtrip():
    # op_tests/test_lmcache_kv_transfer.py:63-84: list caches [2, NB, BS, NH, HS] per layer,
    # paged -> buffer -> paged through the list alias, valid slots restored exactly.
    nl, nb, bs, nh, hs = 2, 2, 4, 2, 3
    hidden = nh * hs
    slots = np.array([0, 3, 5, -1, 7])
    source = [np.arange(2 * nb * bs * nh * hs, dtype=np.float32).reshape(2, nb, bs, nh, hs) + layer * 1000
              for layer in range(nl)]
    destination = [np.zeros_like(layer) for layer in source]
    memory = np.empty((2, nl, slots.size, hidden), np.float32)
    ko.list_to_buffer(source, memory, slots)
    ko.buffer_to_list(memory, destination, slots, 0)
    valid = slots[slots >= 0]
    for src_layer, dst_layer in zip(source, destination):
        for axis in range(2):
            src = src_layer[axis].reshape(-1, hidden)
            dst = dst_layer[axis].reshape(-1, hidden)
            assert np.array_equal(dst[valid], src[valid])
            # untouched slots keep the destination's zeros
            others = np.setdiff1d(np.arange(nb * bs), valid)
            assert np.abs(dst[others]).max() == 0
    # the skipped token's buffer row is zero (the gather zeroes the whole buffer first)
    assert np.abs(memory[:, :, 3]).max() == 0


@pytest.mark.parametrize("skip", [0, 3])
def test_buffer_to_list_per_token_loop(skip):
    # _lmcache_kv_buffer_to_paged_list (lmcache_kv_transfer.py:416-437): for each token with
    # slot >= 0, for each layer, kvcache[0|1, block, offset] = memory[0|1, layer, skip + token].
    rng = np.random.default_rng(11)
    nl, nb, bs, nh, hs, t = 3, 5, 4, 2, 3, 17
    hidden = nh * hs
    slots = _dup_slots(nb * bs, t, rng)
    memory = _distinct((2, nl, skip + t + 2, hidden), base=0.5)
    caches = [_distinct((2, nb, bs, nh, hs), base=-1000.0 * (layer + 1)) for layer in range(nl)]
    got = [c.copy() for c in caches]
    ko.buffer_to_list(memory, got, slots, skip)
    want = [c.copy() for c in caches]
    for token_index, slot in enumerate(slots.tolist()):
        if slot < 0:
            continue
        block_id, block_offset = divmod(slot, bs)
        for layer in range(nl):
            want[layer][0, block_id, block_offset] = memory[0, layer, skip + token_index].reshape(nh, hs)
            want[layer][1, block_id, block_offset] = memory[1, layer, skip + token_index].reshape(nh, hs)
    for layer in range(nl):
        assert np.array_equal(got[layer], want[layer]), f"layer {layer}"


def test_buffer_to_list_rejects_plausible_mistakes():
    # The loop above is only a pin if the mistakes it is meant to catch change the result on
    # its inputs.  Each variant here is a wrong restatement; every one must differ from the
    # oracle on the same inputs.
    rng = np.random.default_rng(12)
    nl, nb, bs, nh, hs, t, skip = 2, 4, 4, 2, 2, 13, 2
    hidden = nh * hs
    slots = _dup_slots(nb * bs, t, rng)
    memory = _distinct((2, nl, skip + t, hidden))
    caches = [np.zeros((2, nb, bs, nh, hs), np.float32) for _ in range(nl)]
    good = [c.copy() for c in caches]
    ko.buffer_to_list(memory, good, slots, skip)

    def variant(axis_of, layer_of, row_of, first_wins=False, wrap_negative=False):
        out = [c.copy() for c in caches]
        order = list(enumerate(slots.tolist()))
        if first_wins:
            order = order[::-1]
        for i, s in order:
            if s < 0 and not wrap_negative:
                continue
            b, o = divmod(s, bs)
            for layer in range(nl):
                for axis in range(2):
                    out[layer][axis, b, o] = memory[axis_of(axis, layer), layer_of(axis, layer), row_of(i)].reshape(
                        nh, hs)
        return out

    mistakes = {
        "axis/layer transposed": variant(lambda a, l: l, lambda a, l: a, lambda i: skip + i),
        "skip dropped": variant(lambda a, l: a, lambda a, l: l, lambda i: i),
        "first writer wins": variant(lambda a, l: a, lambda a, l: l, lambda i: skip + i, first_wins=True),
        "negative slot wraps": variant(lambda a, l: a, lambda a, l: l, lambda i: skip + i, wrap_negative=True),
    }
    for name, out in mistakes.items():
        assert not all(np.array_equal(g, o) for g, o in zip(good, out)), name


# ----- the other scatters, each against its reference loop -------------------------------------


def test_linear_to_paged_multi_layer_per_token_loop():
    # kv_linear_to_paged_multi_layer (kv_transfer.py:3382-3457): per layer, per token,
    # cache[layer, block, :, :, offset] = lin[layer, token].
    rng = np.random.default_rng(13)
    nl, nb, nh, hd, bs, t = 3, 4, 2, 3, 4, 15
    slots = _dup_slots(nb * bs, t, rng)
    lin = _distinct((nl, t, nh, hd))
    cache = _distinct((nl, nb, nh, hd, bs), base=-5000.0)
    got = cache.copy()
    ko.linear_to_paged_multi_layer(lin, got, slots)
    want = cache.copy()
    for layer in range(nl):
        for i, s in enumerate(slots.tolist()):
            if s >= 0:
                b, o = divmod(s, bs)
                want[layer, b, :, :, o] = lin[layer, i]
    assert np.array_equal(got, want)


def test_merged_linear_to_paged_per_token_loop():
    # kv_merged_linear_to_paged (kv_transfer.py:3621-3654): merged[:, 0] -> K, merged[:, 1] -> V.
    rng = np.random.default_rng(14)
    nb, nh, hd, bs, t = 3, 2, 4, 4, 11
    slots = _dup_slots(nb * bs, t, rng)
    merged = _distinct((t, 2, nh, hd))
    kc, vc = _distinct((nb, nh, hd, bs), -100.0), _distinct((nb, nh, hd, bs), -900.0)
    gk, gv = kc.copy(), vc.copy()
    ko.merged_linear_to_paged(merged, gk, gv, slots)
    wk, wv = kc.copy(), vc.copy()
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            b, o = divmod(s, bs)
            wk[b, :, :, o] = merged[i, 0]
            wv[b, :, :, o] = merged[i, 1]
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)


def test_flat_linear_to_paged_per_token_loop():
    # _flat_linear_to_paged_scatter (kv_transfer.py:3818-3838): cache[block, offset] = lin[token].
    rng = np.random.default_rng(15)
    nb, bs, d, t = 4, 4, 5, 14
    slots = _dup_slots(nb * bs, t, rng)
    lin = _distinct((t, d))
    cache = _distinct((nb, bs, d), -77.0)
    got = cache.copy()
    ko.flat_linear_to_paged(lin, got, slots)
    want = cache.copy()
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            want[s // bs, s % bs] = lin[i]
    assert np.array_equal(got, want)


def test_buffer_to_six_d_per_token_loop():
    # lmcache_kv_buffer_to_paged (lmcache_kv_transfer.py:84-96): paged[layer, axis, block, offset]
    # = kv_buffer[axis, layer, token] for cache [NL, 2, NB, BS, NH, HS] and buffer [2, NL, T, H].
    rng = np.random.default_rng(16)
    nl, nb, bs, nh, hs, t = 3, 3, 4, 2, 2, 12
    slots = _dup_slots(nb * bs, t, rng)
    buf = _distinct((2, nl, t, nh * hs))
    paged = _distinct((nl, 2, nb, bs, nh, hs), -3000.0)
    got = paged.copy()
    ko.buffer_to_six_d(buf, got, slots)
    want = paged.copy()
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            b, o = divmod(s, bs)
            for layer in range(nl):
                for axis in range(2):
                    want[layer, axis, b, o] = buf[axis, layer, i].reshape(nh, hs)
    assert np.array_equal(got, want)


def test_buffer_to_mla_and_mla_list_per_token_loops():
    # lmcache_kv_buffer_to_paged_mla (lmcache_kv_transfer.py:118-135) and the list form
    # _lmcache_mla_buffer_to_paged_list (:465-481, memory [1, NL, M, HS], skip prefix).
    rng = np.random.default_rng(17)
    nl, nb, bs, hs, t, skip = 3, 3, 4, 5, 10, 2
    slots = _dup_slots(nb * bs, t, rng)
    buf = _distinct((nl, t, hs))
    paged = _distinct((nl, nb, bs, hs), -400.0)
    got = paged.copy()
    ko.buffer_to_mla(buf, got, slots)
    want = paged.copy()
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            for layer in range(nl):
                want[layer, s // bs, s % bs] = buf[layer, i]
    assert np.array_equal(got, want)
    memory = _distinct((1, nl, skip + t, hs), 0.25)
    lists = [_distinct((nb, bs, hs), -10_000.0 * (layer + 1)) for layer in range(nl)]
    got_l = [c.copy() for c in lists]
    ko.buffer_to_mla_list(memory, got_l, slots, skip)
    want_l = [c.copy() for c in lists]
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            for layer in range(nl):
                want_l[layer][s // bs, s % bs] = memory[0, layer, skip + i]
    for g, w in zip(got_l, want_l):
        assert np.array_equal(g, w)


# ----- helpers ------------------------------------------------------------------------------


def test_split_slots_is_divmod_with_skips():
    # slot = block * block_size + offset (kv_transfer.py:12-14); slot < 0 is skipped.
    slots = np.array([0, 1, 15, 16, 17, -1, 31, -5, 48])
    valid, block, offset = ko.split_slots(slots, 16)
    assert valid.tolist() == [True, True, True, True, True, False, True, False, True]
    for s, v, b, o in zip(slots.tolist(), valid, block.tolist(), offset.tolist()):
        if v:
            assert (b, o) == divmod(s, 16)


def test_apply_batch_byte_loop():
    # lmcache_musa_batch_copy_ext.cpp:80-170: entry i copies size[i] bytes from
    # source[i] + source_offset[i] to destination[i] + destination_offset[i].
    rng = np.random.default_rng(18)
    srcs = [rng.integers(0, 256, size=n, dtype=np.uint8) for n in (40, 64, 9)]
    dst_a = np.zeros(96, np.uint8)
    dst_b = np.full(33, 0xEE, np.uint8)
    dsts = [dst_a, dst_b, dst_a]
    sizes, d_off, s_off = [7, 20, 9], [3, 13, 60], [30, 41, 0]
    got = [dst_a.copy(), dst_b.copy()]
    bo.apply_batch([got[0], got[1], got[0]], srcs, sizes, d_off, s_off)
    want = [dst_a.copy(), dst_b.copy()]
    which = [0, 1, 0]
    for i in range(3):
        for k in range(sizes[i]):
            want[which[i]][d_off[i] + k] = srcs[i][s_off[i] + k]
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    # bytes outside the ranges are untouched
    assert np.all(got[1][:13] == 0xEE) and np.all(got[1][33:] == 0xEE)
    assert dsts[0] is dst_a


def test_split_sizes_known_answers():
    # lmcache_musa_batch_copy_plan.py:129-152; op_tests/test_lmcache_musa_batch_copy.py: 10 bytes
    # at host offset 6 with 8-byte registration chunks are cut at host offset 8 and 16.
    assert bo.split_sizes(10, 6, 8) == [2, 8]
    assert bo.split_sizes(10, 6, None) == [10]
    assert bo.split_sizes(16, 0, 8) == [8, 8]
    assert bo.split_sizes(5, 3, 8) == [5]
    assert sum(bo.split_sizes(1000, 7, 64)) == 1000


def test_cachegen_helpers():
    # tensor.float() (kv_transfer.py:1124): bf16 bits widen by a 16-bit shift; float64 rounds.
    bits = np.array([0x3F80, 0xBF80, 0x7F80, 0x0001], np.uint16)
    assert co.to_f32(bits, "bfloat16").tolist()[:3] == [1.0, -1.0, float("inf")]
    assert co.to_f32(bits, "bfloat16")[3] == np.float32(2.0 ** -133)
    assert co.to_f32(np.array([1 + 2.0 ** -30]), "float64")[0] == np.float32(1.0)
    # min/max with NaN propagation (torch's min()/max() propagate NaN)
    mn, mx = co.minmax(np.array([3.0, -2.0, 7.5], np.float32))
    assert (mn, mx) == (np.float32(-2.0), np.float32(7.5))
    assert all(np.isnan(v) for v in co.minmax(np.array([1.0, np.nan], np.float32)))
    # bincount with minlength
    assert co.histogram(np.array([[0, 2], [2, 2]], np.uint8), 4).tolist() == [1, 0, 3, 0]


# ----- the torch-CPU port timed by bench.py's CPU baseline ----------------------------------------


@pytest.mark.parametrize("gather_name,scatter_name", [
    ("paged_to_linear_reference_ops", "linear_to_paged_reference_ops"),
    ("paged_to_linear_vectorised", "linear_to_paged_vectorised"),
])
def test_torch_cpu_port_matches_the_oracle(gather_name, scatter_name):
    import torch

    from oracle import torch_cpu_port as tp

    rng = np.random.default_rng(19)
    nb, nh, hd, bs, t = 6, 2, 8, 16, 70
    slots = _dup_slots(nb * bs, t, rng)
    cache = rng.integers(0, 1 << 16, size=(nb, nh, hd, bs), dtype=np.uint16)
    lin = rng.integers(0, 1 << 16, size=(t, nh, hd), dtype=np.uint16)
    gather = getattr(tp, gather_name)
    scatter = getattr(tp, scatter_name)
    as_t = lambda a: torch.from_numpy(a.astype(np.int32)).to(torch.int16)  # noqa: E731
    got = gather(as_t(cache), torch.from_numpy(slots)).numpy().astype(np.uint16)
    assert np.array_equal(got, ko.paged_to_linear(cache, slots))
    tc = as_t(cache)
    scatter(as_t(lin), tc, torch.from_numpy(slots))
    want = cache.copy()
    ko.linear_to_paged(lin, want, slots)
    assert np.array_equal(tc.numpy().astype(np.uint16), want)
