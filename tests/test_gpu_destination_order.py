"""GPU parity of the destination-order scatters on slot mappings built to stress them.

A scatter whose tokens cover a good share of the destination (a quarter of the slots for the
paged-A tile and FP8 kernels, half of the rows for the row kernels) runs destination-major:
its claim pass records, per destination slot, the last token that writes it, and the copy walks
the destination in address order, rebuilding runs of consecutive tokens from those tags.  The
mappings below cover most of the cache and put into single blocks every run shape that
reconstruction has to get right -- a block written by two runs from distant tokens, a block
written in reverse (one-slot runs), a run split by a later duplicate token, a partial block,
every other slot, untouched blocks, skipped tokens and repeated slots -- and each result is
compared bit for bit with the oracle (last writer in token order, untouched rows preserved).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from oracle import kv_oracle as ko
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def tricky_slots(rng: np.random.Generator, nb: int, bs: int) -> np.ndarray:
    """A slot mapping over nb blocks of bs slots with the run shapes listed in the module docstring."""
    assert nb >= 12
    half = bs // 2
    order: list[int] = []
    order += list(range(0, half))                               # block 0, first half (second half at the end)
    order += list(range(2 * bs - 1, bs - 1, -1))                # block 1 in reverse
    order += list(range(2 * bs, 3 * bs))                        # block 2, later split by a duplicate
    order += list(range(3 * bs + 1, 4 * bs - 2))                # block 3, partial
    order += list(range(5 * bs, 6 * bs, 2))                     # block 5, every other slot; block 4 untouched
    rest = [b for b in range(6, nb) if b not in (8, 11)]         # blocks 8 and 11 untouched
    for b in rng.permutation(rest).tolist():
        n = bs if rng.random() < 0.8 else int(rng.integers(1, bs))
        order += list(range(b * bs, b * bs + n))
    order.append(2 * bs + half)                                 # duplicate in the middle of block 2's run
    order += list(range(half, bs))                              # block 0, second half
    slots = np.array(order, dtype=np.int64)
    skip = rng.random(len(slots)) < 0.03
    slots[skip] = -1
    dups = rng.choice(len(slots), size=max(1, len(slots) // 40), replace=False)
    tail = slots[dups].copy()                                   # repeat some slots (the later copy wins)
    return np.concatenate([slots, tail, np.array([-1, -1], dtype=np.int64)])


def _covers(slots: np.ndarray, rows: int, share: int) -> bool:
    return len(slots) * share >= rows


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_paged_multi_layer_scatter_in_destination_order(dtype, bs):
    nl, nh, hd, nb = 3, 4, 64, 24
    rng = np.random.default_rng(100 + bs)
    gen = torch.Generator().manual_seed(bs)
    slots = tricky_slots(rng, nb, bs)
    assert _covers(slots, nb * bs, 4)
    t = len(slots)
    kl, vl = (random_payload((nl, t, nh, hd), dtype, gen) for _ in range(2))
    kc, vc = (random_payload((nl, nb, nh, hd, bs), dtype, gen) for _ in range(2))
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged_multi_layer(kl.to(DEV), vl.to(DEV), kc_d, vc_d, torch.from_numpy(slots).to(DEV))
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged_multi_layer(bits(kl), want_k, slots)
    ko.linear_to_paged_multi_layer(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)
    # Single layer and merged K/V through the same kernels.
    musa_aiter.kv_linear_to_paged(kl[1].to(DEV), vl[1].to(DEV), kc_d[0], vc_d[0], torch.from_numpy(slots).to(DEV))
    ko.linear_to_paged(bits(kl[1]), want_k[0], slots)
    ko.linear_to_paged(bits(vl[1]), want_v[0], slots)
    merged = torch.stack([kl[2], vl[2]], 1).contiguous()
    musa_aiter.kv_merged_linear_to_paged(merged.to(DEV), kc_d[2], vc_d[2], torch.from_numpy(slots).to(DEV))
    ko.merged_linear_to_paged(bits(merged), want_k[2], want_v[2], slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


@pytest.mark.parametrize("nh, hd", [(2, 64), (5, 64), (10, 128), (9, 120)])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_paged_scatter_in_destination_order_row_counts(nh, hd, bs):
    # 16-bit scatters over few planes run one workgroup per cache block, its waves consecutive chunks of
    # 512, 256 or 128 rows (block size 8, 16, 32): row counts of 128 ... 1,280 give blocks of one
    # partial chunk, of fewer chunks than waves, and of more (a second grid z) with a partial last chunk.
    nl, nb = 2, 14
    rng = np.random.default_rng(nh * 100 + hd + bs)
    gen = torch.Generator().manual_seed(nh + hd + bs)
    slots = tricky_slots(rng, nb, bs)
    assert _covers(slots, nb * bs, 4)
    t = len(slots)
    kl, vl = (random_payload((nl, t, nh, hd), torch.bfloat16, gen) for _ in range(2))
    kc, vc = (random_payload((nl, nb, nh, hd, bs), torch.bfloat16, gen) for _ in range(2))
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged_multi_layer(kl.to(DEV), vl.to(DEV), kc_d, vc_d, torch.from_numpy(slots).to(DEV))
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged_multi_layer(bits(kl), want_k, slots)
    ko.linear_to_paged_multi_layer(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("lin", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bs", [16, 32])
def test_fp8_quant_store_in_destination_order(fmt, lin, bs):
    nh, hd, nb = 8, 128, 20
    rng = np.random.default_rng(200 + bs)
    slots = tricky_slots(rng, nb, bs)
    assert _covers(slots, nb * bs, 4)
    t = len(slots)
    gen = torch.Generator().manual_seed(7)
    k = (torch.randn((t, nh, hd), generator=gen) * 3).to(lin)
    v = (torch.randn((t, nh, hd), generator=gen) * 3).to(lin)
    ks = (torch.rand(nh, generator=gen) * 0.02 + 0.001).to(torch.float32)
    vs = torch.tensor(0.0071, dtype=torch.float32)
    kc = torch.randint(0, 256, (nb, nh, hd, bs), dtype=torch.uint8, generator=gen)
    vc = torch.randint(0, 256, (nb, nh, hd, bs), dtype=torch.uint8, generator=gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged_fp8(k.to(DEV), v.to(DEV), kc_d, vc_d, torch.from_numpy(slots).to(DEV), ks.to(DEV),
                                      vs.to(DEV), fp8_format=fmt)
    want_k, want_v = kc.numpy().copy(), vc.numpy().copy()
    ko.linear_to_paged_fp8(k.to(torch.float32).numpy(), want_k, slots, ks.numpy(), fmt)
    ko.linear_to_paged_fp8(v.to(torch.float32).numpy(), want_v, slots, vs.numpy(), fmt)
    assert np.array_equal(kc_d.cpu().numpy(), want_k)
    assert np.array_equal(vc_d.cpu().numpy(), want_v)


@pytest.mark.parametrize("nh, hd", [(2, 64), (5, 64), (10, 128), (9, 120)])
@pytest.mark.parametrize("lin", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bs", [16, 32])
def test_fp8_quant_store_in_destination_order_row_counts(nh, hd, lin, bs):
    # A workgroup takes one cache block, its waves consecutive row chunks (256 rows for bf16 at block
    # size 16, 128 for fp32 or block size 32, 64 for both): row counts of 128 ... 1,280 give blocks of
    # one partial chunk, of fewer chunks than waves (idle waves), and of more (a second grid z) with a
    # partial last chunk.
    nb = 14
    rng = np.random.default_rng(nh * 1000 + hd + bs)
    slots = tricky_slots(rng, nb, bs)
    assert _covers(slots, nb * bs, 4)
    t = len(slots)
    gen = torch.Generator().manual_seed(nh + hd)
    k = (torch.randn((t, nh, hd), generator=gen) * 3).to(lin)
    v = (torch.randn((t, nh, hd), generator=gen) * 3).to(lin)
    ks = (torch.rand(nh, generator=gen) * 0.02 + 0.001).to(torch.float32)
    vs = (torch.rand(nh, generator=gen) * 0.02 + 0.001).to(torch.float32)
    kc = torch.randint(0, 256, (nb, nh, hd, bs), dtype=torch.uint8, generator=gen)
    vc = torch.randint(0, 256, (nb, nh, hd, bs), dtype=torch.uint8, generator=gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    s_d = torch.from_numpy(slots).to(DEV)
    musa_aiter.kv_linear_to_paged_fp8(k.to(DEV), v.to(DEV), kc_d, vc_d, s_d, ks.to(DEV), vs.to(DEV), fp8_format="e4m3")
    want_k, want_v = kc.numpy().copy(), vc.numpy().copy()
    ko.linear_to_paged_fp8(k.to(torch.float32).numpy(), want_k, slots, ks.numpy(), "e4m3")
    ko.linear_to_paged_fp8(v.to(torch.float32).numpy(), want_v, slots, vs.numpy(), "e4m3")
    assert np.array_equal(kc_d.cpu().numpy(), want_k)
    assert np.array_equal(vc_d.cpu().numpy(), want_v)


@pytest.mark.parametrize("hidden", [576, 328])
def test_mla_rows_scatter_in_destination_order(hidden):
    # 1,152-byte bf16 rows (whole lines) and 656-byte ones.
    nl, bs, nb = 2, 64, 14
    rng = np.random.default_rng(300 + hidden)
    gen = torch.Generator().manual_seed(hidden)
    slots = tricky_slots(rng, nb, bs)
    assert _covers(slots, nb * bs, 2)
    t = len(slots)
    paged = random_payload((nl, nb, bs, hidden), torch.bfloat16, gen)
    src = random_payload((nl, t, hidden), torch.bfloat16, gen)
    paged_d = paged.to(DEV)
    assert musa_aiter.lmcache_kv_buffer_to_paged_mla(src.to(DEV), paged_d, torch.from_numpy(slots).to(DEV))
    want = bits(paged).copy()
    ko.buffer_to_mla(bits(src), want, slots)
    assert np.array_equal(bits(paged_d), want)


def test_two_x_nl_scatter_in_destination_order():
    nl, bs, nh, hs, nb = 3, 16, 8, 128, 16
    rng = np.random.default_rng(400)
    gen = torch.Generator().manual_seed(400)
    slots = tricky_slots(rng, nb, bs)
    assert _covers(slots, nb * bs, 2)
    t = len(slots)
    caches = [[random_payload((nb, bs, nh, hs), torch.bfloat16, gen) for _ in range(nl)] for _ in range(2)]
    memory = random_payload((2, nl, t + 4, nh * hs), torch.bfloat16, gen)
    caches_d = [[c.to(DEV) for c in axis] for axis in caches]
    assert musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(memory.to(DEV), caches_d, torch.from_numpy(slots).to(DEV),
                                                          4, bs, nh, hs)
    want = [[bits(c).copy() for c in axis] for axis in caches]
    ko.buffer_to_two_x_nl(bits(memory), want, slots, 4)
    for axis in range(2):
        for layer in range(nl):
            assert np.array_equal(bits(caches_d[axis][layer]), want[axis][layer]), (axis, layer)


def test_byte_rows_copy_in_destination_order():
    rows, item = 512, 656
    rng = np.random.default_rng(500)
    gen = torch.Generator().manual_seed(500)
    dst_idx = tricky_slots(rng, rows // 16, 16)
    dst_idx = dst_idx[dst_idx >= 0]                 # byte-row copies take no negative indices
    assert _covers(dst_idx, rows, 2)
    n = len(dst_idx)
    src_idx = rng.integers(0, 700, size=n)
    src = torch.randint(0, 256, (700, item), dtype=torch.uint8, generator=gen)
    dst = torch.randint(0, 256, (rows, item), dtype=torch.uint8, generator=gen)
    dst_d = dst.to(DEV)
    musa_aiter.kv_copy_paged_rows(src.to(DEV), dst_d, torch.from_numpy(src_idx).to(DEV),
                                  torch.from_numpy(dst_idx).to(DEV))
    want = dst.numpy().copy()
    ko.copy_rows(src.numpy(), want, src_idx, dst_idx)
    assert np.array_equal(dst_d.cpu().numpy(), want)


def test_scatters_repeat_with_advancing_epochs():
    # The same caller-owned tag array serves consecutive calls (one epoch each): a second scatter with a
    # different mapping must not see the first call's tags as its own.
    nl, nh, hd, bs, nb = 2, 4, 64, 16, 16
    rng = np.random.default_rng(600)
    gen = torch.Generator().manual_seed(600)
    kc = random_payload((nl, nb, nh, hd, bs), torch.bfloat16, gen)
    vc = random_payload((nl, nb, nh, hd, bs), torch.bfloat16, gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    for rep in range(3):
        slots = tricky_slots(rng, nb, bs)
        if rep == 2:
            slots = slots[: len(slots) // 6]  # below the coverage threshold: the token-order kernel
        t = len(slots)
        kl, vl = (random_payload((nl, t, nh, hd), torch.bfloat16, gen) for _ in range(2))
        musa_aiter.kv_linear_to_paged_multi_layer(kl.to(DEV), vl.to(DEV), kc_d, vc_d, torch.from_numpy(slots).to(DEV))
        ko.linear_to_paged_multi_layer(bits(kl), want_k, slots)
        ko.linear_to_paged_multi_layer(bits(vl), want_v, slots)
        assert np.array_equal(bits(kc_d), want_k), rep
        assert np.array_equal(bits(vc_d), want_v), rep
