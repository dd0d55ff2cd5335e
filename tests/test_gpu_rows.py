"""GPU parity: token-row transfers (LMCache, SGLang-MP 2 x NL, MLA, DSV4 byte rows, strided blocks) vs the oracle.

All comparisons are bit-exact on random bit patterns.  Cases include skipped
and duplicated slots, prefix skips, non-contiguous LMCache buffers, byte rows
whose width is not a multiple of any vector size, and empty transfers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from oracle import kv_oracle as ko
from tests.kvgen import bits, make_slots, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _caches_2xnl(nl, nb, bs, nh, hs, dtype, gen):
    return [[random_payload((nb, bs, nh, hs), dtype, gen) for _ in range(nl)] for _ in range(2)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("kind", ["sequences", "skips", "random"])
@pytest.mark.parametrize("nh,hs", [(8, 128), (2, 3), (4, 6), (8, 96)])
def test_two_x_nl_gather_matches_oracle(dtype, kind, nh, hs):
    nl, bs, tokens, mem_tokens = 3, 16, 200, 230
    rng = np.random.default_rng(41)
    gen = torch.Generator().manual_seed(41)
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=tokens)
    caches = _caches_2xnl(nl, nb, bs, nh, hs, dtype, gen)
    memory = random_payload((2, nl, mem_tokens, nh * hs), dtype, gen).to(DEV)
    caches_d = [[c.to(DEV) for c in axis] for axis in caches]
    assert musa_aiter.lmcache_kv_paged_to_buffer(caches_d, memory, torch.from_numpy(slots).to(DEV), bs, nh, hs) is True
    want = np.empty((2, nl, mem_tokens, nh * hs), dtype=bits(memory).dtype)
    ko.two_x_nl_to_buffer([[bits(c) for c in axis] for axis in caches], want, slots)
    assert np.array_equal(bits(memory), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kind", ["sequences", "skips", "duplicates"])
@pytest.mark.parametrize("skip", [0, 5])
@pytest.mark.parametrize("hs", [128, 96])
def test_two_x_nl_scatter_matches_oracle(dtype, kind, skip, hs):
    nl, bs, nh, tokens = 4, 16, 8, 150
    rng = np.random.default_rng(42)
    gen = torch.Generator().manual_seed(42)
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=tokens)
    caches = _caches_2xnl(nl, nb, bs, nh, hs, dtype, gen)
    memory = random_payload((2, nl, tokens + skip + 3, nh * hs), dtype, gen)
    caches_d = [[c.to(DEV) for c in axis] for axis in caches]
    assert musa_aiter.lmcache_kv_buffer_to_paged(memory.to(DEV), caches_d, torch.from_numpy(slots).to(DEV), skip, bs,
                                                 nh, hs) is True
    want = [[bits(c).copy() for c in axis] for axis in caches]
    ko.buffer_to_two_x_nl(bits(memory), want, slots, skip)
    for axis in range(2):
        for layer in range(nl):
            assert np.array_equal(bits(caches_d[axis][layer]), want[axis][layer]), (axis, layer)


def test_two_x_nl_noncontiguous_memory_and_empty():
    # op_tests/test_lmcache_kv_transfer.py:173-211 on the GPU path.
    nl, nb, bs, nh, hs = 2, 1, 2, 1, 2
    caches = [[(torch.arange(nb * bs * nh * hs, dtype=torch.float32).reshape(nb, bs, nh, hs) + a * 100 + l * 10).to(DEV)
               for l in range(nl)] for a in range(2)]
    backing = torch.empty(nl, 2, 2, nh * hs, device=DEV)
    memory = backing.transpose(0, 1)
    assert not memory.is_contiguous()
    slots = torch.tensor([0, 1], dtype=torch.int64, device=DEV)
    assert musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(caches, memory, slots, bs, nh, hs) is True
    for a in range(2):
        for l in range(nl):
            assert torch.equal(memory[a, l], caches[a][l].reshape(2, nh * hs))
    empty = torch.empty(2, nl, 0, nh * hs, device=DEV)
    assert musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(caches, empty, torch.empty(0, dtype=torch.int64, device=DEV),
                                                          bs, nh, hs) is True


def test_two_x_nl_prefix_skip_reference_scenario():
    # op_tests/test_lmcache_kv_transfer.py:118-140.
    nl, nb, bs, nh, hs = 2, 2, 2, 1, 2
    slots = torch.tensor([0, 3], dtype=torch.int32, device=DEV)
    memory = torch.arange(2 * nl * 4 * nh * hs, dtype=torch.float32).reshape(2, nl, 4, nh * hs).to(DEV)
    dest = [[torch.full((nb, bs, nh, hs), -1.0, device=DEV) for _ in range(nl)] for _ in range(2)]
    assert musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(memory, dest, slots, 2, bs, nh, hs) is True
    for a in range(2):
        for l in range(nl):
            flat = dest[a][l].reshape(-1, nh * hs)
            assert torch.equal(flat[0], memory[a, l, 2]) and torch.equal(flat[3], memory[a, l, 3])
            assert torch.equal(flat[1], torch.full_like(flat[1], -1.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_list_and_six_d_layouts_match_oracle(dtype):
    nl, bs, nh, hs, tokens = 3, 16, 4, 64, 170
    rng = np.random.default_rng(43)
    gen = torch.Generator().manual_seed(43)
    slots, nb = make_slots("skips", rng, block_size=bs, tokens=tokens)
    s_d = torch.from_numpy(slots).to(DEV)
    kvcaches = [random_payload((2, nb, bs, nh, hs), dtype, gen) for _ in range(nl)]
    memory = torch.empty(2, nl, tokens, nh * hs, dtype=dtype, device=DEV)
    kv_d = [c.to(DEV) for c in kvcaches]
    musa_aiter.lmcache_kv_paged_to_buffer(kv_d, memory, s_d, bs, nh, hs)
    want = np.empty((2, nl, tokens, nh * hs), dtype=bits(memory).dtype)
    ko.list_to_buffer([bits(c) for c in kvcaches], want, slots)
    assert np.array_equal(bits(memory), want)
    src = random_payload((2, nl, tokens + 4, nh * hs), dtype, gen)
    musa_aiter.lmcache_kv_buffer_to_paged(src.to(DEV), kv_d, s_d, 4, bs, nh, hs)
    want_caches = [bits(c).copy() for c in kvcaches]
    ko.buffer_to_list(bits(src), want_caches, slots, 4)
    for got, exp in zip(kv_d, want_caches):
        assert np.array_equal(bits(got), exp)
    paged = random_payload((nl, 2, nb, bs, nh, hs), dtype, gen)
    paged_d = paged.to(DEV)
    buf = torch.empty(2, nl, tokens, nh * hs, dtype=dtype, device=DEV)
    musa_aiter.lmcache_paged_to_kv_buffer(paged_d, buf, s_d)
    want = np.empty_like(bits(buf))
    ko.six_d_to_buffer(bits(paged), want, slots)
    assert np.array_equal(bits(buf), want)
    src6 = random_payload((2, nl, tokens, nh * hs), dtype, gen)
    musa_aiter.lmcache_kv_buffer_to_paged(src6.to(DEV), paged_d, s_d)
    want6 = bits(paged).copy()
    ko.buffer_to_six_d(bits(src6), want6, slots)
    assert np.array_equal(bits(paged_d), want6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hidden", [576, 5, 64, 520, 1000])
@pytest.mark.parametrize("kind", ["skips", "duplicates"])
def test_lmcache_mla_layouts_match_oracle(dtype, hidden, kind):
    # bf16 rows of 1,152 and 2,000 bytes (whole 128-byte lines and not) and 1,040 bytes (not a
    # multiple of 32) next to tiny rows and fp32 rows above 2 KiB.
    nl, bs, tokens = 3, 64, 300
    rng = np.random.default_rng(44)
    gen = torch.Generator().manual_seed(44)
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=tokens)
    s_d = torch.from_numpy(slots).to(DEV)
    paged = random_payload((nl, nb, bs, hidden), dtype, gen)
    paged_d = paged.to(DEV)
    buf = torch.empty(nl, tokens, hidden, dtype=dtype, device=DEV)
    musa_aiter.lmcache_paged_to_kv_buffer_mla(paged_d, buf, s_d)
    want = np.empty_like(bits(buf))
    ko.mla_to_buffer(bits(paged), want, slots)
    assert np.array_equal(bits(buf), want)
    src = random_payload((nl, tokens, hidden), dtype, gen)
    musa_aiter.lmcache_kv_buffer_to_paged_mla(src.to(DEV), paged_d, s_d)
    want_p = bits(paged).copy()
    ko.buffer_to_mla(bits(src), want_p, slots)
    assert np.array_equal(bits(paged_d), want_p)
    lists = [random_payload((nb, bs, hidden), dtype, gen) for _ in range(nl)]
    lists_d = [c.to(DEV) for c in lists]
    mem = torch.empty(1, nl, tokens + 6, hidden, dtype=dtype, device=DEV)
    musa_aiter.lmcache_mla_paged_to_buffer(lists_d, mem, s_d, bs, hidden)
    want_m = np.empty_like(bits(mem))
    ko.mla_list_to_buffer([bits(c) for c in lists], want_m, slots)
    assert np.array_equal(bits(mem), want_m)
    src_m = random_payload((1, nl, tokens + 6, hidden), dtype, gen)
    musa_aiter.lmcache_mla_buffer_to_paged(src_m.to(DEV), lists_d, s_d, 6, bs, hidden)
    want_l = [bits(c).copy() for c in lists]
    ko.buffer_to_mla_list(bits(src_m), want_l, slots, 6)
    for got, exp in zip(lists_d, want_l):
        assert np.array_equal(bits(got), exp)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("layers", [None, 4])
def test_mla_split_caches_match_oracle(dtype, layers):
    bs, kv_dim, pe_dim, tokens = 64, 512, 64, 333
    rng = np.random.default_rng(45)
    gen = torch.Generator().manual_seed(45)
    slots, nb = make_slots("skips", rng, block_size=bs, tokens=tokens)
    s_d = torch.from_numpy(slots).to(DEV)
    lead = () if layers is None else (layers,)
    kvc = random_payload(lead + (nb, bs, kv_dim), dtype, gen)
    pec = random_payload(lead + (nb, bs, pe_dim), dtype, gen)
    kvc_d, pec_d = kvc.to(DEV), pec.to(DEV)
    if layers is None:
        okv, ope = musa_aiter.kv_paged_to_mla_linear(kvc_d, pec_d, s_d)
        assert np.array_equal(bits(okv), ko.flat_paged_to_linear(bits(kvc), slots))
        assert np.array_equal(bits(ope), ko.flat_paged_to_linear(bits(pec), slots))
    else:
        okv, ope = musa_aiter.kv_paged_to_mla_linear_multi_layer(kvc_d, pec_d, s_d)
        for layer in range(layers):
            assert np.array_equal(bits(okv[layer]), ko.flat_paged_to_linear(bits(kvc)[layer], slots))
            assert np.array_equal(bits(ope[layer]), ko.flat_paged_to_linear(bits(pec)[layer], slots))
    lin_kv = random_payload(tuple(okv.shape), dtype, gen)
    lin_pe = random_payload(tuple(ope.shape), dtype, gen)
    want_kv, want_pe = bits(kvc).copy(), bits(pec).copy()
    if layers is None:
        musa_aiter.kv_mla_linear_to_paged(lin_kv.to(DEV), lin_pe.to(DEV), kvc_d, pec_d, s_d)
        ko.flat_linear_to_paged(bits(lin_kv), want_kv, slots)
        ko.flat_linear_to_paged(bits(lin_pe), want_pe, slots)
    else:
        assert musa_aiter.kv_mla_linear_to_paged_multi_layer(lin_kv.to(DEV), lin_pe.to(DEV), kvc_d, pec_d, s_d) is True
        for layer in range(layers):
            ko.flat_linear_to_paged(bits(lin_kv)[layer], want_kv[layer], slots)
            ko.flat_linear_to_paged(bits(lin_pe)[layer], want_pe[layer], slots)
    assert np.array_equal(bits(kvc_d), want_kv)
    assert np.array_equal(bits(pec_d), want_pe)


@pytest.mark.parametrize("item_bytes", [1, 1728, 1729, 37439, 37440, 656])
def test_copy_paged_rows_matches_index_copy(item_bytes):
    # op_tests/test_kv_copy_paged_rows_correctness.py:31-104 shapes.
    g = torch.Generator().manual_seed(7)
    src = torch.randint(0, 256, (16, item_bytes), dtype=torch.uint8, generator=g)
    dst = torch.zeros(16, item_bytes, dtype=torch.uint8)
    src_idx = torch.randperm(16, generator=g)[:8]
    dst_idx = torch.randperm(16, generator=g)[:8]
    dst_d = dst.to(DEV)
    musa_aiter.kv_copy_paged_rows(src.to(DEV), dst_d, src_idx.to(DEV), dst_idx.to(DEV))
    want = dst.numpy().copy()
    ko.copy_rows(src.numpy(), want, src_idx.numpy(), dst_idx.numpy())
    assert np.array_equal(dst_d.cpu().numpy(), want)


def test_copy_paged_rows_duplicates_and_layer_table():
    src = torch.randint(0, 256, (8, 256), dtype=torch.uint8)
    dst = torch.zeros(4, 256, dtype=torch.uint8)
    src_idx = torch.arange(8)
    dst_idx = torch.tensor([1, 1, 2, 2, 3, 3, 0, 0])
    dst_d = dst.to(DEV)
    musa_aiter.kv_copy_paged_rows(src.to(DEV), dst_d, src_idx.to(DEV), dst_idx.to(DEV))
    ref = torch.zeros(4, 256, dtype=torch.uint8)
    ref.index_copy_(0, dst_idx, src.index_select(0, src_idx))
    assert torch.equal(dst_d.cpu(), ref)
    layers, pages, item = 43, 64, 1728
    g = torch.Generator().manual_seed(21)
    srcs = [torch.randint(0, 256, (pages, item), dtype=torch.uint8, generator=g) for _ in range(layers)]
    dsts = [torch.zeros(pages, item, dtype=torch.uint8, device=DEV) for _ in range(layers)]
    si = torch.randperm(pages, generator=g)[:16]
    di = torch.randperm(pages, generator=g)[:16]
    musa_aiter.kv_copy_paged_rows_layer_table([s.to(DEV) for s in srcs], dsts, si.to(DEV), di.to(DEV))
    for layer in range(layers):
        ref = torch.zeros(pages, item, dtype=torch.uint8)
        ref.index_copy_(0, di, srcs[layer].index_select(0, si))
        assert torch.equal(dsts[layer].cpu(), ref), layer


def test_multi_pool_shared_indices():
    pages = 32
    specs = [(2, 37440), (3, 1728), (1, 4096), (4, 1024), (1, 512), (2, 256)]
    g = torch.Generator().manual_seed(5)
    idx = torch.randperm(pages, generator=g)[:12]
    pools, refs = [], []
    for layers, item in specs:
        srcs = [torch.randint(0, 256, (pages, item), dtype=torch.uint8, generator=g) for _ in range(layers)]
        dsts = [torch.zeros(pages, item, dtype=torch.uint8, device=DEV) for _ in range(layers)]
        pools.append(musa_aiter.PoolSpec([s.to(DEV) for s in srcs], dsts, item))
        refs.append(srcs)
    musa_aiter.kv_copy_paged_rows_multi_pool(pools, idx.to(DEV), direction="H2D")
    for pool, srcs in zip(pools, refs):
        for src, dst in zip(srcs, pool.dst_ptrs):
            ref = torch.zeros_like(src)
            ref.index_copy_(0, idx, src.index_select(0, idx))
            assert torch.equal(dst.cpu(), ref)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("direction", [0, 1])
def test_strided_block_transfer_matches_oracle(mode, direction):
    nl, bs, nb, row, value, scale = 3, 64, 12, 656, 640, 16
    stride = bs * row + 256  # padded pages
    staging_tokens, offset = 5 * bs + 7, 3
    g = torch.Generator().manual_seed(9)
    pages = [torch.randint(0, 256, (nb * stride,), dtype=torch.uint8, generator=g) for _ in range(nl)]
    staging = torch.randint(0, 256, (nl * staging_tokens * row,), dtype=torch.uint8, generator=g)
    block_ids = torch.tensor([7, 2, 9, 0, 11], dtype=torch.int64)
    pages_d = [p.to(DEV) for p in pages]
    staging_d = staging.to(DEV)
    ok = musa_aiter.lmcache_kv_strided_block_transfer(
        staging_d, [p.data_ptr() for p in pages_d], block_ids.to(DEV), direction, nl, 1, 4, offset, staging_tokens, bs,
        row, stride, mode, value if mode else 0, scale if mode else 0)
    assert ok is True
    want_pages = [p.numpy().copy() for p in pages]
    want_staging = staging.numpy().copy()
    ko.strided_block_transfer(want_staging, want_pages, block_ids.numpy(), direction=direction, idx_start=1, n_valid=4,
                              offset_in_object=offset, staging_tokens=staging_tokens, block_size=bs, row_bytes=row,
                              paged_block_stride=stride, mode=mode, value_bytes=value if mode else 0,
                              scale_bytes=scale if mode else 0)
    assert np.array_equal(staging_d.cpu().numpy(), want_staging)
    for got, exp in zip(pages_d, want_pages):
        assert np.array_equal(got.cpu().numpy(), exp)


@pytest.mark.parametrize("row", [48, 7, 2048])
def test_copy_rows_plane_inner_grid_zero_fills_skipped_and_tail_rows(row):
    # Destination planes interleaved inside rows (a [rows, planes, row] buffer): the row launcher walks
    # planes inside rows.  Skipped tokens and rows past num_tokens of this directly addressed
    # destination must still be zero filled in every plane.
    from musa_aiter.ops import _hip

    planes, rows_out, tokens, src_rows = 5, 40, 33, 64
    rng = np.random.default_rng(row)
    gen = torch.Generator().manual_seed(row)
    srcs = [random_payload((src_rows, row), torch.uint8, gen) for _ in range(planes)]
    idx = rng.integers(-1, src_rows + 3, size=tokens).astype(np.int64)   # -1 and out-of-range skip
    dst = torch.full((rows_out, planes, row), 0xAB, dtype=torch.uint8, device=DEV)
    srcs_d = [s.to(DEV) for s in srcs]
    idx_d = torch.from_numpy(idx).to(DEV)
    _hip.copy_rows(op="plane-inner test", device=dst.device, src_planes=[s.data_ptr() for s in srcs_d],
                   dst_planes=[dst.data_ptr() + p * row for p in range(planes)], num_planes=planes, src_idx=idx_d,
                   dst_idx=None, num_tokens=tokens, num_rows_out=rows_out, src_rows=src_rows, dst_rows=rows_out,
                   row_bytes=row, src_stride=row, dst_stride=planes * row, zero_invalid=True)
    want = np.zeros((rows_out, planes, row), dtype=np.uint8)
    for r in range(tokens):
        if 0 <= idx[r] < src_rows:
            for p in range(planes):
                want[r, p] = srcs[p].numpy()[idx[r]]
    assert np.array_equal(dst.cpu().numpy(), want)
