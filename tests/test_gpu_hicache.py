"""GPU parity: SGLang HiCache transfers vs oracle/hicache_oracle.py, bit-exact.

Covers the eight layout-transfer functions (K/V and MLA, layer-first and page-first), the
reference's own CPU and native test cases run on the GPU, skipped (-1) and duplicated pages,
int32 and host-resident index tables, the caller's current stream, item widths of one to many
vectors, empty tables, a large round trip, the three direct token-range functions (consecutive
pages, breaks inside pages, runs past the tables, broadcast pages) and the reference-named C-ABI
entry musa_aiter_hicache_transfer_bytes.
"""

from __future__ import annotations

import ctypes
import itertools

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops import _hip
from oracle import hicache_oracle as ho
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"

# function -> (src_layout, dst_layout, per_layer, mla)
LAYOUT_FNS = {
    "hicache_transfer_kv_per_layer": ("layer_first", "layer_first", True, False),
    "hicache_transfer_kv_per_layer_pf_lf": ("page_first", "layer_first", True, False),
    "hicache_transfer_kv_all_layer": ("layer_first", "layer_first", False, False),
    "hicache_transfer_kv_all_layer_lf_pf": ("layer_first", "page_first", False, False),
    "hicache_transfer_kv_per_layer_mla": ("layer_first", "layer_first", True, True),
    "hicache_transfer_kv_per_layer_mla_pf_lf": ("page_first", "layer_first", True, True),
    "hicache_transfer_kv_all_layer_mla": ("layer_first", "layer_first", False, True),
    "hicache_transfer_kv_all_layer_mla_lf_pf": ("layer_first", "page_first", False, True),
}


def _shape(layout, layers, pages, item):
    return (layers, pages, item) if layout == "layer_first" else (pages, layers, item)


def _pairs(kind, rng, n, src_pages, dst_pages):
    src = rng.integers(0, src_pages, size=n).astype(np.int64)
    if kind == "duplicates":
        dst = rng.integers(0, max(1, dst_pages // 4), size=n).astype(np.int64)
    else:
        dst = rng.permutation(dst_pages)[:n].astype(np.int64)
    if kind in ("skips", "duplicates"):
        src[rng.random(n) < 0.2] = -1
        dst[rng.random(n) < 0.1] = -1
    return src, dst


def _run_layout(name, dtype, item, kind, *, layers=4, src_pages=37, dst_pages=41, n=29, layer_id=2,
                index_dtype=torch.int64, index_device=DEV, seed=0):
    src_layout, dst_layout, per_layer, mla = LAYOUT_FNS[name]
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    src_idx, dst_idx = _pairs(kind, rng, n, src_pages, dst_pages)
    planes = 1 if mla else 2
    src = [random_payload(_shape(src_layout, layers, src_pages, item), dtype, gen).to(DEV) for _ in range(planes)]
    dst = [random_payload(_shape(dst_layout, layers, dst_pages, item), dtype, gen).to(DEV) for _ in range(planes)]
    want = [bits(d).copy() for d in dst]
    si = torch.from_numpy(src_idx).to(index_dtype).to(index_device)
    di = torch.from_numpy(dst_idx).to(index_dtype).to(index_device)
    fn = getattr(musa_aiter, name)
    kwargs = {"layer_id": layer_id} if per_layer else {}
    if mla:
        assert fn(src[0], dst[0], si, di, **kwargs) is True
    else:
        assert fn(src[0], dst[0], src[1], dst[1], si, di, **kwargs) is True
    start, count = (layer_id, 1) if per_layer else (0, layers)
    ho.transfer(bits(src[0]), want[0], None if mla else bits(src[1]), None if mla else want[1], src_idx, dst_idx,
                src_layout=src_layout, dst_layout=dst_layout, start_layer=start, num_layers=count)
    for p in range(planes):
        assert np.array_equal(bits(dst[p]), want[p]), (name, p)


@pytest.mark.parametrize("name", list(LAYOUT_FNS))
@pytest.mark.parametrize("dtype,item", [(torch.bfloat16, 1024), (torch.float16, 4), (torch.float32, 6),
                                        (torch.uint8, 40), (torch.bfloat16, 40)])
@pytest.mark.parametrize("kind", ["unique", "skips", "duplicates"])
def test_layout_transfers_match_oracle(name, dtype, item, kind):
    _run_layout(name, dtype, item, kind)


@pytest.mark.parametrize("name", ["hicache_transfer_kv_per_layer_pf_lf", "hicache_transfer_kv_all_layer_mla_lf_pf"])
@pytest.mark.parametrize("index_dtype,index_device", [(torch.int32, DEV), (torch.int64, "cpu"), (torch.int32, "cpu")])
def test_layout_transfers_accept_int32_and_host_index_tables(name, index_dtype, index_device):
    _run_layout(name, torch.float16, 64, "skips", index_dtype=index_dtype, index_device=index_device, seed=5)


@pytest.mark.parametrize("name", list(LAYOUT_FNS))
def test_layout_transfers_empty_and_all_skipped_tables(name):
    _run_layout(name, torch.bfloat16, 16, "unique", n=0)
    src_layout, dst_layout, per_layer, mla = LAYOUT_FNS[name]
    k = torch.ones(_shape(src_layout, 2, 3, 8), dtype=torch.float16, device=DEV)
    d = torch.zeros(_shape(dst_layout, 2, 3, 8), dtype=torch.float16, device=DEV)
    args = (k, d) if mla else (k, d, k.clone(), d.clone())
    idx = torch.tensor([-1, -1], dtype=torch.int64, device=DEV)
    assert getattr(musa_aiter, name)(*args, idx, torch.tensor([0, 1], device=DEV)) is True
    assert torch.count_nonzero(d) == 0


def test_reference_cpu_cases_on_gpu():
    # op_tests/test_hicache_transfer.py:27-141 with device tensors.
    key = torch.arange(2 * 4 * 8, dtype=torch.float32, device=DEV).reshape(2, 4, 8)
    value = key + 10000
    dst_k, dst_v = torch.zeros_like(key), torch.zeros_like(value)
    assert musa_aiter.hicache_transfer_kv_per_layer(key, dst_k, value, dst_v, torch.tensor([3, 1], device=DEV),
                                                    torch.tensor([0, 2], device=DEV), layer_id=1)
    torch.cuda.synchronize()
    assert torch.equal(dst_k[1, 0], key[1, 3]) and torch.equal(dst_k[1, 2], key[1, 1])
    assert torch.count_nonzero(dst_k[0]) == 0 and torch.equal(dst_v[1, 0], value[1, 3])

    dst_k, dst_v = torch.full_like(key, -1), torch.full_like(value, -1)
    assert musa_aiter.hicache_transfer_kv_all_layer(key, dst_k, value, dst_v, torch.tensor([-1, 1], device=DEV),
                                                    torch.tensor([0, 2], device=DEV))
    assert torch.equal(dst_k[:, 2], key[:, 1]) and torch.equal(dst_v[:, 2], value[:, 1])
    assert torch.all(dst_k[:, 0] == -1)

    src = torch.arange(2 * 4 * 6, dtype=torch.float32, device=DEV).reshape(2, 4, 6)
    dst = torch.zeros(4, 2, 6, device=DEV)
    assert musa_aiter.hicache_transfer_kv_all_layer_mla_lf_pf(src, dst, torch.tensor([-1, 1, 3], device=DEV),
                                                              torch.tensor([0, 2, 1], device=DEV))
    assert torch.equal(dst[2], src[:, 1]) and torch.equal(dst[1], src[:, 3]) and torch.all(dst[0] == 0)


def test_reference_native_cases_current_stream():
    # op_tests/test_hicache_transfer_musa.py:22-105 with a side stream.
    layers, pages, item = 2, 4, 8
    src_k = torch.arange(layers * pages * item, dtype=torch.float16, device=DEV).reshape(layers, pages, item)
    src_v = src_k + 2000
    dst_k = torch.zeros((pages, layers, item), dtype=torch.float16, device=DEV)
    dst_v = torch.zeros_like(dst_k)
    si = torch.tensor([0, 2], dtype=torch.int64, device=DEV)
    di = torch.tensor([1, 3], dtype=torch.int64, device=DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        assert musa_aiter.hicache_transfer_kv_all_layer_lf_pf(src_k, dst_k, src_v, dst_v, si, di)
    stream.synchronize()
    assert torch.equal(dst_k[1, 0], src_k[0, 0]) and torch.equal(dst_k[1, 1], src_k[1, 0])
    assert torch.equal(dst_k[3, 0], src_k[0, 2]) and torch.equal(dst_v[3, 1], src_v[1, 2])

    src_pf = torch.arange(pages * layers * item, dtype=torch.float16, device=DEV).reshape(pages, layers, item)
    dst_lf = torch.zeros((layers, pages, item), dtype=torch.float16, device=DEV)
    dst_lf_v = torch.zeros_like(dst_lf)
    assert musa_aiter.hicache_transfer_kv_per_layer_pf_lf(src_pf, dst_lf, src_pf + 1000, dst_lf_v,
                                                          torch.tensor([3, 1], device=DEV),
                                                          torch.tensor([0, 2], device=DEV), layer_id=1)
    torch.cuda.synchronize()
    assert torch.equal(dst_lf[1, 0], src_pf[3, 1]) and torch.equal(dst_lf[1, 2], src_pf[1, 1])
    assert torch.equal(dst_lf_v[1, 0], src_pf[3, 1] + 1000)


def test_large_round_trip_layer_first_page_first():
    # Device cache [layers, tokens, item] -> host-style page-first pool and back, all 8 layers.
    layers, pages, item = 8, 4096, 512
    gen = torch.Generator().manual_seed(9)
    dev_k = random_payload((layers, pages, item), torch.bfloat16, gen).to(DEV)
    dev_v = random_payload((layers, pages, item), torch.bfloat16, gen).to(DEV)
    pool_k = torch.zeros((pages, layers, item), dtype=torch.bfloat16, device=DEV)
    pool_v = torch.zeros_like(pool_k)
    sel = torch.randperm(pages, generator=gen)[:3000].to(DEV)
    slots = torch.randperm(pages, generator=gen)[:3000].to(DEV)
    assert musa_aiter.hicache_transfer_kv_all_layer_lf_pf(dev_k, pool_k, dev_v, pool_v, sel, slots)
    back_k, back_v = torch.zeros_like(dev_k), torch.zeros_like(dev_v)
    for layer in range(layers):
        assert musa_aiter.hicache_transfer_kv_per_layer_pf_lf(pool_k, back_k, pool_v, back_v, slots, sel,
                                                              layer_id=layer)
    torch.cuda.synchronize()
    kb, bb = dev_k.view(torch.int16), back_k.view(torch.int16)
    assert torch.equal(bb[:, sel], kb[:, sel])
    assert torch.equal(back_v.view(torch.int16)[:, sel], dev_v.view(torch.int16)[:, sel])
    assert torch.equal(pool_k.view(torch.int16)[slots], kb[:, sel].transpose(0, 1))
    untouched = torch.ones(pages, dtype=torch.bool, device=DEV)
    untouched[sel] = False
    assert torch.count_nonzero(bb[:, untouched]) == 0


# ----- reference-named C-ABI entry ---------------------------------------------------------


@pytest.mark.parametrize("src_layout,dst_layout", list(itertools.product(["layer_first", "page_first"], repeat=2)))
@pytest.mark.parametrize("item_bytes,with_v", [(2048, True), (24, True), (20, False), (8, True)])
def test_c_abi_transfer_bytes_matches_kernel_contract(src_layout, dst_layout, item_bytes, with_v):
    rng = np.random.default_rng(item_bytes)
    layers, src_pages, dst_pages, n, start, count = 5, 23, 19, 17, 1, 3
    src_idx, dst_idx = _pairs("skips", rng, n, src_pages, dst_pages)
    gen = torch.Generator().manual_seed(item_bytes)
    sk = random_payload(_shape(src_layout, layers, src_pages, item_bytes), torch.uint8, gen).to(DEV)
    sv = random_payload(_shape(src_layout, layers, src_pages, item_bytes), torch.uint8, gen).to(DEV)
    dk = random_payload(_shape(dst_layout, layers, dst_pages, item_bytes), torch.uint8, gen).to(DEV)
    dv = random_payload(_shape(dst_layout, layers, dst_pages, item_bytes), torch.uint8, gen).to(DEV)
    want_k, want_v = bits(dk).reshape(-1).copy(), bits(dv).reshape(-1).copy()
    sps, sls = ho.layout_strides(tuple(sk.shape), 1, src_layout)
    dps, dls = ho.layout_strides(tuple(dk.shape), 1, dst_layout)
    si_d = torch.from_numpy(src_idx).to(DEV)
    di_d = torch.from_numpy(dst_idx).to(DEV)
    lib = _hip.library()
    rc = _hip.fn("musa_aiter_hicache_transfer_bytes")(
        _hip.ptr(sk), _hip.ptr(dk), _hip.ptr(sv if with_v else None), _hip.ptr(dv if with_v else None),
        _hip.ptr(si_d), _hip.ptr(di_d), n, start, count, item_bytes, sps, sls, dps, dls,
        _hip.stream_ptr(torch.device(DEV)))
    assert rc == 0 and lib is not None
    torch.cuda.synchronize()
    ho.transfer_bytes(bits(sk).reshape(-1), want_k, bits(sv).reshape(-1) if with_v else None,
                      want_v if with_v else None, src_idx, dst_idx, n, start, count, item_bytes, sps, sls, dps, dls)
    assert np.array_equal(bits(dk).reshape(-1), want_k)
    assert np.array_equal(bits(dv).reshape(-1), want_v)


def test_c_abi_transfer_bytes_noops():
    t = torch.zeros(64, dtype=torch.uint8, device=DEV)
    idx = torch.zeros(1, dtype=torch.int64, device=DEV)
    f = _hip.fn("musa_aiter_hicache_transfer_bytes")
    s = _hip.stream_ptr(torch.device(DEV))
    # Fewer than 8 bytes per item, no items or no layers copy nothing (hicache_transfer.mu:71-76).
    for items, layers, item in ((1, 1, 7), (0, 1, 8), (1, 0, 8)):
        assert f(_hip.ptr(t), _hip.ptr(t), None, None, _hip.ptr(idx), _hip.ptr(idx), items, 0, layers, item,
                 8, 0, 8, 0, s) == 0
    assert f(None, _hip.ptr(t), None, None, _hip.ptr(idx), _hip.ptr(idx), 1, 0, 1, 8, 8, 0, 8, 0, s) != 0
    assert ctypes.c_int(_hip.fn("musa_aiter_hicache_transfer_abi_version")()).value == 1


# ----- direct token ranges ----------------------------------------------------------------


def _direct_tables(kind, rng, groups, page_size, pages):
    sp = rng.choice(pages, size=groups, replace=False) * page_size
    dp = rng.choice(pages, size=groups, replace=False) * page_size
    j = np.tile(np.arange(page_size), groups)
    src = np.repeat(sp, page_size) + j
    dst = np.repeat(dp, page_size) + j
    if kind == "merged":
        # consecutive entries on both sides from unaligned starts: one run spans every page
        src = np.arange(groups * page_size) + int(rng.integers(0, (pages - groups) * page_size + 1))
        dst = np.arange(groups * page_size) + int(rng.integers(0, (pages - groups) * page_size + 1))
    elif kind == "irregular":
        # breaks inside pages: the reference copies from each run's first entry
        mask = rng.random(src.shape[0]) < 0.2
        src = np.where(mask, rng.integers(0, pages * page_size - page_size, size=src.shape[0]), src)
    elif kind == "duplicates":
        dst[page_size:2 * page_size] = dst[:page_size]
    return src.astype(np.int64), dst.astype(np.int64)


@pytest.mark.parametrize("kind", ["regular", "merged", "irregular", "duplicates"])
@pytest.mark.parametrize("page_size", [1, 4, 16])
def test_direct_matches_oracle(kind, page_size):
    rng = np.random.default_rng(page_size * 7 + len(kind))
    gen = torch.Generator().manual_seed(page_size)
    groups, pages = 6, 16
    tokens = pages * page_size + page_size
    src_t, dst_t = _direct_tables(kind, rng, groups, page_size, pages)
    # Three row widths (two share a launch) and a 1-D layer (one element per row).
    shapes = [(tokens, 8, 16), (tokens, 8, 16), (tokens, 24), (tokens,)]
    dtypes = [torch.bfloat16, torch.bfloat16, torch.float32, torch.float16]
    src = [random_payload(s, d, gen).to(DEV) for s, d in zip(shapes, dtypes)]
    dst = [random_payload(s, d, gen).to(DEV) for s, d in zip(shapes, dtypes)]
    want = [bits(d).copy() for d in dst]
    assert musa_aiter.hicache_transfer_kv_direct(src, dst, torch.from_numpy(src_t).to(DEV),
                                                 torch.from_numpy(dst_t).to(DEV), page_size) is True
    ho.direct([bits(s) for s in src], want, src_t, dst_t, page_size)
    for i, d in enumerate(dst):
        assert np.array_equal(bits(d), want[i]), i


def test_direct_reference_cases():
    # op_tests/test_hicache_transfer.py:156-173 and test_hicache_transfer_musa.py:108-123.
    layers, tokens, item = 2, 8, 4
    src_k = torch.arange(layers * tokens * item, dtype=torch.float32, device=DEV).reshape(layers, tokens, item)
    src_v = src_k + 1000
    dst_k, dst_v = torch.zeros_like(src_k), torch.zeros_like(src_v)
    assert musa_aiter.hicache_transfer_kv_direct([src_k[0], src_k[1], src_v[0], src_v[1]],
                                                 [dst_k[0], dst_k[1], dst_v[0], dst_v[1]],
                                                 torch.tensor([0, 1, 4, 5]), torch.tensor([2, 3, 0, 1]), page_size=2)
    torch.cuda.synchronize()
    assert torch.equal(dst_k[:, 2:4], src_k[:, 0:2]) and torch.equal(dst_k[:, 0:2], src_k[:, 4:6])
    assert torch.equal(dst_v[:, 2:4], src_v[:, 0:2])


@pytest.mark.parametrize("kind", ["regular", "irregular", "duplicates"])
@pytest.mark.parametrize("page_size,page_rows", [(1, 1), (4, 4), (16, 16), (4, 1)])
@pytest.mark.parametrize("planes", [1, 2])
def test_per_layer_direct_matches_oracle(kind, page_size, page_rows, planes):
    rng = np.random.default_rng(page_size + 3 * planes + len(kind))
    gen = torch.Generator().manual_seed(page_size + planes)
    groups, pages, layers, item, layer_id = 5, 12, 3, 128, 1
    src_t, dst_t = _direct_tables(kind, rng, groups, page_size, pages)
    src = [random_payload((pages, layers, page_rows, item), torch.bfloat16, gen).to(DEV) for _ in range(planes)]
    dst = [random_payload((pages * page_size + 5, item), torch.bfloat16, gen).to(DEV) for _ in range(planes)]
    want = [bits(d).copy() for d in dst]
    assert musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf(src, dst, torch.from_numpy(src_t).to(DEV),
                                                                 torch.from_numpy(dst_t).to(DEV), layer_id,
                                                                 page_size) is True
    ho.per_layer_direct_pf_lf([bits(s) for s in src], want, src_t, dst_t, layer_id, page_size)
    for i, d in enumerate(dst):
        assert np.array_equal(bits(d), want[i]), i


@pytest.mark.parametrize("kind", ["regular", "irregular", "duplicates"])
@pytest.mark.parametrize("page_size,page_rows", [(1, 1), (4, 4), (16, 16), (1, 4)])
@pytest.mark.parametrize("mla", [False, True])
def test_all_layer_direct_matches_oracle(kind, page_size, page_rows, mla):
    rng = np.random.default_rng(page_size + page_rows + int(mla) + len(kind))
    gen = torch.Generator().manual_seed(page_size + int(mla))
    groups, pages, layers, item = 5, 12, 3, 64
    src_t, dst_t = _direct_tables(kind, rng, groups, page_size, pages)
    tokens = pages * page_size + 5
    src = [random_payload((tokens, item), torch.float16, gen).to(DEV) for _ in range(layers * (1 if mla else 2))]
    dst = [random_payload((pages, layers + 1, page_rows, item), torch.float16, gen).to(DEV)
           for _ in range(1 if mla else 2)]
    want = [bits(d).copy() for d in dst]
    assert musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst, torch.from_numpy(src_t).to(DEV),
                                                                 torch.from_numpy(dst_t).to(DEV), page_size) is True
    ho.all_layer_direct_lf_pf([bits(s) for s in src], want, src_t, dst_t, page_size)
    for i, d in enumerate(dst):
        assert np.array_equal(bits(d), want[i]), i


def test_direct_reference_native_cases():
    # op_tests/test_hicache_transfer_musa.py:108-145.
    page_size, layers, item = 2, 2, 4
    src_tokens = torch.arange(layers * 6 * item, dtype=torch.float16, device=DEV).reshape(layers, 6, item)
    dst_tokens = torch.zeros_like(src_tokens)
    assert musa_aiter.hicache_transfer_kv_direct([src_tokens[0], src_tokens[1]], [dst_tokens[0], dst_tokens[1]],
                                                 torch.tensor([0, 1, 4, 5], device=DEV),
                                                 torch.tensor([2, 3, 0, 1], device=DEV), page_size)
    src_pf = torch.arange(3 * layers * page_size * item, dtype=torch.float16, device=DEV).reshape(3, layers,
                                                                                                 page_size, item)
    dst_lf = torch.zeros(layers, 6, item, dtype=torch.float16, device=DEV)
    assert musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src_pf], [dst_lf[1]],
                                                                 torch.tensor([0, 1], device=DEV),
                                                                 torch.tensor([2, 3], device=DEV), 1, page_size)
    dst_pf = torch.zeros(3, layers, page_size, item, dtype=torch.float16, device=DEV)
    assert musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf([src_tokens[0], src_tokens[1]], [dst_pf],
                                                                 torch.tensor([0, 1], device=DEV),
                                                                 torch.tensor([2, 3], device=DEV), page_size)
    torch.cuda.synchronize()
    assert torch.equal(dst_tokens[:, 2:4], src_tokens[:, 0:2])
    assert torch.equal(dst_lf[1, 2:4], src_pf[0, 1])
    assert torch.equal(dst_pf[1], src_tokens[:, 0:2])


@pytest.mark.parametrize("name,layers", [("hicache_transfer_kv_all_layer_lf_pf", 70),
                                         ("hicache_transfer_kv_all_layer_mla_lf_pf", 131),
                                         ("hicache_transfer_kv_all_layer", 70)])
@pytest.mark.parametrize("kind", ["skips", "duplicates"])
def test_more_planes_than_one_launch_holds(name, layers, kind):
    # More than 128 (layer, K/V) planes: the row kernel splits the planes over launches (plane-inner
    # grids for page-first destinations, plane-major otherwise).
    _run_layout(name, torch.bfloat16, 40, kind, layers=layers, src_pages=13, dst_pages=17, n=11, seed=layers)
