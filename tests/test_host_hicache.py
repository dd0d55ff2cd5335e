"""Host-side contract of the HiCache transfers (CPU only, no kernel launches).

Mirrors the reference's error contracts (hicache_transfer.py:96-193, :502-544, :602-679 and
op_tests/test_hicache_transfer.py:144-260): validation raises before any launch, in the
reference's order, and tensors that pass validation but are not on a ROCm device are rejected
with RuntimeError.  Also checks the host-side run coalescing of the direct path against the
oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops import hicache_transfer as hc
from oracle import hicache_oracle as ho

I64 = torch.int64


def _idx(*values, dtype=I64):
    return torch.tensor(values, dtype=dtype)


def _lf(layers=2, pages=4, item=8, dtype=torch.float16):
    return torch.zeros(layers, pages, item, dtype=dtype)


def test_layout_transfer_validation_order():
    k, v = _lf(), _lf()
    with pytest.raises(TypeError, match="torch.Tensor"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, v, [0], _idx(0))
    with pytest.raises(ValueError, match="1-D"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, v, _idx(0).reshape(1, 1), _idx(0))
    with pytest.raises(ValueError, match="same length"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, v, _idx(0, 1), _idx(0))
    with pytest.raises(ValueError, match="int32 or int64"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, v, _idx(0, dtype=torch.int16), _idx(0))
    with pytest.raises(ValueError, match="same dtype"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k.float(), v, v, _idx(0), _idx(0))
    with pytest.raises(ValueError, match="provided together"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, None, _idx(0), _idx(0))
    with pytest.raises(ValueError, match="requires K and V"):
        hc._transfer(k, k, None, None, _idx(0), _idx(0), src_layout="layer_first", dst_layout="layer_first",
                     start_layer=0, num_layers=1, mla=False)
    with pytest.raises(ValueError, match="MLA HiCache transfer does not accept a value plane"):
        musa_aiter.hicache_transfer_kv_per_layer_mla(k, k, _idx(0), _idx(0), value=v)
    with pytest.raises(ValueError, match="MLA HiCache transfer does not accept a value plane"):
        hc._transfer(k, k, v, v, _idx(0), _idx(0), src_layout="layer_first", dst_layout="layer_first",
                     start_layer=0, num_layers=1, mla=True)
    with pytest.raises(ValueError, match="rank-3"):
        musa_aiter.hicache_transfer_kv_per_layer(k[0], k[0], v[0], v[0], _idx(0), _idx(0))
    with pytest.raises(ValueError, match="contiguous"):
        musa_aiter.hicache_transfer_kv_per_layer(k.transpose(0, 1), k, v, v, _idx(0), _idx(0))
    with pytest.raises(ValueError, match="item byte sizes must match"):
        musa_aiter.hicache_transfer_kv_per_layer(k, _lf(item=4), v, _lf(item=4), _idx(0), _idx(0))
    with pytest.raises(ValueError, match="source K and V layouts must match"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, _lf(pages=5), v, _idx(0), _idx(0))
    with pytest.raises(ValueError, match="destination K and V layouts must match"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, _lf(pages=5), _idx(0), _idx(0))
    with pytest.raises(ValueError, match="non-negative/positive"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, v, _idx(0), _idx(0), layer_id=-1)
    with pytest.raises(ValueError, match="layer range exceeds"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k, v, v, _idx(0), _idx(0), layer_id=2)
    odd = _lf(item=3)
    with pytest.raises(ValueError, match="divisible by 8"):
        musa_aiter.hicache_transfer_kv_per_layer(odd, odd, odd, odd, _idx(0), _idx(0))
    with pytest.raises(ValueError, match="unsupported HiCache layout"):
        hc._layout_geometry(k, "token_first")
    with pytest.raises(ValueError, match="must be positive"):
        hc._layout_geometry(torch.zeros(0, 4, 8), "layer_first")


def test_page_index_checks_follow_pair_order():
    k, v = _lf(), _lf()
    with pytest.raises(ValueError, match="-1 or non-negative"):
        musa_aiter.hicache_transfer_kv_all_layer(k, k, v, v, _idx(0, -2), _idx(1, 2))
    with pytest.raises(ValueError, match="out of range"):
        musa_aiter.hicache_transfer_kv_all_layer(k, k, v, v, _idx(0, 1), _idx(4, 2))
    # The first offending pair decides the message.
    with pytest.raises(ValueError, match="out of range"):
        musa_aiter.hicache_transfer_kv_all_layer(k, k, v, v, _idx(9, -2), _idx(0, 1))
    with pytest.raises(ValueError, match="-1 or non-negative"):
        musa_aiter.hicache_transfer_kv_all_layer(k, k, v, v, _idx(-2, 9), _idx(0, 1))
    # page_first geometry: pages are dim 0.
    pf = torch.zeros(3, 2, 8, dtype=torch.float16)
    with pytest.raises(ValueError, match="out of range"):
        musa_aiter.hicache_transfer_kv_all_layer_lf_pf(k, pf, v, pf.clone(), _idx(0), _idx(3))


def test_layout_transfer_cpu_tensors_are_rejected_not_computed():
    k, v = _lf(), _lf()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.hicache_transfer_kv_per_layer(k, k.clone(), v, v.clone(), _idx(0), _idx(1))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.hicache_transfer_kv_all_layer_mla_lf_pf(k, torch.zeros(4, 2, 8, dtype=torch.float16), _idx(0),
                                                           _idx(1))


def test_direct_validation_contract():
    src, dst = torch.zeros(4, 4), torch.zeros(4, 4)
    with pytest.raises(TypeError, match="tensor lists"):
        musa_aiter.hicache_transfer_kv_direct(src, [dst], _idx(0), _idx(0), 1)
    with pytest.raises(ValueError, match="equal non-zero length"):
        musa_aiter.hicache_transfer_kv_direct([], [], _idx(0), _idx(0), 1)
    with pytest.raises(ValueError, match="tails must match"):
        musa_aiter.hicache_transfer_kv_direct([src], [torch.zeros(4, 2)], _idx(0), _idx(0), 1)
    with pytest.raises(ValueError, match="dtypes must match"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst.half()], _idx(0), _idx(0), 1)
    with pytest.raises(ValueError, match="contiguous"):
        musa_aiter.hicache_transfer_kv_direct([src.t()], [dst], _idx(0), _idx(0), 1)
    # op_tests/test_hicache_transfer.py:250-260
    with pytest.raises(ValueError, match="divisible"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst], _idx(0, 1, 2), _idx(0, 1, 2), page_size=2)
    with pytest.raises(ValueError, match="page_size must be positive"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst], _idx(0), _idx(0), 0)
    with pytest.raises(ValueError, match="non-negative"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst], _idx(0, -1), _idx(0, 1), 2)
    with pytest.raises(ValueError, match="int32 or int64"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst], _idx(0, dtype=torch.int16), _idx(0), 1)
    with pytest.raises(ValueError, match="token range exceeds"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst], _idx(2, 3, 4, 5), _idx(0, 1, 2, 3), 2)
    # A run that starts mid-page reaches past the tables: [0,1,2] then a run of 2 from 3 -> rows 3, 4.
    with pytest.raises(ValueError, match="token range exceeds"):
        musa_aiter.hicache_transfer_kv_direct([src], [dst], _idx(0, 1, 2, 0), _idx(0, 1, 2, 3), 2)


def test_per_layer_direct_validation_contract():
    src = torch.zeros(3, 2, 2, 4)
    dst = torch.zeros(6, 4)
    with pytest.raises(ValueError, match="layer_id must be non-negative"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst], _idx(0, 1), _idx(0, 1), -1, 2)
    with pytest.raises(ValueError, match="one MLA plane or K/V plane pairs"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src] * 3, [dst] * 3, _idx(0, 1), _idx(0, 1), 0, 2)
    with pytest.raises(ValueError, match=r"source \[pages,layers,page,item\]"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([dst], [dst], _idx(0, 1), _idx(0, 1), 0, 2)
    with pytest.raises(ValueError, match="exceeds source layers"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst], _idx(0, 1), _idx(0, 1), 2, 2)
    with pytest.raises(ValueError, match="item shapes/dtypes"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst.half()], _idx(0, 1), _idx(0, 1), 0, 2)
    with pytest.raises(ValueError, match="page range exceeds"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst], _idx(6, 7), _idx(0, 1), 0, 2)
    with pytest.raises(ValueError, match="page range exceeds"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst], _idx(0, 1), _idx(5, 6), 0, 2)
    with pytest.raises(RuntimeError, match="broadcast"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([torch.zeros(3, 2, 3, 4)], [dst], _idx(0, 1),
                                                              _idx(0, 1), 0, 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst], _idx(0, 1), _idx(0, 1), 0, 2)
    # Nothing to copy: no launch, so CPU tensors are fine.
    assert musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf([src], [dst], _idx(), _idx(), 0, 2) is True


def test_all_layer_direct_validation_contract():
    src = [torch.zeros(6, 4) for _ in range(4)]
    dst = [torch.zeros(3, 2, 2, 4), torch.zeros(3, 2, 2, 4)]
    with pytest.raises(ValueError, match="one MLA plane or K/V plane pairs"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst * 2, _idx(0, 1), _idx(0, 1), 2)
    with pytest.raises(ValueError, match="do not match destination planes"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src[:3], dst, _idx(0, 1), _idx(0, 1), 2)
    with pytest.raises(TypeError, match="must be tensors"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src[:3] + [None], dst, _idx(0, 1), _idx(0, 1), 2)
    with pytest.raises(ValueError, match=r"contiguous \[tokens,item\]"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf([torch.zeros(6, 4, 1)] * 4, dst, _idx(0, 1),
                                                              _idx(0, 1), 2)
    with pytest.raises(ValueError, match=r"contiguous \[pages,layers,page,item\]"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, [torch.zeros(3, 2, 8)] * 2, _idx(0, 1),
                                                              _idx(0, 1), 2)
    with pytest.raises(ValueError, match="source and destination item shapes/dtypes"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf([s.half() for s in src], dst, _idx(0, 1), _idx(0, 1), 2)
    with pytest.raises(ValueError, match="K/V item shapes/dtypes"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src[:2] + [torch.zeros(6, 2)] * 2, dst, _idx(0, 1),
                                                              _idx(0, 1), 2)
    with pytest.raises(ValueError, match="destination page exceeds destination"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst, _idx(0, 1), _idx(6, 7), 2)
    with pytest.raises(ValueError, match="source range exceeds source"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst, _idx(5, 6), _idx(0, 1), 2)
    # Groups are checked in order: group 0's short source comes before group 1's bad page.
    with pytest.raises(ValueError, match="source range exceeds source"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst, _idx(5, 6, 0, 1), _idx(0, 1, 6, 7), 2)
    with pytest.raises(IndexError, match="fewer layers"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src[:3] + src[:3], dst, _idx(0, 1), _idx(0, 1), 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst, _idx(0, 1), _idx(0, 1), 2)


@pytest.mark.parametrize("seed", range(40))
def test_direct_run_tokens_match_oracle_runs(seed):
    rng = np.random.default_rng(seed)
    page_size = int(rng.integers(1, 5))
    groups = int(rng.integers(0, 7))
    n = groups * page_size
    # Mostly consecutive tables with random breaks, some inside pages.
    src = np.cumsum(np.where(rng.random(n) < 0.25, rng.integers(2, 6, size=n), 1)) + int(rng.integers(0, 4))
    dst = np.cumsum(np.where(rng.random(n) < 0.25, rng.integers(2, 6, size=n), 1)) + int(rng.integers(0, 4))
    src, dst = src.astype(np.int64), dst.astype(np.int64)
    runs = ho.direct_runs(src.tolist(), dst.tolist(), page_size)
    want_src = np.concatenate([np.arange(s, s + c) for s, _, c in runs]) if runs else np.zeros(0, np.int64)
    want_dst = np.concatenate([np.arange(d, d + c) for _, d, c in runs]) if runs else np.zeros(0, np.int64)
    got_src, got_dst, src_max, dst_max = hc._direct_run_tokens(src, dst, page_size)
    if got_src is None:
        got_src, got_dst = src, dst
    assert np.array_equal(got_src, want_src)
    assert np.array_equal(got_dst, want_dst)
    assert src_max == (int(want_src.max()) if n else -1)
    assert dst_max == (int(want_dst.max()) if n else -1)


# ----- host logic end to end on CPU tensors, through the launch contract -------------------------


@pytest.fixture
def emulate(monkeypatch):
    """Routes the host layer's launches to a CPU emulator of the row-copy contract."""
    from musa_aiter.ops import _hip
    from tests.row_emulator import RowCopyEmulator

    monkeypatch.setattr(hc, "_require_rocm", lambda *args, **kwargs: None)

    def install(*tensors):
        emu = RowCopyEmulator(*tensors)
        monkeypatch.setattr(_hip, "copy_rows_paged", emu)
        return emu

    return install


def _u16(shape, rng):
    return torch.from_numpy(rng.integers(0, 2**16, size=shape, dtype=np.uint16).view(np.int16).copy())


LAYOUTS = {
    "hicache_transfer_kv_per_layer": ("layer_first", "layer_first", True, False),
    "hicache_transfer_kv_per_layer_pf_lf": ("page_first", "layer_first", True, False),
    "hicache_transfer_kv_all_layer": ("layer_first", "layer_first", False, False),
    "hicache_transfer_kv_all_layer_lf_pf": ("layer_first", "page_first", False, False),
    "hicache_transfer_kv_per_layer_mla": ("layer_first", "layer_first", True, True),
    "hicache_transfer_kv_per_layer_mla_pf_lf": ("page_first", "layer_first", True, True),
    "hicache_transfer_kv_all_layer_mla": ("layer_first", "layer_first", False, True),
    "hicache_transfer_kv_all_layer_mla_lf_pf": ("layer_first", "page_first", False, True),
}


@pytest.mark.parametrize("name", list(LAYOUTS))
@pytest.mark.parametrize("duplicates", [False, True])
def test_layout_host_logic_matches_oracle(emulate, name, duplicates):
    src_layout, dst_layout, per_layer, mla = LAYOUTS[name]
    rng = np.random.default_rng(len(name) + duplicates)
    layers, src_pages, dst_pages, item, n = 3, 9, 10, 4, 8
    shape = lambda layout, pages: (layers, pages, item) if layout == "layer_first" else (pages, layers, item)  # noqa
    planes = 1 if mla else 2
    src = [_u16(shape(src_layout, src_pages), rng) for _ in range(planes)]
    dst = [_u16(shape(dst_layout, dst_pages), rng) for _ in range(planes)]
    si = rng.integers(-1, src_pages, size=n)
    di = rng.integers(-1, dst_pages // 2, size=n) if duplicates else rng.permutation(dst_pages)[:n] - (rng.random(n) < 0.2)
    want = [d.numpy().copy() for d in dst]
    emu = emulate(*src, *dst)
    kwargs = {"layer_id": 1} if per_layer else {}
    args = (src[0], dst[0]) if mla else (src[0], dst[0], src[1], dst[1])
    assert getattr(musa_aiter, name)(*args, torch.from_numpy(si), torch.from_numpy(di).to(torch.int32), **kwargs)
    assert emu.launches == 1
    start, count = (1, 1) if per_layer else (0, layers)
    ho.transfer(src[0].numpy(), want[0], None if mla else src[1].numpy(), None if mla else want[1], si, di,
                src_layout=src_layout, dst_layout=dst_layout, start_layer=start, num_layers=count)
    for p in range(planes):
        assert np.array_equal(dst[p].numpy(), want[p])


def _tables(kind, rng, groups, page_size, pages):
    sp = rng.choice(pages, size=groups, replace=False) * page_size
    dp = rng.choice(pages, size=groups, replace=False) * page_size
    j = np.tile(np.arange(page_size), groups)
    src, dst = np.repeat(sp, page_size) + j, np.repeat(dp, page_size) + j
    if kind == "irregular":
        mask = rng.random(src.shape[0]) < 0.3
        src = np.where(mask, rng.integers(0, pages * page_size - page_size, size=src.shape[0]), src)
    elif kind == "duplicates":
        dst[page_size:2 * page_size] = dst[:page_size]
    return src.astype(np.int64), dst.astype(np.int64)


@pytest.mark.parametrize("kind", ["regular", "irregular", "duplicates"])
@pytest.mark.parametrize("page_size", [1, 2, 4])
def test_direct_host_logic_matches_oracle(emulate, kind, page_size):
    rng = np.random.default_rng(page_size + 10 * len(kind))
    groups, pages = 4, 8
    tokens = pages * page_size + page_size
    src_t, dst_t = _tables(kind, rng, groups, page_size, pages)
    src = [_u16((tokens, 3, 2), rng), _u16((tokens, 3, 2), rng), _u16((tokens, 5), rng), _u16((tokens,), rng)]
    dst = [_u16(tuple(s.shape), rng) for s in src]
    want = [d.numpy().copy() for d in dst]
    emu = emulate(*src, *dst)
    assert musa_aiter.hicache_transfer_kv_direct(src, dst, torch.from_numpy(src_t), torch.from_numpy(dst_t),
                                                 page_size)
    assert emu.launches == 3  # one per distinct row width
    ho.direct([s.numpy() for s in src], want, src_t, dst_t, page_size)
    for d, w in zip(dst, want):
        assert np.array_equal(d.numpy(), w)


@pytest.mark.parametrize("kind", ["regular", "irregular", "duplicates"])
@pytest.mark.parametrize("page_size,page_rows", [(1, 1), (4, 4), (4, 1)])
@pytest.mark.parametrize("planes", [1, 2])
def test_per_layer_direct_host_logic_matches_oracle(emulate, kind, page_size, page_rows, planes):
    rng = np.random.default_rng(page_size + page_rows + planes + len(kind))
    groups, pages, layers, item = 3, 6, 3, 5
    src_t, dst_t = _tables(kind, rng, groups, page_size, pages)
    src = [_u16((pages, layers, page_rows, item), rng) for _ in range(planes)]
    dst = [_u16((pages * page_size + 3, item), rng) for _ in range(planes)]
    want = [d.numpy().copy() for d in dst]
    emu = emulate(*src, *dst)
    assert musa_aiter.hicache_transfer_kv_per_layer_direct_pf_lf(src, dst, torch.from_numpy(src_t),
                                                                 torch.from_numpy(dst_t), 2, page_size)
    assert emu.launches == 1
    ho.per_layer_direct_pf_lf([s.numpy() for s in src], want, src_t, dst_t, 2, page_size)
    for d, w in zip(dst, want):
        assert np.array_equal(d.numpy(), w)


@pytest.mark.parametrize("kind", ["regular", "irregular", "duplicates"])
@pytest.mark.parametrize("page_size,page_rows", [(1, 1), (4, 4), (1, 4)])
@pytest.mark.parametrize("mla", [False, True])
def test_all_layer_direct_host_logic_matches_oracle(emulate, kind, page_size, page_rows, mla):
    rng = np.random.default_rng(page_size + page_rows + int(mla) + len(kind))
    groups, pages, layers, item = 3, 6, 3, 5
    src_t, dst_t = _tables(kind, rng, groups, page_size, pages)
    src = [_u16((pages * page_size + 3, item), rng) for _ in range(layers * (1 if mla else 2))]
    dst = [_u16((pages, layers + 1, page_rows, item), rng) for _ in range(1 if mla else 2)]
    want = [d.numpy().copy() for d in dst]
    emu = emulate(*src, *dst)
    assert musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src, dst, torch.from_numpy(src_t),
                                                                 torch.from_numpy(dst_t), page_size)
    assert emu.launches == 1
    ho.all_layer_direct_lf_pf([s.numpy() for s in src], want, src_t, dst_t, page_size)
    for d, w in zip(dst, want):
        assert np.array_equal(d.numpy(), w)


def test_direct_tensors_must_share_one_device(monkeypatch):
    # All layers and planes of a direct transfer go in one launch on one device.
    monkeypatch.setattr(hc, "_require_rocm", lambda *args, **kwargs: None)
    with pytest.raises(ValueError, match="one device"):
        hc._require_one_rocm_device("op", [torch.zeros(2), torch.zeros(2, device="meta")])
    assert hc._require_one_rocm_device("op", [torch.zeros(2), torch.zeros(3)]) == torch.device("cpu")
