"""GPU parity: dense preload for attention and whole-block copies vs the oracle.

Covers kv_load_and_reshape_flash, kv_reshape_and_cache_back_flash,
kv_load_and_dequantize_fp8_flash, kv_triton_indexed_to_dense and
kv_copy_paged_blocks(_fp8) through the public API and through the
reference-named C symbols (bound with ctypes as the reference's shims bind
them), on seeded random bit patterns, compared bit-for-bit with
oracle/kv_oracle.py.  Block tables hold whole sequences, shared blocks,
unused columns and (C-ABI only, which the Python layer rejects) invalid ids;
sequence lengths include 0 and lengths ending mid-block.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops import _hip
from oracle import kv_oracle as ko
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]
SUFFIX = {torch.bfloat16: "bfloat16", torch.float16: "half", torch.float32: "float"}
SHAPES = [  # (num_heads, head_dim, block_size): tile kernel sizes, then the element kernel
    (8, 128, 16),
    (4, 64, 32),
    (2, 32, 8),
    (3, 7, 16),
    (2, 16, 5),
]


def _tables(rng, seq_lens, bs, *, extra_cols=1, spare=5, share=False):
    """Block tables giving each sequence distinct blocks (or, with ``share``, reusing some)."""
    need = [(int(n) + bs - 1) // bs for n in seq_lens]
    max_blocks = max(need + [1]) + extra_cols
    nb = sum(need) + spare
    perm = rng.permutation(nb)
    tables = rng.integers(0, nb, size=(len(seq_lens), max_blocks)).astype(np.int64)
    pos = 0
    for b, k in enumerate(need):
        tables[b, :k] = perm[pos:pos + k]
        pos += k
    if share and len(seq_lens) > 1:
        k = min(need[0], need[-1])
        tables[-1, :k] = tables[0, :k]
    return tables, nb


def _dev(a: np.ndarray, dtype=torch.int64) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def _fn(name: str, nargs_ptr: int, nargs_i64: int):
    fn = getattr(_hip.library(), name)
    fn.argtypes = [ctypes.c_void_p] * nargs_ptr + [ctypes.c_longlong] * nargs_i64 + [ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# ----- kv_load_and_reshape_flash --------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_load_and_reshape_flash_matches_oracle(dtype, shape):
    nh, hd, bs = shape
    rng = np.random.default_rng(31)
    seq_lens = rng.integers(0, 5 * bs + 3, size=7)
    seq_lens[1] = 0
    seq_lens[2] = 3 * bs  # ends on a block boundary
    tables, nb = _tables(rng, seq_lens, bs)
    gen = torch.Generator().manual_seed(7)
    kc = random_payload((nb, nh, hd, bs), dtype, gen)
    vc = random_payload((nb, nh, hd, bs), dtype, gen)
    dense_len = int(seq_lens.max()) + 2
    ok, ov = musa_aiter.kv_load_and_reshape_flash(kc.to(DEV), vc.to(DEV), _dev(tables, torch.int32),
                                                  _dev(seq_lens, torch.int32), max_seq_len=dense_len)
    assert ok.shape == (7, dense_len, nh, hd) and ok.dtype == dtype
    assert np.array_equal(bits(ok), ko.load_and_reshape_flash(bits(kc), tables, seq_lens, dense_len))
    assert np.array_equal(bits(ov), ko.load_and_reshape_flash(bits(vc), tables, seq_lens, dense_len))


def test_load_and_reshape_flash_out_buffers_are_overwritten():
    nh, hd, bs = 8, 128, 16
    rng = np.random.default_rng(2)
    seq_lens = np.array([40, 17, 0, 33])
    tables, nb = _tables(rng, seq_lens, bs)
    gen = torch.Generator().manual_seed(3)
    kc, vc = (random_payload((nb, nh, hd, bs), torch.bfloat16, gen) for _ in range(2))
    shape = (4, 48, nh, hd)
    out_k = torch.full(shape, 7.0, dtype=torch.bfloat16, device=DEV)  # stale values past seq_lens must go
    out_v = torch.full((4, 48, hd, nh), 7.0, dtype=torch.bfloat16, device=DEV).transpose(2, 3)  # non-contiguous
    rk, rv = musa_aiter.kv_load_and_reshape_flash(kc.to(DEV), vc.to(DEV), _dev(tables), _dev(seq_lens),
                                                  max_seq_len=48, out_k=out_k, out_v=out_v)
    assert rk is out_k and rv is out_v
    assert np.array_equal(bits(out_k), ko.load_and_reshape_flash(bits(kc), tables, seq_lens, 48))
    assert np.array_equal(bits(out_v), ko.load_and_reshape_flash(bits(vc), tables, seq_lens, 48))


@pytest.mark.parametrize("shape", [(8, 128, 16), (2, 16, 5)])
def test_load_and_reshape_flash_c_abi_skips_invalid_blocks(shape):
    # The reference-named symbol with block ids the Python layer would reject, a table narrower than
    # the dense length and a negative length: such positions are zeros (kv_transfer_float.mu:1006-1030).
    nh, hd, bs = shape
    rng = np.random.default_rng(4)
    seq_lens = np.array([5 * bs, 2 * bs + 1, -3, 4 * bs])
    tables, nb = _tables(rng, np.maximum(seq_lens, 0), bs, extra_cols=0)
    tables = tables[:, :4]  # logical block 4 of sequence 0 is past max_blocks
    tables[1, 1] = -1
    tables[3, 2] = nb + 5
    gen = torch.Generator().manual_seed(5)
    kc, vc = (random_payload((nb, nh, hd, bs), torch.float16, gen).to(DEV) for _ in range(2))
    dense_len = 5 * bs
    ok = torch.full((4, dense_len, nh, hd), 3.0, dtype=torch.float16, device=DEV)
    ov = torch.full_like(ok, 3.0)
    t_d, s_d = _dev(tables), _dev(seq_lens)  # kept alive until the launch has been read back
    fn = _fn("musa_aiter_kv_load_and_reshape_flash_half", 6, 7)
    rc = fn(kc.data_ptr(), vc.data_ptr(), t_d.data_ptr(), s_d.data_ptr(), ok.data_ptr(),
            ov.data_ptr(), 4, dense_len, tables.shape[1], nb, nh, hd, bs, _stream())
    assert rc == 0
    assert np.array_equal(bits(ok), ko.load_and_reshape_flash(bits(kc), tables, seq_lens, dense_len))
    assert np.array_equal(bits(ov), ko.load_and_reshape_flash(bits(vc), tables, seq_lens, dense_len))


# ----- kv_reshape_and_cache_back_flash ----------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("share", [False, True])
def test_reshape_and_cache_back_matches_oracle(dtype, shape, share):
    nh, hd, bs = shape
    rng = np.random.default_rng(41)
    seq_lens = rng.integers(1, 4 * bs + 3, size=6)
    seq_lens[2] = 0
    tables, nb = _tables(rng, seq_lens, bs, share=share)
    dense_len = int(seq_lens.max()) + 1
    gen = torch.Generator().manual_seed(8)
    dk, dv = (random_payload((6, dense_len, nh, hd), dtype, gen) for _ in range(2))
    kc, vc = (random_payload((nb, nh, hd, bs), dtype, gen) for _ in range(2))
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    assert musa_aiter.kv_reshape_and_cache_back_flash(dk.to(DEV), dv.to(DEV), kc_d, vc_d, _dev(tables, torch.int16),
                                                      _dev(seq_lens, torch.int32)) is True
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.reshape_and_cache_back_flash(bits(dk), want_k, tables, seq_lens)
    ko.reshape_and_cache_back_flash(bits(dv), want_v, tables, seq_lens)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


def test_reshape_and_cache_back_c_abi_last_sequence_wins():
    nh, hd, bs = 4, 64, 16
    nb = 6
    tables = np.array([[2, 3, 0], [2, 5, 1], [4, 3, 1]])  # block 2, 3 and 1 are shared
    seq_lens = np.array([40, 20, 37])
    dense_len = 40
    gen = torch.Generator().manual_seed(9)
    dk, dv = (random_payload((3, dense_len, nh, hd), torch.bfloat16, gen).to(DEV) for _ in range(2))
    kc, vc = (random_payload((nb, nh, hd, bs), torch.bfloat16, gen).to(DEV) for _ in range(2))
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    t_d, s_d = _dev(tables), _dev(seq_lens)
    fn = _fn("musa_aiter_kv_reshape_and_cache_back_flash_bfloat16", 6, 7)
    rc = fn(dk.data_ptr(), dv.data_ptr(), t_d.data_ptr(), s_d.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), 3, dense_len, 3, nb, nh, hd, bs, _stream())
    assert rc == 0
    ko.reshape_and_cache_back_flash(bits(dk), want_k, tables, seq_lens)
    ko.reshape_and_cache_back_flash(bits(dv), want_v, tables, seq_lens)
    assert np.array_equal(bits(kc), want_k)
    assert np.array_equal(bits(vc), want_v)


def test_flash_round_trip_at_serving_size():
    # Size-independent property at a decode-batch shape: write back, read back, equal up to seq_lens.
    nh, hd, bs, batch = 8, 128, 16, 64
    rng = np.random.default_rng(12)
    seq_lens = rng.integers(1, 2049, size=batch)
    seq_lens[0] = 2048
    tables, nb = _tables(rng, seq_lens, bs)
    dense_len = 2048
    gen = torch.Generator(device=DEV).manual_seed(1)
    dk = torch.randn((batch, dense_len, nh, hd), dtype=torch.bfloat16, device=DEV, generator=gen)
    dv = torch.randn((batch, dense_len, nh, hd), dtype=torch.bfloat16, device=DEV, generator=gen)
    kc = torch.zeros((nb, nh, hd, bs), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    t, s = _dev(tables), _dev(seq_lens)
    musa_aiter.kv_reshape_and_cache_back_flash(dk, dv, kc, vc, t, s)
    rk, rv = musa_aiter.kv_load_and_reshape_flash(kc, vc, t, s, max_seq_len=dense_len)
    mask = (torch.arange(dense_len, device=DEV)[None, :] < s[:, None])[:, :, None, None]
    assert torch.equal(rk, torch.where(mask, dk, torch.zeros_like(dk)))
    assert torch.equal(rv, torch.where(mask, dv, torch.zeros_like(dv)))


# ----- kv_load_and_dequantize_fp8_flash ----------------------------------------------------------

FP8_SHAPES = [(8, 128, 16), (4, 64, 32), (2, 16, 5), (3, 8, 16)]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("out_dtype", DTYPES)
@pytest.mark.parametrize("shape", FP8_SHAPES)
@pytest.mark.parametrize("per_head", [False, True])
def test_load_and_dequantize_fp8_flash_matches_oracle(fmt, out_dtype, shape, per_head):
    nh, hd, bs = shape
    rng = np.random.default_rng(51)
    seq_lens = rng.integers(0, 4 * bs + 5, size=5)
    tables, nb = _tables(rng, seq_lens, bs)
    gen = torch.Generator().manual_seed(6)
    kc = random_payload((nb, nh, hd, bs), torch.uint8, gen)
    vc = random_payload((nb, nh, hd, bs), torch.uint8, gen)
    if per_head:
        ks = (rng.random(nh) * 2 + 0.05).astype(np.float32)
        vs = (rng.random(nh) * 2 + 0.05).astype(np.float32)
        k_scale, v_scale = torch.from_numpy(ks).to(DEV), torch.from_numpy(vs).to(DEV)
    else:
        ks, vs = np.float32(0.375), np.float32(1.5)
        k_scale, v_scale = 0.375, 1.5
    dense_len = int(seq_lens.max()) + 3
    kd = kc.to(DEV).view(torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2)
    ok, ov = musa_aiter.kv_load_and_dequantize_fp8_flash(kd, vc.to(DEV), _dev(tables), _dev(seq_lens), k_scale,
                                                         v_scale, max_seq_len=dense_len, out_dtype=out_dtype,
                                                         fp8_format=fmt)
    name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[out_dtype]
    want_k = ko.load_and_dequantize_fp8_flash(bits(kc), tables, seq_lens, ks, fmt, name, dense_len)
    want_v = ko.load_and_dequantize_fp8_flash(bits(vc), tables, seq_lens, vs, fmt, name, dense_len)
    assert np.array_equal(bits(ok), want_k)
    assert np.array_equal(bits(ov), want_v)


# ----- kv_triton_indexed_to_dense ----------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES + [torch.uint8])
@pytest.mark.parametrize("nh_hd", [(8, 128), (2, 8), (3, 5)])
def test_triton_indexed_to_dense_matches_oracle(dtype, nh_hd):
    nh, hd = nh_hd
    rng = np.random.default_rng(61)
    ntok = 300
    lengths = rng.integers(0, 70, size=9)
    indptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    indices = rng.integers(0, ntok, size=int(indptr[-1])).astype(np.int64)
    gen = torch.Generator().manual_seed(4)
    key, value = (random_payload((ntok, nh, hd), dtype, gen) for _ in range(2))
    dense_len = 50  # shorter than some sequences: they are cut
    ok, ov = musa_aiter.ops.kv_transfer.kv_triton_indexed_to_dense(
        key.to(DEV), value.to(DEV), _dev(indptr, torch.int32), _dev(indices, torch.int32), max_seq_len=dense_len)
    assert np.array_equal(bits(ok), ko.triton_indexed_to_dense(bits(key), indptr, indices, dense_len))
    assert np.array_equal(bits(ov), ko.triton_indexed_to_dense(bits(value), indptr, indices, dense_len))


def test_triton_indexed_to_dense_c_abi_invalid_entries_are_zero():
    nh, hd, ntok = 4, 32, 40
    indptr = np.array([0, 5, 3, 12, 20, 30])  # a decreasing pair and an end past kv_indices
    indices = np.array([1, 39, -1, 40, 7, 8, 9, 10, 11, 12, 50, 2, 3, 4, 5, 6, 7, 8, 9, 0, 1, 2, 3, 4, 5])
    gen = torch.Generator().manual_seed(5)
    key, value = (random_payload((ntok, nh, hd), torch.float32, gen).to(DEV) for _ in range(2))
    dense_len = 9
    ok = torch.full((5, dense_len, nh, hd), 2.0, device=DEV)
    ov = torch.full_like(ok, 2.0)
    p_d, i_d = _dev(indptr), _dev(indices)
    fn = _fn("musa_aiter_kv_triton_indexed_to_dense_float", 6, 6)
    rc = fn(key.data_ptr(), value.data_ptr(), p_d.data_ptr(), i_d.data_ptr(), ok.data_ptr(),
            ov.data_ptr(), 5, dense_len, indices.size, ntok, nh, hd, _stream())
    assert rc == 0
    assert np.array_equal(bits(ok), ko.triton_indexed_to_dense(bits(key), indptr, indices, dense_len))
    assert np.array_equal(bits(ov), ko.triton_indexed_to_dense(bits(value), indptr, indices, dense_len))


# ----- kv_copy_paged_blocks(_fp8) -----------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES + [torch.uint8])
@pytest.mark.parametrize("layers", [None, 3])
def test_copy_paged_blocks_matches_oracle(dtype, layers):
    nh, hd, bs, sb, db = 8, 128, 16, 20, 24
    rng = np.random.default_rng(71)
    pairs = np.stack([rng.permutation(sb)[:12], rng.permutation(db)[:12]], axis=1).astype(np.int64)
    pairs[3, 0] = -1
    pairs[7, 1] = -1
    pairs[9, 1] = pairs[2, 1]  # a destination named twice: the later pair wins
    gen = torch.Generator().manual_seed(11)
    lead = () if layers is None else (layers,)
    sk, sv = (random_payload(lead + (sb, nh, hd, bs), dtype, gen) for _ in range(2))
    dk, dv = (random_payload(lead + (db, nh, hd, bs), dtype, gen) for _ in range(2))
    dk_d, dv_d = dk.to(DEV), dv.to(DEV)
    op = musa_aiter.kv_copy_paged_blocks_fp8 if dtype == torch.uint8 else musa_aiter.kv_copy_paged_blocks
    copied = op(sk.to(DEV), sv.to(DEV), dk_d, dv_d, _dev(pairs, torch.int32))
    want_k, want_v = bits(dk).copy(), bits(dv).copy()
    assert copied == ko.copy_paged_blocks(bits(sk), want_k, pairs, multi_layer=layers is not None) == 10
    ko.copy_paged_blocks(bits(sv), want_v, pairs, multi_layer=layers is not None)
    assert np.array_equal(bits(dk_d), want_k)
    assert np.array_equal(bits(dv_d), want_v)


@pytest.mark.parametrize("name,dtype", [("musa_aiter_kv_copy_paged_blocks_bfloat16", torch.bfloat16),
                                        ("musa_aiter_kv_copy_paged_blocks_fp8_vec8", torch.uint8)])
def test_copy_paged_blocks_c_abi_skips_out_of_range(name, dtype):
    nl, nh, hd, bs, sb, db = 2, 2, 16, 8, 5, 6
    # Out-of-range ids on either side; the last two pairs name earlier destinations with invalid
    # sources, which must not undo the earlier copies.
    pairs = np.array([[4, 0], [5, 1], [0, 6], [1, 2], [-2, 3], [2, 5], [-1, 0], [6, 2]])
    gen = torch.Generator().manual_seed(12)
    sk, sv = (random_payload((nl, sb, nh, hd, bs), dtype, gen).to(DEV) for _ in range(2))
    dk, dv = (random_payload((nl, db, nh, hd, bs), dtype, gen).to(DEV) for _ in range(2))
    want_k, want_v = bits(dk).copy(), bits(dv).copy()
    m_d = _dev(pairs)
    fn = _fn(name, 5, 7)
    rc = fn(sk.data_ptr(), sv.data_ptr(), dk.data_ptr(), dv.data_ptr(), m_d.data_ptr(), pairs.shape[0], nl,
            sb, db, nh, hd, bs, _stream())
    assert rc == 0
    ko.copy_paged_blocks(bits(sk), want_k, pairs, multi_layer=True)
    ko.copy_paged_blocks(bits(sv), want_v, pairs, multi_layer=True)
    assert np.array_equal(bits(dk), want_k)
    assert np.array_equal(bits(dv), want_v)
