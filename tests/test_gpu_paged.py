"""GPU parity: paged [NB, NH, HD, BS] <-> linear transfers through the HIP library vs the oracle.

Every case runs the public API (which calls libmusa_aiter_kv_hip.so through
ctypes) on seeded inputs with random bit patterns and compares the result
bit-for-bit with oracle/kv_oracle.py.  Shapes cover the fast tile kernel
(block sizes 8/16/32, head_dim a multiple of 8) and the generic element
kernel (other block sizes and head dims), separate / merged / multi-layer
layouts, skipped and duplicated slots and fill_skipped="preserve".
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from oracle import kv_oracle as ko
from tests.kvgen import bits, make_slots, random_payload, sequence_slots

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [  # (num_heads, head_dim, block_size); the cache size follows the slot pattern
    (8, 128, 16),
    (2, 64, 8),
    (4, 32, 32),
    (3, 40, 16),
    (2, 8, 16),
    (3, 7, 16),   # head_dim not a multiple of 8: element kernel
    (2, 16, 5),   # block size outside {8,16,32}: element kernel
]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _case(dtype, shape, kind, tokens, seed, layers=None):
    nh, hd, bs = shape
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    slots, nb = make_slots(kind, rng, block_size=bs, tokens=tokens)
    cshape = (nb, nh, hd, bs) if layers is None else (layers, nb, nh, hd, bs)
    kc = random_payload(cshape, dtype, gen)
    vc = random_payload(cshape, dtype, gen)
    return slots, kc, vc


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["sequences", "random", "skips"])
def test_paged_to_linear_matches_oracle(dtype, shape, kind):
    slots, kc, vc = _case(dtype, shape, kind, tokens=257, seed=11)
    ok, ov = musa_aiter.kv_paged_to_linear(kc.to(DEV), vc.to(DEV), torch.from_numpy(slots).to(DEV))
    assert np.array_equal(bits(ok), ko.paged_to_linear(bits(kc), slots))
    assert np.array_equal(bits(ov), ko.paged_to_linear(bits(vc), slots))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["sequences", "random", "skips", "duplicates"])
def test_linear_to_paged_matches_oracle(dtype, shape, kind):
    nh, hd, bs = shape
    slots, kc, vc = _case(dtype, shape, kind, tokens=203, seed=12)
    gen = torch.Generator().manual_seed(5)
    kl = random_payload((len(slots), nh, hd), dtype, gen)
    vl = random_payload((len(slots), nh, hd), dtype, gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged(kl.to(DEV), vl.to(DEV), kc_d, vc_d, torch.from_numpy(slots).to(DEV))
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged(bits(kl), want_k, slots)
    ko.linear_to_paged(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(8, 128, 16), (3, 7, 16), (4, 32, 32)])
def test_multi_layer_roundtrip_and_oracle(dtype, shape):
    nh, hd, bs = shape
    layers = 3
    slots, kc, vc = _case(dtype, shape, "skips", tokens=300, seed=13, layers=layers)
    s_d = torch.from_numpy(slots).to(DEV)
    ok, ov = musa_aiter.kv_paged_to_linear_multi_layer(kc.to(DEV), vc.to(DEV), s_d)
    assert np.array_equal(bits(ok), ko.paged_to_linear_multi_layer(bits(kc), slots))
    assert np.array_equal(bits(ov), ko.paged_to_linear_multi_layer(bits(vc), slots))
    gen = torch.Generator().manual_seed(6)
    kl = random_payload((layers, len(slots), nh, hd), dtype, gen)
    vl = random_payload((layers, len(slots), nh, hd), dtype, gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged_multi_layer(kl.to(DEV), vl.to(DEV), kc_d, vc_d, s_d)
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged_multi_layer(bits(kl), want_k, slots)
    ko.linear_to_paged_multi_layer(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layers", [None, 2])
def test_merged_layouts_match_oracle(dtype, layers):
    shape = (8, 128, 16)
    nh, hd, bs = shape
    slots, kc, vc = _case(dtype, shape, "skips", tokens=150, seed=14, layers=layers)
    s_d = torch.from_numpy(slots).to(DEV)
    if layers is None:
        merged = musa_aiter.kv_paged_to_merged_linear(kc.to(DEV), vc.to(DEV), s_d)
        want = ko.paged_to_merged_linear(bits(kc), bits(vc), slots)
    else:
        merged = musa_aiter.kv_paged_to_merged_linear_multi_layer(kc.to(DEV), vc.to(DEV), s_d)
        want = np.stack([ko.paged_to_merged_linear(bits(kc)[layer], bits(vc)[layer], slots)
                         for layer in range(layers)])
    assert np.array_equal(bits(merged), want)
    gen = torch.Generator().manual_seed(9)
    src = random_payload(tuple(merged.shape), dtype, gen)
    kc_d, vc_d = torch.zeros_like(kc).to(DEV), torch.zeros_like(vc).to(DEV)
    if layers is None:
        musa_aiter.kv_merged_linear_to_paged(src.to(DEV), kc_d, vc_d, s_d)
        want_k, want_v = np.zeros_like(bits(kc)), np.zeros_like(bits(vc))
        ko.merged_linear_to_paged(bits(src), want_k, want_v, slots)
    else:
        musa_aiter.kv_merged_linear_to_paged_multi_layer(src.to(DEV), kc_d, vc_d, s_d)
        want_k, want_v = np.zeros_like(bits(kc)), np.zeros_like(bits(vc))
        for layer in range(layers):
            ko.merged_linear_to_paged(bits(src)[layer], want_k[layer], want_v[layer], slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


def test_fill_skipped_preserve_keeps_rows():
    shape = (8, 128, 16)
    nh, hd, bs = shape
    slots, kc, vc = _case(torch.bfloat16, shape, "skips", tokens=120, seed=15)
    gen = torch.Generator().manual_seed(3)
    out_k = random_payload((len(slots), nh, hd), torch.bfloat16, gen)
    out_v = random_payload((len(slots), nh, hd), torch.bfloat16, gen)
    want_k = ko.paged_to_linear(bits(kc), slots, fill_skipped="preserve", out=bits(out_k).copy())
    want_v = ko.paged_to_linear(bits(vc), slots, fill_skipped="preserve", out=bits(out_v).copy())
    ok_d, ov_d = out_k.to(DEV), out_v.to(DEV)
    rk, rv = musa_aiter.kv_paged_to_linear(kc.to(DEV), vc.to(DEV), torch.from_numpy(slots).to(DEV),
                                           fill_skipped="preserve", out_k=ok_d, out_v=ov_d)
    assert rk.data_ptr() == ok_d.data_ptr()
    assert np.array_equal(bits(ok_d), want_k)
    assert np.array_equal(bits(ov_d), want_v)


def test_reference_duplicate_slot_scenario():
    # op_tests/test_kv_transfer.py:281-303: last writer wins for repeated slots.
    nb, kvh, d, blk = 3, 2, 5, 4
    slots = torch.tensor([0, 1, 0, -1, 7, 7, 11], dtype=torch.int32)
    k_lin = torch.randn(len(slots), kvh, d)
    v_lin = torch.randn(len(slots), kvh, d)
    k_cache = torch.zeros(nb, kvh, d, blk, device=DEV)
    v_cache = torch.zeros_like(k_cache)
    musa_aiter.kv_linear_to_paged(k_lin.to(DEV), v_lin.to(DEV), k_cache, v_cache, slots.to(DEV))
    kr, vr = musa_aiter.kv_paged_to_linear(k_cache, v_cache, slots.to(DEV))
    kr, vr = kr.cpu(), vr.cpu()
    for got, want in ((0, 2), (2, 2), (4, 5), (5, 5)):
        assert torch.equal(kr[got], k_lin[want]) and torch.equal(vr[got], v_lin[want])
    assert kr[3].abs().max() == 0 and vr[3].abs().max() == 0


def test_noncontiguous_linear_and_int16_slots():
    shape = (8, 128, 16)
    nh, hd, bs = shape
    slots, kc, vc = _case(torch.bfloat16, shape, "sequences", tokens=64, seed=16)
    gen = torch.Generator().manual_seed(4)
    big = random_payload((len(slots), 3, nh, hd), torch.bfloat16, gen).to(DEV)
    kl, vl = big[:, 0], big[:, 2]  # strided token rows
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged(kl, vl, kc_d, vc_d, torch.from_numpy(slots).to(torch.int16).to(DEV))
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged(bits(kl), want_k, slots)
    ko.linear_to_paged(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


def test_empty_and_out_of_bounds():
    kc = torch.zeros(4, 2, 8, 16, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    ok, ov = musa_aiter.kv_paged_to_linear(kc, vc, torch.zeros(0, dtype=torch.int64, device=DEV))
    assert ok.shape == (0, 2, 8) and ov.shape == (0, 2, 8)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_paged_to_linear(kc, vc, torch.tensor([0, 64], device=DEV))


def test_large_roundtrip_properties():
    # Llama-3-8B KV row shape at 4 layers and ~33k tokens: scatter then gather is the identity on
    # written slots, skipped tokens read back as zeros, and untouched blocks keep their bytes.
    layers, nb, nh, hd, bs = 4, 4096, 8, 128, 16
    rng = np.random.default_rng(21)
    lengths = [int(x) for x in rng.integers(128, 1024, size=48)]
    slots = sequence_slots(rng, lengths, num_blocks=nb, block_size=bs)
    slots[rng.random(len(slots)) < 0.01] = -1
    s_d = torch.from_numpy(slots).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(1)
    kl = torch.randn((layers, len(slots), nh, hd), generator=gen, device=DEV, dtype=torch.bfloat16)
    vl = torch.randn((layers, len(slots), nh, hd), generator=gen, device=DEV, dtype=torch.bfloat16)
    kc = torch.full((layers, nb, nh, hd, bs), 3.0, device=DEV, dtype=torch.bfloat16)
    vc = torch.full_like(kc, -3.0)
    musa_aiter.kv_linear_to_paged_multi_layer(kl, vl, kc, vc, s_d)
    rk, rv = musa_aiter.kv_paged_to_linear_multi_layer(kc, vc, s_d)
    valid = s_d >= 0
    assert torch.equal(rk[:, valid], kl[:, valid]) and torch.equal(rv[:, valid], vl[:, valid])
    assert int(torch.count_nonzero(rk[:, ~valid])) == 0
    used = torch.zeros(nb * bs, dtype=torch.bool, device=DEV)
    used[s_d[valid]] = True
    untouched = ~used.view(nb, bs)
    kc_t = kc.permute(0, 1, 4, 2, 3)  # [L, NB, BS, NH, HD]
    assert bool((kc_t[:, untouched] == 3.0).all())


@pytest.mark.parametrize("layers,tokens,kind", [
    (2, 2500, "duplicates"),    # scatter: 1,256 workgroups, the loads-first form
    (16, 2500, "duplicates"),   # scatter: 10,048 workgroups, the chunk-by-chunk form
    (16, 1500, "skips"),        # gather: 32 planes, 12,032 workgroups, the XCD-contiguous order
    (8, 1500, "sequences"),     # gather: 16 planes, natural order
])
def test_kernel_forms_either_side_of_the_launch_thresholds(layers, tokens, kind):
    # The tile kernels pick a form by launch size (scatters of at most 8,192 workgroups; gathers
    # over at least 32 planes and more than 8,192 workgroups): every form against the oracle,
    # with repeated, skipped and partial-block slots.
    shape = (8, 128, 16)
    nh, hd, _ = shape
    slots, kc, vc = _case(torch.bfloat16, shape, kind, tokens=tokens, seed=31 + layers, layers=layers)
    s_d = torch.from_numpy(slots).to(DEV)
    ok, ov = musa_aiter.kv_paged_to_linear_multi_layer(kc.to(DEV), vc.to(DEV), s_d)
    assert np.array_equal(bits(ok), ko.paged_to_linear_multi_layer(bits(kc), slots))
    assert np.array_equal(bits(ov), ko.paged_to_linear_multi_layer(bits(vc), slots))
    gen = torch.Generator().manual_seed(7)
    kl = random_payload((layers, len(slots), nh, hd), torch.bfloat16, gen)
    vl = random_payload((layers, len(slots), nh, hd), torch.bfloat16, gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged_multi_layer(kl.to(DEV), vl.to(DEV), kc_d, vc_d, s_d)
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged_multi_layer(bits(kl), want_k, slots)
    ko.linear_to_paged_multi_layer(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("layers,tokens,kind", [
    (1, 200, "decode"),          # at most 256 tokens: gathers may take the per-token form too,
    (4, 256, "random"),          # scatters resolve repeated slots in LDS
    (1, 301, "decode"),          # short launches: loads-first scatter, 128-thread gather
    (3, 301, "decode"),
    (2, 40000, "decode"),        # scatter above 8,192 workgroups: chunk-by-chunk form
    (16, 5000, "decode"),        # gather over 32 planes above 8,192 workgroups: XCD-contiguous order
    (2, 3000, "duplicates"),     # claimed slots in per-token tiles
])
def test_short_run_tiles_match_oracle(dtype, bs, layers, tokens, kind):
    # Tiles whose runs average fewer than 8 tokens move each token's rows
    # directly instead of through the LDS transpose; the decode pattern puts
    # such tiles next to tiles of whole blocks in one launch.
    shape = (4, 64, bs)
    nh, hd, _ = shape
    slots, kc, vc = _case(dtype, shape, kind, tokens=tokens, seed=51 + bs + layers, layers=layers)
    if kind == "decode":
        slots[np.random.default_rng(bs).random(len(slots)) < 0.05] = -1
    s_d = torch.from_numpy(slots).to(DEV)
    ok, ov = musa_aiter.kv_paged_to_linear_multi_layer(kc.to(DEV), vc.to(DEV), s_d)
    assert np.array_equal(bits(ok), ko.paged_to_linear_multi_layer(bits(kc), slots))
    assert np.array_equal(bits(ov), ko.paged_to_linear_multi_layer(bits(vc), slots))
    gen = torch.Generator().manual_seed(9)
    kl = random_payload((layers, len(slots), nh, hd), dtype, gen)
    vl = random_payload((layers, len(slots), nh, hd), dtype, gen)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    musa_aiter.kv_linear_to_paged_multi_layer(kl.to(DEV), vl.to(DEV), kc_d, vc_d, s_d)
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    ko.linear_to_paged_multi_layer(bits(kl), want_k, slots)
    ko.linear_to_paged_multi_layer(bits(vl), want_v, slots)
    assert np.array_equal(bits(kc_d), want_k)
    assert np.array_equal(bits(vc_d), want_v)


@pytest.mark.parametrize("dtype,shape,tokens", [
    (torch.float32, (4, 32, 32), 3000),   # 32 planes x 188 tiles x 2 row groups (12,032 workgroups): XCD order
    (torch.float16, (2, 64, 8), 5000),    # 32 planes x 313 tiles x 1 row group (10,016 workgroups): XCD order
    # 240-byte token rows (not whole 128-byte lines) keep non-temporal stores in both forms
    (torch.bfloat16, (3, 40, 16), 5000),  # 10,016 workgroups: XCD order
    (torch.bfloat16, (3, 40, 16), 600),   # 1,216 workgroups: the short 128-thread form
])
def test_xcd_order_gathers_other_shapes(dtype, shape, tokens):
    slots, kc, vc = _case(dtype, shape, "skips", tokens=tokens, seed=41, layers=16)
    s_d = torch.from_numpy(slots).to(DEV)
    ok, ov = musa_aiter.kv_paged_to_linear_multi_layer(kc.to(DEV), vc.to(DEV), s_d)
    assert np.array_equal(bits(ok), ko.paged_to_linear_multi_layer(bits(kc), slots))
    assert np.array_equal(bits(ov), ko.paged_to_linear_multi_layer(bits(vc), slots))


@pytest.mark.parametrize("n", [1, 100, 4097, 300_001])
def test_index_max_matches_torch(n):
    # The host-side bounds checks read the largest slot through musa_aiter_hip_index_max: one to 64
    # workgroups writing their maxima to pinned host memory.  Negative (skipped) slots included.
    from musa_aiter.ops import _hip

    rng = np.random.default_rng(n)
    vals = rng.integers(-(2 ** 40), 2 ** 40, size=n).astype(np.int64)
    for case in range(3):
        if case == 1:
            vals = -np.abs(vals) - 1  # all skipped
        if case == 2:
            vals[rng.integers(0, n)] = 2 ** 62  # one large entry anywhere
        t = torch.from_numpy(vals.copy()).to(DEV)
        assert _hip.index_max(t) == int(t.max().item())
