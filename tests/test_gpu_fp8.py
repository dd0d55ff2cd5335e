"""GPU parity: fused FP8 quant-store / dequant-gather vs the oracle, bit-exact.

The linear inputs enumerate every bf16 (or fp16) bit pattern, so each test
covers the whole input domain of the encoder for its scales, including
subnormals, +-0, +-Inf and NaNs; scales include per-head amax/448 values and
powers of two +-1 ulp.  Dequantised outputs are compared bit-for-bit with the
oracle (stricter than the 1-ulp bound the path promises).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from oracle import kv_oracle as ko
from tests.kvgen import bits, make_slots

pytestmark = pytest.mark.gpu
DEV = "cuda"
NH, HD, BS = 8, 128, 16
LIN_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _all_patterns(dtype: torch.dtype) -> torch.Tensor:
    """[512, NH, HD] tensor holding every 16-bit pattern once (bf16/fp16) or a spread of fp32 values."""
    if dtype == torch.float32:
        gen = torch.Generator().manual_seed(0)
        raw = torch.randint(-(2 ** 31), 2 ** 31 - 1, (512 * NH * HD,), dtype=torch.int32, generator=gen)
        return raw.view(torch.float32).reshape(512, NH, HD)
    raw = torch.arange(-(2 ** 15), 2 ** 15, dtype=torch.int32).to(torch.int16)
    return raw.view(dtype).reshape(-1, NH, HD)


def _lin_f32(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.float32).numpy()


def _scales(kind: str, rng: np.random.Generator) -> torch.Tensor:
    if kind == "scalar":
        return torch.tensor(1.7 / 448.0, dtype=torch.float32)
    if kind == "per_head":
        vals = np.array([1.0, 0.125, 2.0 / 448.0, 50.0 / 448.0, np.nextafter(np.float32(2.0), np.float32(0.0)),
                         np.nextafter(np.float32(0.5), np.float32(1.0)), 3.0, 7.3e-5], dtype=np.float32)
        return torch.from_numpy(vals)
    raise ValueError(kind)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("lin", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("scale_kind", ["scalar", "per_head"])
def test_quant_store_then_dequant_gather_exhaustive(fmt, lin, scale_kind):
    dtype = LIN_DTYPES[lin]
    rng = np.random.default_rng(31)
    x = _all_patterns(dtype)
    tokens = x.shape[0]
    slots, nb = make_slots("sequences", rng, block_size=BS, tokens=tokens)
    slots[rng.random(tokens) < 0.05] = -1
    xv = x.flip(0).contiguous()
    ks, vs = _scales(scale_kind, rng), _scales(scale_kind, rng).flip(0).contiguous()
    kc = torch.zeros(nb, NH, HD, BS, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    s_d = torch.from_numpy(slots).to(DEV)
    musa_aiter.kv_linear_to_paged_fp8(x.to(DEV), xv.to(DEV), kc_d, vc_d, s_d, ks.to(DEV), vs.to(DEV), fp8_format=fmt)
    want_k, want_v = kc.numpy().copy(), vc.numpy().copy()
    ko.linear_to_paged_fp8(_lin_f32(x), want_k, slots, ks.numpy(), fmt)
    ko.linear_to_paged_fp8(_lin_f32(xv), want_v, slots, vs.numpy(), fmt)
    got_k, got_v = kc_d.cpu().numpy(), vc_d.cpu().numpy()
    assert np.array_equal(got_k, want_k), np.argwhere(got_k != want_k)[:5]
    assert np.array_equal(got_v, want_v)
    for out_name, out_dtype in LIN_DTYPES.items():
        rk, rv = musa_aiter.kv_paged_fp8_to_linear(kc_d, vc_d, s_d, ks.to(DEV), vs.to(DEV), out_dtype=out_dtype,
                                                   fp8_format=fmt)
        assert np.array_equal(bits(rk), ko.paged_fp8_to_linear(want_k, slots, ks.numpy(), fmt, out_name))
        assert np.array_equal(bits(rv), ko.paged_fp8_to_linear(want_v, slots, vs.numpy(), fmt, out_name))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_multi_layer_layer_head_scales_and_merged(fmt):
    layers, tokens = 3, 600
    rng = np.random.default_rng(32)
    slots, nb = make_slots("skips", rng, block_size=BS, tokens=tokens)
    gen = torch.Generator().manual_seed(2)
    kl = (torch.randn((layers, tokens, NH, HD), generator=gen) * 2.0).to(torch.bfloat16)
    vl = (torch.randn((layers, tokens, NH, HD), generator=gen) * 2.0).to(torch.bfloat16)
    ks = torch.rand((layers, NH), generator=gen) * 0.02 + 1e-3
    vs = torch.rand((layers, NH), generator=gen) * 0.02 + 1e-3
    kc = torch.zeros(layers, nb, NH, HD, BS, dtype=torch.uint8, device=DEV)
    vc = torch.zeros_like(kc)
    s_d = torch.from_numpy(slots).to(DEV)
    merged = torch.stack((kl, vl), dim=2).to(DEV)
    musa_aiter.kv_merged_linear_to_paged_fp8_multi_layer(merged, kc, vc, s_d, ks.to(DEV), vs.to(DEV), fp8_format=fmt)
    want_k = np.zeros((layers, nb, NH, HD, BS), np.uint8)
    want_v = np.zeros_like(want_k)
    for layer in range(layers):
        ko.linear_to_paged_fp8(_lin_f32(kl[layer]), want_k[layer], slots, ks.numpy(), fmt, layer=layer)
        ko.linear_to_paged_fp8(_lin_f32(vl[layer]), want_v[layer], slots, vs.numpy(), fmt, layer=layer)
    assert np.array_equal(kc.cpu().numpy(), want_k)
    assert np.array_equal(vc.cpu().numpy(), want_v)
    out = musa_aiter.kv_paged_fp8_to_merged_linear_multi_layer(kc, vc, s_d, ks.to(DEV), vs.to(DEV), fp8_format=fmt)
    for layer in range(layers):
        assert np.array_equal(bits(out[layer, :, 0]),
                              ko.paged_fp8_to_linear(want_k[layer], slots, ks.numpy(), fmt, "bfloat16", layer=layer))
        assert np.array_equal(bits(out[layer, :, 1]),
                              ko.paged_fp8_to_linear(want_v[layer], slots, vs.numpy(), fmt, "bfloat16", layer=layer))


def test_float8_dtype_caches_and_block_size_32():
    bs, tokens = 32, 500
    rng = np.random.default_rng(33)
    slots, nb = make_slots("sequences", rng, block_size=bs, tokens=tokens)
    gen = torch.Generator().manual_seed(3)
    kl = torch.randn((tokens, NH, HD), generator=gen).to(torch.float16)
    kc = torch.zeros(nb, NH, HD, bs, dtype=torch.float8_e4m3fn, device=DEV)
    vc = torch.zeros_like(kc)
    s_d = torch.from_numpy(slots).to(DEV)
    musa_aiter.kv_linear_to_paged_fp8(kl.to(DEV), kl.to(DEV), kc, vc, s_d, 0.02, 0.02)
    want = np.zeros((nb, NH, HD, bs), np.uint8)
    ko.linear_to_paged_fp8(_lin_f32(kl), want, slots, np.float32(0.02), "e4m3")
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), want)


def test_reference_fp8_roundtrip_tolerances():
    # op_tests/test_kv_transfer.py:402-427 scenario and tolerances, on the GPU path.
    nb, kvh, d, blk = 3, 2, 8, 4
    t = 5
    k_lin = torch.linspace(-1.5, 1.5, steps=t * kvh * d, dtype=torch.float32).reshape(t, kvh, d)
    v_lin = torch.linspace(1.25, -1.25, steps=t * kvh * d, dtype=torch.float32).reshape(t, kvh, d)
    k_cache = torch.zeros(nb, kvh, d, blk, dtype=torch.uint8, device=DEV)
    v_cache = torch.zeros_like(k_cache)
    slots = torch.tensor([0, 7, -1, 5, 9], dtype=torch.int32, device=DEV)
    scale = torch.tensor(0.125, dtype=torch.float32)
    musa_aiter.kv_linear_to_paged_fp8(k_lin.to(DEV), v_lin.to(DEV), k_cache, v_cache, slots, scale, scale)
    rk, rv = musa_aiter.kv_paged_fp8_to_linear(k_cache, v_cache, slots, scale, scale, out_dtype=torch.float32)
    valid = (slots >= 0).cpu()
    torch.testing.assert_close(rk.cpu()[valid], k_lin[valid], atol=0.065, rtol=0.08)
    torch.testing.assert_close(rv.cpu()[valid], v_lin[valid], atol=0.065, rtol=0.08)
    assert rk.cpu()[~valid].abs().max() == 0


def test_raw_symbol_scalar_scale_matches_api():
    # The reference-named C symbol, bound with ctypes exactly as the reference's shim does.
    import ctypes

    from musa_aiter.ops import _hip

    lib = _hip.library()
    tokens = 100
    rng = np.random.default_rng(34)
    slots, nb = make_slots("sequences", rng, block_size=BS, tokens=tokens)
    gen = torch.Generator().manual_seed(4)
    kl = torch.randn((tokens, NH, HD), generator=gen).to(torch.bfloat16).to(DEV)
    kc = torch.zeros(nb, NH, HD, BS, dtype=torch.uint8, device=DEV)
    vc = torch.zeros_like(kc)
    scale = torch.tensor(0.01, dtype=torch.float32, device=DEV)
    s_d = torch.from_numpy(slots).to(DEV)
    fn = lib.musa_aiter_kv_linear_to_paged_fp8_e4m3
    fn.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_longlong] * 5 + [ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    rc = fn(kl.data_ptr(), kl.data_ptr(), s_d.data_ptr(), kc.data_ptr(), vc.data_ptr(), scale.data_ptr(),
            scale.data_ptr(), tokens, nb, NH, HD, BS, 2, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    want = np.zeros((nb, NH, HD, BS), np.uint8)
    ko.linear_to_paged_fp8(_lin_f32(kl.cpu()), want, slots, np.float32(0.01), "e4m3")
    assert np.array_equal(kc.cpu().numpy(), want)


def _fast_range_inputs(lin: str, rng: np.random.Generator) -> torch.Tensor:
    """Inputs whose every lane tile lies in the quantiser's hoisted-reciprocal range (zero allowed)."""
    if lin == "float32":
        mag = np.exp2(rng.uniform(-60.0, 60.0, size=48 * NH * HD)).astype(np.float32)
        vals = np.where(rng.random(mag.size) < 0.5, -mag, mag).astype(np.float32)
        vals[rng.random(vals.size) < 0.01] = 0.0
        return torch.from_numpy(vals.reshape(-1, NH, HD))
    dtype = LIN_DTYPES[lin]
    raw = torch.arange(0, 2 ** 16, dtype=torch.int32).to(torch.int16).view(dtype).float()
    finite = torch.isfinite(raw) & ((raw == 0) | ((raw.abs() >= 2.0 ** -60) & (raw.abs() < 2.0 ** 60)))
    vals = raw[finite].to(dtype)
    vals = vals[torch.from_numpy(rng.permutation(vals.numel()))]
    pad = (-vals.numel()) % (NH * HD)
    vals = torch.cat([vals, vals[:pad]])
    return vals.reshape(-1, NH, HD)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("lin", ["bfloat16", "float16", "float32"])
def test_quant_store_fast_reciprocal_range_many_scales(fmt, lin):
    """Tiles in the hoisted-reciprocal range, log-uniform per-head scales and the range edges."""
    rng = np.random.default_rng(41)
    x = _fast_range_inputs(lin, rng)
    tokens = x.shape[0]
    slots, nb = make_slots("sequences", rng, block_size=BS, tokens=tokens)
    s_d = torch.from_numpy(slots).to(DEV)
    edges = np.array([2.0 ** -60, np.nextafter(np.float32(2.0 ** 60), np.float32(0.0)), 2.0 ** -61, 2.0 ** 60],
                     dtype=np.float32)
    for rep in range(6):
        ks = np.exp2(rng.uniform(-50.0, 50.0, size=NH)).astype(np.float32)
        ks *= np.float32(1.0) + rng.random(NH).astype(np.float32)
        if rep == 0:
            ks[:4] = edges
        vs = np.exp2(rng.uniform(-12.0, 4.0, size=NH)).astype(np.float32)
        kc_d = torch.zeros(nb, NH, HD, BS, dtype=torch.uint8, device=DEV)
        vc_d = torch.zeros_like(kc_d)
        musa_aiter.kv_linear_to_paged_fp8(x.to(DEV), x.flip(0).contiguous().to(DEV), kc_d, vc_d, s_d,
                                          torch.from_numpy(ks).to(DEV), torch.from_numpy(vs).to(DEV), fp8_format=fmt)
        want_k = np.zeros((nb, NH, HD, BS), np.uint8)
        want_v = np.zeros_like(want_k)
        ko.linear_to_paged_fp8(_lin_f32(x), want_k, slots, ks, fmt)
        ko.linear_to_paged_fp8(_lin_f32(x.flip(0).contiguous()), want_v, slots, vs, fmt)
        got_k, got_v = kc_d.cpu().numpy(), vc_d.cpu().numpy()
        assert np.array_equal(got_k, want_k), (rep, np.argwhere(got_k != want_k)[:5])
        assert np.array_equal(got_v, want_v), (rep, np.argwhere(got_v != want_v)[:5])


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("bs", [16, 32])
def test_quant_store_bf16_tiny_inputs_scale_window_edges(fmt, bs):
    """Every finite bf16 pattern (subnormals and values below 2^-60 included) with per-head scales at and
    beyond the edges of the bf16 fast window [2^-45, 2^15): the fast tiles, the fallback tiles and the
    partial runs must all give the reference bytes."""
    rng = np.random.default_rng(43)
    raw = torch.arange(0, 2 ** 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    vals = raw[torch.isfinite(raw.float())]
    vals = vals[torch.from_numpy(rng.permutation(vals.numel()))]
    pad = (-vals.numel()) % (NH * HD)
    x = torch.cat([vals, vals[:pad]]).reshape(-1, NH, HD)
    tokens = x.shape[0]
    slots, nb = make_slots("sequences", rng, block_size=bs, tokens=tokens)
    s_d = torch.from_numpy(slots).to(DEV)
    ks = np.array([2.0 ** -46, 2.0 ** -45, np.nextafter(np.float32(2.0 ** 15), np.float32(0.0)), 2.0 ** 15,
                   2.0 ** 20, 2.0 ** -50, 1.0, 0.01], dtype=np.float32)
    vs = ks[::-1].copy()
    kc_d = torch.zeros(nb, NH, HD, bs, dtype=torch.uint8, device=DEV)
    vc_d = torch.zeros_like(kc_d)
    musa_aiter.kv_linear_to_paged_fp8(x.to(DEV), x.flip(0).contiguous().to(DEV), kc_d, vc_d, s_d,
                                      torch.from_numpy(ks).to(DEV), torch.from_numpy(vs).to(DEV), fp8_format=fmt)
    want_k = np.zeros((nb, NH, HD, bs), np.uint8)
    want_v = np.zeros_like(want_k)
    ko.linear_to_paged_fp8(_lin_f32(x), want_k, slots, ks, fmt)
    ko.linear_to_paged_fp8(_lin_f32(x.flip(0).contiguous()), want_v, slots, vs, fmt)
    got_k, got_v = kc_d.cpu().numpy(), vc_d.cpu().numpy()
    assert np.array_equal(got_k, want_k), np.argwhere(got_k != want_k)[:5]
    assert np.array_equal(got_v, want_v), np.argwhere(got_v != want_v)[:5]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("lin", ["bfloat16", "float16"])
def test_quant_store_matches_reference_golden_codes(fmt, lin):
    # Every 16-bit pattern under each scale of tests/golden/fp8_codec_golden.npz (the reference's own
    # encoder outputs): token t, head h, dim d holds flat index k = t*1024 + h*128 + d, i.e. the int16
    # value k - 32768, whose bit pattern is k ^ 0x8000.
    import os

    golden = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fp8_codec_golden.npz"))
    table = golden[f"encode_{fmt}_{'bf16' if lin == 'bfloat16' else 'fp16'}"]
    x = _all_patterns(LIN_DTYPES[lin]).to(DEV)
    tokens = x.shape[0]
    slots = torch.arange(tokens, dtype=torch.int64, device=DEV)
    nb = tokens // BS
    flat = np.arange(tokens * NH * HD)
    for i, s in enumerate(golden["scales"]):
        kc = torch.zeros(nb, NH, HD, BS, dtype=torch.uint8, device=DEV)
        vc = torch.zeros_like(kc)
        scale = torch.tensor(float(s), dtype=torch.float32, device=DEV)
        musa_aiter.kv_linear_to_paged_fp8(x, x, kc, vc, slots, scale, scale, fp8_format=fmt)
        got = kc.permute(0, 3, 1, 2).reshape(-1).cpu().numpy()   # slot-major = token-major rows
        assert np.array_equal(got, table[i][flat ^ 0x8000]), float(s)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("lin", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("inputs", ["all_patterns", "fast_range"])
def test_quant_store_decode_shaped_tiles(fmt, lin, bs, inputs):
    """Decode-shaped slots (one to six tokens per sequence at random block offsets, every eighth
    sequence longer), token order (the cache is mostly unused): tiles of short runs quantise
    each token's rows element by element; every bit pattern reaches the exact path, the
    fast-range inputs the fast one."""
    dtype = LIN_DTYPES[lin]
    rng = np.random.default_rng(61 + bs)
    x = _all_patterns(dtype) if inputs == "all_patterns" else _fast_range_inputs(lin, rng)
    tokens = x.shape[0]
    slots, nb = make_slots("decode", rng, block_size=bs, tokens=tokens, spare_blocks=300)
    slots[rng.random(tokens) < 0.05] = -1
    assert 4 * tokens < nb * bs  # below the destination-order coverage
    xv = x.flip(0).contiguous()
    for scale_kind in ("scalar", "per_head"):
        ks, vs = _scales(scale_kind, rng), _scales(scale_kind, rng).flip(0).contiguous()
        kc_d = torch.zeros(nb, NH, HD, bs, dtype=torch.uint8, device=DEV)
        vc_d = torch.zeros_like(kc_d)
        s_d = torch.from_numpy(slots).to(DEV)
        musa_aiter.kv_linear_to_paged_fp8(x.to(DEV), xv.to(DEV), kc_d, vc_d, s_d, ks.to(DEV), vs.to(DEV),
                                          fp8_format=fmt)
        want_k = np.zeros((nb, NH, HD, bs), np.uint8)
        want_v = np.zeros_like(want_k)
        ko.linear_to_paged_fp8(_lin_f32(x), want_k, slots, ks.numpy(), fmt)
        ko.linear_to_paged_fp8(_lin_f32(xv), want_v, slots, vs.numpy(), fmt)
        got_k, got_v = kc_d.cpu().numpy(), vc_d.cpu().numpy()
        assert np.array_equal(got_k, want_k), (scale_kind, np.argwhere(got_k != want_k)[:5])
        assert np.array_equal(got_v, want_v), (scale_kind, np.argwhere(got_v != want_v)[:5])
        # The same slots back (at most 256 tokens: the dequant-gather's per-token tiles).
        for out_name, out_dtype in LIN_DTYPES.items():
            rk, rv = musa_aiter.kv_paged_fp8_to_linear(kc_d, vc_d, s_d, ks.to(DEV), vs.to(DEV), out_dtype=out_dtype,
                                                       fp8_format=fmt)
            assert np.array_equal(bits(rk), ko.paged_fp8_to_linear(want_k, slots, ks.numpy(), fmt, out_name))
            assert np.array_equal(bits(rv), ko.paged_fp8_to_linear(want_v, slots, vs.numpy(), fmt, out_name))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("tokens", [200, 512])
def test_quant_store_decode_shaped_duplicates(fmt, tokens):
    """Repeated slots in token order keep the last writer in per-token tiles: found in the
    kernel's LDS table for calls of at most 256 tokens, by the claim pass above."""
    rng = np.random.default_rng(71)
    x = _all_patterns(torch.bfloat16).repeat(8, 1, 1)[:tokens].contiguous()  # 64 tokens of patterns, repeated
    slots, nb = make_slots("duplicates", rng, block_size=BS, tokens=tokens, spare_blocks=300)
    ks = _scales("per_head", rng)
    kc_d = torch.zeros(nb, NH, HD, BS, dtype=torch.uint8, device=DEV)
    vc_d = torch.zeros_like(kc_d)
    s_d = torch.from_numpy(slots).to(DEV)
    musa_aiter.kv_linear_to_paged_fp8(x.to(DEV), x.to(DEV), kc_d, vc_d, s_d, ks.to(DEV), ks.to(DEV), fp8_format=fmt)
    want = np.zeros((nb, NH, HD, BS), np.uint8)
    ko.linear_to_paged_fp8(_lin_f32(x), want, slots, ks.numpy(), fmt)
    assert np.array_equal(kc_d.cpu().numpy(), want)
    assert np.array_equal(vc_d.cpu().numpy(), want)
