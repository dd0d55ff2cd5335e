"""Pins the FP8 codec of the oracle (oracle/kv_oracle.py) independently of the oracle's own text.

Reference function: musa_aiter/ops/kv_transfer.py:2161-2200 (_fp8_quantize_to_uint8,
_fp8_dequantize_from_uint8).  Checks, over every bf16 and fp16 bit pattern and
a set of scales:

1. torch's own float8_e4m3fn / float8_e5m2 casts (c10's round-to-nearest-even
   encoders, an independent implementation) on the range where the reference
   encoder is an IEEE cast: finite |w| >= min normal (E4M3: all of it, since
   both saturate to the 0x7F pattern above 464; E5M2: |w| <= 73728);
2. the non-IEEE rules as known answers: flush below the minimum normal to a
   signed zero, -0.0 -> 0x00, +Inf/NaN -> 0x00, -Inf -> 0x80, E4M3 464 -> 0x7E
   and above -> 0x7F, E5M2 codes above 61440 kept finite (0x7D..0x7F);
3. op-level agreement with the same steps written with torch ops (the ops the
   reference uses: log2, floor, pow, round), which pins numpy-vs-torch
   differences in those primitives (log2 rounding near powers of two);
4. decoding against torch's float8 -> float32 casts for every normal code and
   known answers for the codes torch treats as NaN/Inf;
5. the reference's own encoder and decoder: tests/golden/fp8_codec_golden.npz holds their
   outputs for every bf16 and fp16 pattern and every code under eight scales, written in this
   build container by tests/golden/make_fp8_golden.py.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import kv_oracle as ko
from tests import torch_ref

FORMATS = {"e4m3": (torch.float8_e4m3fn, 2.0 ** -6, float("inf")), "e5m2": (torch.float8_e5m2, 2.0 ** -14, 73728.0)}

SCALES = [
    1.0, 0.125, 0.25, 2.0, 3.0, 0.1, 1.7 / 448.0, 6.5 / 448.0, 50.0 / 448.0, 7.3e-5, 1e-3,
    float(np.nextafter(np.float32(2.0), np.float32(0.0))), float(np.nextafter(np.float32(2.0), np.float32(10.0))),
    float(np.nextafter(np.float32(0.5), np.float32(0.0))), 1e30, 1e-30,
]


def _all_bf16_as_f32() -> np.ndarray:
    return (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)


def _all_f16_as_f32() -> np.ndarray:
    return np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)


def _torch_steps_quantize(x: torch.Tensor, scale: torch.Tensor, fmt: str) -> torch.Tensor:
    """The encoder's steps written with torch primitives (tests/torch_ref.py; bench.py checks with it)."""
    return torch_ref.fp8_quantize(x, scale, fmt)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("source", ["bf16", "f16"])
def test_encoder_matches_torch_float8_cast_on_ieee_range(fmt, source):
    dtype, min_normal, upper = FORMATS[fmt]
    x = _all_bf16_as_f32() if source == "bf16" else _all_f16_as_f32()
    for scale in SCALES:
        with np.errstate(all="ignore"):
            w = (x / np.float32(scale)).astype(np.float32)
        ours = ko.fp8_quantize(x, np.float32(scale), fmt)
        sel = np.isfinite(w) & (np.abs(w) >= min_normal) & (np.abs(w) <= upper)
        theirs = torch.from_numpy(w[sel]).to(dtype).view(torch.uint8).numpy()
        mismatch = np.nonzero(ours[sel] != theirs)[0]
        assert mismatch.size == 0, (fmt, source, scale, w[sel][mismatch[:5]], ours[sel][mismatch[:5]],
                                    theirs[mismatch[:5]])


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_encoder_agrees_with_torch_primitives_exhaustively(fmt):
    x = np.concatenate([_all_bf16_as_f32(), _all_f16_as_f32()])
    xt = torch.from_numpy(x)
    for scale in SCALES:
        ours = ko.fp8_quantize(x, np.float32(scale), fmt)
        theirs = _torch_steps_quantize(xt, torch.tensor(scale, dtype=torch.float32), fmt).numpy()
        assert np.array_equal(ours, theirs), (fmt, scale, np.nonzero(ours != theirs)[0][:5])


def test_encoder_per_head_scale_broadcast():
    x = np.linspace(-3.0, 3.0, 2 * 8, dtype=np.float32).reshape(2, 8)
    scale = np.array([[0.125], [0.5]], dtype=np.float32)
    assert np.array_equal(ko.fp8_quantize(x, scale, "e4m3")[0], ko.fp8_quantize(x[0], np.float32(0.125), "e4m3"))
    assert np.array_equal(ko.fp8_quantize(x, scale, "e4m3")[1], ko.fp8_quantize(x[1], np.float32(0.5), "e4m3"))


def _f32(v: float) -> np.float32:
    return np.float32(v)


E4M3_KAT = [
    (0.0, 0x00), (-0.0, 0x00), (1.0, 0x38), (-1.0, 0xB8), (1.125, 0x39), (448.0, 0x7E), (-448.0, 0xFE),
    (464.0, 0x7E), (float(np.nextafter(_f32(464.0), _f32(1e9))), 0x7F), (480.0, 0x7F), (1e9, 0x7F), (-1e9, 0xFF),
    (float("inf"), 0x00), (float("-inf"), 0x80), (float("nan"), 0x00), (2.0 ** -6, 0x08),
    (float(np.nextafter(_f32(2.0 ** -6), _f32(0.0))), 0x00), (-(2.0 ** -7), 0x80), (2.0 ** -20, 0x00),
    (2.0 ** -6 * (1 + 1 / 16), 0x08), (2.0 ** -6 * (1 + 3 / 16), 0x0A), (float(np.nextafter(_f32(2.0), _f32(0.0))), 0x40),
    (1e-45, 0x00), (-1e-45, 0x80),
]
E5M2_KAT = [
    (0.0, 0x00), (-0.0, 0x00), (1.0, 0x3C), (-1.0, 0xBC), (57344.0, 0x7B), (61440.0, 0x7C), (65536.0, 0x7C),
    (73728.0, 0x7C), (float(np.nextafter(_f32(73728.0), _f32(1e9))), 0x7D), (98304.0, 0x7E), (114688.0, 0x7F),
    (1e9, 0x7F), (-1e9, 0xFF), (float("inf"), 0x00), (float("-inf"), 0x80), (float("nan"), 0x00),
    (2.0 ** -14, 0x04), (float(np.nextafter(_f32(2.0 ** -14), _f32(0.0))), 0x00), (-(2.0 ** -15), 0x80),
]


@pytest.mark.parametrize("fmt,table", [("e4m3", E4M3_KAT), ("e5m2", E5M2_KAT)])
def test_encoder_known_answers(fmt, table):
    w = np.array([v for v, _ in table], dtype=np.float32)
    got = ko.fp8_quantize(w, np.float32(1.0), fmt)
    want = np.array([b for _, b in table], dtype=np.uint8)
    assert np.array_equal(got, want), list(zip(w.tolist(), got.tolist(), want.tolist()))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_encoder_just_below_powers_of_two(fmt):
    # floor(log2(w)) may round up just below 2^e; the mantissa carry must give the same byte as exact rounding.
    dtype, min_normal, upper = FORMATS[fmt]
    emax = ko.FP8_FORMATS[fmt][3]
    e = np.arange(int(np.log2(min_normal)) + 1, emax + 1)
    w = np.nextafter(np.float32(2.0) ** e.astype(np.float32), np.float32(0.0)).astype(np.float32)
    w = np.concatenate([w, -w])
    theirs = torch.from_numpy(w).to(dtype).view(torch.uint8).numpy()
    assert np.array_equal(ko.fp8_quantize(w, np.float32(1.0), fmt), theirs)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_decoder_matches_torch_float8_cast_on_normal_codes(fmt):
    dtype, _, _ = FORMATS[fmt]
    codes = np.arange(256, dtype=np.uint8)
    mant = ko.FP8_FORMATS[fmt][1]
    exp_field = (codes.astype(np.int32) >> mant) & ((1 << (7 - mant)) - 1)
    top = (1 << (7 - mant)) - 1
    normal = (exp_field != 0) & ~((fmt == "e4m3") & ((codes & 0x7F) == 0x7F)) & ~((fmt == "e5m2") & (exp_field == top))
    ours = ko.fp8_dequantize_f32(codes, np.float32(1.0), fmt)
    theirs = torch.from_numpy(codes).view(dtype).to(torch.float32).numpy()
    assert np.array_equal(ours[normal].view(np.uint32), theirs[normal].view(np.uint32))


def test_decoder_known_answers():
    e4 = ko.fp8_dequantize_f32(np.array([0x7F, 0xFF, 0x80, 0x00, 0x01, 0x07, 0x81, 0x08, 0x38], np.uint8), 1.0, "e4m3")
    assert e4.tolist()[:2] == [480.0, -480.0]
    assert e4.view(np.uint32).tolist()[2:7] == [0x80000000, 0, 0, 0, 0x80000000]
    assert e4.tolist()[7:] == [2.0 ** -6, 1.0]
    e5 = ko.fp8_dequantize_f32(np.array([0x7C, 0x7D, 0x7F, 0xFF, 0x03, 0x83, 0x3C], np.uint8), 1.0, "e5m2")
    assert e5.tolist()[:4] == [65536.0, 81920.0, 114688.0, -114688.0]
    assert e5.view(np.uint32).tolist()[4:6] == [0, 0x80000000]
    assert e5.tolist()[6] == 1.0


def test_decoder_scale_multiply_is_fp32_then_rounded():
    codes = np.arange(256, dtype=np.uint8)
    for scale in SCALES:
        v = ko.fp8_dequantize_f32(codes, np.float32(scale), "e4m3")
        base = ko.fp8_dequantize_f32(codes, np.float32(1.0), "e4m3")
        with np.errstate(all="ignore"):
            assert np.array_equal(v.view(np.uint32), (base * np.float32(scale)).astype(np.float32).view(np.uint32))


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F7FFFFF, 0x00000001,
                         0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7F8000], dtype=np.uint32)
    x = np.concatenate([bits, specials]).view(np.float32)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ours = ko.f32_to_bf16_bits(x)
    # NaN payloads differ between torch's scalar (0x7FC0) and vectorised (0xFFFF) CPU
    # paths; the FP8 dequant path never produces NaN (finite code times finite scale).
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert np.isnan(ko.bf16_bits_to_f32(ours[nan])).all() and np.isnan(ko.bf16_bits_to_f32(theirs[nan])).all()


def test_f16_rounding_matches_torch():
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.standard_normal(1 << 18).astype(np.float32) * np.float32(3e4),
                        rng.standard_normal(1 << 18).astype(np.float32) * np.float32(1e-5),
                        np.array([65504.0, 65520.0, 65519.99, 1e-8, -0.0, 6e-8, 3e-8], np.float32)])
    theirs = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ko.to_storage(x, "float16"), theirs)


def test_division_matches_torch_exhaustively():
    x = _all_bf16_as_f32()
    for scale in SCALES:
        with np.errstate(all="ignore"):
            ours = (x / np.float32(scale)).astype(np.float32)
        theirs = (torch.from_numpy(x) / torch.tensor(scale, dtype=torch.float32)).numpy()
        assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_torch_decode_table_matches_oracle_on_every_code(fmt):
    # tests/torch_ref.py's decoder (used by bench.py's checks) against the oracle's, all 256 codes and two scales.
    codes = np.arange(256, dtype=np.uint8)
    for scale in (1.0, 0.0123):
        mine = torch_ref.fp8_dequantize(torch.from_numpy(codes), torch.tensor(scale), fmt, torch.float32).numpy()
        want = ko.fp8_dequantize_f32(codes, np.float32(scale), fmt)
        assert np.array_equal(mine.view(np.uint32), want.view(np.uint32))
    assert torch_ref.FP8_FORMATS[fmt] == ko.FP8_FORMATS[fmt]


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fp8_codec_golden.npz")


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("source", ["bf16", "fp16"])
def test_encoder_matches_reference_golden_table(fmt, source):
    golden = np.load(GOLDEN)
    x = _all_bf16_as_f32() if source == "bf16" else _all_f16_as_f32()
    table = golden[f"encode_{fmt}_{source}"]
    for i, s in enumerate(golden["scales"]):
        want = table[i]
        got = ko.fp8_quantize(x, s, fmt)
        assert np.array_equal(got, want), (float(s), np.flatnonzero(got != want)[:5])
        via_torch = torch_ref.fp8_quantize(torch.from_numpy(x), torch.tensor(float(s), dtype=torch.float32), fmt)
        assert np.array_equal(via_torch.numpy(), want), float(s)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_decoder_matches_reference_golden_table(fmt):
    golden = np.load(GOLDEN)
    codes = np.arange(256, dtype=np.uint8)
    for i, s in enumerate(golden["scales"]):
        f32 = ko.fp8_dequantize_f32(codes, s, fmt)
        assert np.array_equal(f32.view(np.uint32), golden[f"decode_{fmt}_f32"][i])
        assert np.array_equal(ko.f32_to_bf16_bits(f32), golden[f"decode_{fmt}_bf16"][i])
        with np.errstate(over="ignore"):  # values beyond fp16's range round to +-Inf, as torch's cast does
            f16 = f32.astype(np.float16)
        assert np.array_equal(f16.view(np.uint16), golden[f"decode_{fmt}_fp16"][i])
