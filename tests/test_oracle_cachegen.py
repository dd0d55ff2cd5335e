"""Pins the CacheGen codec of the oracle (oracle/cachegen_oracle.py) independently of its text.

Reference functions: musa_aiter/ops/kv_transfer.py:1111-1215 (kv_cachegen_encode,
kv_cachegen_decode).  Checks:

1. the reference's own scenarios (op_tests/test_kv_transfer.py:218-250);
2. torch on the CPU evaluating the reference's expressions (an independent implementation of
   its rounding, reciprocal, linspace, cumsum and division) over random tensors;
3. known answers built so that a plausible mistake changes the result: a true division in
   place of torch's reciprocal-times-integer scale, rounding half away from zero in the torch
   path, float32 accumulation in the CDF, plain multiply-add in the codebook;
4. exact arithmetic (fractions) for the fused multiply-add helper and the CDF quotient;
5. closed forms of the codebook (two bins, integer ranges).
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import cachegen_oracle as cg

F32 = np.float32


def _torch_encode(x: torch.Tensor, num_bins: int):
    """The reference's torch path (kv_transfer.py:1124-1172) run on the CPU."""
    work = x.float()
    min_val, max_val = work.min(), work.max()
    if bool((max_val == min_val).item()):
        cdf = torch.zeros(num_bins + 1)
        cdf[1:] = 1.0
        return (torch.zeros_like(x, dtype=torch.uint8), torch.full((num_bins,), min_val.item()), cdf)
    scale = (num_bins - 1) / (max_val - min_val)
    enc = torch.round((work - min_val) * scale).clamp_(0, num_bins - 1).to(torch.long)
    codebook = torch.linspace(min_val.item(), max_val.item(), num_bins, dtype=torch.float32)
    counts = torch.bincount(enc.reshape(-1), minlength=num_bins).to(torch.float32)
    cdf = torch.empty(num_bins + 1)
    cdf[0] = 0.0
    cdf[1:] = torch.cumsum(counts, dim=0) / float(enc.numel())
    return enc.to(torch.uint8), codebook, cdf


def _bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- 1. the reference's own scenarios ---------------------------------------------------------

def test_reference_roundtrip_and_cdf():
    x = np.linspace(-1.0, 1.0, 17, dtype=np.float32).reshape(1, 17)
    enc, book, cdf = cg.encode(x, 16)
    dec = cg.decode(enc, book)
    assert enc.dtype == np.uint8 and book.shape == (16,) and cdf.shape == (17,)
    assert cdf[0] == 0 and cdf[-1] == 1 and np.all(cdf[1:] >= cdf[:-1])
    assert dec.shape == x.shape
    assert np.max(np.abs(dec - x)) <= 2.0 / 15.0


def test_reference_constant_tensor():
    x = np.full((2, 3), 5.0, np.float32)
    enc, book, cdf = cg.encode(x, 8)
    assert enc.max() == 0
    np.testing.assert_array_equal(cg.decode(enc, book), x)
    assert cdf[0] == 0 and np.all(cdf[1:] == 1)


def test_rejects_bad_bins_and_decode_overflow():
    with pytest.raises(ValueError, match="num_bins must be in"):
        cg.encode(np.zeros(4, np.float32), 1)
    with pytest.raises(ValueError, match="num_bins must be in"):
        cg.encode(np.zeros(4, np.float32), 257)
    with pytest.raises(ValueError, match="exceeds codebook size"):
        cg.decode(np.array([0, 4], np.uint8), np.zeros(4, np.float32))


def test_empty_tensor():
    enc, book, cdf = cg.encode(np.zeros((0, 5), np.float32), 7)
    assert enc.shape == (0, 5) and enc.dtype == np.uint8
    assert np.all(book == 0) and book.shape == (7,) and np.all(cdf == 0) and cdf.shape == (8,)


# ---- 2. torch on the CPU over random tensors --------------------------------------------------

@pytest.mark.parametrize("seed", range(6))
def test_torch_path_matches_torch_cpu(seed):
    rng = np.random.default_rng(seed)
    for _ in range(25):
        n = int(rng.integers(1, 3000))
        nb = int(rng.choice([2, 3, 16, 100, 255, 256, int(rng.integers(2, 257))]))
        x = (rng.standard_normal(n) * 10.0 ** rng.integers(-4, 5) + rng.standard_normal()).astype(np.float32)
        if rng.random() < 0.2:
            x = np.round(x * 4) / 4  # many exact ties
        e_ref, b_ref, c_ref = _torch_encode(torch.from_numpy(x), nb)
        e, b, c = cg.encode(x, nb)
        np.testing.assert_array_equal(e, e_ref.numpy())
        np.testing.assert_array_equal(_bits(b), _bits(b_ref.numpy()))
        np.testing.assert_array_equal(_bits(c), _bits(c_ref.numpy()))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float64])
def test_other_input_dtypes_match_torch_cpu(dtype):
    rng = np.random.default_rng(11)
    x = torch.from_numpy((rng.standard_normal(4000) * 3).astype(np.float64)).to(dtype)
    e_ref, b_ref, c_ref = _torch_encode(x, 256)
    if dtype == torch.bfloat16:
        raw, name = x.view(torch.int16).numpy().view(np.uint16), "bfloat16"
    else:
        raw, name = x.numpy(), str(dtype).split(".")[1]
    e, b, c = cg.encode(raw, 256, dtype=name)
    np.testing.assert_array_equal(e, e_ref.numpy())
    np.testing.assert_array_equal(_bits(b), _bits(b_ref.numpy()))
    np.testing.assert_array_equal(_bits(c), _bits(c_ref.numpy()))


def test_linspace_matches_torch_cpu():
    rng = np.random.default_rng(3)
    for _ in range(3000):
        a, b = np.sort((rng.standard_normal(2) * 10.0 ** rng.integers(-5, 6)).astype(np.float32))
        n = int(rng.integers(2, 257))
        ref = torch.linspace(float(a), float(b), n, dtype=torch.float32).numpy()
        np.testing.assert_array_equal(_bits(cg.linspace_f32(float(a), float(b), n)), _bits(ref))


# ---- 3. known answers that separate plausible mistakes -----------------------------------------

def test_scale_is_reciprocal_times_bins():
    # (nb - 1) / d == 231 / 1.8889903 rounds differently from (1 / d) * 231 in float32, and
    # the element 0.51109046 lands in bin 63 only with the reciprocal form.
    mx, x, nb = F32(1.8889903), F32(0.51109046), 232
    assert cg.torch_scale(F32(0), mx, nb) != F32(F32(nb - 1) / mx)
    work = torch.tensor([0.0, float(x), float(mx)])
    ref = _torch_encode(work, nb)[0].numpy()
    enc = cg.encode(np.array([0.0, x, mx], np.float32), nb)[0]
    assert ref[1] == 63 and enc[1] == 63
    wrong = cg.torch_bins(np.array([x], np.float32), F32(0), F32(F32(nb - 1) / mx), nb)
    assert wrong[0] == 62


def test_torch_path_rounds_half_to_even_native_half_up():
    x = np.array([0.0, 0.5, 1.5, 2.5, 3.0], np.float32)  # scale is exactly 1 for 4 bins over [0, 3]
    assert torch.equal(_torch_encode(torch.from_numpy(x), 4)[0], torch.tensor([0, 0, 2, 2, 3], dtype=torch.uint8))
    np.testing.assert_array_equal(cg.encode(x, 4)[0], [0, 0, 2, 2, 3])
    np.testing.assert_array_equal(cg.encode(x, 4, native=True)[0], [0, 1, 2, 3, 3])
    # the native rounding applies to float32 input only, as in the reference
    np.testing.assert_array_equal(cg.encode(x.astype(np.float16), 4, native=True, dtype="float16")[0],
                                  [0, 0, 2, 2, 3])


def test_native_scale_is_double_quotient():
    # 255 / (max - min) in double, then one rounding to float32
    mn, mx = F32(-0.7), F32(1.3)
    exact = Fraction(255) / (Fraction(float(mx)) - Fraction(float(mn)))
    assert Fraction(float(cg.native_scale(mn, mx, 256))) == Fraction(float(F32(float(exact))))


def test_cdf_accumulates_in_double_and_divides():
    counts = np.array([2**24 + 1, 1, 1, 3, 0, 7], dtype=np.int64)
    numel = int(counts.sum())
    ref = torch.empty(counts.size + 1)
    ref[0] = 0
    ref[1:] = torch.cumsum(torch.from_numpy(counts).to(torch.float32), dim=0) / float(numel)
    got = cg.cdf(counts, numel)
    np.testing.assert_array_equal(_bits(got), _bits(ref.numpy()))
    # float32 accumulation would lose the second and third ones (2**24 + 1 rounds to 2**24)
    f32_acc = np.cumsum(counts.astype(np.float32)).astype(np.float32) / F32(numel)
    assert not np.array_equal(_bits(got[1:]), _bits(f32_acc))


def test_cdf_is_correctly_rounded_quotient_below_2_24():
    rng = np.random.default_rng(4)
    counts = rng.integers(0, 5000, 256)
    numel = int(counts.sum())
    got = cg.cdf(counts, numel)
    pref = np.cumsum(counts)
    for k in range(256):
        want = F32(float(Fraction(int(pref[k]), numel)))  # exact quotient, one rounding
        assert got[k + 1] == want
    assert got[-1] == 1.0


def test_codebook_uses_fused_multiply_add():
    rng = np.random.default_rng(9)
    seen = False
    for _ in range(500):
        a, b = np.sort((rng.standard_normal(2) * 100).astype(np.float32))
        n = int(rng.integers(3, 257))
        ref = torch.linspace(float(a), float(b), n).numpy()
        step = F32(F32(b - a) / F32(n - 1))
        i = np.arange(n)
        plain = np.where(i < n // 2, a + step * i.astype(np.float32),
                         b - step * (n - 1 - i).astype(np.float32)).astype(np.float32)
        if not np.array_equal(_bits(plain), _bits(ref)):
            seen = True
            np.testing.assert_array_equal(_bits(cg.linspace_f32(float(a), float(b), n)), _bits(ref))
    assert seen  # the unfused form differs from torch somewhere in this sample


# ---- 4. exact arithmetic ------------------------------------------------------------------------

def test_fma_helper_is_correctly_rounded():
    rng = np.random.default_rng(8)
    a = (rng.standard_normal(2000) * 10.0 ** rng.integers(-8, 8, 2000)).astype(np.float32)
    b = (rng.standard_normal(2000) * 10.0 ** rng.integers(-8, 8, 2000)).astype(np.float32)
    c = (rng.standard_normal(2000) * 10.0 ** rng.integers(-8, 8, 2000)).astype(np.float32)
    got = cg.fma_f32(a, b, c)
    for k in range(a.size):
        exact = Fraction(float(a[k])) * Fraction(float(b[k])) + Fraction(float(c[k]))
        f = F32(float(exact))
        cands = [np.nextafter(f, F32(-np.inf)), f, np.nextafter(f, F32(np.inf))]
        best = min(cands, key=lambda q: (abs(Fraction(float(q)) - exact), int(_bits(q)) & 1))
        assert got[k] == best, (a[k], b[k], c[k])


def test_native_bins_truncate_after_fused_add():
    # value + 0.5 is rounded once to float32 (0.5 - 2**-25 + 0.5 ties to 1.0, 0.5 - 2**-24 + 0.5
    # is exact), then truncated; +inf saturates, NaN -> 0
    mn, scale = F32(0.0), F32(1.0)
    x = np.array([0.5 - 2**-24, 0.5 - 2**-25, 0.5, 1.4999999, 254.5, 300.0, np.inf, np.nan], np.float32)
    np.testing.assert_array_equal(cg.native_bins(x, mn, scale, 256), [0, 1, 1, 1, 255, 255, 255, 0])


# ---- 5. closed forms ----------------------------------------------------------------------------

def test_codebook_closed_forms():
    rng = np.random.default_rng(6)
    for _ in range(200):
        a, b = np.sort(rng.standard_normal(2).astype(np.float32))
        np.testing.assert_array_equal(_bits(cg.codebook(a, b, 2)), _bits([a, b]))
    np.testing.assert_array_equal(cg.codebook(F32(0), F32(255), 256), np.arange(256, dtype=np.float32))
    np.testing.assert_array_equal(cg.codebook(F32(-8), F32(8), 17), np.arange(-8, 9, dtype=np.float32))
    assert np.all(cg.codebook(F32(-0.0), F32(-0.0), 5) == 0)


def test_encode_error_bound_and_monotone_bins():
    rng = np.random.default_rng(12)
    x = rng.standard_normal(50000).astype(np.float32)
    for nb in (2, 16, 256):
        enc, book, cdf = cg.encode(x, nb)
        lo, hi = float(x.min()), float(x.max())
        bound = (hi - lo) / (nb - 1) / 2 + 8 * float(np.finfo(np.float32).eps) * max(abs(lo), abs(hi))
        assert np.max(np.abs(cg.decode(enc, book) - x)) <= bound
        order = np.argsort(x, kind="stable")
        assert np.all(np.diff(enc[order].astype(np.int64)) >= 0)
        np.testing.assert_array_equal(np.round(cdf[1:] * x.size).astype(np.int64),
                                      np.cumsum(np.bincount(enc, minlength=nb)))
