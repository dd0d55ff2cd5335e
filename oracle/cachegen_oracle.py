"""numpy restatement of the reference's CacheGen-style KV codec -- TEST INFRASTRUCTURE ONLY.

Follows musa_aiter 0.5.0 ``musa_aiter/ops/kv_transfer.py``:

- ``kv_cachegen_encode`` (:1111-1172): uint8 uniform bins over [min, max] of the
  tensor (in float32), a ``torch.linspace`` dequant codebook and the empirical
  CDF of the bins;
- ``kv_cachegen_decode`` (:1175-1215): ``codebook[encoded]``, optionally cast;
- the gated native variant (:1048-1108 with ``kv_transfer_float.mu:828-898``),
  which differs from the torch path only in how the bin is rounded.

Every float32 step is written out so that the rounding of each operation is the
one torch (CPU) or the reference kernel performs.  Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg use this module.

How each part is pinned (tests/test_oracle_cachegen.py):

- torch-path bins: against torch evaluating the reference's own expression on
  the CPU, including inputs built so that a true division in place of torch's
  reciprocal-times-integer scale, or rounding half away from zero, changes a bin;
- codebook: against ``torch.linspace`` on the CPU over random ranges and sizes,
  and closed forms (two bins give [min, max]; integer ranges give integers);
- CDF: against torch's ``cumsum`` / division on the CPU, including counts past
  2**24 where float32 accumulation would differ, and the exact quotient;
- the reference's own test scenarios (op_tests/test_kv_transfer.py:218-250).

Parity unpinned: the native variant's rounding step.  The reference kernel
computes ``value = (x - min) * scale`` and then ``(int64)(value + 0.5f)``; built
with the CUDA-language default (floating-point contraction on), the multiply and
add become one fused multiply-add, which is what ``native_bins`` restates.  No
output of the compiled reference kernel is available to confirm it.  Inputs
holding NaN are also unpinned: the torch path's behaviour there depends on the
device (a NaN cast to int64), and this restatement gives such elements bin 0.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def to_f32(values: np.ndarray, dtype: str) -> np.ndarray:
    """``tensor.float()`` (kv_transfer.py:1124): bf16 (given as uint16 bits) and fp16 widen
    exactly, float64 rounds to nearest even, float32 is kept."""
    if dtype == "bfloat16":
        return (values.astype(np.uint32) << 16).view(np.float32)
    return np.asarray(values).astype(np.float32)


def _round_once_f32(hi: np.ndarray, lo: np.ndarray) -> np.ndarray:
    """float32 nearest-even rounding of the exact sum ``hi + lo`` (both float64, ``hi`` the
    rounded sum and ``lo`` its exact error), via round-to-odd in double: when the sum is not
    exact, an even ``hi`` moves one ulp toward the true value, so the single rounding to float32
    that follows is correct (double keeps more than 24 + 2 bits)."""
    hi = np.asarray(hi, dtype=np.float64)
    lo = np.asarray(lo, dtype=np.float64)
    bits = hi.view(np.uint64)
    inexact = (lo != 0) & ((bits & np.uint64(1)) == 0) & np.isfinite(hi)
    toward = np.where(lo > 0, np.inf, -np.inf)
    adj = np.where(inexact, np.nextafter(hi, toward), hi)
    with np.errstate(over="ignore"):
        return adj.astype(np.float32)


def fma_f32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """float32 fused multiply-add ``RN(a * b + c)`` for float32 operands whose product is exact
    in double (true for any two float32 values)."""
    p = np.asarray(a, np.float64) * np.asarray(b, np.float64)
    c = np.asarray(c, np.float64)
    with np.errstate(invalid="ignore"):
        s = p + c
        bb = s - p
        err = (p - (s - bb)) + (c - bb)  # TwoSum: s + err == p + c exactly
    err = np.where(np.isfinite(s), err, 0.0)
    return _round_once_f32(s, err)


def minmax(x: np.ndarray) -> tuple[np.float32, np.float32]:
    """``work.min()`` / ``work.max()`` (kv_transfer.py:1129-1130): NaN propagates."""
    return F32(np.min(x)), F32(np.max(x))


def torch_scale(mn: np.float32, mx: np.float32, num_bins: int) -> np.float32:
    """``(num_bins - 1) / (max_val - min_val)`` on float32 0-d tensors (kv_transfer.py:1155).
    torch evaluates ``int / tensor`` as ``tensor.reciprocal() * int``."""
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        d = F32(mx - mn)
        r = F32(F32(1.0) / d)
        return F32(r * F32(num_bins - 1))


def native_scale(mn: np.float32, mx: np.float32, num_bins: int) -> np.float32:
    """``float((num_bins - 1) / (max_item - min_item))`` in Python doubles, passed as a C float
    (kv_transfer.py:1058-1060)."""
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        return F32(np.float64(num_bins - 1) / (np.float64(mx) - np.float64(mn)))


def torch_bins(x: np.ndarray, mn: np.float32, scale: np.float32, num_bins: int) -> np.ndarray:
    """``torch.round((work - min_val) * scale).clamp_(0, num_bins - 1)`` (kv_transfer.py:1156):
    two float32 operations, round half to even, clamp; NaN gives bin 0."""
    with np.errstate(over="ignore", invalid="ignore"):
        v = (x.astype(np.float32) - F32(mn)).astype(np.float32) * F32(scale)
        r = np.rint(v.astype(np.float32))
        out = np.where(r >= num_bins - 1, num_bins - 1, np.where(r > 0, r, 0))
    return np.nan_to_num(out, nan=0).astype(np.uint8)


def native_bins(x: np.ndarray, mn: np.float32, scale: np.float32, num_bins: int) -> np.ndarray:
    """Bins of the reference kernel (kv_transfer_float.mu:828-848): ``t = x - min`` in float32,
    ``value + 0.5f`` fused with the multiply by ``scale``, truncation toward zero, clamp to
    [0, num_bins - 1]; NaN gives bin 0 and +inf saturates."""
    with np.errstate(over="ignore", invalid="ignore"):
        t = (x.astype(np.float32) - F32(mn)).astype(np.float32)
        v = fma_f32(t, np.full_like(t, scale), np.full_like(t, 0.5))
        tr = np.trunc(v)
        out = np.where(v >= num_bins - 1, num_bins - 1, np.where(v > 0, tr, 0))
    return np.nan_to_num(out, nan=0).astype(np.uint8)


def linspace_f32(start: float, end: float, steps: int) -> np.ndarray:
    """``torch.linspace(start, end, steps, dtype=torch.float32)`` (used at kv_transfer.py:1146,
    :1158): ``step = (end - start) / (steps - 1)`` in float32; the first ``steps // 2`` values
    are ``start + step * i`` and the rest ``end - step * (steps - 1 - i)``, each one fused
    multiply-add."""
    s, e = F32(start), F32(end)
    with np.errstate(over="ignore", invalid="ignore"):
        step = F32(F32(e - s) / F32(steps - 1))
    i = np.arange(steps)
    half = steps // 2
    lo = fma_f32(np.full(steps, step, np.float32), i.astype(np.float32), np.full(steps, s, np.float32))
    hi = fma_f32(np.full(steps, -step, np.float32), (steps - 1 - i).astype(np.float32),
                 np.full(steps, e, np.float32))
    return np.where(i < half, lo, hi).astype(np.float32)


def codebook(mn: np.float32, mx: np.float32, num_bins: int) -> np.ndarray:
    """Dequant codebook: ``torch.full(min)`` for a constant tensor (kv_transfer.py:1133), else
    ``linspace(min, max, num_bins)`` (:1146, :1158)."""
    if mx == mn:
        return np.full(num_bins, mn, dtype=np.float32)
    return linspace_f32(float(mn), float(mx), num_bins)


def histogram(bins: np.ndarray, num_bins: int) -> np.ndarray:
    """``torch.bincount(encoded, minlength=num_bins)`` (kv_transfer.py:1147, :1159)."""
    return np.bincount(bins.reshape(-1).astype(np.int64), minlength=num_bins).astype(np.int64)


def cdf(counts: np.ndarray, numel: int) -> np.ndarray:
    """``cdf[0] = 0; cdf[1:] = torch.cumsum(counts, 0) / float(numel)`` with float32 ``counts``
    (kv_transfer.py:1147-1151, :1159-1162), as torch computes it on the CPU: each count rounded
    to float32, the running sum accumulated in double and rounded to float32, then a float32
    division by ``numel`` rounded to float32."""
    c32 = counts.astype(np.float32).astype(np.float64)
    prefix = np.cumsum(c32).astype(np.float32)
    out = np.empty(counts.size + 1, dtype=np.float32)
    out[0] = 0.0
    out[1:] = prefix / F32(numel)
    return out


def encode(x: np.ndarray, num_bins: int = 256, *, native: bool = False, dtype: str = "float32"
           ) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``kv_cachegen_encode`` (kv_transfer.py:1111-1172): returns (encoded uint8 with the input's
    shape, codebook float32[num_bins], cdf float32[num_bins + 1]).  ``native`` selects the
    gated native kernel's rounding, which the reference uses for float32 input only."""
    if num_bins < 2 or num_bins > 256:
        raise ValueError("kv_cachegen_encode: num_bins must be in [2, 256]")
    work = to_f32(np.asarray(x), dtype)
    if work.size == 0:
        return (np.empty(work.shape, np.uint8), np.zeros(num_bins, np.float32),
                np.zeros(num_bins + 1, np.float32))
    mn, mx = minmax(work)
    if mx == mn:
        enc = np.zeros(work.shape, np.uint8)
        c = np.zeros(num_bins + 1, np.float32)
        c[1:] = 1.0
        return enc, np.full(num_bins, mn, np.float32), c
    if native and dtype == "float32":
        enc = native_bins(work, mn, native_scale(mn, mx, num_bins), num_bins)
    else:
        enc = torch_bins(work, mn, torch_scale(mn, mx, num_bins), num_bins)
    return enc, codebook(mn, mx, num_bins), cdf(histogram(enc, num_bins), work.size)


def decode(encoded: np.ndarray, table: np.ndarray) -> np.ndarray:
    """``codebook[encoded.long()]`` (kv_transfer.py:1214); a cast to ``dtype`` applies to each
    value, so casting the table first gives the same result."""
    if encoded.size and int(encoded.max()) >= table.size:
        raise ValueError("kv_cachegen_decode: encoded bin exceeds codebook size")
    return table[encoded.astype(np.int64)]
