"""torch restatements of the reference's FP8 steps and paged-row indexing -- checkers, not product code.

``bench.py`` checks its timed kernels' results with these (the numpy oracle is
kept to the tests and the CPU-baseline leg), and tests/test_oracle_fp8.py pins
them against oracle/kv_oracle.py over every bf16 / fp16 bit pattern and every
FP8 code.  Run them on CPU tensors: the pinning covers torch's CPU ``log2``.
"""

from __future__ import annotations

import torch

# (exponent bits, mantissa bits, bias, max unbiased exponent) -- reference kv_transfer.py:2103-2107
FP8_FORMATS = {"e4m3": (4, 3, 7, 8), "e5m2": (5, 2, 15, 16)}


def fp8_quantize(x: torch.Tensor, scale: torch.Tensor, fmt: str) -> torch.Tensor:
    """The reference encoder's steps (kv_transfer.py:2161-2183) written with torch ops: uint8 codes."""
    _, mant, bias, emax = FP8_FORMATS[fmt]
    work = x.to(torch.float32) / scale
    sign = work < 0
    a = work.abs()
    a = torch.where(torch.isfinite(a), a, torch.zeros_like(a))
    clipped = a.clamp(max=(2.0 - 2.0 ** (-mant)) * (2.0 ** emax))
    nonzero = clipped >= 2.0 ** (1 - bias)
    safe = torch.where(nonzero, clipped, torch.ones_like(clipped))
    e = torch.floor(torch.log2(safe)).to(torch.int32).clamp(min=1 - bias, max=emax)
    base = torch.pow(torch.tensor(2.0, dtype=torch.float32), e.to(torch.float32))
    m = torch.round((safe / base - 1.0) * (2 ** mant)).to(torch.int32)
    ovf = m == 2 ** mant
    e = torch.where(ovf, e + 1, e).clamp(max=emax)
    m = torch.where(ovf, torch.zeros_like(m), m).clamp(min=0, max=2 ** mant - 1)
    ef = torch.where(nonzero, e + bias, torch.zeros_like(e))
    m = torch.where(nonzero, m, torch.zeros_like(m))
    return ((sign.to(torch.int32) << 7) | (ef << mant) | m).to(torch.uint8)


def fp8_decode_table(fmt: str) -> torch.Tensor:
    """float32 value of every code under the reference decoder (kv_transfer.py:2186-2200): [256]."""
    _, mant, bias, _ = FP8_FORMATS[fmt]
    codes = torch.arange(256, dtype=torch.int32)
    ef = (codes >> mant) & ((1 << (7 - mant)) - 1)
    m = (codes & ((1 << mant) - 1)).to(torch.float32)
    value = (1.0 + m / (2 ** mant)) * torch.pow(torch.tensor(2.0), (ef - bias).to(torch.float32))
    value = torch.where(ef != 0, value, torch.zeros_like(value))
    return torch.where((codes >> 7) == 1, -value, value)


def fp8_dequantize(codes: torch.Tensor, scale: torch.Tensor, fmt: str, out_dtype: torch.dtype) -> torch.Tensor:
    """``decode(code) * scale`` in float32, rounded to ``out_dtype`` (the reference's dequantize path)."""
    table = fp8_decode_table(fmt).to(codes.device)
    return (table[codes.to(torch.int64)] * scale.to(torch.float32)).to(out_dtype)


def paged_rows(cache: torch.Tensor) -> torch.Tensor:
    """Paged cache [NB, NH, HD, BS] as slot-major rows [NB * BS, NH, HD] (slot = block * BS + offset)."""
    nb, nh, hd, bs = cache.shape
    return cache.permute(0, 3, 1, 2).reshape(nb * bs, nh, hd)
