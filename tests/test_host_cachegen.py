"""Host-side contract of the CacheGen codec, no GPU needed.

Follows musa_aiter/ops/kv_transfer.py:1111-1215: validation messages and order (before any
device check), empty tensors answered without a launch, CPU tensors rejected instead of computed,
the native-rounding gate (float32 input and MUSA_AITER_NATIVE_KV_TRANSFER=1 only), and the
reference's invalid-input test (op_tests/test_kv_transfer.py:241-250).
"""

from __future__ import annotations

import pytest
import torch

import musa_aiter
from musa_aiter.ops import kv_transfer


def test_reference_invalid_inputs():
    with pytest.raises(ValueError, match="tensor must use a floating dtype"):
        musa_aiter.kv_cachegen_encode(torch.arange(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="encoded must be uint8"):
        musa_aiter.kv_cachegen_decode(torch.zeros(2, dtype=torch.int32), torch.zeros(4))


@pytest.mark.parametrize("bins", [-1, 0, 1, 257, 1000])
def test_num_bins_range_checked_first(bins):
    with pytest.raises(ValueError, match=r"num_bins must be in \[2, 256\]"):
        musa_aiter.kv_cachegen_encode(torch.arange(4, dtype=torch.int32), num_bins=bins)


def test_decode_validation_order_and_messages():
    codes = torch.zeros(3, dtype=torch.uint8)
    with pytest.raises(ValueError, match="1-D with 2..256 bins"):
        musa_aiter.kv_cachegen_decode(codes, torch.zeros(2, 2))
    with pytest.raises(ValueError, match="1-D with 2..256 bins"):
        musa_aiter.kv_cachegen_decode(codes, torch.zeros(257))
    with pytest.raises(ValueError, match="1-D with 2..256 bins"):
        musa_aiter.kv_cachegen_decode(codes, torch.zeros(1))
    with pytest.raises(ValueError, match="floating dtype"):
        musa_aiter.kv_cachegen_decode(codes, torch.zeros(4, dtype=torch.int64))


def test_empty_tensors_need_no_device():
    enc, book, cdf = musa_aiter.kv_cachegen_encode(torch.zeros(0, 4, dtype=torch.float16), num_bins=9)
    assert enc.shape == (0, 4) and enc.dtype == torch.uint8
    assert book.dtype == torch.float32 and book.shape == (9,) and not bool(book.any())
    assert cdf.dtype == torch.float32 and cdf.shape == (10,) and not bool(cdf.any())
    out = musa_aiter.kv_cachegen_decode(torch.zeros(2, 0, dtype=torch.uint8), torch.zeros(4, dtype=torch.float64),
                                        dtype=torch.float16)
    assert out.shape == (2, 0) and out.dtype == torch.float16


def test_cpu_tensors_are_rejected_not_computed():
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        musa_aiter.kv_cachegen_encode(torch.randn(16))
    with pytest.raises(RuntimeError, match="ROCm GPU device"):
        musa_aiter.kv_cachegen_decode(torch.zeros(16, dtype=torch.uint8), torch.randn(4))


def test_native_rounding_gate(monkeypatch):
    monkeypatch.delenv("MUSA_AITER_NATIVE_KV_TRANSFER", raising=False)
    assert not kv_transfer._cachegen_native_rounding(torch.zeros(1))
    monkeypatch.setenv("MUSA_AITER_NATIVE_KV_TRANSFER", "1")
    assert kv_transfer._cachegen_native_rounding(torch.zeros(1))
    for dtype in (torch.float16, torch.bfloat16, torch.float64):
        assert not kv_transfer._cachegen_native_rounding(torch.zeros(1, dtype=dtype))
    monkeypatch.setenv("MUSA_AITER_NATIVE_KV_TRANSFER", "0")
    assert not kv_transfer._cachegen_native_rounding(torch.zeros(1))
