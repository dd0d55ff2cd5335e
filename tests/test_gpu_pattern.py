"""GPU check of the block-pattern copy that bench.py times as the access-pattern ceiling.

musa_aiter_hip_block_pattern_copy has no reference counterpart; these cases pin what it writes, so a
ceiling is a real copy of the bytes it claims: whole blocks in the given order (1:1), the XOR of a
source block's two halves into a half-size block (2:1, the FP8 quant-store's traffic) and one half
written twice (1:2, the dequant-gather's), block ids outside their regions skipped, with
non-temporal and with write-through stores alike.  Expected values are computed on the CPU with
numpy from the same inputs.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from musa_aiter.ops import _hip

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _copy(src, dst, src_blocks, dst_blocks, n, sreg, dreg, sbytes, dbytes, planes, sps, dps, wt):
    fn = getattr(_hip.library(), "musa_aiter_hip_block_pattern_copy")
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 8 + [ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    rc = fn(src.data_ptr(), dst.data_ptr(), None if src_blocks is None else src_blocks.data_ptr(),
            None if dst_blocks is None else dst_blocks.data_ptr(), n, sreg, dreg, sbytes, dbytes, planes, sps, dps,
            wt, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return rc


def _want(src_np, dst_np, sb, db, n, sreg, dreg, sbytes, dbytes, planes, sps, dps):
    """Byte-level restatement: block i of every plane, source block sb[i] -> destination block db[i]."""
    out = dst_np.copy()
    for p in range(planes):
        for i in range(n):
            s = i if sb is None else int(sb[i])
            d = i if db is None else int(db[i])
            if not (0 <= s < sreg and 0 <= d < dreg):
                continue
            blk = src_np[p * sps + s * sbytes: p * sps + (s + 1) * sbytes]
            if sbytes == dbytes:
                res = blk
            elif sbytes == 2 * dbytes:  # unit u (2 KiB) -> XOR of its two KiB halves
                u = blk.reshape(-1, 2, 1024)
                res = (u[:, 0] ^ u[:, 1]).reshape(-1)
            else:  # unit u (1 KiB) written to both halves of a 2 KiB destination unit
                u = blk.reshape(-1, 1, 1024)
                res = np.concatenate([u, u], axis=1).reshape(-1)
            out[p * dps + d * dbytes: p * dps + (d + 1) * dbytes] = res
    return out


@pytest.mark.parametrize("write_through", [0, 1])
@pytest.mark.parametrize("ratio", ["1:1", "2:1", "1:2"])
def test_block_pattern_copy_writes_the_blocks_it_times(ratio, write_through):
    rng = np.random.default_rng(61)
    planes, n = 3, 37
    sbytes, dbytes = {"1:1": (4096, 4096), "2:1": (8192, 4096), "1:2": (4096, 8192)}[ratio]
    sreg, dreg = 50, 45
    sps, dps = sreg * sbytes + 1024, dreg * dbytes + 2048
    src_np = rng.integers(0, 256, size=planes * sps, dtype=np.uint8)
    dst_np = rng.integers(0, 256, size=planes * dps, dtype=np.uint8)
    sb = rng.permutation(sreg)[:n].astype(np.int32)
    sb[[3, 11]] = [-1, sreg + 2]                      # skipped: outside the source region
    db = rng.permutation(dreg)[:n].astype(np.int32) if n <= dreg else None
    db[20] = dreg                                      # skipped: outside the destination region
    src = torch.from_numpy(src_np).to(DEV)
    dst = torch.from_numpy(dst_np).to(DEV)
    assert _copy(src, dst, torch.from_numpy(sb).to(DEV), torch.from_numpy(db).to(DEV), n, sreg, dreg, sbytes, dbytes,
                 planes, sps, dps, write_through) == 0
    want = _want(src_np, dst_np, sb, db, n, sreg, dreg, sbytes, dbytes, planes, sps, dps)
    assert np.array_equal(dst.cpu().numpy(), want)


def test_block_pattern_copy_in_order_and_rejects_bad_sizes():
    rng = np.random.default_rng(62)
    n, bytes_ = 9, 2048
    src_np = rng.integers(0, 256, size=n * bytes_, dtype=np.uint8)
    src = torch.from_numpy(src_np).to(DEV)
    dst = torch.zeros(n * bytes_, dtype=torch.uint8, device=DEV)
    assert _copy(src, dst, None, None, n, n, n, bytes_, bytes_, 1, 0, 0, 1) == 0
    assert np.array_equal(dst.cpu().numpy(), src_np)
    # block sizes must be whole KiB in a 1:1, 2:1 or 1:2 ratio
    assert _copy(src, dst, None, None, n, n, n, 1536, 1536, 1, 0, 0, 0) != 0
    assert _copy(src, dst, None, None, n, n, n, 3072, 1024, 1, 0, 0, 0) != 0
