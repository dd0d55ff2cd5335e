"""CPU stand-in for the ``_hip.copy_rows_paged`` launch -- host-logic tests only.

It applies the documented contract of ``musa_aiter_hip_copy_rows_paged`` to CPU tensors, so
the host layer's plane addresses, strides, page addressing and token tables can be checked on
a machine without a GPU.  Every address the host passes is mapped back to one of the tensors
registered with the emulator and bounds-checked (an address outside them fails the test), and
rows move through numpy byte views, never through raw pointers.
"""

from __future__ import annotations

import numpy as np
import torch


class RowCopyEmulator:
    def __init__(self, *tensors: torch.Tensor):
        self._buffers = []
        for t in tensors:
            assert t.device.type == "cpu" and t.is_contiguous()
            flat = t.reshape(-1).view(torch.uint8).numpy()
            self._buffers.append((t.data_ptr(), flat.shape[0], flat))
        self.launches = 0

    def _locate(self, addr: int, nbytes: int) -> tuple[np.ndarray, int]:
        for base, size, flat in self._buffers:
            if base <= addr and addr + nbytes <= base + size:
                return flat, addr - base
        raise AssertionError(f"row [{addr:#x}, +{nbytes}) lies outside every registered tensor")

    @staticmethod
    def _offset(r: int, page_rows: int, page_stride: int, stride: int) -> int:
        if page_rows <= 0:
            return r * stride
        return (r // page_rows) * page_stride + (r % page_rows) * stride

    def __call__(self, *, op, device, src_planes, dst_planes, src_idx, dst_idx, src_rows, dst_rows, row_bytes,
                 src_stride, dst_stride, src_page_rows=0, src_page_stride=0, dst_page_rows=0, dst_page_stride=0,
                 dedupe=True):
        s = src_idx.cpu().numpy().astype(np.int64)
        d = dst_idx.cpu().numpy().astype(np.int64)
        assert s.shape == d.shape and len(src_planes) == len(dst_planes)
        if s.shape[0] == 0 or row_bytes <= 0:
            return
        self.launches += 1
        valid = (s >= 0) & (s < src_rows) & (d >= 0) & (d < dst_rows)
        tokens = np.flatnonzero(valid)
        if dedupe:
            last = {}
            for u in tokens:
                last[int(d[u])] = int(u)
            tokens = sorted(last.values())
        # All reads happen before the writes, as in one kernel launch over distinct rows.
        moves = []
        for sp, dp in zip(src_planes, dst_planes):
            for u in tokens:
                src_buf, so = self._locate(int(sp) + self._offset(int(s[u]), src_page_rows, src_page_stride,
                                                                  src_stride), row_bytes)
                dst_buf, do = self._locate(int(dp) + self._offset(int(d[u]), dst_page_rows, dst_page_stride,
                                                                  dst_stride), row_bytes)
                moves.append((dst_buf, do, src_buf[so:so + row_bytes].copy()))
        for dst_buf, do, row in moves:
            dst_buf[do:do + row_bytes] = row
