"""Dispatch trace records (mirrors the reference's musa_aiter/dispatch.py:10-36).

When ``MUSA_AITER_TRACE_DISPATCH`` is truthy every hot-path call prints one
``[MUSA_AITER DISPATCH] op=... backend=... device=... dtype=... reason=...``
line to stderr, in the reference's format, so existing log scrapers keep
working.  The backend label of this package is ``rocm-hip``.
"""

from __future__ import annotations

import os
import sys
from dataclasses import dataclass
from typing import Any

_TRUTHY = {"1", "true", "TRUE", "yes", "YES"}


@dataclass(frozen=True)
class DispatchRecord:
    op: str
    backend: str
    device: str
    dtype: str
    reason: str


def trace_enabled() -> bool:
    return os.environ.get("MUSA_AITER_TRACE_DISPATCH", "0") in _TRUTHY


def emit(record: DispatchRecord) -> None:
    if not trace_enabled():
        return
    sys.stderr.write(
        f"[MUSA_AITER DISPATCH] op={record.op} backend={record.backend} device={record.device} "
        f"dtype={record.dtype} reason={record.reason}\n"
    )


def tensor_device_dtype(x: Any) -> tuple[str, str]:
    return str(getattr(x, "device", "unknown")), str(getattr(x, "dtype", "unknown"))
