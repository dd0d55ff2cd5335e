"""Fallback policy (same environment contract as the reference's policy.py:7-44).

``MUSA_AITER_FALLBACK_POLICY`` accepts ``allow`` (default), ``warn`` and
``require-native`` (aliases ``1``, ``native``, ``require_native``).  This
package ships no reference fallback: every KV op runs the HIP kernels or
raises, so ``ensure_reference_allowed`` only matters for callers that ask
whether a fallback *would* be permitted.
"""

from __future__ import annotations

import os
import warnings
from enum import Enum


class FallbackPolicy(str, Enum):
    ALLOW = "allow"
    WARN = "warn"
    REQUIRE_NATIVE = "require-native"


_ALIASES = {"1": "require-native", "0": "allow", "require_native": "require-native", "native": "require-native"}


def current_policy() -> FallbackPolicy:
    raw = os.environ.get("MUSA_AITER_FALLBACK_POLICY", "allow").strip().lower()
    raw = _ALIASES.get(raw, raw)
    try:
        return FallbackPolicy(raw)
    except ValueError:
        return FallbackPolicy.ALLOW


def ensure_reference_allowed(op: str, native_available: bool = False) -> None:
    if native_available:
        return
    policy = current_policy()
    if policy == FallbackPolicy.REQUIRE_NATIVE:
        raise RuntimeError(
            f"{op}: native backend required by MUSA_AITER_FALLBACK_POLICY=require-native, "
            "but no native backend is available in this environment."
        )
    if policy == FallbackPolicy.WARN:
        warnings.warn(f"{op}: using reference fallback because native backend is unavailable.", RuntimeWarning,
                      stacklevel=2)
