"""Native-gate helpers (environment contract of the reference's ops/native_gate.py:19-55).

The reference runs its MUSA kernels only when a gate variable such as
``MUSA_AITER_NATIVE_KV_TRANSFER=1`` is set.  On ROCm the HIP backend is the
only backend of this package, so the gates are informational: a set gate is
reported as requested, an unset gate does not disable the kernels.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Iterable


@dataclass(frozen=True)
class NativeGateDecision:
    operation: str
    requested: bool
    available: bool
    mode: str
    reason: str


def native_requested(*env_names: str) -> bool:
    """True when any of the given gate variables is exactly ``"1"``."""
    return any(os.environ.get(name, "0") == "1" for name in env_names)


def decide_native_gate(operation: str, env_names: Iterable[str], *, available: bool,
                       native_required: bool = False) -> NativeGateDecision:
    requested = native_requested(*tuple(env_names))
    if not requested:
        return NativeGateDecision(operation, False, available, "reference", "native_gate_off")
    if available:
        return NativeGateDecision(operation, True, True, "native", "native_available")
    return NativeGateDecision(operation, True, False, "error" if native_required else "fallback",
                              "native_unavailable")


__all__ = ["NativeGateDecision", "decide_native_gate", "native_requested"]
