"""LMCache buffer format descriptors (interface of the reference's ops/lmcache_format.py:12-139).

``describe_lmcache_format`` classifies an LMCache memory tensor as
``KV_2LTD`` ``[2, NL, T, H]``, ``KV_T2D`` ``[T, 2, H]`` or ``KV_2TD``
``[2, T, H]``; ``describe_sglang_split_list`` describes SGLang-MP
``[K_layers, V_layers]`` lists of ``[NB, BS, NH, HS]`` tensors.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Sequence

import torch

from .kv_layout import KVLayoutKind, KVLayoutSpec, KVOrganization


class LMCacheFormat(str, Enum):
    KV_2LTD = "kv_2ltd"
    KV_T2D = "kv_t2d"
    KV_2TD = "kv_2td"
    SGLANG_SPLIT_LIST = "sglang_split_list"


@dataclass(frozen=True)
class LMCacheFormatFacts:
    format: LMCacheFormat
    spec: KVLayoutSpec


_SUPPORTED = (torch.float32, torch.float16, torch.bfloat16, torch.uint8)


def _dtype_name(tensor: torch.Tensor) -> str:
    """The dtype's short name; raises for dtypes LMCache buffers do not use."""
    if tensor.dtype not in _SUPPORTED:
        raise ValueError(f"unsupported LMCache dtype={tensor.dtype}")
    return str(tensor.dtype).removeprefix("torch.")


def _linear(tensor: torch.Tensor, kind: KVLayoutKind, organization: KVOrganization, layers: int, tokens: int,
            hidden: int) -> KVLayoutSpec:
    return KVLayoutSpec.linear(num_layers=layers, num_tokens=tokens, num_heads=1, head_size=hidden,
                               dtype_name=_dtype_name(tensor), organization=organization, kind=kind,
                               device_kind=tensor.device.type)


def describe_lmcache_format(memory_tensor: torch.Tensor) -> LMCacheFormatFacts:
    if not isinstance(memory_tensor, torch.Tensor) or not memory_tensor.is_contiguous():
        raise ValueError("LMCache memory tensor must be contiguous")
    shape = tuple(int(x) for x in memory_tensor.shape)
    if len(shape) == 4:
        if shape[0] != 2:
            raise ValueError("KV_2LTD memory tensor must have leading K/V dimension 2")
        _dtype_name(memory_tensor)  # a bad dtype is reported before the layout is built
        _, layers, tokens, hidden = shape
        spec = _linear(memory_tensor, KVLayoutKind.KV_2LTD, KVOrganization.SEPARATE, layers, tokens, hidden)
        return LMCacheFormatFacts(LMCacheFormat.KV_2LTD, spec)
    if len(shape) != 3:
        raise ValueError("LMCache memory tensor rank must be 3 or 4")
    _dtype_name(memory_tensor)  # a bad dtype is reported before the 3-D shape errors
    first, second, hidden = shape
    if first == 2 and second == 2:
        raise ValueError("3-D LMCache tensor is ambiguous when both leading dimensions are 2")
    if second == 2:
        spec = _linear(memory_tensor, KVLayoutKind.KV_T2D, KVOrganization.MERGED, 1, first, hidden)
        return LMCacheFormatFacts(LMCacheFormat.KV_T2D, spec)
    if first == 2:
        spec = _linear(memory_tensor, KVLayoutKind.KV_2TD, KVOrganization.SEPARATE, 1, second, hidden)
        return LMCacheFormatFacts(LMCacheFormat.KV_2TD, spec)
    raise ValueError("3-D LMCache memory tensor must be [T, 2, H] or [2, T, H]")


def describe_sglang_split_list(kvcaches: Sequence[Sequence[torch.Tensor]]) -> LMCacheFormatFacts:
    if len(kvcaches) != 2:
        raise ValueError("SGLang split-list must contain K and V layer lists")
    if not kvcaches[0] or not kvcaches[1]:
        raise ValueError("SGLang split-list must be non-empty")
    if len(kvcaches[0]) != len(kvcaches[1]):
        raise ValueError("SGLang K/V layer lists must have the same length")
    first = kvcaches[0][0]
    if not isinstance(first, torch.Tensor) or first.dim() != 4:
        raise ValueError("SGLang split-list entries must be [NB, BS, NH, HS] tensors")
    dtype_name = _dtype_name(first)
    for axis in kvcaches:
        for tensor in axis:
            if not isinstance(tensor, torch.Tensor) or tensor.shape != first.shape:
                raise ValueError("all SGLang split-list entries must share one shape")
            if tensor.dtype != first.dtype:
                raise ValueError("all SGLang split-list entries must share one dtype")
    nb, block_size, num_heads, head_size = (int(x) for x in first.shape)
    row_bytes = num_heads * head_size * first.element_size()
    spec = KVLayoutSpec(
        kind=KVLayoutKind.TWO_X_NL,
        num_layers=len(kvcaches[0]),
        num_blocks=nb,
        block_size=block_size,
        num_heads=num_heads,
        head_size=head_size,
        row_bytes=row_bytes,
        block_stride_bytes=block_size * row_bytes,
        dtype_name=dtype_name,
        organization=KVOrganization.SPLIT_LIST,
        is_contiguous=False,
        pointer_table_length=2 * len(kvcaches[0]),
        device_kind=first.device.type,
    )
    return LMCacheFormatFacts(LMCacheFormat.SGLANG_SPLIT_LIST, spec)
