"""Operator capability registry (API of the reference's musa_aiter/registry.py:8-56).

Only the KV-cache movement family is registered: it is the path this package
implements.  Every row lists the single backend label ``rocm-hip`` (the gfx950
HIP kernels behind ``libmusa_aiter_kv_hip.so``), which is what
``python -m musa_aiter.cli list-ops --family kvcache`` prints.  Devices are
torch device types: ROCm tensors report ``cuda``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable


@dataclass(frozen=True)
class OperatorCapability:
    name: str
    family: str
    status: str
    dtypes: tuple[str, ...]
    devices: tuple[str, ...]
    backends: tuple[str, ...]
    description: str
    notes: tuple[str, ...] = field(default_factory=tuple)
    vendor_backends: tuple[str, ...] = field(default_factory=tuple)


_REGISTRY: dict[str, OperatorCapability] = {}

BACKEND = "rocm-hip"
DEVICES = ("cuda",)
VENDOR = ("handwritten-hip-gfx950",)


def register(capability: OperatorCapability) -> OperatorCapability:
    if capability.name in _REGISTRY:
        raise ValueError(f"duplicate operator capability: {capability.name}")
    _REGISTRY[capability.name] = capability
    return capability


def get(name: str) -> OperatorCapability:
    return _REGISTRY[name]


def list_capabilities(family: str | None = None) -> list[OperatorCapability]:
    values: Iterable[OperatorCapability] = _REGISTRY.values()
    if family is not None:
        values = [cap for cap in values if cap.family == family]
    return sorted(values, key=lambda cap: (cap.family, cap.name))


def as_dict() -> dict[str, dict]:
    return {
        name: {
            "name": cap.name,
            "family": cap.family,
            "status": cap.status,
            "dtypes": list(cap.dtypes),
            "devices": list(cap.devices),
            "backends": list(cap.backends),
            "description": cap.description,
            "notes": list(cap.notes),
            "vendor_backends": list(cap.vendor_backends),
        }
        for name, cap in sorted(_REGISTRY.items())
    }


_FLOAT = ("float32", "float16", "bfloat16")
_FP8_STORE = ("float16", "bfloat16", "float32", "uint8", "float8_e4m3fn", "float8_e5m2")
_FP8_LOAD = ("uint8", "float8_e4m3fn", "float8_e5m2", "float16", "bfloat16", "float32")


def _kv(name: str, status: str, dtypes: tuple[str, ...], description: str, notes: tuple[str, ...] = ()) -> None:
    register(OperatorCapability(name, "kvcache", status, dtypes, DEVICES, (BACKEND,), description, notes, VENDOR))


# Paged-A [NB, NH, HD, BS] <-> token-major linear.
_kv("kv_paged_to_linear", "hip-native", _FLOAT, "Paged KV -> token-major linear gather (single layer).")
_kv("kv_linear_to_paged", "hip-native", _FLOAT, "Token-major linear -> paged KV scatter (single layer).")
_kv("kv_paged_to_linear_multi_layer", "hip-native", _FLOAT, "Paged KV -> linear gather, stacked layers, one launch.")
_kv("kv_linear_to_paged_multi_layer", "hip-native", _FLOAT, "Linear -> paged KV scatter, stacked layers, one launch.")
_kv("kv_paged_to_merged_linear", "hip-native", _FLOAT, "Paged KV -> merged [T, 2, kv_heads, head_dim] gather.")
_kv("kv_merged_linear_to_paged", "hip-native", _FLOAT, "Merged [T, 2, kv_heads, head_dim] -> paged KV scatter.")
_kv("kv_paged_to_merged_linear_multi_layer", "hip-native", _FLOAT, "Paged KV -> merged [L, T, 2, H, D] gather.")
_kv("kv_merged_linear_to_paged_multi_layer", "hip-native", _FLOAT, "Merged [L, T, 2, H, D] -> paged KV scatter.")
# FP8 codec fused into the transfers.
_kv("kv_linear_to_paged_fp8", "hip-native", _FP8_STORE, "Linear KV -> paged FP8 cache quantize scatter (scalar or per-head scales).")
_kv("kv_paged_fp8_to_linear", "hip-native", _FP8_LOAD, "Paged FP8 cache -> linear dequantize gather (scalar or per-head scales).")
_kv("kv_linear_to_paged_fp8_multi_layer", "hip-native", _FP8_STORE, "Multi-layer FP8 quantize scatter (scalar, [H] or [L, H] scales).")
_kv("kv_paged_fp8_to_linear_multi_layer", "hip-native", _FP8_LOAD, "Multi-layer FP8 dequantize gather (scalar, [H] or [L, H] scales).")
_kv("kv_merged_linear_to_paged_fp8", "hip-native", _FP8_STORE, "Merged linear KV -> paged FP8 cache quantize scatter.")
_kv("kv_paged_fp8_to_merged_linear", "hip-native", _FP8_LOAD, "Paged FP8 cache -> merged linear dequantize gather.")
_kv("kv_merged_linear_to_paged_fp8_multi_layer", "hip-native", _FP8_STORE, "Merged multi-layer FP8 quantize scatter.")
_kv("kv_paged_fp8_to_merged_linear_multi_layer", "hip-native", _FP8_LOAD, "Merged multi-layer FP8 dequantize gather.")
# MLA / DSA flat caches.
_kv("kv_paged_to_mla_linear", "hip-native", _FLOAT, "MLA flat caches [NB, BS, D] -> token-major kv and rope rows.")
_kv("kv_mla_linear_to_paged", "hip-native", _FLOAT, "Token-major kv and rope rows -> MLA flat caches.")
_kv("kv_paged_to_mla_linear_multi_layer", "hip-native", _FLOAT, "Stacked MLA flat caches -> layer-major rows.")
_kv("kv_mla_linear_to_paged_multi_layer", "hip-native", _FLOAT, "Layer-major rows -> stacked MLA flat caches.")
# Dense preload for attention and whole-block copies.
_kv("kv_load_and_reshape_flash", "hip-native", _FLOAT,
    "Paged KV blocks -> dense Flash-style [batch, seq, kv_heads, head_dim] through block tables.")
_kv("kv_load_and_dequantize_fp8_flash", "hip-native", ("uint8", "float8_e4m3fn", "float8_e5m2"),
    "Paged FP8 blocks -> dense dequantized Flash-style tensors through block tables.")
_kv("kv_reshape_and_cache_back_flash", "hip-native", _FLOAT,
    "Dense Flash-style KV tensors -> paged KV blocks through block tables.")
_kv("kv_copy_paged_blocks", "hip-native", _FLOAT, "Copy selected paged KV blocks between same-layout caches.")
_kv("kv_copy_paged_blocks_fp8", "hip-native", ("uint8", "float8_e4m3fn", "float8_e5m2"),
    "Raw FP8 paged KV block copy between same-layout caches.")
_kv("kv_cachegen_encode", "hip-native", ("float32", "float16", "bfloat16", "float64"),
    "CacheGen-style uniform-bin uint8 KV encode with dequant codebook and empirical CDF, on device.")
_kv("kv_cachegen_decode", "hip-native", ("uint8",), "CacheGen-style uint8 codebook decode through an LDS table.")
# DSV4 opaque byte rows.
_kv("kv_copy_paged_rows", "hip-native", ("uint8",), "Opaque byte-row gather/scatter between row pools (per layer).")
_kv("kv_copy_paged_rows_layer_table", "hip-native", ("uint8",), "Opaque byte-row copy across a layer table, one launch.")
_kv("kv_copy_paged_rows_multi_pool", "hip-native", ("uint8",), "Opaque byte-row copy over several pools sharing one index set.")
# LMCache converters.
_kv("lmcache_kv_paged_to_buffer_two_x_nl", "hip-native", _FLOAT,
    "Gather SGLang MP 2 x NL x [NB, BS, NH, HS] split K/V caches into an LMCache [2, NL, T, NH*HS] buffer.")
_kv("lmcache_kv_buffer_to_paged_two_x_nl", "hip-native", _FLOAT,
    "Scatter an LMCache [2, NL, T, NH*HS] buffer into SGLang MP 2 x NL x [NB, BS, NH, HS] split K/V caches.")
_kv("lmcache_kv_paged_to_buffer", "hip-native", _FLOAT, "LMCache list / nested-list caches -> [2, NL, T, NH*HS] buffer.")
_kv("lmcache_kv_buffer_to_paged", "hip-native", _FLOAT, "LMCache buffer -> legacy 6-D, list or nested-list caches.")
_kv("lmcache_paged_to_kv_buffer", "hip-native", _FLOAT, "Legacy 6-D [NL, 2, NB, BS, NH, HS] cache -> LMCache buffer.")
_kv("lmcache_kv_buffer_to_paged_mla", "hip-native", _FLOAT, "LMCache MLA buffer [NL, T, D] -> [NL, NB, BS, D] cache.")
_kv("lmcache_paged_to_kv_buffer_mla", "hip-native", _FLOAT, "[NL, NB, BS, D] MLA cache -> LMCache MLA buffer.")
_kv("lmcache_mla_buffer_to_paged", "hip-native", _FLOAT, "LMCache [1, NL, T, D] buffer -> per-layer MLA list caches.")
_kv("lmcache_mla_paged_to_buffer", "hip-native", _FLOAT, "Per-layer MLA list caches -> LMCache [1, NL, T, D] buffer.")
_kv("lmcache_kv_strided_block_transfer", "hip-native", ("uint8",),
    "Block-granular byte copy between an LMCache staging object and padded per-layer pages (modes 0 and 1).")
_kv("lmcache_musa_memcpy_batch_async", "hip-native", ("uint8",),
    "Opt-in asynchronous host/device byte-copy batch for LMCache direct transfer: one batch-copy kernel launch "
    "over pinned host memory, or the DMA engines.")
# SGLang HiCache layer-first / page-first transfers (any element type: items are byte rows).
_HICACHE = ("float32", "float16", "bfloat16", "uint8")
_kv("hicache_transfer_kv_per_layer", "hip-native", _HICACHE,
    "SGLang HiCache per-layer layer-first transfer with two index tables.")
_kv("hicache_transfer_kv_per_layer_pf_lf", "hip-native", _HICACHE,
    "SGLang HiCache per-layer page-first -> layer-first transfer.")
_kv("hicache_transfer_kv_all_layer", "hip-native", _HICACHE, "SGLang HiCache all-layer layer-first transfer, one launch.")
_kv("hicache_transfer_kv_all_layer_lf_pf", "hip-native", _HICACHE,
    "SGLang HiCache all-layer layer-first -> page-first transfer, one launch.")
_kv("hicache_transfer_kv_per_layer_mla", "hip-native", _HICACHE, "SGLang HiCache per-layer MLA layer-first transfer.")
_kv("hicache_transfer_kv_per_layer_mla_pf_lf", "hip-native", _HICACHE,
    "SGLang HiCache per-layer MLA page-first -> layer-first transfer.")
_kv("hicache_transfer_kv_all_layer_mla", "hip-native", _HICACHE, "SGLang HiCache all-layer MLA layer-first transfer.")
_kv("hicache_transfer_kv_all_layer_mla_lf_pf", "hip-native", _HICACHE,
    "SGLang HiCache all-layer MLA layer-first -> page-first transfer.")
_kv("hicache_transfer_kv_direct", "hip-native", _HICACHE,
    "SGLang direct HiCache token-range copy over per-layer tensors, one launch.")
_kv("hicache_transfer_kv_per_layer_direct_pf_lf", "hip-native", _HICACHE,
    "SGLang direct HiCache page-first pages -> one layer-first layer.")
_kv("hicache_transfer_kv_all_layer_direct_lf_pf", "hip-native", _HICACHE,
    "SGLang direct HiCache layer-first rows -> all-layer page-first pages, one launch.")
