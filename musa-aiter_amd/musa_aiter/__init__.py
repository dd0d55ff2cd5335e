"""MI355X-native KV-cache movement with the public KV API of musa_aiter 0.5.0.

Importing this package gives the reference's KV transfer names (paged <->
linear, merged, FP8 quant-store / dequant-gather, MLA flat rows, DSV4 byte
rows, LMCache / SGLang-MP converters, LMCache host <-> device copy batches,
SGLang HiCache transfers, layout descriptors) backed by hand-written gfx950 HIP
kernels in ``_lib/libmusa_aiter_kv_hip.so``.
"""

from musa_aiter.version import __version__, REFERENCE_API_VERSION
from musa_aiter.dispatch import DispatchRecord, emit, tensor_device_dtype
from musa_aiter.policy import FallbackPolicy, current_policy, ensure_reference_allowed
from musa_aiter import registry
from musa_aiter.ops.native_gate import NativeGateDecision, decide_native_gate, native_requested
from musa_aiter.ops.kv_layout import (
    KVFormatFacts,
    KVLayoutKind,
    KVLayoutSpec,
    KVOrganization,
    KVScaleKind,
)
from musa_aiter.ops.lmcache_format import (
    LMCacheFormat,
    LMCacheFormatFacts,
    describe_lmcache_format,
    describe_sglang_split_list,
)
from musa_aiter.ops.kv_transfer_plan import (
    KVTransferEntry,
    KVTransferPlan,
    assess_direct_eligibility,
    validate_transfer_plan,
)
from musa_aiter.ops.kv_backend import (
    KVBackend,
    KVBackendCapabilities,
    KVBackendDecision,
    hip_capabilities,
    select_kv_backend,
)
from musa_aiter.ops.kv_transfer import (
    BuildResult,
    InterleavedFp8Layout,
    PoolSpec,
    build_native_fp8_kv_cache,
    build_native_kv_transfer,
    clear_dsv4_ptr_table_cache,
    is_native_fp8_kv_cache_available,
    is_native_fp8_kv_vectorized_available,
    is_native_kv_transfer_available,
    kv_cachegen_decode,
    kv_cachegen_encode,
    kv_copy_paged_blocks,
    kv_copy_paged_blocks_fp8,
    kv_copy_paged_rows,
    kv_copy_paged_rows_layer_table,
    kv_copy_paged_rows_multi_pool,
    kv_linear_to_paged,
    kv_load_and_dequantize_fp8_flash,
    kv_load_and_reshape_flash,
    kv_linear_to_paged_fp8,
    kv_linear_to_paged_fp8_multi_layer,
    kv_linear_to_paged_multi_layer,
    kv_merged_linear_to_paged,
    kv_merged_linear_to_paged_fp8,
    kv_merged_linear_to_paged_fp8_multi_layer,
    kv_merged_linear_to_paged_multi_layer,
    kv_mla_linear_to_paged,
    kv_mla_linear_to_paged_multi_layer,
    kv_paged_fp8_to_linear,
    kv_paged_fp8_to_linear_multi_layer,
    kv_paged_fp8_to_merged_linear,
    kv_paged_fp8_to_merged_linear_multi_layer,
    kv_paged_to_linear,
    kv_paged_to_linear_multi_layer,
    kv_paged_to_merged_linear,
    kv_paged_to_merged_linear_multi_layer,
    kv_paged_to_mla_linear,
    kv_paged_to_mla_linear_multi_layer,
    kv_reshape_and_cache_back_flash,
    kv_transfer_stats,
    kv_triton_indexed_to_dense,
    native_fp8_kv_cache_abi_version,
    native_kv_transfer_abi_version,
    reset_kv_transfer_stats,
)
from musa_aiter.ops.lmcache_kv_transfer import (
    clear_native_lmcache_kv_transfer_cache,
    is_native_lmcache_kv_transfer_available,
    is_native_lmcache_two_x_nl_kv_transfer_available,
    lmcache_kv_buffer_to_paged,
    lmcache_kv_buffer_to_paged_mla,
    lmcache_kv_buffer_to_paged_two_x_nl,
    lmcache_kv_paged_to_buffer,
    lmcache_kv_paged_to_buffer_two_x_nl,
    lmcache_kv_strided_block_transfer,
    lmcache_mla_buffer_to_paged,
    lmcache_mla_paged_to_buffer,
    lmcache_paged_to_kv_buffer,
    lmcache_paged_to_kv_buffer_mla,
    native_lmcache_kv_transfer_abi_version,
)
from musa_aiter.ops.lmcache_musa_batch_copy import (
    is_native_lmcache_musa_batch_copy_available,
    lmcache_musa_memcpy_batch_async,
    native_lmcache_musa_batch_copy_abi_version,
    native_lmcache_musa_batch_copy_runtime_versions,
)
from musa_aiter.ops.hicache_transfer import (
    build_native_hicache_transfer,
    hicache_transfer_kv_all_layer,
    hicache_transfer_kv_all_layer_direct_lf_pf,
    hicache_transfer_kv_all_layer_lf_pf,
    hicache_transfer_kv_all_layer_mla,
    hicache_transfer_kv_all_layer_mla_lf_pf,
    hicache_transfer_kv_direct,
    hicache_transfer_kv_per_layer,
    hicache_transfer_kv_per_layer_direct_pf_lf,
    hicache_transfer_kv_per_layer_mla,
    hicache_transfer_kv_per_layer_mla_pf_lf,
    hicache_transfer_kv_per_layer_pf_lf,
    is_native_hicache_transfer_available,
    native_hicache_transfer_abi_version,
)

list_capabilities = registry.list_capabilities

__all__ = [name for name in dir() if not name.startswith("_")]
