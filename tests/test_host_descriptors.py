"""The layout / transfer-plan / backend / LMCache-format descriptors (CPU only, metadata only).

Restates the reference's contract tests against this package's modules:
op_tests/test_kv_layout_contract.py (7 tests), test_kv_transfer_plan.py (6), test_kv_backend.py (7)
and test_lmcache_format_matrix.py (5), with the same constructors, arguments and assertions, plus
cases beyond them where a rule has more than one branch.
"""

from __future__ import annotations

import pytest
import torch

import musa_aiter
from musa_aiter.ops.kv_backend import KVBackend, KVBackendCapabilities, KVBackendDecision, select_kv_backend
from musa_aiter.ops.kv_layout import KVLayoutKind, KVLayoutSpec, KVOrganization, KVScaleKind
from musa_aiter.ops.kv_transfer_plan import (
    KVTransferEntry,
    KVTransferPlan,
    assess_direct_eligibility,
    validate_transfer_plan,
)
from musa_aiter.ops.lmcache_format import LMCacheFormat, describe_lmcache_format, describe_sglang_split_list


# ----- layout contract: op_tests/test_kv_layout_contract.py --------------------------------------


def test_standard_paged_layout_exposes_hidden_size_and_kind():
    # :13-28
    spec = KVLayoutSpec.standard_paged(num_layers=2, num_blocks=4, block_size=16, num_heads=8, head_size=64,
                                       dtype_name="float16", row_bytes=128, block_stride_bytes=2048)
    assert spec.kind is KVLayoutKind.STANDARD_PAGED
    assert spec.organization is KVOrganization.SEPARATE
    assert spec.hidden_size == 512
    assert spec.is_paged is True


def test_layout_spec_rejects_non_positive_row_bytes():
    # :31-42
    with pytest.raises(ValueError, match="row_bytes"):
        KVLayoutSpec.standard_paged(num_layers=1, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                    dtype_name="float16", row_bytes=0, block_stride_bytes=32)


def test_layout_spec_rejects_block_stride_smaller_than_row():
    # :45-56
    with pytest.raises(ValueError, match="block_stride_bytes"):
        KVLayoutSpec.standard_paged(num_layers=1, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                    dtype_name="float16", row_bytes=32, block_stride_bytes=16)


def test_blocked_scale_requires_value_and_scale_bytes():
    # :59-71
    with pytest.raises(ValueError, match="scale_bytes"):
        KVLayoutSpec.dsv4(num_layers=1, num_blocks=4, block_size=16, row_bytes=132, block_stride_bytes=8640,
                          dtype_name="uint8", scale_kind=KVScaleKind.BLOCKED, value_bytes=128, scale_bytes=0)


def test_page_first_constructor_preserves_non_contiguous_layout_fact():
    # :74-88
    spec = KVLayoutSpec.page_first(num_layers=2, num_blocks=8, block_size=16, num_heads=4, head_size=32,
                                   dtype_name="bfloat16", row_bytes=64, block_stride_bytes=1024)
    assert spec.kind is KVLayoutKind.PAGE_FIRST
    assert spec.is_contiguous is False
    assert spec.requires_layout_transform is True


def test_dsv4_blocked_scale_facts_preserve_byte_geometry():
    # :91-107
    spec = KVLayoutSpec.dsv4(num_layers=1, num_blocks=8, block_size=64, row_bytes=132, block_stride_bytes=8640,
                             dtype_name="uint8", scale_kind=KVScaleKind.BLOCKED, value_bytes=128, scale_bytes=4)
    assert spec.kind is KVLayoutKind.DSV4_BLOCKED_SCALE
    assert spec.format_facts().value_bytes == 128
    assert spec.format_facts().scale_bytes == 4
    assert spec.format_facts().requires_transform is True


def test_public_package_exports_layout_contract():
    # :110-114
    assert musa_aiter.KVLayoutSpec is KVLayoutSpec
    assert musa_aiter.KVLayoutKind is KVLayoutKind


def test_layout_facts_of_the_other_constructors():
    # Beyond the reference tests: a standard paged cache and a linear buffer are contiguous and
    # transform-free, so their facts allow a direct batch; a page-first pool does not.
    paged = KVLayoutSpec.standard_paged(num_layers=1, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                        dtype_name="float16", row_bytes=32, block_stride_bytes=512)
    linear = KVLayoutSpec.linear(num_layers=1, num_tokens=32, num_heads=2, head_size=8, dtype_name="float16")
    page_first = KVLayoutSpec.page_first(num_layers=1, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                         dtype_name="float16", row_bytes=32, block_stride_bytes=512)
    assert paged.format_facts().supports_direct_batch and linear.format_facts().supports_direct_batch
    assert not page_first.format_facts().supports_direct_batch
    assert linear.is_paged is False and linear.hidden_size == 16
    with pytest.raises(ValueError):
        KVLayoutSpec.standard_paged(num_layers=0, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                    dtype_name="float16", row_bytes=32, block_stride_bytes=512)


# ----- transfer plan: op_tests/test_kv_transfer_plan.py -------------------------------------------


def _paged() -> KVLayoutSpec:
    return KVLayoutSpec.standard_paged(num_layers=1, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                       dtype_name="float16", row_bytes=32, block_stride_bytes=512)


def _linear(tokens: int = 32) -> KVLayoutSpec:
    return KVLayoutSpec.linear(num_layers=1, num_tokens=tokens, num_heads=2, head_size=8, dtype_name="float16")


def _plan(*entries: KVTransferEntry, direct_eligible: bool = False, reason: str | None = None) -> KVTransferPlan:
    return KVTransferPlan(source=_paged(), destination=_linear(), direction="d2d", num_tokens=32,
                          skip_prefix_n_tokens=0, entries=tuple(entries), stream_id=None,
                          direct_eligible=direct_eligible, direct_reject_reason=reason)


def test_validate_transfer_plan_accepts_non_overlapping_entries():
    # :49-55
    plan = _plan(KVTransferEntry(0, 0, 16, layer=0, block=0), KVTransferEntry(32, 16, 16, layer=0, block=1))
    assert validate_transfer_plan(plan) is plan


def test_plan_rejects_overlapping_destinations():
    # :58-65
    plan = _plan(KVTransferEntry(0, 0, 16), KVTransferEntry(32, 8, 16))
    with pytest.raises(ValueError, match="destination.*overlap"):
        validate_transfer_plan(plan)


def test_plan_rejects_prefix_larger_than_token_count():
    # :68-82
    plan = KVTransferPlan(source=_paged(), destination=_linear(), direction="d2d", num_tokens=4,
                          skip_prefix_n_tokens=5, entries=(), stream_id=None, direct_eligible=False,
                          direct_reject_reason="empty")
    with pytest.raises(ValueError, match="skip_prefix_n_tokens"):
        validate_transfer_plan(plan)


def test_page_first_plan_is_not_direct_eligible():
    # :85-100
    source = KVLayoutSpec.page_first(num_layers=1, num_blocks=4, block_size=16, num_heads=2, head_size=8,
                                     dtype_name="float16", row_bytes=32, block_stride_bytes=512)
    eligible, reason = assess_direct_eligibility(source, _linear())
    assert eligible is False
    assert "layout transform" in reason


def test_same_geometry_can_use_direct_batch_copy():
    # :103-116
    eligible, reason = assess_direct_eligibility(_linear(), _linear())
    assert eligible is True
    assert reason is None


def test_direct_plan_requires_reason_when_rejected():
    # :119-122
    plan = _plan(direct_eligible=False)
    assert validate_transfer_plan(plan) is plan


def test_touching_destination_ranges_do_not_overlap():
    # Beyond the reference tests: half-open ranges that only touch are accepted; a range inside
    # another one is an overlap even when its start is not adjacent in entry order.
    assert validate_transfer_plan(_plan(KVTransferEntry(0, 0, 16), KVTransferEntry(16, 16, 16))) is not None
    with pytest.raises(ValueError, match="destination.*overlap"):
        validate_transfer_plan(_plan(KVTransferEntry(0, 0, 32), KVTransferEntry(40, 48, 4),
                                     KVTransferEntry(64, 8, 4)))


# ----- backend selection: op_tests/test_kv_backend.py ---------------------------------------------


def _backend_plan(*, direct_eligible: bool, reason: str | None = None) -> KVTransferPlan:
    linear = KVLayoutSpec.linear(num_layers=1, num_tokens=4, num_heads=2, head_size=8, dtype_name="float16")
    return KVTransferPlan(source=linear, destination=linear, direction="d2d", num_tokens=4, skip_prefix_n_tokens=0,
                          entries=(KVTransferEntry(0, 0, 16),), stream_id=None, direct_eligible=direct_eligible,
                          direct_reject_reason=reason)


def test_specialized_native_has_priority_over_direct():
    # :35-51
    decision = select_kv_backend(_backend_plan(direct_eligible=True),
                                 capabilities=KVBackendCapabilities(specialized_native=True, fused_native=True,
                                                                    direct_batch=True, reference=True))
    assert decision == KVBackendDecision(backend=KVBackend.SPECIALIZED_NATIVE, accepted=True,
                                         reason="exact specialized native capability is available",
                                         requires_sync=False)


def test_direct_is_selected_only_for_direct_eligible_plan():
    # :54-62
    decision = select_kv_backend(_backend_plan(direct_eligible=True),
                                 capabilities=KVBackendCapabilities(direct_batch=True))
    assert decision.backend is KVBackend.DIRECT_BATCH
    assert decision.accepted is True
    assert decision.requires_sync is False


def test_non_direct_plan_falls_back_with_plan_reason():
    # :65-73
    decision = select_kv_backend(_backend_plan(direct_eligible=False, reason="layout transform is required"),
                                 capabilities=KVBackendCapabilities(direct_batch=True, reference=True))
    assert decision.backend is KVBackend.REFERENCE
    assert decision.accepted is True
    assert "layout transform is required" in decision.reason


def test_require_native_rejects_when_no_native_backend_is_available():
    # :76-85
    decision = select_kv_backend(_backend_plan(direct_eligible=True),
                                 capabilities=KVBackendCapabilities(reference=True), require_native=True)
    assert decision.backend is KVBackend.REJECTED
    assert decision.accepted is False
    assert "native backend required" in decision.reason


def test_invalid_plan_is_rejected_before_backend_selection():
    # :88-104
    valid = _backend_plan(direct_eligible=True)
    invalid = KVTransferPlan(source=valid.source, destination=valid.destination, direction="d2d", num_tokens=4,
                             skip_prefix_n_tokens=5, entries=valid.entries, stream_id=None, direct_eligible=True,
                             direct_reject_reason=None)
    with pytest.raises(ValueError, match="skip_prefix_n_tokens"):
        select_kv_backend(invalid)


def test_lmcache_batch_copy_wrapper_uses_plan_selector():
    # :107-118
    from musa_aiter.ops.lmcache_musa_batch_copy import select_lmcache_batch_copy_backend

    decision = select_lmcache_batch_copy_backend(_backend_plan(direct_eligible=True), native_available=True)
    assert decision.backend is KVBackend.DIRECT_BATCH
    assert decision.accepted is True


def test_public_package_exports_backend_selector():
    # :121-125
    assert musa_aiter.KVBackend is KVBackend
    assert musa_aiter.select_kv_backend is select_kv_backend


def test_backend_priority_order_without_the_higher_tiers():
    # Beyond the reference tests: fused native comes after specialized and before direct; with no
    # native capability at all a reference-capable selection takes the reference path.
    fused = select_kv_backend(_backend_plan(direct_eligible=True),
                              capabilities=KVBackendCapabilities(fused_native=True, direct_batch=True))
    assert fused.backend is KVBackend.FUSED_NATIVE and fused.accepted is True
    ref = select_kv_backend(_backend_plan(direct_eligible=True), capabilities=KVBackendCapabilities(reference=True))
    assert ref.backend is KVBackend.REFERENCE and ref.accepted is True


# ----- LMCache formats: op_tests/test_lmcache_format_matrix.py -------------------------------------


def test_kv_2ltd_format_is_identified_from_memory_shape():
    # :14-20
    facts = describe_lmcache_format(torch.zeros(2, 3, 5, 16))
    assert facts.format is LMCacheFormat.KV_2LTD
    assert facts.spec.kind is KVLayoutKind.KV_2LTD
    assert facts.spec.num_layers == 3
    assert facts.spec.num_tokens == 5


def test_kv_t2d_and_kv_2td_are_not_ambiguous():
    # :23-31
    t2d = describe_lmcache_format(torch.zeros(5, 2, 16))
    two_td = describe_lmcache_format(torch.zeros(2, 5, 16))
    assert t2d.format is LMCacheFormat.KV_T2D
    assert t2d.spec.organization is KVOrganization.MERGED
    assert two_td.format is LMCacheFormat.KV_2TD
    assert two_td.spec.organization is KVOrganization.SEPARATE


def test_sglang_split_list_format_preserves_layer_count_and_geometry():
    # :34-46
    caches = [[torch.zeros(4, 16, 2, 8) for _ in range(3)], [torch.zeros(4, 16, 2, 8) for _ in range(3)]]
    facts = describe_sglang_split_list(caches)
    assert facts.format is LMCacheFormat.SGLANG_SPLIT_LIST
    assert facts.spec.kind is KVLayoutKind.TWO_X_NL
    assert facts.spec.num_layers == 3
    assert facts.spec.block_size == 16


def test_format_rejects_wrong_rank_and_empty_split_list():
    # :49-53
    with pytest.raises(ValueError, match="rank"):
        describe_lmcache_format(torch.zeros(2, 3))
    with pytest.raises(ValueError, match="non-empty"):
        describe_sglang_split_list([[], []])


def test_format_facts_are_exported_from_package():
    # :56-60
    assert musa_aiter.LMCacheFormat is LMCacheFormat
    assert musa_aiter.describe_lmcache_format is describe_lmcache_format


def test_format_dtype_errors_come_before_shape_errors():
    # lmcache_format.py:58 and :77 check the dtype before the 3-D shape rules: an unsupported dtype
    # is reported even where the shape alone would be ambiguous or unclassifiable.
    with pytest.raises(ValueError, match="unsupported LMCache dtype"):
        describe_lmcache_format(torch.zeros(2, 2, 4, dtype=torch.int64))
    with pytest.raises(ValueError, match="unsupported LMCache dtype"):
        describe_lmcache_format(torch.zeros(3, 5, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="unsupported LMCache dtype"):
        describe_lmcache_format(torch.zeros(2, 3, 5, 4, dtype=torch.float64))
    with pytest.raises(ValueError, match="ambiguous"):
        describe_lmcache_format(torch.zeros(2, 2, 4))
    with pytest.raises(ValueError, match=r"\[T, 2, H\] or \[2, T, H\]"):
        describe_lmcache_format(torch.zeros(3, 5, 4))
    assert describe_lmcache_format(torch.zeros(2, 5, 4, dtype=torch.uint8)).spec.dtype_name == "uint8"
