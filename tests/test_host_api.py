"""Host-side contract of the public API (CPU only, no kernel launches).

Mirrors the reference's error contracts (op_tests/test_kv_transfer.py:490-560,
test_lmcache_kv_transfer.py:213-296, test_kv_copy_paged_rows*.py): validation
raises ValueError / TypeError / IndexError before any launch, and tensors that
are not on a ROCm device are rejected with RuntimeError instead of silently
taking a CPU path.  Also pins the registry rows, the dispatch trace format,
the CLI and the layout descriptors.
"""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch

import musa_aiter
from musa_aiter import registry
from musa_aiter.dispatch import DispatchRecord, emit


def test_validation_errors_precede_device_check():
    kc = torch.zeros(2, 1, 4, 4)
    vc = torch.zeros(2, 1, 4, 4)
    with pytest.raises(ValueError, match="4-D"):
        musa_aiter.kv_paged_to_linear(torch.zeros(2, 4, 4), vc, torch.tensor([0]))
    with pytest.raises(ValueError, match="shapes must match"):
        musa_aiter.kv_paged_to_linear(kc, torch.zeros(2, 1, 4, 2), torch.tensor([0]))
    with pytest.raises(ValueError, match="integer-valued"):
        musa_aiter.kv_paged_to_linear(kc, vc, torch.tensor([0.0]))
    with pytest.raises(ValueError, match="1-D"):
        musa_aiter.kv_paged_to_linear(kc, vc, torch.tensor([[0]]))
    with pytest.raises(ValueError, match="preserve requires"):
        musa_aiter.kv_paged_to_linear(kc, vc, torch.tensor([0]), fill_skipped="preserve")
    with pytest.raises(ValueError, match="last dims must match"):
        musa_aiter.kv_linear_to_paged(torch.zeros(2, 1, 3), torch.zeros(2, 1, 3), kc, vc, torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="layer count mismatch"):
        musa_aiter.kv_linear_to_paged_multi_layer(torch.zeros(3, 2, 1, 4), torch.zeros(3, 2, 1, 4),
                                                  torch.zeros(2, 2, 1, 4, 4), torch.zeros(2, 2, 1, 4, 4),
                                                  torch.tensor([0, 1]))


def test_cpu_tensors_are_rejected_not_computed():
    kc = torch.zeros(2, 1, 4, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.kv_paged_to_linear(kc, kc.clone(), torch.tensor([0, 3]))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.kv_linear_to_paged(torch.zeros(1, 1, 4), torch.zeros(1, 1, 4), kc, kc.clone(), torch.tensor([0]))
    caches = [[torch.zeros(1, 2, 1, 4) for _ in range(2)] for _ in range(2)]
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.lmcache_kv_paged_to_buffer(caches, torch.zeros(2, 2, 2, 4), torch.tensor([0, 1]), 2, 1, 4)


def test_fp8_validation_contract():
    # op_tests/test_kv_transfer.py:490-519
    k_lin = torch.zeros(2, 1, 4)
    k_cache = torch.zeros(1, 1, 4, 2, dtype=torch.uint8)
    slots = torch.tensor([0, 1], dtype=torch.int32)
    for bad in (0.0, -1.0, float("inf")):
        with pytest.raises(ValueError, match="positive and finite"):
            musa_aiter.kv_linear_to_paged_fp8(k_lin, k_lin, k_cache, k_cache.clone(), slots, bad, 1.0)
    with pytest.raises(ValueError, match="uint8"):
        musa_aiter.kv_linear_to_paged_fp8(k_lin, k_lin, k_cache.float(), k_cache, slots, 1.0, 1.0)
    with pytest.raises(ValueError, match="unsupported FP8"):
        musa_aiter.kv_linear_to_paged_fp8(k_lin, k_lin, k_cache, k_cache, slots, 1.0, 1.0, fp8_format="bad")
    with pytest.raises(ValueError, match=r"scalar or \[kv_heads\]"):
        musa_aiter.kv_linear_to_paged_fp8(k_lin, k_lin, k_cache, k_cache, slots, torch.ones(3), 1.0)


def test_slot_bounds_contract():
    # op_tests/test_kv_transfer.py:522-560
    kc = torch.zeros(2, 1, 4, 4)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_paged_to_linear(kc, kc.clone(), torch.tensor([0, 8]))
    big = torch.zeros(2, 2, 1, 4, 4)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_linear_to_paged_multi_layer(torch.zeros(2, 2, 1, 4), torch.zeros(2, 2, 1, 4), big, big.clone(),
                                                  torch.tensor([0, 13]))


def test_slot_bounds_come_before_output_and_dtype_checks():
    # The reference checks slot bounds right after the device check
    # (kv_transfer.py:3153, :3234, :3351, :3858): a call that is wrong in
    # several ways reports the bad slot first.
    kc = torch.zeros(2, 1, 4, 4)
    bad = torch.tensor([0, 8])
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_paged_to_linear(kc, kc.clone(), bad, out_k=torch.zeros(5), fill_skipped="preserve")
    big = torch.zeros(2, 2, 1, 4, 4)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_paged_to_linear_multi_layer(big, big.clone(), bad, out_k=torch.zeros(5), out_v=torch.zeros(5))
    ints = torch.zeros(2, 1, 4, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_linear_to_paged(torch.zeros(2, 1, 4, dtype=torch.int32), torch.zeros(2, 1, 4, dtype=torch.int32),
                                      ints, ints.clone(), bad)
    flat = torch.zeros(2, 4, 3)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_paged_to_mla_linear(flat, flat.clone(), bad, out_kv=torch.zeros(1))


def test_lmcache_contracts():
    # op_tests/test_lmcache_kv_transfer.py:213-241, :276-295
    memory = torch.zeros(2, 2, 2, 4)
    bad_layers = [[torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 1, 4)], [torch.zeros(1, 2, 1, 4)]]
    with pytest.raises(ValueError, match="layer"):
        musa_aiter.lmcache_kv_paged_to_buffer(bad_layers, memory, torch.tensor([0, 1]), 2, 1, 4)
    good = [[torch.zeros(1, 2, 1, 4) for _ in range(2)] for _ in range(2)]
    with pytest.raises(ValueError, match="int32 or int64"):
        musa_aiter.lmcache_kv_paged_to_buffer(good, memory, torch.tensor([0.0, 1.0]), 2, 1, 4)
    with pytest.raises(ValueError, match="transfer range"):
        musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(memory, good, torch.tensor([0, 1]), 1, 2, 1, 4)
    with pytest.raises(ValueError, match="out of range"):
        musa_aiter.lmcache_kv_buffer_to_paged(torch.zeros(2, 1, 2, 4), torch.zeros(1, 2, 1, 4, 1, 4),
                                              torch.tensor([0, 8], dtype=torch.int32))
    with pytest.raises(ValueError, match="rank"):
        musa_aiter.lmcache_kv_buffer_to_paged(torch.zeros(1, 2, 3), torch.zeros(1, 2, 1, 4, 1, 4), torch.tensor([0]))
    with pytest.raises(TypeError):
        musa_aiter.lmcache_kv_buffer_to_paged(memory, [torch.zeros(2, 1, 2, 1, 4)], torch.tensor([0, 1]), 0, 2)


def test_cache_list_checks_keep_the_reference_order():
    """The per-cache checks of the list paths run in the reference's order (every shape, then
    devices, then dtypes, then contiguity) whichever cache fails first; the host module's single
    pass only decides whether they need to run."""
    nb, bs, nh, hs = 3, 2, 1, 4
    mem = torch.zeros(2, 3, 5, nh * hs)
    good = torch.zeros(2, nb, bs, nh, hs)
    wrong_dtype = torch.zeros(2, nb, bs, nh, hs, dtype=torch.float16)
    wrong_shape = torch.zeros(2, nb, bs + 1, nh, hs)
    slots = torch.tensor([0, 1])
    with pytest.raises(ValueError, match="rank must be 5"):  # the shape error of cache 2 wins over cache 1's dtype
        musa_aiter.lmcache_kv_paged_to_buffer([good, wrong_dtype, wrong_shape], mem, slots, bs, nh, hs)
    with pytest.raises(RuntimeError, match="ROCm GPU device"):  # all caches valid: the CPU device is rejected
        musa_aiter.lmcache_kv_paged_to_buffer([good, good, good], mem, slots, bs, nh, hs)
    mla_mem = torch.zeros(1, 2, 5, hs)
    mla_good, mla_bad = torch.zeros(nb, bs, hs), torch.zeros(nb, bs, hs + 1)
    with pytest.raises(ValueError, match="rank must be 3"):
        musa_aiter.lmcache_mla_paged_to_buffer([mla_good.half(), mla_bad], mla_mem, slots, bs, hs)
    k = [torch.zeros(nb, bs, nh, hs) for _ in range(2)]
    v = [torch.zeros(nb, bs, nh, hs), torch.zeros(nb, bs, nh, hs + 1)]
    with pytest.raises(ValueError, match=r"cache\[1\]\[1\] must have shape"):
        musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl([k, v], torch.zeros(2, 2, 5, nh * hs), slots, bs, nh, hs)
    v[1] = torch.zeros(nb, bs, nh, hs, dtype=torch.float16)
    with pytest.raises(ValueError, match="cache dtype must match memory_tensor"):
        musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl([k, v], torch.zeros(2, 2, 5, nh * hs), slots, bs, nh, hs)


def test_byte_row_contracts():
    src = torch.zeros(4, 8, dtype=torch.uint8)
    with pytest.raises(TypeError):
        musa_aiter.kv_copy_paged_rows([1], src, torch.tensor([0]), torch.tensor([0]))
    with pytest.raises(ValueError, match="uint8"):
        musa_aiter.kv_copy_paged_rows(src.float(), src, torch.tensor([0]), torch.tensor([0]))
    with pytest.raises(IndexError, match="out of bounds"):
        musa_aiter.kv_copy_paged_rows(src, src.clone(), torch.tensor([4]), torch.tensor([0]))
    with pytest.raises(IndexError, match="negative"):
        musa_aiter.kv_copy_paged_rows(src, src.clone(), torch.tensor([0]), torch.tensor([-1]))
    layout = musa_aiter.InterleavedFp8Layout(value_bytes=4, scale_bytes=2, scale_granularity=2)
    with pytest.raises(ValueError, match="layout.item_bytes"):
        musa_aiter.kv_copy_paged_rows(src, src.clone(), torch.tensor([0]), torch.tensor([0]), layout=layout)
    with pytest.raises(ValueError, match="direction"):
        musa_aiter.kv_copy_paged_rows_multi_pool([], torch.tensor([0]), direction="X")


def test_strided_block_transfer_rejects_without_launch():
    ids = torch.zeros(4, dtype=torch.int64)
    assert musa_aiter.lmcache_kv_strided_block_transfer(0, [0], ids, 0, 1, 0, 1, 0, 4, 2, 6, 16, 0) is False
    assert musa_aiter.lmcache_kv_strided_block_transfer(0, [0], ids, 0, 1, 0, 1, 0, 4, 2, 8, 16, 0) is False


def test_kvcache_registry_rows_and_backend():
    caps = registry.list_capabilities(family="kvcache")
    names = {c.name for c in caps}
    assert names == {
        "kv_paged_to_linear", "kv_linear_to_paged", "kv_paged_to_linear_multi_layer", "kv_linear_to_paged_multi_layer",
        "kv_paged_to_merged_linear", "kv_merged_linear_to_paged", "kv_paged_to_merged_linear_multi_layer",
        "kv_merged_linear_to_paged_multi_layer", "kv_linear_to_paged_fp8", "kv_paged_fp8_to_linear",
        "kv_linear_to_paged_fp8_multi_layer", "kv_paged_fp8_to_linear_multi_layer", "kv_merged_linear_to_paged_fp8",
        "kv_paged_fp8_to_merged_linear", "kv_merged_linear_to_paged_fp8_multi_layer",
        "kv_paged_fp8_to_merged_linear_multi_layer", "kv_paged_to_mla_linear", "kv_mla_linear_to_paged",
        "kv_load_and_reshape_flash", "kv_load_and_dequantize_fp8_flash", "kv_reshape_and_cache_back_flash",
        "kv_copy_paged_blocks", "kv_copy_paged_blocks_fp8",
        "kv_paged_to_mla_linear_multi_layer", "kv_mla_linear_to_paged_multi_layer", "kv_copy_paged_rows",
        "kv_copy_paged_rows_layer_table", "kv_copy_paged_rows_multi_pool", "lmcache_kv_paged_to_buffer_two_x_nl",
        "lmcache_kv_buffer_to_paged_two_x_nl", "lmcache_kv_paged_to_buffer", "lmcache_kv_buffer_to_paged",
        "lmcache_paged_to_kv_buffer", "lmcache_kv_buffer_to_paged_mla", "lmcache_paged_to_kv_buffer_mla",
        "lmcache_mla_buffer_to_paged", "lmcache_mla_paged_to_buffer", "lmcache_kv_strided_block_transfer",
        "hicache_transfer_kv_per_layer", "hicache_transfer_kv_per_layer_pf_lf", "hicache_transfer_kv_all_layer",
        "hicache_transfer_kv_all_layer_lf_pf", "hicache_transfer_kv_per_layer_mla",
        "hicache_transfer_kv_per_layer_mla_pf_lf", "hicache_transfer_kv_all_layer_mla",
        "hicache_transfer_kv_all_layer_mla_lf_pf", "hicache_transfer_kv_direct",
        "hicache_transfer_kv_per_layer_direct_pf_lf", "hicache_transfer_kv_all_layer_direct_lf_pf",
        "lmcache_musa_memcpy_batch_async", "kv_cachegen_encode", "kv_cachegen_decode",
    }
    for cap in caps:
        assert cap.backends == ("rocm-hip",)
        assert callable(getattr(musa_aiter, cap.name))


def test_dispatch_trace_format(monkeypatch, capsys):
    monkeypatch.setenv("MUSA_AITER_TRACE_DISPATCH", "1")
    emit(DispatchRecord("kv_paged_to_linear", "rocm-hip", "cuda:0", "torch.bfloat16", "why"))
    err = capsys.readouterr().err
    assert err.strip() == ("[MUSA_AITER DISPATCH] op=kv_paged_to_linear backend=rocm-hip device=cuda:0 "
                           "dtype=torch.bfloat16 reason=why")
    monkeypatch.setenv("MUSA_AITER_TRACE_DISPATCH", "0")
    emit(DispatchRecord("x", "y", "z", "w", "v"))
    assert capsys.readouterr().err == ""


def test_policy_and_gate(monkeypatch):
    from musa_aiter.policy import FallbackPolicy, current_policy

    monkeypatch.setenv("MUSA_AITER_FALLBACK_POLICY", "1")
    assert current_policy() is FallbackPolicy.REQUIRE_NATIVE
    with pytest.raises(RuntimeError):
        musa_aiter.ensure_reference_allowed("op")
    musa_aiter.ensure_reference_allowed("op", native_available=True)
    monkeypatch.setenv("MUSA_AITER_NATIVE_KV_TRANSFER", "1")
    d = musa_aiter.decide_native_gate("op", ["MUSA_AITER_NATIVE_KV_TRANSFER"], available=False, native_required=True)
    assert (d.mode, d.reason) == ("error", "native_unavailable")


def test_cli_list_ops():
    out = subprocess.run([sys.executable, "-m", "musa_aiter.cli", "list-ops", "--family", "kvcache"],
                         capture_output=True, text=True, check=True,
                         env={**__import__("os").environ, "PYTHONPATH": ":".join(sys.path)}).stdout
    assert "kv_paged_to_linear_multi_layer" in out and "backends=rocm-hip" in out


def test_layout_descriptors():
    spec = musa_aiter.InterleavedFp8Layout(value_bytes=128, scale_bytes=4, scale_granularity=16).as_kv_layout_spec(
        num_layers=2, num_blocks=8, block_size=16)
    facts = spec.format_facts()
    assert (facts.value_bytes, facts.scale_bytes, facts.requires_transform) == (128, 4, True)
    lin = musa_aiter.KVLayoutSpec.linear(num_layers=2, num_tokens=4, num_heads=8, head_size=128, dtype_name="bfloat16")
    assert lin.row_bytes == 2048 and lin.format_facts().supports_direct_batch
    with pytest.raises(ValueError):
        musa_aiter.KVLayoutSpec.linear(num_layers=1, num_tokens=1, num_heads=1, head_size=1, dtype_name="int7")
    fmt = musa_aiter.describe_lmcache_format(torch.zeros(2, 3, 5, 16, dtype=torch.bfloat16))
    assert fmt.format is musa_aiter.LMCacheFormat.KV_2LTD and fmt.spec.num_tokens == 5
    assert musa_aiter.describe_lmcache_format(torch.zeros(7, 2, 4)).spec.num_tokens == 7
    split = musa_aiter.describe_sglang_split_list([[torch.zeros(4, 16, 2, 8)] * 3, [torch.zeros(4, 16, 2, 8)] * 3])
    assert split.spec.pointer_table_length == 6
    plan = musa_aiter.KVTransferPlan(lin, lin, "d2d", 4, 0, (musa_aiter.KVTransferEntry(0, 0, 8),
                                                             musa_aiter.KVTransferEntry(0, 4, 8)), None, True, None)
    with pytest.raises(ValueError, match="overlap"):
        musa_aiter.validate_transfer_plan(plan)
    ok_plan = musa_aiter.KVTransferPlan(lin, lin, "d2d", 4, 0, (musa_aiter.KVTransferEntry(0, 0, 8),), None, True, None)
    decision = musa_aiter.select_kv_backend(ok_plan, capabilities=musa_aiter.KVBackendCapabilities(reference=False),
                                            require_native=True)
    assert decision.backend is musa_aiter.KVBackend.REJECTED
    assert musa_aiter.select_kv_backend(ok_plan, capabilities=musa_aiter.hip_capabilities()).accepted


def test_abi_version_probes():
    assert musa_aiter.native_lmcache_kv_transfer_abi_version() == 1
    assert musa_aiter.native_kv_transfer_abi_version() == 1
    assert musa_aiter.native_fp8_kv_cache_abi_version() == 1
    assert musa_aiter.native_hicache_transfer_abi_version() == 1
    assert musa_aiter.is_native_hicache_transfer_available() is True


def test_dense_preload_validation_contract():
    # op_tests/test_kv_transfer.py:335-346, test_kv_flash_reverse.py:45-55, kv_transfer.py:1303-1328
    kc = torch.zeros(2, 1, 2, 4)
    tables = torch.tensor([[0, 2]], dtype=torch.int32)
    with pytest.raises(ValueError, match="invalid block id 2"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables, torch.tensor([5], dtype=torch.int32),
                                             out_k=torch.empty(1, 5, 1, 2), out_v=torch.empty(1, 5, 1, 2))
    with pytest.raises(ValueError, match="max_seq_len is smaller"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables, torch.tensor([5]), max_seq_len=4)
    with pytest.raises(ValueError, match="enough columns"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables, torch.tensor([3]), max_seq_len=9)
    with pytest.raises(ValueError, match="non-negative"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables, torch.tensor([-1]))
    with pytest.raises(ValueError, match="block_tables must use an integer dtype"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables.float(), torch.tensor([3]))
    with pytest.raises(ValueError, match="out_k must match"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables, torch.tensor([3]), out_k=torch.empty(1, 4, 1, 2))
    with pytest.raises(ValueError, match="dense"):
        musa_aiter.kv_reshape_and_cache_back_flash(torch.zeros(2, 7, 3), torch.zeros(2, 7, 3), torch.zeros(4, 2, 3, 4),
                                                   torch.zeros(4, 2, 3, 4),
                                                   torch.tensor([[0, 1], [2, 3]], dtype=torch.int32),
                                                   torch.tensor([4, 4], dtype=torch.int32))
    dense = torch.zeros(2, 4, 1, 2)
    with pytest.raises(ValueError, match="seq_lens exceeds"):
        musa_aiter.kv_reshape_and_cache_back_flash(dense, dense.clone(), kc, kc.clone(),
                                                   torch.tensor([[0, 1], [1, 0]]), torch.tensor([4, 5]))
    with pytest.raises(ValueError, match="invalid block id -1"):
        musa_aiter.kv_reshape_and_cache_back_flash(dense, dense.clone(), kc, kc.clone(),
                                                   torch.tensor([[0, 1], [-1, 0]]), torch.tensor([4, 2]))
    with pytest.raises(ValueError, match="integer tensors"):
        musa_aiter.kv_load_and_dequantize_fp8_flash(kc.to(torch.uint8), kc.to(torch.uint8), tables,
                                                    torch.tensor([3.0]), 1.0, 1.0)
    with pytest.raises(ValueError, match="out_k must match"):
        musa_aiter.kv_load_and_dequantize_fp8_flash(kc.to(torch.uint8), kc.to(torch.uint8), tables,
                                                    torch.tensor([3]), 1.0, 1.0, out_k=torch.empty(1, 3, 1, 2))
    key = torch.zeros(8, 2, 4)
    with pytest.raises(ValueError, match=r"kv_indptr must be \[batch \+ 1\]"):
        musa_aiter.ops.kv_transfer.kv_triton_indexed_to_dense(key, key.clone(), torch.tensor([0]), torch.tensor([0]),
                                                             max_seq_len=2)
    with pytest.raises(ValueError, match="max_seq_len must be non-negative"):
        musa_aiter.ops.kv_transfer.kv_triton_indexed_to_dense(key, key.clone(), torch.tensor([0, 1]),
                                                             torch.tensor([0]), max_seq_len=-1)
    with pytest.raises(ValueError, match="be contiguous"):
        musa_aiter.ops.kv_transfer.kv_triton_indexed_to_dense(key, key.clone(), torch.tensor([0, 1]),
                                                             torch.tensor([0]), max_seq_len=2,
                                                             out_k=torch.zeros(1, 2, 4, 2).transpose(2, 3))


def test_block_copy_validation_contract():
    # op_tests/test_kv_transfer.py:387-399
    src = torch.zeros(2, 1, 2, 3)
    with pytest.raises(ValueError, match="out of bounds"):
        musa_aiter.kv_copy_paged_blocks(src, src.clone(), src.clone(), src.clone(), torch.tensor([[2, 0]]))
    with pytest.raises(ValueError, match=r"\[num_pairs, 2\]"):
        musa_aiter.kv_copy_paged_blocks(src, src.clone(), src.clone(), src.clone(), torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="tails must match"):
        musa_aiter.kv_copy_paged_blocks(src, src.clone(), torch.zeros(2, 1, 2, 4), torch.zeros(2, 1, 2, 4),
                                        torch.tensor([[0, 1]]))
    with pytest.raises(ValueError, match="FP8 cache storage"):
        musa_aiter.kv_copy_paged_blocks_fp8(src, src.clone(), src.clone(), src.clone(), torch.tensor([[0, 1]]))
    # Nothing to copy: no launch, so CPU tensors are fine.
    assert musa_aiter.kv_copy_paged_blocks(src, src.clone(), src.clone(), src.clone(), torch.tensor([[-1, 0]])) == 0


def test_dense_preload_cpu_tensors_are_rejected_not_computed():
    kc = torch.zeros(2, 1, 2, 4)
    tables = torch.tensor([[0, 1]])
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.kv_load_and_reshape_flash(kc, kc.clone(), tables, torch.tensor([5]))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.kv_reshape_and_cache_back_flash(torch.zeros(1, 5, 1, 2), torch.zeros(1, 5, 1, 2), kc, kc.clone(),
                                                   tables, torch.tensor([5]))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.kv_load_and_dequantize_fp8_flash(kc.to(torch.uint8), kc.to(torch.uint8), tables,
                                                    torch.tensor([5]), 1.0, 1.0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.ops.kv_transfer.kv_triton_indexed_to_dense(torch.zeros(4, 1, 2), torch.zeros(4, 1, 2),
                                                             torch.tensor([0, 2]), torch.tensor([1, 3]), max_seq_len=2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        musa_aiter.kv_copy_paged_blocks(kc, kc.clone(), kc.clone(), kc.clone(), torch.tensor([[0, 1]]))
