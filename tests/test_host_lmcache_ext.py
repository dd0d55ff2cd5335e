"""Host-side contract of the LMCache extension surface (no GPU needed).

Follows musa_aiter/ops/lmcache_kv_transfer_ext.py:17-56 of the reference (gate variable, one load
attempt, recorded error) and the argument checks of csrc/kvcache/lmcache_kv_transfer_ext.cpp:164-229
and :565-585 (messages, order, RuntimeError as TORCH_CHECK raises), on CPU tensors, which fail the
device check after the checks that precede it.
"""

from __future__ import annotations

import pytest
import torch

from musa_aiter.ops import lmcache_kv_transfer_ext as ext_mod


@pytest.fixture
def fresh(monkeypatch):
    monkeypatch.setattr(ext_mod, "_EXT_MODULE", None)
    monkeypatch.setattr(ext_mod, "_EXT_ATTEMPTED", False)
    monkeypatch.setattr(ext_mod, "_EXT_ERROR", None)
    return ext_mod


def test_gate_and_single_load(fresh, monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_CPP_EXTENSION", "0")
    assert fresh.load_lmcache_kv_transfer_ext() is None
    monkeypatch.delenv("MUSA_AITER_LMCACHE_CPP_EXTENSION")
    ext = fresh.load_lmcache_kv_transfer_ext()
    assert isinstance(ext, fresh.HipLMCacheKVTransferExtension)
    assert fresh.load_lmcache_kv_transfer_ext() is ext
    assert fresh.lmcache_kv_transfer_ext_error() is None
    for name in ("kv_buffer_to_paged_list2", "paged_to_kv_buffer_list2", "kv_buffer_to_paged_two_x_nl",
                 "paged_to_kv_buffer_two_x_nl"):
        assert callable(getattr(ext, name))


def test_failed_load_is_recorded_once(fresh, monkeypatch):
    def broken():
        raise OSError("no library")

    with monkeypatch.context() as m:
        m.setattr(fresh._hip, "library", broken)
        assert fresh.load_lmcache_kv_transfer_ext() is None
        assert isinstance(fresh.lmcache_kv_transfer_ext_error(), OSError)
    assert fresh.load_lmcache_kv_transfer_ext() is None  # one attempt per process, as the reference


def _list2_args(**over):
    args = dict(memory=torch.zeros(2, 2, 4, 8, dtype=torch.float16),
                kvcaches=[torch.zeros(2, 3, 16, 2, 4, dtype=torch.float16)] * 2,
                slots=torch.zeros(4, dtype=torch.long))
    args.update(over)
    return args


def test_list2_checks():
    ext = ext_mod.HipLMCacheKVTransferExtension()
    a = _list2_args(kvcaches=[torch.zeros(2, 3, 16, 2, 4)] * 3)
    with pytest.raises(RuntimeError, match="expects exactly 2 layers"):
        ext.kv_buffer_to_paged_list2(a["memory"], a["kvcaches"], a["slots"], 0, 16, 2, 4)
    a = _list2_args()
    with pytest.raises(RuntimeError, match="memory_tensor must be a ROCm GPU tensor"):
        ext.kv_buffer_to_paged_list2(a["memory"], a["kvcaches"], a["slots"], 0, 16, 2, 4)
    with pytest.raises(RuntimeError, match="memory_tensor must be a ROCm GPU tensor"):
        ext.paged_to_kv_buffer_list2(a["kvcaches"], a["memory"], a["slots"], 16, 2, 4)


def test_two_x_nl_checks():
    ext = ext_mod.HipLMCacheKVTransferExtension()
    mem = torch.zeros(2, 2, 4, 8, dtype=torch.float16)
    caches = [[torch.zeros(3, 16, 2, 4, dtype=torch.float16)] * 2] * 2
    with pytest.raises(RuntimeError, match="split cache must contain K and V groups"):
        ext.kv_buffer_to_paged_two_x_nl(mem, caches[:1], torch.zeros(4, dtype=torch.long), 0, 16, 2, 4)
    with pytest.raises(RuntimeError, match="memory_tensor must be contiguous ROCm GPU"):
        ext.paged_to_kv_buffer_two_x_nl(caches, mem, torch.zeros(4, dtype=torch.long), 16, 2, 4)
