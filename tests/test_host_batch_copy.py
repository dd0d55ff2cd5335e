"""Host-side contract of the LMCache host/device copy batches (CPU only, no copies).

Restates the reference's op_tests/test_lmcache_musa_batch_copy.py (:17-460): the opt-in gate,
the plan's validation and splitting at host registration boundaries, chunking, the fail-closed
cases and the submission to the extension object, with the GPU endpoint faked by device-kind
monkeypatching as the reference does.  Also pins the product plan builder against the oracle's
byte-level splitting rule and checks the HIP extension object's argument checks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops import lmcache_musa_batch_copy as batch
from musa_aiter.ops import lmcache_musa_batch_copy_ext as ext
from oracle import batch_copy_oracle as bo


def _fake_kinds(monkeypatch, source, destination, direction="h2d"):
    kinds = {id(source): "cpu", id(destination): "gpu"} if direction == "h2d" else \
        {id(source): "gpu", id(destination): "cpu"}
    monkeypatch.setattr(batch, "_tensor_device_kind", lambda tensor: kinds[id(tensor)])


class _Recorder:
    def __init__(self, results=None, abi=1):
        self.calls = []
        self._results = results
        self._abi = abi

    def abi_version(self):
        return self._abi

    def batch_memcpy_supported(self):
        return True

    def execute_batch_copy(self, *args):
        self.calls.append(args)
        return True if self._results is None else self._results(len(self.calls))


def test_public_api_is_exported():
    from musa_aiter.registry import get

    assert musa_aiter.native_lmcache_musa_batch_copy_abi_version() == 1
    assert callable(musa_aiter.is_native_lmcache_musa_batch_copy_available)
    assert callable(musa_aiter.lmcache_musa_memcpy_batch_async)
    assert callable(musa_aiter.native_lmcache_musa_batch_copy_runtime_versions)
    cap = get("lmcache_musa_memcpy_batch_async")
    assert cap.family == "kvcache" and cap.backends == ("rocm-hip",)


def test_opt_in_and_empty_batch_is_a_noop(monkeypatch):
    monkeypatch.delenv("MUSA_AITER_LMCACHE_BATCH_COPY", raising=False)
    monkeypatch.delenv("LMCACHE_MUSA_DIRECT_COPY", raising=False)
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: pytest.fail("extension must stay lazy"))
    assert musa_aiter.is_native_lmcache_musa_batch_copy_available() is False
    assert musa_aiter.lmcache_musa_memcpy_batch_async([], [], []) is True
    assert musa_aiter.native_lmcache_musa_batch_copy_runtime_versions() is None


def test_gate_alias_and_real_extension_probe(monkeypatch):
    monkeypatch.delenv("MUSA_AITER_LMCACHE_BATCH_COPY", raising=False)
    monkeypatch.setenv("LMCACHE_MUSA_DIRECT_COPY", "1")
    assert batch.is_native_lmcache_musa_batch_copy_available() is True
    versions = batch.native_lmcache_musa_batch_copy_runtime_versions()
    assert versions is not None and versions[0] > 0


def test_plan_splits_at_host_registration_boundaries():
    plan = batch._build_batch_copy_plan(direction="h2d", sizes=[10], source_capacities=[32],
                                        destination_capacities=[32], source_offsets=[4], destination_offsets=[8],
                                        host_registration_offsets=[6], pin_chunk_size=8)
    assert plan.direction == "h2d" and plan.total_bytes == 10 and plan.input_entry_count == 1
    assert [(e.source_offset, e.destination_offset, e.size) for e in plan.entries] == [(4, 8, 2), (6, 10, 8)]


def test_plan_preserves_entry_order_and_d2h_host_offsets():
    plan = batch._build_batch_copy_plan(direction="d2h", sizes=[3, 5], source_capacities=[16, 16],
                                        destination_capacities=[16, 16], source_offsets=[1, 2],
                                        destination_offsets=[3, 4], host_registration_offsets=[5, 0],
                                        pin_chunk_size=8)
    assert plan.total_bytes == 8
    assert [(e.input_index, e.size) for e in plan.entries] == [(0, 3), (1, 5)]


@pytest.mark.parametrize(("kwargs", "message"), [
    ({"direction": "sideways"}, "direction"),
    ({"sizes": [4, 5]}, "same length"),
    ({"sizes": [0]}, "positive"),
    ({"source_offsets": [-1]}, "non-negative"),
    ({"destination_capacities": [3]}, "destination range"),
    ({"source_capacities": [3]}, "source range"),
    ({"pin_chunk_size": 0}, "pin_chunk_size"),
    ({"sizes": [True]}, "integers"),
    ({"destination_keys": [[1]]}, "hashable"),
])
def test_plan_rejects_invalid_contract(kwargs, message):
    values = {"direction": "h2d", "sizes": [4], "source_capacities": [8], "destination_capacities": [8],
              "source_offsets": [0], "destination_offsets": [0], "host_registration_offsets": [0],
              "pin_chunk_size": 8}
    values.update(kwargs)
    with pytest.raises(ValueError, match=message):
        batch._build_batch_copy_plan(**values)


def test_plan_rejects_overlapping_destinations():
    with pytest.raises(ValueError, match="overlapping destination"):
        batch._build_batch_copy_plan(direction="h2d", sizes=[6, 4], source_capacities=[16, 16],
                                     destination_capacities=[16, 16], source_offsets=[0, 0],
                                     destination_offsets=[0, 4], destination_keys=[7, 7])
    # Same offsets in different destinations are fine.
    batch._build_batch_copy_plan(direction="h2d", sizes=[6, 4], source_capacities=[16, 16],
                                 destination_capacities=[16, 16], destination_offsets=[0, 4],
                                 destination_keys=[7, 8])


def test_plan_chunks_entries_without_changing_order():
    plan = batch._build_batch_copy_plan(direction="h2d", sizes=[2, 3, 4, 5, 6], source_capacities=[20] * 5,
                                        destination_capacities=[20] * 5, destination_keys=list(range(5)))
    chunks = batch._chunk_batch_copy_plan(plan, 2)
    assert [[e.input_index for e in c] for c in chunks] == [[0, 1], [2, 3], [4]]
    assert sum(e.size for c in chunks for e in c) == plan.total_bytes
    with pytest.raises(ValueError, match="max_batch_entries"):
        batch._chunk_batch_copy_plan(plan, 0)


def test_batch_limit_environment_override(monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_MAX_ENTRIES", "17")
    assert batch._resolve_max_batch_entries(None) == 17
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_MAX_ENTRIES", "0")
    with pytest.raises(ValueError, match="must be positive"):
        batch._resolve_max_batch_entries(None)
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_MAX_ENTRIES", "x")
    with pytest.raises(ValueError, match="must be an integer"):
        batch._resolve_max_batch_entries(None)
    with pytest.raises(ValueError, match="positive integer"):
        batch._resolve_max_batch_entries(True)


@pytest.mark.parametrize("seed", range(30))
def test_plan_split_matches_byte_level_rule(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 6))
    sizes = [int(x) for x in rng.integers(1, 200, size=n)]
    pin = int(rng.integers(1, 64)) if seed % 5 else None
    src_off = [int(x) for x in rng.integers(0, 50, size=n)]
    dst_off = [int(sum(sizes[:i])) for i in range(n)]
    host_off = [int(x) for x in rng.integers(0, 300, size=n)]
    plan = batch._build_batch_copy_plan(direction="h2d", sizes=sizes, source_capacities=[400] * n,
                                        destination_capacities=[2000] * n, source_offsets=src_off,
                                        destination_offsets=dst_off, host_registration_offsets=host_off,
                                        pin_chunk_size=pin, destination_keys=[0] * n)
    want = []
    for i in range(n):
        s, d = src_off[i], dst_off[i]
        for piece in bo.split_sizes(sizes[i], host_off[i], pin):
            want.append((i, s, d, piece))
            s, d = s + piece, d + piece
    assert [(e.input_index, e.source_offset, e.destination_offset, e.size) for e in plan.entries] == want


def test_submission_splits_the_plan(monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
    source, destination = torch.arange(16, dtype=torch.uint8), torch.zeros(16, dtype=torch.uint8)
    _fake_kinds(monkeypatch, source, destination)
    rec = _Recorder()
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: rec)
    assert batch.lmcache_musa_memcpy_batch_async([destination], [source], [10], destination_offsets=[2],
                                                 source_offsets=[1], host_registration_offsets=[6], pin_chunk_size=8,
                                                 require_pinned_host=False, prefer_overlap_with_compute=True)
    assert len(rec.calls) == 1
    dsts, srcs, d_off, s_off, sizes, overlap = rec.calls[0]
    assert dsts == [destination, destination] and srcs == [source, source]
    assert d_off == [2, 4] and s_off == [1, 3] and sizes == [2, 8] and overlap is True


def test_submission_chunks_and_fails_closed(monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
    source, destination = torch.arange(10, dtype=torch.uint8), torch.zeros(10, dtype=torch.uint8)
    _fake_kinds(monkeypatch, source, destination)
    rec = _Recorder()
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: rec)
    assert batch.lmcache_musa_memcpy_batch_async([destination] * 5, [source] * 5, [2] * 5,
                                                 destination_offsets=[0, 2, 4, 6, 8], source_offsets=[0, 2, 4, 6, 8],
                                                 require_pinned_host=False, max_batch_entries=2)
    assert [c[4] for c in rec.calls] == [[2, 2], [2, 2], [2]]
    assert all(c[5] is False for c in rec.calls)

    partial = _Recorder(results=lambda k: k == 1)
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: partial)
    with pytest.raises(RuntimeError, match="earlier chunk"):
        batch.lmcache_musa_memcpy_batch_async([destination] * 4, [source] * 4, [1] * 4,
                                              destination_offsets=[0, 1, 2, 3], source_offsets=[0, 1, 2, 3],
                                              require_pinned_host=False, max_batch_entries=2)
    first_fails = _Recorder(results=lambda k: False)
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: first_fails)
    assert batch.lmcache_musa_memcpy_batch_async([destination], [source], [8], require_pinned_host=False) is False

    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: None)
    assert batch.lmcache_musa_memcpy_batch_async([destination], [source], [8], require_pinned_host=False) is False
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: _Recorder(abi=2))
    assert batch.is_native_lmcache_musa_batch_copy_available() is False
    assert batch.lmcache_musa_memcpy_batch_async([destination], [source], [8], require_pinned_host=False) is False


def test_submission_validation(monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
    source, destination = torch.zeros(8, dtype=torch.uint8), torch.zeros(8, dtype=torch.uint8)
    _fake_kinds(monkeypatch, source, destination)
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext",
                        lambda: pytest.fail("invalid batches must not reach the backend"))
    with pytest.raises(ValueError, match="pinned memory"):
        batch.lmcache_musa_memcpy_batch_async([destination], [source], [8])
    with pytest.raises(ValueError, match="destination range"):
        batch.lmcache_musa_memcpy_batch_async([destination], [source], [9], require_pinned_host=False)
    with pytest.raises(ValueError, match="same length"):
        batch.lmcache_musa_memcpy_batch_async([destination], [source, source], [8], require_pinned_host=False)
    with pytest.raises(TypeError, match="torch.Tensor"):
        batch.lmcache_musa_memcpy_batch_async([destination], [b"x"], [8], require_pinned_host=False)
    with pytest.raises(ValueError, match="contiguous"):
        batch.lmcache_musa_memcpy_batch_async([torch.zeros(4, 4).t()], [source], [8], require_pinned_host=False)
    with pytest.raises(ValueError, match="host registration boundary"):
        batch.lmcache_musa_memcpy_batch_async_internal([], [], [], host_registration_offsets=None, pin_chunk_size=8)
    with pytest.raises(ValueError, match="host registration boundary"):
        batch.lmcache_musa_memcpy_batch_async_internal([], [], [], host_registration_offsets=[], pin_chunk_size=None)


def test_cpu_only_batches_are_not_taken(monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: pytest.fail("no GPU endpoint"))
    a, b = torch.zeros(8, dtype=torch.uint8), torch.zeros(8, dtype=torch.uint8)
    assert batch.lmcache_musa_memcpy_batch_async([a], [b], [8], require_pinned_host=False) is False


def test_extension_argument_checks(monkeypatch):
    # The reference extension's prepare_copy (lmcache_musa_batch_copy_ext.cpp:76-170), with the
    # GPU endpoint faked by tensor identity.
    gpu_ids = set()
    monkeypatch.setattr(ext, "_gpu", lambda t: id(t) in gpu_ids)
    e = ext.HipBatchCopyExtension()
    host, dev = torch.zeros(16, dtype=torch.uint8), torch.zeros(16, dtype=torch.uint8)
    dev2 = torch.zeros(16, dtype=torch.uint8)
    gpu_ids.update({id(dev), id(dev2)})
    with pytest.raises(RuntimeError, match="same length"):
        e._prepare([dev], [host, host], [0], [0], [1])
    with pytest.raises(RuntimeError, match="offset vectors"):
        e._prepare([dev], [host], [0, 0], [0], [1])
    with pytest.raises(RuntimeError, match="exactly one GPU endpoint"):
        e._prepare([host], [host], [0], [0], [1])
    with pytest.raises(RuntimeError, match="mix h2d and d2h"):
        e._prepare([dev, host], [host, dev], [0, 0], [0, 0], [1, 1])
    with pytest.raises(RuntimeError, match="destination_offsets\\[0\\] must be non-negative"):
        e._prepare([dev], [host], [-1], [0], [1])
    with pytest.raises(RuntimeError, match="copy_sizes\\[0\\] must be positive"):
        e._prepare([dev], [host], [0], [0], [0])
    with pytest.raises(RuntimeError, match="destination range at index 0"):
        e._prepare([dev], [host], [8], [0], [9])
    with pytest.raises(RuntimeError, match="source range at index 0"):
        e._prepare([dev], [host], [0], [8], [9])
    with pytest.raises(RuntimeError, match="overlapping destination"):
        e._prepare([dev, dev], [host, host], [0, 4], [0, 8], [6, 4])
    dsts, srcs, lens, to_gpu, _, _, _ = e._prepare([dev, dev2], [host, host], [0, 0], [3, 5], [4, 4])
    assert to_gpu and lens == [4, 4] and dsts == [dev.data_ptr(), dev2.data_ptr()]
    assert srcs == [host.data_ptr() + 3, host.data_ptr() + 5]
