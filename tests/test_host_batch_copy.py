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
from musa_aiter.ops.lmcache_musa_batch_copy_plan import plan_columns
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


def _plan_by_entry(sizes, src_cap, dst_cap, src_off, dst_off, host_off, pin, keys):
    """The plan's rules restated one entry at a time (entries in order, rules in order), the overlap
    check as a pairwise scan, and the split from oracle/batch_copy_oracle.split_sizes."""
    for i, (n, so, do, ho, sc, dc) in enumerate(zip(sizes, src_off, dst_off, host_off, src_cap, dst_cap)):
        if n <= 0:
            return f"sizes[{i}] must be positive"
        if min(so, do, ho) < 0:
            return "copy offsets must be non-negative"
        if dc < 0 or do + n > dc:
            return f"destination range at index {i} exceeds tensor capacity"
        if sc < 0 or so + n > sc:
            return f"source range at index {i} exceeds tensor capacity"
    for a in range(len(sizes)):
        for b in range(a + 1, len(sizes)):
            if keys[a] == keys[b] and dst_off[a] < dst_off[b] + sizes[b] and dst_off[b] < dst_off[a] + sizes[a]:
                return "overlapping destination ranges are invalid in an unordered batch"
    out = []
    for i in range(len(sizes)):
        s, d, h = src_off[i], dst_off[i], host_off[i]
        for piece in bo.split_sizes(sizes[i], host_off[i], pin):
            out.append((i, s, d, piece, h))
            s, d, h = s + piece, d + piece, h + piece
    return out


@pytest.mark.parametrize("seed", range(60))
def test_column_plan_matches_per_entry_rules(seed):
    # Larger random batches with planted violations (non-positive sizes, negative offsets, ranges past a
    # capacity, overlaps within one destination) and, for some seeds, offsets near 2**62 that take the
    # one-entry-at-a-time path: same pieces or the same first error as the per-entry restatement.
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(1, 400))
    big = (1 << 62) if seed % 7 == 0 else 0
    sizes = [int(x) for x in rng.integers(1, 5000, size=n)]
    keys = [int(x) for x in rng.integers(0, 4, size=n)]
    dst_off = [0] * n
    cursor = {}
    for i in range(n):  # disjoint ranges per destination unless an overlap is planted below
        dst_off[i] = cursor.get(keys[i], big) + int(rng.integers(0, 3))
        cursor[keys[i]] = dst_off[i] + sizes[i]
    src_off = [int(x) + big for x in rng.integers(0, 1000, size=n)]
    host_off = [int(x) for x in rng.integers(0, 1 << 20, size=n)]
    src_cap = [so + sz + int(rng.integers(0, 10)) for so, sz in zip(src_off, sizes)]
    dst_cap = [do + sz + int(rng.integers(0, 10)) for do, sz in zip(dst_off, sizes)]
    pin = int(rng.integers(1, 9000)) if seed % 3 else None
    kind = seed % 6
    j = int(rng.integers(0, n))
    if kind == 1:
        sizes[j] = -int(rng.integers(0, 3))
    elif kind == 2:
        host_off[j] = -1
    elif kind == 3:
        dst_cap[j] = dst_off[j] + sizes[j] - 1
    elif kind == 4:
        src_cap[j] = -5
    elif kind == 5 and n > 1:
        k = (j + 1) % n
        keys[k], dst_off[k] = keys[j], dst_off[j] + sizes[j] // 2
        dst_cap[k] = max(dst_cap[k], dst_off[k] + sizes[k])
    if seed % 4 == 1:  # host offsets left to default to the source offsets (one column used twice)
        host_off = None
    want = _plan_by_entry(sizes, src_cap, dst_cap, src_off, dst_off, src_off if host_off is None else host_off, pin,
                          keys)
    args = dict(direction="h2d", sizes=sizes, source_capacities=src_cap, destination_capacities=dst_cap,
                source_offsets=src_off, destination_offsets=dst_off, host_registration_offsets=host_off,
                pin_chunk_size=pin, destination_keys=keys)
    if isinstance(want, str):
        with pytest.raises(ValueError) as err:
            batch._build_batch_copy_plan(**args)
        assert str(err.value) == want
    else:
        plan = batch._build_batch_copy_plan(**args)
        got = [(e.input_index, e.source_offset, e.destination_offset, e.size, e.host_registration_offset)
               for e in plan.entries]
        assert got == want
        assert plan.total_bytes == sum(sizes) and plan.input_entry_count == n
        assert all(type(v) is int for e in plan.entries for v in (e.source_offset, e.size))
    # The submission path's form: every column that fits int64 as an int64 array, the keys too.
    as_arrays = {k: (np.array(v, dtype=np.int64) if isinstance(v, list) and all(abs(x) < 1 << 62 for x in v) else v)
                 for k, v in args.items()}
    if isinstance(want, str):
        with pytest.raises(ValueError) as err:
            plan_columns(**as_arrays, int64_arrays=True)
        assert str(err.value) == want
    else:
        c = plan_columns(**as_arrays, int64_arrays=True)
        got = list(zip(c.input_index.tolist(), c.source_offset.tolist(), c.destination_offset.tolist(),
                       c.size.tolist(), c.host_registration_offset.tolist()))
        assert got == want and c.total_bytes == sum(sizes) and type(c.total_bytes) is int
    with pytest.raises(ValueError, match="source_capacities must have the same length"):
        plan_columns(**{**as_arrays, "source_capacities": np.zeros(n + 1, dtype=np.int64)}, int64_arrays=True)
    for name in ("sizes", "source_capacities"):  # arrays only where the submission path asks for them
        with pytest.raises(ValueError, match=f"{name} must contain integers"):
            batch._build_batch_copy_plan(**{**args, name: np.array(args[name], dtype=np.int64)})


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
    # Offsets must be Python ints, as in the reference: not a numpy array, not bools (gate on and off).
    for gate in ("1", "0"):
        monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", gate)
        with pytest.raises(ValueError, match="destination_offsets must contain integers"):
            batch.lmcache_musa_memcpy_batch_async([destination], [source], [8], require_pinned_host=False,
                                                  destination_offsets=np.zeros(1, dtype=np.int64))
        with pytest.raises(ValueError, match="source_offsets must contain integers"):
            batch.lmcache_musa_memcpy_batch_async([destination], [source], [8], require_pinned_host=False,
                                                  source_offsets=[False])
        with pytest.raises(ValueError, match="sizes must contain integers"):
            batch.lmcache_musa_memcpy_batch_async([destination], [source], np.array([8]), require_pinned_host=False)
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
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
    assert to_gpu and lens.tolist() == [4, 4] and dsts.tolist() == [dev.data_ptr(), dev2.data_ptr()]
    assert srcs.tolist() == [host.data_ptr() + 3, host.data_ptr() + 5]


def _prepare_by_entry(dsts, srcs, d_offs, s_offs, sizes, is_gpu):
    """The extension's checks restated one entry at a time (lmcache_musa_batch_copy_ext.cpp:76-170 order):
    the first error message, or the (destination address, source address, size) triples."""
    to_gpu = device = None
    out = []
    for i, (dst, src) in enumerate(zip(dsts, srcs)):
        if not dst.is_contiguous() or not src.is_contiguous():
            return "batch-copy tensors must be contiguous"
        if is_gpu(dst) == is_gpu(src):
            return "each entry must have exactly one GPU endpoint"
        if to_gpu is None:
            to_gpu = is_gpu(dst)
        if is_gpu(dst) != to_gpu:
            return "one batch cannot mix h2d and d2h copies"
        gpu_t, host_t = (dst, src) if to_gpu else (src, dst)
        if host_t.device.type != "cpu":
            return "the non-GPU endpoint must be a CPU tensor"
        if device is None:
            device = gpu_t.device
        if d_offs[i] < 0:
            return f"destination_offsets[{i}] must be non-negative"
        if s_offs[i] < 0:
            return f"source_offsets[{i}] must be non-negative"
        if sizes[i] <= 0:
            return f"copy_sizes[{i}] must be positive"
        if d_offs[i] + sizes[i] > dst.numel() * dst.element_size():
            return f"destination range at index {i} exceeds tensor capacity"
        if s_offs[i] + sizes[i] > src.numel() * src.element_size():
            return f"source range at index {i} exceeds tensor capacity"
        out.append((dst.data_ptr() + d_offs[i], src.data_ptr() + s_offs[i], sizes[i]))
    spans = sorted((d, d + n) for d, _, n in out)
    if any(b[0] < a[1] for a, b in zip(spans, spans[1:])):
        return "overlapping destination ranges are invalid in an unordered batch"
    return out


@pytest.mark.parametrize("seed", range(40))
def test_extension_column_checks_match_per_entry_checks(monkeypatch, seed):
    # Groups of up to 300 entries over a few host and (faked) GPU tensors with one planted fault each;
    # the column-wise checks must raise the per-entry restatement's first error or return its triples.
    gpu_ids = set()
    monkeypatch.setattr(ext, "_gpu", lambda t: id(t) in gpu_ids)
    rng = np.random.default_rng(2000 + seed)
    hosts = [torch.zeros(int(rng.integers(1, 64)) * 64, dtype=torch.uint8) for _ in range(3)]
    gpus = [torch.zeros(int(rng.integers(1, 64)) * 64, dtype=torch.uint8) for _ in range(3)]
    gpu_ids.update(id(t) for t in gpus)
    n = int(rng.integers(1, 300))
    h2d = bool(seed % 2)
    dsts, srcs, d_offs, s_offs, sizes, cursor = [], [], [], [], [], {}
    for _ in range(n):
        g, h = gpus[int(rng.integers(0, 3))], hosts[int(rng.integers(0, 3))]
        dst, src = (g, h) if h2d else (h, g)
        size = int(rng.integers(1, 8))
        d_off = cursor.get(id(dst), 0)
        cursor[id(dst)] = d_off + size
        dsts.append(dst)
        srcs.append(src)
        d_offs.append(d_off)
        s_offs.append(int(rng.integers(0, max(1, src.numel() - size))))
        sizes.append(size)
    j = int(rng.integers(0, n))
    fault = seed % 8
    if fault == 1:
        dsts[j] = torch.zeros(4, 4, dtype=torch.uint8).t()
    elif fault == 2:
        srcs[j] = dsts[j]
    elif fault == 3:
        dsts[j], srcs[j] = srcs[j], dsts[j]
    elif fault == 4:
        d_offs[j] = -1
    elif fault == 5:
        sizes[j] = 0
    elif fault == 6:
        s_offs[j] = srcs[j].numel()
    elif fault == 7 and n > 1:
        k = (j + 1) % n
        dsts[k], d_offs[k] = dsts[j], d_offs[j]
    want = _prepare_by_entry(dsts, srcs, d_offs, s_offs, sizes, ext._gpu)
    if isinstance(want, str):
        with pytest.raises(RuntimeError) as err:
            ext.HipBatchCopyExtension._prepare(dsts, srcs, d_offs, s_offs, sizes)
        assert str(err.value) == want
        return
    got_d, got_s, got_n, to_gpu, _, gpu_t, host_t = ext.HipBatchCopyExtension._prepare(dsts, srcs, d_offs, s_offs,
                                                                                        sizes)
    assert list(zip(got_d.tolist(), got_s.tolist(), got_n.tolist())) == want
    assert to_gpu == h2d
    assert {id(t) for t in gpu_t} == {id(t) for t in (*dsts, *srcs) if id(t) in gpu_ids}
    assert {id(t) for t in host_t} == {id(t) for t in (*dsts, *srcs) if id(t) not in gpu_ids}


def _distinct(dsts, srcs):
    both = (*dsts, *srcs)
    _, first, which = np.unique(np.array([id(t) for t in both], dtype=np.uint64), return_index=True,
                                return_inverse=True)
    return [both[i] for i in first], which[:len(dsts)], which[len(dsts):]


@pytest.mark.parametrize("seed", range(24))
def test_column_submission_matches_list_submission(monkeypatch, seed):
    # The public call hands this package's extension its plan as columns (execute_batch_copy_columns);
    # any other extension object gets the reference's lists.  Both must submit the same
    # (destination address, source address, size) groups, or raise the same first error.
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
    rng = np.random.default_rng(3000 + seed)
    h2d = bool(seed % 2)
    hosts = [torch.zeros(int(rng.integers(8, 64)) * 64, dtype=torch.uint8) for _ in range(3)]
    gpus = [torch.zeros(int(rng.integers(8, 64)) * 64, dtype=torch.uint8) for _ in range(3)]
    gpu_ids = {id(t) for t in gpus}
    monkeypatch.setattr(ext, "_gpu", lambda t: id(t) in gpu_ids)
    monkeypatch.setattr(batch, "_tensor_device_kind", lambda t: "gpu" if id(t) in gpu_ids else "cpu")
    n = int(rng.integers(1, 200))
    dsts, srcs, d_offs, s_offs, sizes, cursor = [], [], [], [], [], {}
    for _ in range(n):
        g, h = gpus[int(rng.integers(0, 3))], hosts[int(rng.integers(0, 3))]
        dst, src = (g, h) if h2d else (h, g)
        size = int(rng.integers(1, 40))
        d_off = cursor.get(id(dst), 0)
        if d_off + size > dst.numel():
            continue
        cursor[id(dst)] = d_off + size
        dsts.append(dst)
        srcs.append(src)
        d_offs.append(d_off)
        s_offs.append(int(rng.integers(0, src.numel() - size + 1)))
        sizes.append(size)
    pin = [None, 16, 24][seed % 3]
    limit = int(rng.integers(1, 64))
    if seed % 4 == 3 and len(dsts) > 1:  # the GPU side of one entry on a second (fake) device
        other = torch.zeros(64, dtype=torch.uint8, device="meta")
        monkeypatch.setattr(batch, "_tensor_device_kind", lambda t: "gpu" if id(t) in gpu_ids else "cpu")
        gpu_ids.add(id(other))
        j = int(rng.integers(0, len(dsts)))
        if h2d:
            dsts[j], d_offs[j] = other, 0
        else:
            srcs[j], s_offs[j] = other, 0
        sizes[j] = min(sizes[j], 64)

    class Lists(_Recorder):
        def execute_batch_copy(self, d, s, do, so, sz, overlap):
            dd, ss, nn, to_gpu, _, _, _ = ext.HipBatchCopyExtension._prepare(d, s, do, so, sz)
            self.calls.append((dd.tolist(), ss.tolist(), nn.tolist(), to_gpu))
            return True

    launched = []
    monkeypatch.setattr(ext.HipBatchCopyExtension, "_launch",
                        lambda self, p, mode: launched.append((p[0].tolist(), p[1].tolist(), p[2].tolist(), p[3]))
                        or True)

    def run(extension):
        monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: extension)
        try:
            return batch.lmcache_musa_memcpy_batch_async(
                dsts, srcs, sizes, destination_offsets=d_offs, source_offsets=s_offs, require_pinned_host=False,
                host_registration_offsets=None, pin_chunk_size=pin, max_batch_entries=limit)
        except (RuntimeError, ValueError) as exc:
            return type(exc), str(exc)

    lists = Lists()
    want = run(lists)
    got = run(ext.HipBatchCopyExtension())
    assert got == want
    assert launched == lists.calls
    assert want is not True or sum(len(c[2]) for c in launched) >= len(sizes)


def test_host_helper_reads_plain_int_lists_only():
    # The helper that reads the caller's lists into int64 columns takes lists and tuples of plain ints
    # within (-2^61, 2^61) and declines everything else, which the plan then checks item by item.
    from musa_aiter.ops import _hip
    column = _hip.host().int64_column
    values = [0, -5, 7, (1 << 61) - 1, -(1 << 61) + 1]
    assert np.frombuffer(column(values), dtype=np.int64).tolist() == values
    assert np.frombuffer(column(tuple(values)), dtype=np.int64).tolist() == values
    assert column([]) == b""

    class Sub(int):
        pass

    for declined in ([1 << 61], [-(1 << 61)], [1 << 70], [True], [np.int64(1)], [Sub(3)], [1, 2.0], range(3),
                     np.arange(3)):
        assert column(declined) is None, declined


def test_host_helper_numbers_distinct_objects_by_identity():
    # Entries' objects numbered by identity in order of first appearance, destinations then sources;
    # equal but distinct objects get their own numbers.
    from musa_aiter.ops import _hip
    index = _hip.host().object_index
    a, b, c = torch.zeros(4), torch.zeros(4), torch.ones(2)
    packed, distinct = index([b, a, b, b], (c, a, c, b))
    assert np.frombuffer(packed, dtype=np.int64).tolist() == [0, 1, 0, 0, 2, 1, 2, 0]
    assert [id(t) for t in distinct] == [id(b), id(a), id(c)]
    packed, distinct = index([], [])
    assert packed == b"" and distinct == []
    with pytest.raises(TypeError):
        index(iter([a]), [a])


def test_missing_host_helper_falls_back_to_false(monkeypatch, tmp_path):
    # With the backend requested but neither the host helper module nor the extension loadable, the
    # call returns False (the caller keeps its own transfer path) instead of raising.
    from musa_aiter.ops import _hip

    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")
    monkeypatch.setattr(_hip, "HOST_PATH", tmp_path / "missing_kv_host.so")
    monkeypatch.setattr(_hip, "_host", None)
    monkeypatch.setattr(batch, "load_lmcache_musa_batch_copy_ext", lambda: None)
    source, destination = torch.arange(10, dtype=torch.uint8), torch.zeros(10, dtype=torch.uint8)
    _fake_kinds(monkeypatch, source, destination)
    assert batch.lmcache_musa_memcpy_batch_async([destination], [source], [8], require_pinned_host=False) is False
