"""GPU parity: LMCache host/device copy batches vs oracle/batch_copy_oracle.py, bit-exact.

Restates the reference's native tests (op_tests/test_lmcache_musa_batch_copy_musa.py:21-160) on
ROCm and adds random batches through every submission path (the batch-copy kernel over pinned
host memory on its normal and its bounded grid, one hipMemcpyAsync per range), pageable host
memory, every relative alignment of source and destination, ranges crossing the kernel's 64 KiB
tiles, more ranges than the kernel arguments hold (one launch over per-tile descriptors in a ring of
pinned buffers, with batches queued back to back), and the C-ABI entry called directly.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops import _hip
from oracle import batch_copy_oracle as bo

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _requested(monkeypatch):
    monkeypatch.setenv("MUSA_AITER_LMCACHE_BATCH_COPY", "1")


def _host(n, *, pinned=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g)
    return t.pin_memory() if pinned else t


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
def test_reference_round_trip(direction):
    host = torch.arange(256, dtype=torch.uint8).pin_memory()
    device = torch.zeros(256, dtype=torch.uint8, device=DEV)
    if direction == "h2d":
        dsts, srcs = [device], [host]
    else:
        device.copy_(host)
        torch.cuda.synchronize()
        host.zero_()
        dsts, srcs = [host], [device]
    assert musa_aiter.lmcache_musa_memcpy_batch_async(dsts, srcs, [96], destination_offsets=[64], source_offsets=[32])
    torch.cuda.synchronize()
    if direction == "h2d":
        assert torch.equal(device[64:160].cpu(), host[32:128])
        assert not device[:64].any() and not device[160:].any()
    else:
        assert torch.equal(host[64:160], torch.arange(32, 128, dtype=torch.uint8))


def test_reference_current_non_default_stream():
    host = torch.arange(128, dtype=torch.uint8).pin_memory()
    device = torch.zeros(128, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        assert musa_aiter.lmcache_musa_memcpy_batch_async([device], [host], [128])
        device.add_(1)
    stream.synchronize()
    assert torch.equal(device.cpu(), host + 1)


def test_reference_observes_non_default_stream_producer():
    host = torch.zeros(128, dtype=torch.uint8).pin_memory()
    device = torch.zeros(128, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        device.fill_(37)
        assert musa_aiter.lmcache_musa_memcpy_batch_async([host], [device], [128])
    stream.synchronize()
    assert torch.equal(host, torch.full_like(host, 37))


def test_reference_split_at_host_registration_boundary():
    host = torch.arange(64, dtype=torch.uint8).pin_memory()
    device = torch.zeros(64, dtype=torch.uint8, device=DEV)
    assert musa_aiter.lmcache_musa_memcpy_batch_async([device], [host], [20], destination_offsets=[10],
                                                      source_offsets=[6], host_registration_offsets=[6],
                                                      pin_chunk_size=8)
    torch.cuda.synchronize()
    assert torch.equal(device[10:30].cpu(), host[6:26])


def test_reference_chunks_large_entry_tables_in_stream_order():
    versions = musa_aiter.native_lmcache_musa_batch_copy_runtime_versions()
    assert versions is not None and versions[0] > 0 and versions[1] > 0
    count = 1300
    host = (torch.arange(count) % 251).to(torch.uint8).pin_memory()
    device = torch.zeros(count, dtype=torch.uint8, device=DEV)
    offsets = list(range(count))
    assert musa_aiter.lmcache_musa_memcpy_batch_async([device] * count, [host] * count, [1] * count,
                                                      destination_offsets=offsets, source_offsets=offsets,
                                                      max_batch_entries=512)
    torch.cuda.synchronize()
    assert torch.equal(device.cpu(), host)


def _random_batch(rng, count, max_size, host_bytes, dev_bytes):
    """Disjoint destination ranges (sorted slots, shuffled order) with random source offsets."""
    sizes = [int(x) for x in rng.integers(1, max_size + 1, size=count)]
    slot = max(sizes) + 17
    order = rng.permutation(count)
    dst_off = [int(order[i] * slot + rng.integers(0, 17)) for i in range(count)]
    src_off = [int(rng.integers(0, host_bytes - s)) for s in sizes]
    assert max(d + s for d, s in zip(dst_off, sizes)) <= dev_bytes
    return sizes, dst_off, src_off


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
@pytest.mark.parametrize("pinned,overlap", [(True, False), (True, True), (False, False)])
@pytest.mark.parametrize("max_size", [40, 3000, 200_000])
def test_random_batches_match_oracle(direction, pinned, overlap, max_size):
    rng = np.random.default_rng(max_size + 3 * int(pinned) + int(overlap) + (7 if direction == "d2h" else 0))
    count = 150  # more than one kernel launch holds
    other = max_size + 64
    gpu_bytes = count * (max_size + 40)
    sizes, dst_off, src_off = _random_batch(rng, count, max_size, other, gpu_bytes)
    host_a = _host(other, pinned=pinned, seed=1)           # the side the copies read (h2d) ...
    gpu = torch.randint(0, 256, (gpu_bytes,), dtype=torch.uint8, device=DEV)
    if direction == "h2d":
        dsts, srcs = [gpu] * count, [host_a] * count
        want = [gpu.cpu().numpy().copy()]
        src_np = [host_a.numpy()]
    else:
        # d2h: the device holds the source bytes, the host buffer receives them.
        src_dev = torch.randint(0, 256, (other,), dtype=torch.uint8, device=DEV)
        host_b = _host(gpu_bytes, pinned=pinned, seed=2)
        dsts, srcs = [host_b] * count, [src_dev] * count
        want = [host_b.numpy().copy()]
        src_np = [src_dev.cpu().numpy()]
    torch.cuda.synchronize()
    assert musa_aiter.lmcache_musa_memcpy_batch_async(dsts, srcs, sizes, destination_offsets=dst_off,
                                                      source_offsets=src_off, require_pinned_host=pinned,
                                                      prefer_overlap_with_compute=overlap)
    torch.cuda.synchronize()
    bo.apply_batch(want * count, src_np * count, sizes, dst_off, src_off)
    got = gpu.cpu().numpy() if direction == "h2d" else host_b.numpy()
    assert np.array_equal(got, want[0])


@pytest.mark.parametrize("rel", range(16))
def test_every_relative_alignment(rel):
    # Source offset rel .. 15 bytes past 16-byte alignment, destination at 5: vector widths 1..16.
    host = _host(1 << 20, seed=rel)
    device = torch.zeros(1 << 20, dtype=torch.uint8, device=DEV)
    size = 200_000 + rel
    assert musa_aiter.lmcache_musa_memcpy_batch_async([device], [host], [size], destination_offsets=[5 + 16],
                                                      source_offsets=[(5 + rel) % 16 + 32])
    torch.cuda.synchronize()
    s = (5 + rel) % 16 + 32
    assert torch.equal(device[21:21 + size].cpu(), host[s:s + size])
    assert not device[:21].any() and not device[21 + size:].any()


def test_c_abi_batch_copy_direct_call():
    host = _host(1 << 16, seed=9)
    device = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    dsts = (ctypes.c_void_p * 3)(device.data_ptr(), device.data_ptr() + 4096, device.data_ptr() + 40_000)
    srcs = (ctypes.c_void_p * 3)(host.data_ptr() + 7, host.data_ptr(), host.data_ptr() + 1000)
    sizes = (ctypes.c_uint64 * 3)(4000, 30_000, 0)
    rc = _hip.fn("musa_aiter_hip_batch_copy")(dsts, srcs, sizes, 3, 0, 0, _hip.stream_ptr(torch.device(DEV)))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(device[:4000].cpu(), host[7:4007])
    assert torch.equal(device[4096:34096].cpu(), host[:30000])
    assert not device[34096:].any()
    assert _hip.fn("musa_aiter_hip_batch_copy")(dsts, srcs, sizes, 3, 2, 0, None) != 0
    assert _hip.fn("musa_aiter_hip_batch_copy")(dsts, srcs, sizes, 3, 0, 3, None) != 0
    assert _hip.fn("musa_aiter_hip_batch_copy_abi_version")() == 1


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
def test_copy_loop_and_bounded_grid_paths(direction):
    from musa_aiter.ops import lmcache_musa_batch_copy_ext as ext

    extension = ext.load_lmcache_musa_batch_copy_ext()
    rng = np.random.default_rng(5)
    count, other = 40, 300_000
    sizes, dst_off, src_off = _random_batch(rng, count, 200_000, other, count * 200_040)
    for run in (lambda *a: extension.execute_copy_loop(*a), lambda *a: extension.execute_batch_copy(*a, True)):
        if direction == "h2d":
            src = _host(other, seed=6)
            dst = torch.zeros(count * 200_040, dtype=torch.uint8, device=DEV)
            src_np = src.numpy()
        else:
            src = torch.randint(0, 256, (other,), dtype=torch.uint8, device=DEV)
            dst = _host(count * 200_040, seed=7)
            src_np = src.cpu().numpy()
        want = (dst.cpu().numpy() if direction == "h2d" else dst.numpy()).copy()
        torch.cuda.synchronize()
        assert run([dst] * count, [src] * count, dst_off, src_off, sizes)
        torch.cuda.synchronize()
        bo.apply_batch([want] * count, [src_np] * count, sizes, dst_off, src_off)
        got = dst.cpu().numpy() if direction == "h2d" else dst.numpy()
        assert np.array_equal(got, want)


def test_tensors_stay_alive_until_the_stream_passes():
    from musa_aiter.ops import lmcache_musa_batch_copy_ext as ext

    extension = ext.load_lmcache_musa_batch_copy_ext()
    host = _host(1 << 22, seed=4)
    device = torch.zeros(1 << 22, dtype=torch.uint8, device=DEV)
    assert musa_aiter.lmcache_musa_memcpy_batch_async([device], [host], [1 << 22])
    torch.cuda.synchronize()
    assert len(extension.in_flight) == 0
    assert torch.equal(device.cpu(), host)


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
def test_queued_large_batches_reuse_descriptor_slots(direction):
    # Batches of more than 96 ranges run as one launch over per-tile descriptors in a ring of pinned
    # buffers; twelve batches queued without a sync cycle the ring three times, each with its own data.
    rng = np.random.default_rng(21 if direction == "h2d" else 22)
    calls, count, size = 12, 200, 4096 + 24
    dev = torch.zeros(calls * count * size, dtype=torch.uint8, device=DEV)
    hosts = [_host(count * size, seed=100 + c) for c in range(calls)]
    if direction == "d2h":
        dev.copy_(torch.randint(0, 256, dev.shape, dtype=torch.uint8, device=DEV))
        hosts = [torch.zeros(count * size, dtype=torch.uint8).pin_memory() for _ in range(calls)]
    torch.cuda.synchronize()
    perms = [rng.permutation(count) for _ in range(calls)]
    for c in range(calls):
        dev_off = [int(c * count * size + p * size) for p in perms[c]]
        host_off = [i * size for i in range(count)]
        if direction == "h2d":
            ok = musa_aiter.lmcache_musa_memcpy_batch_async([dev] * count, [hosts[c]] * count, [size] * count,
                                                            destination_offsets=dev_off, source_offsets=host_off)
        else:
            ok = musa_aiter.lmcache_musa_memcpy_batch_async([hosts[c]] * count, [dev] * count, [size] * count,
                                                            destination_offsets=host_off, source_offsets=dev_off)
        assert ok
    torch.cuda.synchronize()
    got_dev = dev.cpu().numpy()
    for c in range(calls):
        h = hosts[c].numpy()
        for i, p in enumerate(perms[c]):
            d0 = c * count * size + p * size
            assert np.array_equal(got_dev[d0:d0 + size], h[i * size:(i + 1) * size]), (c, i)


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
def test_batch_alternating_between_host_allocations(direction):
    # One batch whose host side alternates between two pinned buffers and a pageable one: the
    # library's cached pinned range must switch allocations, and pageable ranges keep hipMemcpyAsync.
    rng = np.random.default_rng(31 if direction == "h2d" else 32)
    count, size = 240, 3000
    hosts = [_host(count * size, seed=40), _host(count * size, seed=41), _host(count * size, pinned=False, seed=42)]
    dev = torch.randint(0, 256, (count * (size + 16),), dtype=torch.uint8, device=DEV)
    which = rng.integers(0, 3, size=count)
    host_off = [int(i * size) for i in range(count)]
    dev_off = [int(p * (size + 16) + 3) for p in rng.permutation(count)]
    if direction == "d2h":
        for h in hosts:
            h.zero_()
    want_dev = dev.cpu().numpy().copy()
    want_hosts = [h.numpy().copy() for h in hosts]
    torch.cuda.synchronize()
    for i in range(count):
        h = want_hosts[which[i]]
        if direction == "h2d":
            want_dev[dev_off[i]:dev_off[i] + size] = h[host_off[i]:host_off[i] + size]
        else:
            h[host_off[i]:host_off[i] + size] = want_dev[dev_off[i]:dev_off[i] + size]
    picked = [hosts[k] for k in which]
    if direction == "h2d":
        ok = musa_aiter.lmcache_musa_memcpy_batch_async([dev] * count, picked, [size] * count,
                                                        destination_offsets=dev_off, source_offsets=host_off,
                                                        require_pinned_host=False)
    else:
        ok = musa_aiter.lmcache_musa_memcpy_batch_async(picked, [dev] * count, [size] * count,
                                                        destination_offsets=host_off, source_offsets=dev_off,
                                                        require_pinned_host=False)
    assert ok
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy(), want_dev)
    for h, w in zip(hosts, want_hosts):
        assert np.array_equal(h.numpy(), w)


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
@pytest.mark.parametrize("pin,limit", [(None, 37), (4096, 64), (1000, 1 << 20)])
def test_many_tensors_in_groups_match_oracle(direction, pin, limit):
    # Entries spread over three device and three pinned host tensors, cut at registration boundaries
    # and sent in groups of `limit` pieces: the public call hands each group to the extension as
    # columns over the batch's distinct tensors.
    rng = np.random.default_rng(500 + (pin or 0) + limit + (1 if direction == "d2h" else 0))
    devs = [torch.randint(0, 256, (int(n),), dtype=torch.uint8, device=DEV) for n in rng.integers(40_000, 90_000, 3)]
    hosts = [_host(int(n), seed=int(k)) for k, n in enumerate(rng.integers(40_000, 90_000, 3))]
    dst_side, src_side = (devs, hosts) if direction == "h2d" else (hosts, devs)
    before = [t.cpu().numpy().copy() for t in dst_side]
    srcs_np = [t.cpu().numpy() for t in src_side]
    dsts, srcs, sizes, d_off, s_off = [], [], [], [], []
    cursor = [0] * 3
    while len(sizes) < 300:
        i, j = int(rng.integers(0, 3)), int(rng.integers(0, 3))
        size = int(rng.integers(1, 3000))
        if cursor[i] + size > dst_side[i].numel():
            break
        dsts.append(dst_side[i])
        srcs.append(src_side[j])
        d_off.append(cursor[i])
        s_off.append(int(rng.integers(0, src_side[j].numel() - size + 1)))
        sizes.append(size)
        cursor[i] += size + int(rng.integers(0, 64))
    order = rng.permutation(len(sizes))  # the batch is unordered
    pick = lambda xs: [xs[k] for k in order]
    dsts, srcs, sizes, d_off, s_off = pick(dsts), pick(srcs), pick(sizes), pick(d_off), pick(s_off)
    host_off = s_off if direction == "h2d" else d_off
    torch.cuda.synchronize()
    assert musa_aiter.lmcache_musa_memcpy_batch_async(dsts, srcs, sizes, destination_offsets=d_off,
                                                      source_offsets=s_off, host_registration_offsets=host_off,
                                                      pin_chunk_size=pin, max_batch_entries=limit)
    torch.cuda.synchronize()
    index = {id(t): k for k, t in enumerate(dst_side)}
    sindex = {id(t): k for k, t in enumerate(src_side)}
    bo.apply_batch([before[index[id(t)]] for t in dsts], [srcs_np[sindex[id(t)]] for t in srcs], sizes, d_off, s_off)
    for got, want in zip(dst_side, before):
        assert np.array_equal(got.cpu().numpy(), want)
