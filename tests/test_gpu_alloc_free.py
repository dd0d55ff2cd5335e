"""The Python host layer makes the HIP library allocate no memory of its own.

The reference's shims hand their kernels only caller-owned tensors
(musa_aiter/ops/kv_transfer.py:380-437).  Scatters here need last-writer claim
tags; the host layer passes a tensor from torch's caching allocator for them
(musa_aiter_hip_claims), so ``musa_aiter_hip_allocated_bytes`` -- the device and
pinned host bytes the library itself has allocated -- must not move across any
public scatter, whatever other tests ran before in the process.  Each case also
checks its result, with repeated slots so that the claims decide the outcome.
"""

from __future__ import annotations

import ctypes
import gc

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops import _hip
from musa_aiter.ops.lmcache_kv_transfer_ext import HipLMCacheKVTransferExtension
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _repeated_slots(rng, slots: int, t: int) -> torch.Tensor:
    s = rng.integers(0, max(2, slots // 4), size=t)
    s[rng.random(t) < 0.1] = -1
    s[-1] = s[0]
    return torch.from_numpy(s.astype(np.int64)).to(DEV)


def _last_writer(t: int, s: np.ndarray) -> dict[int, int]:
    win = {}
    for i, v in enumerate(s.tolist()):
        if v >= 0:
            win[v] = i
    return win


def test_public_scatters_allocate_nothing_in_the_library():
    rng = np.random.default_rng(5)
    gen = torch.Generator().manual_seed(5)
    nl, nb, bs, nh, hd, t = 2, 24, 16, 4, 64, 300
    torch.cuda.synchronize()
    before = _hip.allocated_bytes()

    # paged-A multi-layer scatter, single layer, merged, MLA split, FP8 quant-store
    kl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
    vl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
    kc = torch.zeros((nl, nb, nh, hd, bs), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    slots = _repeated_slots(rng, nb * bs, t)
    musa_aiter.kv_linear_to_paged_multi_layer(kl, vl, kc, vc, slots)
    musa_aiter.kv_linear_to_paged(kl[0], vl[0], kc[1], vc[1], slots)
    musa_aiter.kv_merged_linear_to_paged(torch.stack([kl[0], vl[0]], 1).contiguous(), kc[0], vc[0], slots)
    kv = random_payload((t, 96), torch.bfloat16, gen).to(DEV)
    pe = random_payload((t, 32), torch.bfloat16, gen).to(DEV)
    kvc = torch.zeros((nb, bs, 96), dtype=torch.bfloat16, device=DEV)
    pec = torch.zeros((nb, bs, 32), dtype=torch.bfloat16, device=DEV)
    musa_aiter.kv_mla_linear_to_paged(kv, pe, kvc, pec, slots)
    k8 = torch.zeros((nb, nh, hd, bs), dtype=torch.uint8, device=DEV)
    v8 = torch.zeros_like(k8)
    musa_aiter.kv_linear_to_paged_fp8(kl[0], vl[0], k8, v8, slots, 0.05, 0.05)

    # LMCache 2 x NL, MLA rows, the extension object's scatters
    caches = [[torch.zeros((nb, bs, nh, hd), dtype=torch.bfloat16, device=DEV) for _ in range(nl)]
              for _ in range(2)]
    mem = random_payload((2, nl, t, nh * hd), torch.bfloat16, gen).to(DEV)
    assert musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(mem, caches, slots, 0, bs, nh, hd)
    mla = torch.zeros((nl, nb, bs, 96), dtype=torch.bfloat16, device=DEV)
    assert musa_aiter.lmcache_kv_buffer_to_paged_mla(random_payload((nl, t, 96), torch.bfloat16, gen).to(DEV),
                                                     mla, slots)
    ext = HipLMCacheKVTransferExtension()
    ext_caches = [[torch.zeros((nb, bs, nh, hd), dtype=torch.bfloat16, device=DEV) for _ in range(nl)]
                  for _ in range(2)]
    assert ext.kv_buffer_to_paged_two_x_nl(mem, ext_caches, slots, 0, bs, nh, hd)
    list_caches = [torch.zeros((2, nb, bs, nh, hd), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    assert ext.kv_buffer_to_paged_list2(mem, list_caches, slots, 0, bs, nh, hd)

    # block-table write-back, whole-block copies, byte rows, HiCache direct
    batch, dense = 3, 40
    tables = torch.from_numpy(rng.integers(0, nb, size=(batch, 3))).to(DEV)  # blocks shared across rows
    seq_lens = torch.tensor([40, 17, 33], device=DEV)
    dk = random_payload((batch, dense, nh, hd), torch.bfloat16, gen).to(DEV)
    musa_aiter.kv_reshape_and_cache_back_flash(dk, dk, kc[0], vc[0], tables, seq_lens)
    pairs = torch.tensor([[0, 5], [1, 5], [2, 6]], device=DEV)
    musa_aiter.kv_copy_paged_blocks(kc[0], vc[0], kc[0], vc[0], pairs)
    rows_src = torch.randint(0, 256, (64, 656), dtype=torch.uint8, device=DEV)
    rows_dst = torch.zeros((32, 656), dtype=torch.uint8, device=DEV)
    musa_aiter.kv_copy_paged_rows(rows_src, rows_dst, torch.arange(20, device=DEV),
                                  torch.tensor([3, 3, 4] + list(range(5, 22)), device=DEV))
    src_pool = [random_payload((64, 128), torch.bfloat16, gen).to(DEV) for _ in range(2)]
    dst_pool = [torch.zeros((64, 128), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    assert musa_aiter.hicache_transfer_kv_direct(src_pool, dst_pool, torch.arange(8, device=DEV),
                                                 torch.tensor([4, 5, 6, 7, 0, 1, 2, 3], device=DEV), 4)
    torch.cuda.synchronize()
    assert _hip.allocated_bytes() == before

    # Spot checks that the claims decided the repeated slots: last writer in token order (layer 1
    # of the paged caches was last written by the single-layer scatter of kl[0]).
    win = _last_writer(t, slots.cpu().numpy())
    keys = torch.tensor(list(win.keys()), device=DEV)
    toks = torch.tensor(list(win.values()), device=DEV)
    flat = kc[1].permute(0, 3, 1, 2).reshape(nb * bs, nh * hd)
    assert np.array_equal(bits(flat[keys]), bits(kl[0].reshape(t, nh * hd)[toks]))
    for a in range(2):
        for layer in range(nl):
            got = ext_caches[a][layer].reshape(nb * bs, nh * hd)
            assert np.array_equal(bits(got[keys]), bits(mem[a, layer][toks])), (a, layer)
            assert np.array_equal(bits(got), bits(caches[a][layer].reshape(nb * bs, nh * hd))), (a, layer)
            lc = list_caches[layer][a].reshape(nb * bs, nh * hd)
            assert np.array_equal(bits(lc[keys]), bits(mem[a, layer][toks])), (a, layer)


def test_config2_shape_scatter_allocates_nothing_in_the_library():
    # configs[1]'s shape through the public API: 32 layers of [8192, 8, 128, 16] bf16 caches.
    from tests.kvgen import sequence_lengths, sequence_slots

    nl, nb, bs, nh, hd = 32, 8192, 16, 8, 128
    rng = np.random.default_rng(1002)
    lengths = sequence_lengths(rng, 64, 128, 4096, num_blocks=nb, block_size=bs)
    slots_np = sequence_slots(rng, lengths, num_blocks=nb, block_size=bs)
    t = int(slots_np.shape[0])
    print(f"configs[1] shape through the public API: {t} tokens x {nl} layers", flush=True)
    slots = torch.from_numpy(slots_np).to(DEV)
    kl = torch.randn((nl, t, nh, hd), device=DEV, dtype=torch.bfloat16)
    vl = torch.randn((nl, t, nh, hd), device=DEV, dtype=torch.bfloat16)
    kc = torch.empty((nl, nb, nh, hd, bs), device=DEV, dtype=torch.bfloat16)
    vc = torch.empty_like(kc)
    torch.cuda.synchronize()
    before = _hip.allocated_bytes()
    for _ in range(3):
        musa_aiter.kv_linear_to_paged_multi_layer(kl, vl, kc, vc, slots)
    ok, ov = musa_aiter.kv_paged_to_linear_multi_layer(kc, vc, slots)
    torch.cuda.synchronize()
    assert _hip.allocated_bytes() == before
    assert torch.equal(ok.view(torch.int16), kl.view(torch.int16))
    assert torch.equal(ov.view(torch.int16), vl.view(torch.int16))
    del kl, vl, kc, vc, ok, ov
    gc.collect()
    torch.cuda.empty_cache()


def test_claim_arrays_of_destroyed_graphs_are_reused():
    # A scatter captured through a reference-named C entry takes a claim array from the library;
    # destroying its graph returns the array, so capturing and destroying graphs in a loop keeps
    # the number of arrays the library holds for graphs bounded.
    nl, nb, bs, nh, hs, t = 2, 16, 16, 2, 64, 96
    rng = np.random.default_rng(19)
    gen = torch.Generator().manual_seed(19)
    entry = getattr(_hip.library(), "lmcache_kv_buffer_to_paged_two_x_nl_coalesced_u16")
    entry.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64), ctypes.c_void_p] + [ctypes.c_int64] * 8 + \
        [ctypes.c_void_p]
    entry.restype = ctypes.c_int
    count = _hip.fn("musa_aiter_hip_graph_claim_arrays")
    held = []
    for rep in range(8):
        caches = [[torch.zeros((nb, bs, nh, hs), dtype=torch.bfloat16, device=DEV) for _ in range(nl)]
                  for _ in range(2)]
        ptrs = _hip.u64_array([c.data_ptr() for grp in caches for c in grp])
        mem = random_payload((2, nl, t, nh * hs), torch.bfloat16, gen).to(DEV)
        slots = torch.from_numpy(rng.integers(0, nb * bs // 8, size=t)).to(DEV)  # many repeats

        def call():
            rc = entry(mem.data_ptr(), ptrs, slots.data_ptr(), nl, t, t, 0, nb, bs, nh, hs,
                       torch.cuda.current_stream().cuda_stream)
            assert rc == 0

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            call()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        want = [[c.clone() for c in grp] for grp in caches]
        for grp in caches:
            for c in grp:
                c.zero_()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
        g.replay()
        torch.cuda.synchronize()
        for a in range(2):
            for layer in range(nl):
                assert np.array_equal(bits(caches[a][layer]), bits(want[a][layer])), (rep, a, layer)
        held.append(int(count()))
        del g
        gc.collect()
        torch.cuda.synchronize()
    print(f"claim arrays held for graphs after each capture: {held}", flush=True)
    assert held[-1] - held[0] <= 1
