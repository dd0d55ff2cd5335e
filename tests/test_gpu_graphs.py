"""HIP graph capture of the entry points that never synchronise with the host.

kv_cachegen_encode, kv_cachegen_decode (256-entry codebook), the LMCache 2 x NL gather and scatter
and kv_triton_indexed_to_dense launch only kernels on the current stream (no host reads, no
memsets), so a caller can capture them in a graph.  A captured scatter whose slots may repeat
clears and re-claims its slots on every replay instead of relying on the eager path's per-call
epoch, which a replay would repeat.  Each case is captured once and replayed several times with
new inputs copied into the captured tensors and eager calls in between; every replay must equal
the eager result of the same inputs bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from musa_aiter.ops.kv_transfer import kv_triton_indexed_to_dense
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(fn):
    """Warm up on a side stream, then capture ``fn`` into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def test_cachegen_encode_decode_replays():
    x = torch.randn(1 << 20, device=DEV)
    g, (enc, book, cdf) = _capture(lambda: musa_aiter.kv_cachegen_encode(x, num_bins=256))
    gd, dec = _capture(lambda: musa_aiter.kv_cachegen_decode(enc, book))
    for rep in range(4):
        x.copy_(torch.randn(1 << 20, device=DEV) * (rep + 1) + rep)
        torch.cuda.synchronize()
        g.replay()
        gd.replay()
        torch.cuda.synchronize()
        e_ref, b_ref, c_ref = musa_aiter.kv_cachegen_encode(x.clone(), num_bins=256)
        d_ref = musa_aiter.kv_cachegen_decode(e_ref, b_ref)
        _ = torch.ones(1000, device=DEV).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(enc, e_ref) and torch.equal(book, b_ref) and torch.equal(cdf, c_ref), rep
        assert torch.equal(dec, d_ref), rep


def test_lmcache_two_x_nl_replays():
    nl, nb, bs, nh, hs, t = 4, 20, 16, 4, 32, 200
    rng = np.random.default_rng(5)
    gen = torch.Generator().manual_seed(5)
    caches = [[random_payload((nb, bs, nh, hs), torch.bfloat16, gen).to(DEV) for _ in range(nl)] for _ in range(2)]
    mem = torch.zeros(2, nl, t, nh * hs, dtype=torch.bfloat16, device=DEV)
    slots = torch.zeros(t, dtype=torch.long, device=DEV)
    g, _ = _capture(lambda: musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(caches, mem, slots, bs, nh, hs))
    for rep in range(3):
        s = rng.permutation(nb * bs)[:t]
        s[rng.random(t) < 0.1] = -1
        slots.copy_(torch.from_numpy(s))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = torch.empty_like(mem)
        musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(caches, want, slots, bs, nh, hs)
        torch.cuda.synchronize()
        assert np.array_equal(bits(mem), bits(want)), rep
    # scatter: replay writes the (changing) buffer back through changing slots; later replays
    # repeat slots (last token wins) and skip some, so stale claims of earlier replays would show
    src = random_payload((2, nl, t, nh * hs), torch.bfloat16, gen).to(DEV)
    gs, _ = _capture(lambda: musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(src, caches, slots, 0, bs, nh, hs))
    for rep in range(4):
        if rep == 0:
            s = rng.permutation(nb * bs)[:t]
        else:
            s = rng.integers(0, nb * bs // 4, size=t)
            s[rng.random(t) < 0.1] = -1
        slots.copy_(torch.from_numpy(s))
        src.copy_(random_payload((2, nl, t, nh * hs), torch.bfloat16, gen).to(DEV))
        before = [[c.clone() for c in grp] for grp in caches]
        torch.cuda.synchronize()
        gs.replay()
        torch.cuda.synchronize()
        musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(src, before, slots, 0, bs, nh, hs)
        torch.cuda.synchronize()
        for a in range(2):
            for layer in range(nl):
                assert np.array_equal(bits(caches[a][layer]), bits(before[a][layer])), (rep, a, layer)


def test_triton_indexed_to_dense_replays():
    ntok, nh, hd, batch, dense = 300, 4, 64, 3, 48
    rng = np.random.default_rng(8)
    gen = torch.Generator().manual_seed(8)
    k = random_payload((ntok, nh, hd), torch.float16, gen).to(DEV)
    v = random_payload((ntok, nh, hd), torch.float16, gen).to(DEV)
    indptr = torch.tensor([0, 40, 40, 100], dtype=torch.long, device=DEV)
    indices = torch.zeros(100, dtype=torch.long, device=DEV)
    g, (ok, ov) = _capture(lambda: kv_triton_indexed_to_dense(k, v, indptr, indices, max_seq_len=dense))
    for rep in range(3):
        indices.copy_(torch.from_numpy(rng.integers(0, ntok, size=100)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        wk, wv = kv_triton_indexed_to_dense(k, v, indptr, indices, max_seq_len=dense)
        torch.cuda.synchronize()
        assert np.array_equal(bits(ok), bits(wk)) and np.array_equal(bits(ov), bits(wv)), rep


def test_graphs_on_the_default_capture_stream_get_their_own_claim_arrays():
    # torch captures every graph on one process-wide stream; two graphs captured there must not
    # share a claim array, or replays of both on different streams would clear each other's tags.
    from musa_aiter.ops import _hip

    nl, nb, bs, nh, hs, t = 2, 16, 16, 2, 64, 96
    rng = np.random.default_rng(9)
    gen = torch.Generator().manual_seed(9)
    count = _hip.fn("musa_aiter_hip_graph_claim_arrays")
    graphs, cases = [], []
    before = int(count())
    for _ in range(2):
        caches = [[random_payload((nb, bs, nh, hs), torch.bfloat16, gen).to(DEV) for _ in range(nl)]
                  for _ in range(2)]
        src = random_payload((2, nl, t, nh * hs), torch.bfloat16, gen).to(DEV)
        slots = torch.from_numpy(rng.integers(0, nb * bs // 8, size=t)).to(DEV)  # many repeats
        g, _ = _capture(lambda c=caches, m=src, s=slots: musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(
            m, c, s, 0, bs, nh, hs))
        graphs.append(g)
        cases.append((caches, src, slots))
    assert int(count()) - before == 2
    # both graphs still replay correctly, on two different streams
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    want = []
    for caches, src, slots in cases:
        ref = [[c.clone() for c in grp] for grp in caches]
        musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(src, ref, slots, 0, bs, nh, hs)
        want.append(ref)
    torch.cuda.synchronize()
    for g, s in zip(graphs, streams):
        with torch.cuda.stream(s):
            g.replay()
    torch.cuda.synchronize()
    for (caches, _, _), ref in zip(cases, want):
        for a in range(2):
            for layer in range(nl):
                assert np.array_equal(bits(caches[a][layer]), bits(ref[a][layer])), (a, layer)
