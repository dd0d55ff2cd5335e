"""HIP graph capture of the entry points that never synchronise with the host.

kv_cachegen_encode, kv_cachegen_decode (256-entry codebook), the LMCache 2 x NL gather and scatter,
kv_triton_indexed_to_dense and the reference-named C entries (the multi-layer paged scatter and
gather, the FP8 quant-store and dequant-gather) launch only kernels on the current stream (no host
reads, no memsets), so a caller can capture them in a graph.  A captured scatter whose slots may repeat
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


def test_graphs_on_the_default_capture_stream_get_their_own_claim_tags():
    # torch captures every graph on one process-wide stream; two graphs captured there must not
    # share claim tags, or replays of both on different streams would clear each other's tags.  A
    # captured public-API scatter takes its tags from the graph's own memory pool.
    nl, nb, bs, nh, hs, t = 2, 16, 16, 2, 64, 96
    rng = np.random.default_rng(9)
    gen = torch.Generator().manual_seed(9)
    graphs, cases = [], []
    for _ in range(2):
        caches = [[random_payload((nb, bs, nh, hs), torch.bfloat16, gen).to(DEV) for _ in range(nl)]
                  for _ in range(2)]
        src = random_payload((2, nl, t, nh * hs), torch.bfloat16, gen).to(DEV)
        slots = torch.from_numpy(rng.integers(0, nb * bs // 8, size=t)).to(DEV)  # many repeats
        g, _ = _capture(lambda c=caches, m=src, s=slots: musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(
            m, c, s, 0, bs, nh, hs))
        graphs.append(g)
        cases.append((caches, src, slots))
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


def _abi(name: str, nptr: int, ni64: int, fp8: bool = False):
    """A reference-named C entry: pointers, int64 sizes, then the stream; the FP8 entries put an int
    dtype code before the stream and an int scale mode after it."""
    import ctypes

    from musa_aiter.ops import _hip

    fn = getattr(_hip.library(), name)
    tail = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] if fp8 else [ctypes.c_void_p]
    fn.argtypes = [ctypes.c_void_p] * nptr + [ctypes.c_longlong] * ni64 + tail
    fn.restype = ctypes.c_int
    return fn


def _cur_stream():
    import ctypes

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_reference_abi_multi_layer_scatter_then_gather_replays():
    # The headline pair through the reference-named C entries (kv_transfer.py:2446-2480 argument
    # order): a multi-layer scatter whose slots repeat and skip, then the gather of other slots,
    # captured as one graph; every replay takes new linear rows, slots and cache contents.
    nl, nb, nh, hd, bs, t = 3, 64, 4, 64, 16, 300
    rng = np.random.default_rng(10)
    gen = torch.Generator().manual_seed(10)
    scatter = _abi("musa_aiter_kv_linear_to_paged_multi_layer_bfloat16", 5, 6)
    gather = _abi("musa_aiter_kv_paged_to_linear_multi_layer_bfloat16", 5, 6)
    kl = torch.empty((nl, t, nh, hd), dtype=torch.bfloat16, device=DEV)
    vl = torch.empty_like(kl)
    kc = torch.empty((nl, nb, nh, hd, bs), dtype=torch.bfloat16, device=DEV)
    vc = torch.empty_like(kc)
    ss = torch.zeros(t, dtype=torch.long, device=DEV)
    gs = torch.zeros(t, dtype=torch.long, device=DEV)
    ok = torch.empty_like(kl)
    ov = torch.empty_like(vl)

    def step(kl, vl, kc, vc, ss, gs, ok, ov):
        assert scatter(kl.data_ptr(), vl.data_ptr(), ss.data_ptr(), kc.data_ptr(), vc.data_ptr(), nl, t, nb, nh, hd,
                       bs, _cur_stream()) == 0
        assert gather(kc.data_ptr(), vc.data_ptr(), gs.data_ptr(), ok.data_ptr(), ov.data_ptr(), nl, t, nb, nh, hd,
                      bs, _cur_stream()) == 0

    bufs = (kl, vl, kc, vc, ss, gs, ok, ov)
    g, _ = _capture(lambda: step(*bufs))
    for rep in range(3):
        for x in (kl, vl, kc, vc):
            x.copy_(random_payload(tuple(x.shape), torch.bfloat16, gen))
        scat = rng.integers(-1, nb * bs // 4, size=t)  # many repeated destinations
        gath = rng.permutation(nb * bs)[:t]
        gath[rng.random(t) < 0.1] = -1
        ss.copy_(torch.from_numpy(scat))
        gs.copy_(torch.from_numpy(gath))
        ref = tuple(x.clone() for x in bufs)
        step(*ref)  # eager, on other buffers, between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, want in zip((kc, vc, ok, ov), ref[2:4] + ref[6:8]):
            assert np.array_equal(bits(got), bits(want)), rep


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_reference_abi_fp8_quant_store_then_dequant_replays(fmt):
    # FP8 vec4 entries with per-head scales (scale mode 1, kv_transfer.py:2401-2440): the quant-store
    # with repeated slots and the dequant-gather of the same slots, captured together.
    nb, nh, hd, bs, t = 64, 4, 64, 16, 256
    rng = np.random.default_rng(11)
    gen = torch.Generator(device=DEV).manual_seed(11)
    quant = _abi(f"musa_aiter_kv_linear_to_paged_fp8_vec4_{fmt}", 7, 5, fp8=True)
    deq = _abi(f"musa_aiter_kv_paged_fp8_to_linear_vec4_{fmt}", 7, 5, fp8=True)
    kl = torch.empty((t, nh, hd), dtype=torch.bfloat16, device=DEV)
    vl = torch.empty_like(kl)
    kc = torch.zeros((nb, nh, hd, bs), dtype=torch.uint8, device=DEV)
    vc = torch.zeros_like(kc)
    ks = torch.empty(nh, dtype=torch.float32, device=DEV)
    vs = torch.empty_like(ks)
    slots = torch.zeros(t, dtype=torch.long, device=DEV)
    ok = torch.empty_like(kl)
    ov = torch.empty_like(vl)

    def step(kl, vl, kc, vc, ks, vs, slots, ok, ov):
        assert quant(kl.data_ptr(), vl.data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(),
                     vs.data_ptr(), t, nb, nh, hd, bs, 2, _cur_stream(), 1) == 0
        assert deq(kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), ks.data_ptr(), vs.data_ptr(), ok.data_ptr(),
                   ov.data_ptr(), t, nb, nh, hd, bs, 2, _cur_stream(), 1) == 0

    bufs = (kl, vl, kc, vc, ks, vs, slots, ok, ov)
    g, _ = _capture(lambda: step(*bufs))
    for rep in range(3):
        for x in (kl, vl):
            x.copy_((torch.randn(tuple(x.shape), generator=gen, device=DEV) * 3.0).to(torch.bfloat16))
        for s, x in ((ks, kl), (vs, vl)):
            s.copy_(x.float().abs().amax(dim=(0, 2)) / (448.0 if fmt == "e4m3" else 57344.0))
        s_np = rng.integers(-1, nb * bs // 3, size=t)
        slots.copy_(torch.from_numpy(s_np))
        ref = tuple(x.clone() for x in bufs)
        step(*ref)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, want in zip((kc, vc, ok, ov), ref[2:4] + ref[7:9]):
            assert np.array_equal(bits(got), bits(want)), rep
