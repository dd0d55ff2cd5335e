"""The allocation-free paged-A entry point against the allocating one, through the C ABI.

``musa_aiter_hip_paged_tiles_noalloc`` keeps a scatter's last-writer claim tags in
a static device array instead of library-allocated scratch.  Each case runs
the same call through ``musa_aiter_hip_paged_tiles`` and through the new entry on
identical caches and compares every byte, twice in a row with the second call
smaller (fewer tokens, fewer blocks, other repeated slots), so stale tags left
in the shared array by the first call would show.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from musa_aiter.ops import _hip
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"
COPY, E4M3 = 0, 1
LIN_BF16 = 2


def _entry(name):
    f = getattr(_hip.library(), name)
    f.argtypes = _hip._SIGNATURES[name]
    f.restype = ctypes.c_int
    return f


def _call(name, *, scatter, codec, cache_elt, kc, vc, kl, vl, slots, nl, t, nb, nh, hd, bs, scale=None,
          fill_zeros=1, dedupe=1):
    p = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    # The allocating entry takes a claims argument (NULL: the library's own tags) before the stream.
    claims = () if name.endswith("_noalloc") else (None,)
    rc = _entry(name)(scatter, codec, cache_elt, 2, LIN_BF16, p(kc), p(vc), p(kl), p(vl), p(slots), nl, t, nb,
                      nh, hd, bs, nh * hd, t * nh * hd, p(scale), p(scale), 0, fill_zeros, dedupe, *claims,
                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0, f"{name}: {rc}"


def _slots(rng, nb, bs, t):
    """Repeated slots (a small pool), skips, and a repeat of the first slot at the end."""
    s = rng.integers(0, max(2, nb * bs // 4), size=t)
    s[rng.random(t) < 0.1] = -1
    s[-1] = s[0]
    return torch.from_numpy(s.astype(np.int64)).to(DEV)


@pytest.mark.parametrize("codec", [COPY, E4M3])
def test_noalloc_scatter_matches_allocating_entry_twice(codec):
    rng = np.random.default_rng(71 + codec)
    gen = torch.Generator().manual_seed(71 + codec)
    nh, hd, bs = 8, 128, 16
    cache_dtype, cache_elt = (torch.bfloat16, 2) if codec == COPY else (torch.uint8, 1)
    scale = torch.tensor([0.02], dtype=torch.float32, device=DEV) if codec != COPY else None
    for step, (nl, nb, t) in enumerate([(3, 96, 700), (2, 40, 150)]):  # the second call is smaller
        print(f"noalloc case codec={codec} step={step} nl={nl} nb={nb} t={t}", flush=True)
        kl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
        vl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
        if codec != COPY:
            kl, vl = kl[:1].contiguous(), vl[:1].contiguous()
            nl = 1
        slots = _slots(rng, nb, bs, t)
        base_k = random_payload((nl, nb, nh, hd, bs), cache_dtype, gen).to(DEV)
        base_v = random_payload((nl, nb, nh, hd, bs), cache_dtype, gen).to(DEV)
        ak, av, bk, bv = base_k.clone(), base_v.clone(), base_k.clone(), base_v.clone()
        common = dict(scatter=1, codec=codec, cache_elt=cache_elt, kl=kl, vl=vl, slots=slots, nl=nl, t=t, nb=nb,
                      nh=nh, hd=hd, bs=bs, scale=scale)
        _call("musa_aiter_hip_paged_tiles", kc=ak, vc=av, **common)
        _call("musa_aiter_hip_paged_tiles_noalloc", kc=bk, vc=bv, **common)
        torch.cuda.synchronize()
        assert np.array_equal(bits(ak), bits(bk)) and np.array_equal(bits(av), bits(bv)), step
        assert not np.array_equal(bits(ak), bits(base_k)), step  # the scatter wrote something


def test_noalloc_gather_matches_allocating_entry():
    rng = np.random.default_rng(73)
    gen = torch.Generator().manual_seed(73)
    nl, nb, nh, hd, bs, t = 2, 64, 8, 128, 16, 333
    kc = random_payload((nl, nb, nh, hd, bs), torch.bfloat16, gen).to(DEV)
    vc = random_payload((nl, nb, nh, hd, bs), torch.bfloat16, gen).to(DEV)
    slots = _slots(rng, nb, bs, t)
    outs = [[torch.full((nl, t, nh, hd), 7.0, dtype=torch.bfloat16, device=DEV) for _ in range(2)] for _ in range(2)]
    for name, (ok, ov) in zip(("musa_aiter_hip_paged_tiles", "musa_aiter_hip_paged_tiles_noalloc"), outs):
        _call(name, scatter=0, codec=COPY, cache_elt=2, kc=kc, vc=vc, kl=ok, vl=ov, slots=slots, nl=nl, t=t, nb=nb,
              nh=nh, hd=hd, bs=bs, dedupe=0)
    torch.cuda.synchronize()
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0])) and np.array_equal(bits(outs[0][1]), bits(outs[1][1]))


def test_noalloc_after_eager_and_on_a_side_stream():
    # Interleaved with the allocating entry and run on a second stream (one call at a time).
    rng = np.random.default_rng(74)
    gen = torch.Generator().manual_seed(74)
    nl, nb, nh, hd, bs, t = 1, 32, 8, 128, 16, 257
    side = torch.cuda.Stream()
    for rep in range(3):
        kl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
        vl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
        slots = _slots(rng, nb, bs, t)
        ak = torch.zeros((nl, nb, nh, hd, bs), dtype=torch.bfloat16, device=DEV)
        av, bk, bv = torch.zeros_like(ak), torch.zeros_like(ak), torch.zeros_like(ak)
        common = dict(scatter=1, codec=COPY, cache_elt=2, kl=kl, vl=vl, slots=slots, nl=nl, t=t, nb=nb, nh=nh,
                      hd=hd, bs=bs)
        _call("musa_aiter_hip_paged_tiles", kc=ak, vc=av, **common)
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            _call("musa_aiter_hip_paged_tiles_noalloc", kc=bk, vc=bv, **common)
        torch.cuda.synchronize()
        assert np.array_equal(bits(ak), bits(bk)) and np.array_equal(bits(av), bits(bv)), rep


def test_noalloc_scatter_and_gather_replay_from_a_graph():
    # Captured once, replayed with new inputs (repeated and skipped slots): every replay equals the
    # allocating entry run eagerly on the same inputs, bit for bit.
    rng = np.random.default_rng(75)
    gen = torch.Generator().manual_seed(75)
    nl, nb, nh, hd, bs, t = 2, 48, 8, 128, 16, 400
    kl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
    vl = random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV)
    slots = _slots(rng, nb, bs, t)
    kc = torch.zeros((nl, nb, nh, hd, bs), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    ok = torch.empty_like(kl)
    ov = torch.empty_like(vl)
    scatter = dict(scatter=1, codec=COPY, cache_elt=2, kc=kc, vc=vc, kl=kl, vl=vl, slots=slots, nl=nl, t=t, nb=nb,
                   nh=nh, hd=hd, bs=bs)
    gather = dict(scatter, scatter=0, kl=ok, vl=ov, dedupe=0)

    def step():
        _call("musa_aiter_hip_paged_tiles_noalloc", **scatter)
        _call("musa_aiter_hip_paged_tiles_noalloc", **gather)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        kl.copy_(random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV))
        vl.copy_(random_payload((nl, t, nh, hd), torch.bfloat16, gen).to(DEV))
        slots.copy_(_slots(rng, nb, bs, t))
        base = random_payload((nl, nb, nh, hd, bs), torch.bfloat16, gen).to(DEV)
        kc.copy_(base)
        vc.copy_(base)
        wk, wv = base.clone(), base.clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        wok, wov = torch.empty_like(kl), torch.empty_like(vl)
        _call("musa_aiter_hip_paged_tiles", **dict(scatter, kc=wk, vc=wv))
        _call("musa_aiter_hip_paged_tiles", **dict(gather, kc=wk, vc=wv, kl=wok, vl=wov))
        torch.cuda.synchronize()
        assert np.array_equal(bits(kc), bits(wk)) and np.array_equal(bits(vc), bits(wv)), rep
        assert np.array_equal(bits(ok), bits(wok)) and np.array_equal(bits(ov), bits(wov)), rep
