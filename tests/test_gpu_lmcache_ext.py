"""GPU parity of the LMCache extension surface (reference csrc/kvcache/lmcache_kv_transfer_ext.cpp:389-592).

The four methods of the object load_lmcache_kv_transfer_ext() returns, against the oracle's
native row semantics (oracle/kv_oracle.py native_gather_rows / native_scatter_rows), bit-exactly:
list2 scatter with a prefix skip and gather, the 2 x NL scatter with a prefix skip and gather,
skipped, out-of-range and repeated slots, the range check of the 2 x NL scatter, and the timing
line of the list2 calls.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from musa_aiter.ops.lmcache_kv_transfer_ext import load_lmcache_kv_transfer_ext
from oracle import kv_oracle as ko
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _payload(shape, dtype, seed):
    return random_payload(shape, dtype, torch.Generator().manual_seed(seed)).to(DEV)


def _slots(rng, nb, bs, t, dup):
    s = rng.integers(-1, nb * bs // 3, size=t) if dup else rng.permutation(nb * bs)[:t]
    if not dup:
        s[rng.random(t) < 0.15] = -1
    s[rng.random(t) < 0.05] = nb * bs + 3
    return s.astype(np.int64)


def _inside(s, nb, bs):
    s = s.copy()
    s[(s < 0) | (s >= nb * bs)] = -1
    return s


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_list2_methods(dtype, capsys, monkeypatch):
    ext = load_lmcache_kv_transfer_ext()
    assert ext is not None
    nb, bs, nh, hs, t, skip = 13, 16, 8, 16, 150, 4
    hidden, m = nh * hs, t + skip + 3
    rng = np.random.default_rng(1)
    gs, ds = _slots(rng, nb, bs, t, False), _slots(rng, nb, bs, t, True)
    kv = [_payload((2, nb, bs, nh, hs), dtype, 10 + layer) for layer in range(2)]
    mem = _payload((2, 2, m, hidden), dtype, 20)
    want = bits(mem).copy()
    assert ext.paged_to_kv_buffer_list2(kv, mem, torch.from_numpy(gs).to(DEV), bs, nh, hs) is True
    for layer in range(2):
        for a in range(2):
            ko.native_gather_rows(bits(kv[layer])[a].reshape(nb * bs, hidden), _inside(gs, nb, bs), want[a, layer])
    assert np.array_equal(bits(mem), want)
    wkv = [bits(c).copy().reshape(2, nb * bs, hidden) for c in kv]
    monkeypatch.setenv("MUSA_AITER_LMCACHE_CPP_TIMING", "1")
    assert ext.kv_buffer_to_paged_list2(mem, kv, torch.from_numpy(ds).to(DEV), skip, bs, nh, hs) is True
    line = capsys.readouterr().err
    assert "[musa_aiter_lmcache_timing] op=to_gpu_buffer_to_paged impl=rocm-hip tokens=150" in line
    assert f"bytes={2 * 2 * t * hidden * 2}" in line and "device_ms=" in line and "bandwidth_gbps=" in line
    for layer in range(2):
        for a in range(2):
            ko.native_scatter_rows(want[a, layer], _inside(ds, nb, bs), wkv[layer][a], skip)
        assert np.array_equal(bits(kv[layer]).reshape(2, nb * bs, hidden), wkv[layer])


@pytest.mark.parametrize("nl", [1, 4])
def test_two_x_nl_methods(nl):
    ext = load_lmcache_kv_transfer_ext()
    nb, bs, nh, hs, t, skip = 9, 16, 4, 32, 100, 7
    hidden, m = nh * hs, t + skip
    rng = np.random.default_rng(nl)
    gs, ds = _slots(rng, nb, bs, t, False), _slots(rng, nb, bs, t, True)
    caches = [[_payload((nb, bs, nh, hs), torch.bfloat16, 30 + 10 * a + layer) for layer in range(nl)]
              for a in range(2)]
    mem = _payload((2, nl, m, hidden), torch.bfloat16, 40)
    want = bits(mem).copy()
    assert ext.paged_to_kv_buffer_two_x_nl(caches, mem, torch.from_numpy(gs).to(DEV), bs, nh, hs) is True
    for a in range(2):
        for layer in range(nl):
            ko.native_gather_rows(bits(caches[a][layer]).reshape(nb * bs, hidden), _inside(gs, nb, bs),
                                  want[a, layer])
    assert np.array_equal(bits(mem), want)
    wc = [[bits(c).copy().reshape(nb * bs, hidden) for c in g] for g in caches]
    assert ext.kv_buffer_to_paged_two_x_nl(mem, caches, torch.from_numpy(ds).to(DEV), skip, bs, nh, hs) is True
    for a in range(2):
        for layer in range(nl):
            ko.native_scatter_rows(want[a, layer], _inside(ds, nb, bs), wc[a][layer], skip)
            assert np.array_equal(bits(caches[a][layer]).reshape(nb * bs, hidden), wc[a][layer])
    with pytest.raises(RuntimeError, match="transfer range exceeds memory_tensor token extent"):
        ext.kv_buffer_to_paged_two_x_nl(mem, caches, torch.from_numpy(ds).to(DEV), skip + 1, bs, nh, hs)
    with pytest.raises(RuntimeError, match="skip_prefix_n_tokens must be non-negative"):
        ext.kv_buffer_to_paged_two_x_nl(mem, caches, torch.from_numpy(ds).to(DEV), -1, bs, nh, hs)
    with pytest.raises(RuntimeError, match="split cache must be \\[NB, BS, NH, HS\\]"):
        ext.paged_to_kv_buffer_two_x_nl(caches, mem, torch.from_numpy(gs).to(DEV), bs * 2, nh, hs)
