"""GPU parity at the full BASELINE sizes, through properties that do not need the CPU oracle.

The oracle finishes in seconds only on smaller inputs, so at the full shapes of the five BASELINE
configs these tests check, for every token:

* configs[0] (one fp16 layer, 1,024 blocks of 16, 32 sequences of 1-512 tokens): the gather
  equals torch indexing of the cache;
* configs[1] (32 layers bf16, 8,192 blocks of 16, 64 sequences of 128-4,096 tokens): a scatter
  followed by a gather returns the input bit for bit; every cache row named by a slot equals its
  linear row by torch indexing; every cache row no slot names keeps its previous bits;
* configs[2] (FP8, one layer of the same shape; E4M3 with per-kv-head scales amax/448 or a scalar
  scale, E5M2 with per-head scales amax/57344): every cache byte equals the reference encoder's
  steps restated in torch (tests/torch_ref.py, evaluated on CPU copies), every dequantised row
  equals the reference decoder's steps, untouched cache bytes keep their sentinel;
* configs[3] (SGLang MP caches 2 x 32 x [4,096, 16, 8, 128] bf16, sixteen 256-token chunks of
  random sequences): each chunk's gather equals torch indexing, and a scatter of the gathered
  buffer into zeroed caches restores exactly the named rows;
* configs[4] (MLA, 61 layers, block size 64, 576 bf16 values per row, 128 sequences of
  256-8,192 tokens): the gather equals torch indexing of the cache, and a scatter of the gathered
  rows into a zeroed cache restores every named row and leaves every other row zero.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import musa_aiter
from tests import torch_ref
from tests.kvgen import sequence_lengths, sequence_slots

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _release_memory():
    torch.cuda.empty_cache()
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _slots(seed, num_seqs, lo, hi, nb, bs):
    rng = np.random.default_rng(seed)
    lengths = sequence_lengths(rng, num_seqs, lo, hi, num_blocks=nb, block_size=bs)
    return sequence_slots(rng, lengths, num_blocks=nb, block_size=bs)


def _unnamed(slots, rows):
    mask = torch.ones(rows, dtype=torch.bool, device=DEV)
    mask[slots] = False
    return mask


def test_config1_single_layer_fp16_gather_full_size():
    nb, bs, nh, hd = 1024, 16, 8, 128
    slots_np = _slots(1001, 32, 1, 512, nb, bs)
    slots = torch.from_numpy(slots_np).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(11)
    kc = torch.randn((nb, nh, hd, bs), generator=gen, device=DEV, dtype=torch.float16)
    vc = torch.randn((nb, nh, hd, bs), generator=gen, device=DEV, dtype=torch.float16)
    ok, ov = musa_aiter.kv_paged_to_linear(kc, vc, slots)
    torch.cuda.synchronize()
    for cache, out in ((kc, ok), (vc, ov)):
        assert torch.equal(out.view(torch.int16), torch_ref.paged_rows(cache).view(torch.int16)[slots])


def test_config4_sglang_mp_two_x_nl_chunks_full_size():
    nl, nb, bs, nh, hs, chunk = 32, 4096, 16, 8, 128, 256
    gen = torch.Generator(device=DEV).manual_seed(14)
    caches = [[torch.randn((nb, bs, nh, hs), generator=gen, device=DEV, dtype=torch.bfloat16) for _ in range(nl)]
              for _ in range(2)]
    back = [[torch.zeros_like(c) for c in grp] for grp in caches]
    all_slots = torch.from_numpy(_slots(1004, 64, 256, 2048, nb, bs)).to(DEV)
    rng = np.random.default_rng(1004)
    named = torch.zeros(nb * bs, dtype=torch.bool, device=DEV)
    mem = torch.empty((2, nl, chunk, nh * hs), dtype=torch.bfloat16, device=DEV)
    for c in range(16):
        start = int(rng.integers(0, all_slots.numel() - chunk))
        slots = all_slots[start:start + chunk].contiguous()
        named[slots] = True
        assert musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(caches, mem, slots, bs, nh, hs)
        assert musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(mem, back, slots, 0, bs, nh, hs)
        for a in range(2):
            for layer in range(nl):
                rows = caches[a][layer].view(nb * bs, nh * hs).view(torch.int16)
                assert torch.equal(mem[a, layer].view(torch.int16), rows[slots]), (c, a, layer)
    torch.cuda.synchronize()
    for a in range(2):
        for layer in range(nl):
            src = caches[a][layer].view(nb * bs, nh * hs).view(torch.int16)
            dst = back[a][layer].view(nb * bs, nh * hs).view(torch.int16)
            assert torch.equal(dst[named], src[named]), (a, layer)
            assert not bool(dst[~named].any()), (a, layer)


def test_config2_multi_layer_bf16_round_trip_full_size():
    nl, nb, bs, nh, hd = 32, 8192, 16, 8, 128
    slots_np = _slots(1002, 64, 128, 4096, nb, bs)
    t = int(slots_np.shape[0])
    print(f"configs[1] full size: {t} tokens x {nl} layers", flush=True)
    slots = torch.from_numpy(slots_np).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(12)
    kl = torch.randn((nl, t, nh, hd), generator=gen, device=DEV, dtype=torch.bfloat16)
    vl = torch.randn((nl, t, nh, hd), generator=gen, device=DEV, dtype=torch.bfloat16)
    kc = torch.randn((nl, nb, nh, hd, bs), generator=gen, device=DEV, dtype=torch.bfloat16)
    vc = torch.randn((nl, nb, nh, hd, bs), generator=gen, device=DEV, dtype=torch.bfloat16)
    kc0, vc0 = kc.clone(), vc.clone()
    musa_aiter.kv_linear_to_paged_multi_layer(kl, vl, kc, vc, slots)
    ok, ov = torch.empty_like(kl), torch.empty_like(vl)
    musa_aiter.kv_paged_to_linear_multi_layer(kc, vc, slots, out_k=ok, out_v=ov)
    torch.cuda.synchronize()
    assert torch.equal(ok.view(torch.int16), kl.view(torch.int16))
    assert torch.equal(ov.view(torch.int16), vl.view(torch.int16))
    del ok, ov
    unnamed = _unnamed(slots, nb * bs)
    for cache, before, lin in ((kc, kc0, kl), (vc, vc0, vl)):
        for layer in range(nl):
            rows = torch_ref.paged_rows(cache[layer]).view(torch.int16)
            assert torch.equal(rows[slots], lin[layer].view(torch.int16)), layer
            assert torch.equal(rows[unnamed], torch_ref.paged_rows(before[layer]).view(torch.int16)[unnamed]), layer


@pytest.mark.parametrize("fmt,per_head,fmax", [("e4m3", True, 448.0), ("e4m3", False, 448.0),
                                               ("e5m2", True, 57344.0)])
def test_config3_fp8_full_size(fmt, per_head, fmax):
    # per-kv-head scales amax/448 (the headline), a scalar scale (global amax/448), and
    # E5M2 with per-head scales amax/57344.  The expected codes and dequantised values are computed
    # from CPU copies, where tests/test_oracle_fp8.py pins tests/torch_ref.py against the oracle.
    nb, bs, nh, hd = 8192, 16, 8, 128
    slots_np = _slots(1003, 64, 128, 4096, nb, bs)
    t = int(slots_np.shape[0])
    print(f"configs[2] full size: {t} tokens, {fmt}, per_head={per_head}", flush=True)
    slots = torch.from_numpy(slots_np).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(13)
    lin = []
    for _ in range(2):
        x = torch.randn((t, nh, hd), generator=gen, device=DEV) * 2.0
        x.mul_(torch.where(torch.rand(x.shape, generator=gen, device=DEV) < 0.01, 50.0, 1.0))
        lin.append(x.to(torch.bfloat16))
    kl, vl = lin
    if per_head:
        ks = (kl.float().abs().amax(dim=(0, 2)) / fmax).contiguous()
        vs = (vl.float().abs().amax(dim=(0, 2)) / fmax).contiguous()
    else:
        ks = (kl.float().abs().amax() / fmax).reshape(1).contiguous()
        vs = (vl.float().abs().amax() / fmax).reshape(1).contiguous()
    kc = torch.full((nb, nh, hd, bs), 0x5A, dtype=torch.uint8, device=DEV)
    vc = torch.full_like(kc, 0x5A)
    musa_aiter.kv_linear_to_paged_fp8(kl, vl, kc, vc, slots, ks, vs, fp8_format=fmt)
    ok, ov = musa_aiter.kv_paged_fp8_to_linear(kc, vc, slots, ks, vs, out_dtype=torch.bfloat16, fp8_format=fmt)
    torch.cuda.synchronize()
    unnamed = _unnamed(slots, nb * bs)
    for cache, x, scale, out in ((kc, kl, ks, ok), (vc, vl, vs, ov)):
        rows = torch_ref.paged_rows(cache)
        scale_cpu = scale.cpu().reshape(-1, 1)
        want = torch_ref.fp8_quantize(x.cpu(), scale_cpu, fmt)
        assert torch.equal(rows[slots].cpu(), want)
        want_deq = torch_ref.fp8_dequantize(want, scale_cpu, fmt, torch.bfloat16)
        assert torch.equal(out.cpu().view(torch.int16), want_deq.view(torch.int16))
        assert bool((rows[unnamed] == 0x5A).all())
        del want, want_deq


def test_config5_mla_rows_full_size():
    nl, bs, hs = 61, 64, 576
    rng = np.random.default_rng(1005)
    lengths = [int(x) for x in rng.integers(256, 8193, size=128)]
    nb = sum((n + bs - 1) // bs for n in lengths)
    slots_np = sequence_slots(rng, lengths, num_blocks=nb, block_size=bs)
    t = int(slots_np.shape[0])
    print(f"configs[4] full size: {t} tokens x {nl} layers, {nb} blocks", flush=True)
    slots = torch.from_numpy(slots_np).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(15)
    paged = torch.randn((nl, nb, bs, hs), generator=gen, device=DEV, dtype=torch.bfloat16)
    buf = torch.empty((nl, t, hs), dtype=torch.bfloat16, device=DEV)
    assert musa_aiter.lmcache_paged_to_kv_buffer_mla(paged, buf, slots)
    back = torch.zeros_like(paged)
    assert musa_aiter.lmcache_kv_buffer_to_paged_mla(buf, back, slots)
    torch.cuda.synchronize()
    unnamed = _unnamed(slots, nb * bs)
    for layer in range(nl):
        src = paged[layer].view(nb * bs, hs).view(torch.int16)
        dst = back[layer].view(nb * bs, hs).view(torch.int16)
        assert torch.equal(buf[layer].view(torch.int16), src[slots]), layer
        assert torch.equal(dst[slots], src[slots]), layer
        assert not bool(dst[unnamed].any()), layer
