"""GPU parity of every reference-named C entry, called through ctypes as the reference's shims bind them.

The public-API tests reach the kernels through the library's generic entries; this file calls
the symbols a reference build binds (kv_transfer.py:288-976, :2401-2980;
lmcache_kv_transfer.py:628-761) with the reference's argument orders, on seeded random bit
patterns, and compares bit-exactly with oracle/kv_oracle.py.  It follows the reference's native
kernels where they differ from its Python path: a gather writes zeros for a slot that is negative
or past the cache and leaves buffer rows outside the transfer untouched; a scatter skips such
slots (kv_transfer_float.mu:16-56, :1592-1680, :2233-2308, :2518-2560).  Scatters use duplicate
destinations too: the last token wins.  Families: paged-A single / multi-layer / merged / merged
multi-layer / MLA split (float, half, bfloat16); FP8 scalar, vec4, multi-layer and shape-specialised
entries (E4M3, E5M2, fp16 / bf16 / fp32 linear sides, every scale mode); LMCache 6-D, MLA, 2 x NL
per plane and coalesced, list, list2 and MLA lists; DSV4 byte rows; the dense preload and block
copies for every element suffix; the ABI probes.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from musa_aiter.ops import _hip
from oracle import kv_oracle as ko
from tests.kvgen import bits, random_payload

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
SUFFIX = {torch.float32: "float", torch.float16: "half", torch.bfloat16: "bfloat16"}
P, I64, I32 = ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int


def _bind(name: str, argtypes: list):
    fn = getattr(_hip.library(), name)
    fn.argtypes = argtypes
    fn.restype = ctypes.c_int
    return fn


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(a: np.ndarray, dtype=torch.int64) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


def _slots(rng, nb: int, bs: int, t: int, *, dup: bool) -> np.ndarray:
    """Gathers: distinct slots with skips; scatters: repeated destinations.  Both with slots past
    the cache, which the native entries treat as skipped."""
    if dup:
        s = rng.integers(-1, max(2, nb * bs // 3), size=t)
    else:
        s = rng.permutation(nb * bs)[:t]
        s[rng.random(t) < 0.15] = -1
    s[rng.random(t) < 0.05] = nb * bs + int(rng.integers(0, 50))
    return s.astype(np.int64)


def _inside(slots: np.ndarray, nb: int, bs: int) -> np.ndarray:
    s = slots.copy()
    s[(s < 0) | (s >= nb * bs)] = -1
    return s


def _payload(shape, dtype, seed):
    return random_payload(shape, dtype, torch.Generator().manual_seed(seed)).to(DEV)


# ---- paged-A [NB, NH, HD, BS] <-> linear (kv_transfer.py:350-959) ------------------------------

SHAPES = [(4, 64, 16), (2, 16, 8), (3, 7, 5)]  # tiled kernels, then the element-wise kernel


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_paged_gathers(dtype, shape):
    nh, hd, bs = shape
    sfx, nl, nb, t = SUFFIX[dtype], 3, 41, 173
    rng = np.random.default_rng(hd + bs)
    slots = _slots(rng, nb, bs, t, dup=False)
    sv, s_d = _inside(slots, nb, bs), _dev(slots)
    kc, vc = _payload((nl, nb, nh, hd, bs), dtype, 1), _payload((nl, nb, nh, hd, bs), dtype, 2)
    kb, vb = bits(kc), bits(vc)
    # single layer (layer 0 of the stacked caches is a contiguous cache)
    ok, ov = _payload((t, nh, hd), dtype, 3), _payload((t, nh, hd), dtype, 4)
    fn = _bind(f"musa_aiter_kv_paged_to_linear_{sfx}", [P] * 5 + [I64] * 5 + [P])
    assert fn(kc[0].data_ptr(), vc[0].data_ptr(), s_d.data_ptr(), ok.data_ptr(), ov.data_ptr(), t, nb, nh, hd, bs,
              _stream()) == 0
    assert np.array_equal(bits(ok), ko.paged_to_linear(kb[0], sv))
    assert np.array_equal(bits(ov), ko.paged_to_linear(vb[0], sv))
    # multi-layer
    ok, ov = _payload((nl, t, nh, hd), dtype, 5), _payload((nl, t, nh, hd), dtype, 6)
    fn = _bind(f"musa_aiter_kv_paged_to_linear_multi_layer_{sfx}", [P] * 5 + [I64] * 6 + [P])
    assert fn(kc.data_ptr(), vc.data_ptr(), s_d.data_ptr(), ok.data_ptr(), ov.data_ptr(), nl, t, nb, nh, hd, bs,
              _stream()) == 0
    assert np.array_equal(bits(ok), ko.paged_to_linear_multi_layer(kb, sv))
    assert np.array_equal(bits(ov), ko.paged_to_linear_multi_layer(vb, sv))
    # merged [T, 2, NH, HD]
    out = _payload((t, 2, nh, hd), dtype, 7)
    fn = _bind(f"musa_aiter_kv_paged_to_merged_linear_{sfx}", [P] * 4 + [I64] * 5 + [P])
    assert fn(kc[1].data_ptr(), vc[1].data_ptr(), s_d.data_ptr(), out.data_ptr(), t, nb, nh, hd, bs, _stream()) == 0
    assert np.array_equal(bits(out), ko.paged_to_merged_linear(kb[1], vb[1], sv))
    # merged multi-layer [NL, T, 2, NH, HD]
    out = _payload((nl, t, 2, nh, hd), dtype, 8)
    fn = _bind(f"musa_aiter_kv_paged_to_merged_linear_multi_layer_{sfx}", [P] * 4 + [I64] * 6 + [P])
    assert fn(kc.data_ptr(), vc.data_ptr(), s_d.data_ptr(), out.data_ptr(), nl, t, nb, nh, hd, bs, _stream()) == 0
    want = np.stack([ko.paged_to_merged_linear(kb[layer], vb[layer], sv) for layer in range(nl)])
    assert np.array_equal(bits(out), want)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_paged_scatters(dtype, shape):
    nh, hd, bs = shape
    sfx, nl, nb, t = SUFFIX[dtype], 3, 29, 211
    rng = np.random.default_rng(3 * hd + bs)
    slots = _slots(rng, nb, bs, t, dup=True)
    sv, s_d = _inside(slots, nb, bs), _dev(slots)

    def caches(seed):
        kc, vc = _payload((nl, nb, nh, hd, bs), dtype, seed), _payload((nl, nb, nh, hd, bs), dtype, seed + 1)
        return kc, vc, bits(kc).copy(), bits(vc).copy()

    kl, vl = _payload((nl, t, nh, hd), dtype, 11), _payload((nl, t, nh, hd), dtype, 12)
    klb, vlb = bits(kl), bits(vl)
    # single layer into layer 2
    kc, vc, wk, wv = caches(20)
    fn = _bind(f"musa_aiter_kv_linear_to_paged_{sfx}", [P] * 5 + [I64] * 5 + [P])
    assert fn(kl[0].data_ptr(), vl[0].data_ptr(), s_d.data_ptr(), kc[2].data_ptr(), vc[2].data_ptr(), t, nb, nh, hd,
              bs, _stream()) == 0
    ko.linear_to_paged(klb[0], wk[2], sv)
    ko.linear_to_paged(vlb[0], wv[2], sv)
    assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv)
    # multi-layer
    kc, vc, wk, wv = caches(30)
    fn = _bind(f"musa_aiter_kv_linear_to_paged_multi_layer_{sfx}", [P] * 5 + [I64] * 6 + [P])
    assert fn(kl.data_ptr(), vl.data_ptr(), s_d.data_ptr(), kc.data_ptr(), vc.data_ptr(), nl, t, nb, nh, hd, bs,
              _stream()) == 0
    ko.linear_to_paged_multi_layer(klb, wk, sv)
    ko.linear_to_paged_multi_layer(vlb, wv, sv)
    assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv)
    # merged
    merged = _payload((nl, t, 2, nh, hd), dtype, 13)
    mb = bits(merged)
    kc, vc, wk, wv = caches(40)
    fn = _bind(f"musa_aiter_kv_merged_linear_to_paged_{sfx}", [P] * 4 + [I64] * 5 + [P])
    assert fn(merged[1].data_ptr(), s_d.data_ptr(), kc[0].data_ptr(), vc[0].data_ptr(), t, nb, nh, hd, bs,
              _stream()) == 0
    ko.merged_linear_to_paged(mb[1], wk[0], wv[0], sv)
    assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv)
    # merged multi-layer
    kc, vc, wk, wv = caches(50)
    fn = _bind(f"musa_aiter_kv_merged_linear_to_paged_multi_layer_{sfx}", [P] * 4 + [I64] * 6 + [P])
    assert fn(merged.data_ptr(), s_d.data_ptr(), kc.data_ptr(), vc.data_ptr(), nl, t, nb, nh, hd, bs,
              _stream()) == 0
    for layer in range(nl):
        ko.merged_linear_to_paged(mb[layer], wk[layer], wv[layer], sv)
    assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dims", [(512, 64), (5, 3)])
def test_mla_split_entries(dtype, dims):
    kv_dim, pe_dim = dims
    sfx, nb, bs, t = SUFFIX[dtype], 23, 16, 150
    rng = np.random.default_rng(kv_dim)
    gslots, dslots = _slots(rng, nb, bs, t, dup=False), _slots(rng, nb, bs, t, dup=True)
    kv, pe = _payload((nb, bs, kv_dim), dtype, 60), _payload((nb, bs, pe_dim), dtype, 61)
    okv, ope = _payload((t, kv_dim), dtype, 62), _payload((t, pe_dim), dtype, 63)
    g_d = _dev(gslots)
    fn = _bind(f"musa_aiter_kv_paged_to_mla_linear_{sfx}", [P] * 5 + [I64] * 5 + [P])
    assert fn(kv.data_ptr(), pe.data_ptr(), g_d.data_ptr(), okv.data_ptr(), ope.data_ptr(), t, nb, bs, kv_dim,
              pe_dim, _stream()) == 0
    gv = _inside(gslots, nb, bs)
    assert np.array_equal(bits(okv), ko.flat_paged_to_linear(bits(kv), gv))
    assert np.array_equal(bits(ope), ko.flat_paged_to_linear(bits(pe), gv))
    wkv, wpe = bits(kv).copy(), bits(pe).copy()
    d_d = _dev(dslots)
    fn = _bind(f"musa_aiter_kv_mla_linear_to_paged_{sfx}", [P] * 5 + [I64] * 5 + [P])
    assert fn(okv.data_ptr(), ope.data_ptr(), d_d.data_ptr(), kv.data_ptr(), pe.data_ptr(), t, nb, bs, kv_dim,
              pe_dim, _stream()) == 0
    dv = _inside(dslots, nb, bs)
    ko.flat_linear_to_paged(bits(okv), wkv, dv)
    ko.flat_linear_to_paged(bits(ope), wpe, dv)
    assert np.array_equal(bits(kv), wkv) and np.array_equal(bits(pe), wpe)


# ---- FP8 entries (kv_transfer.py:2401-2980) ------------------------------------------------------

LIN = {1: (torch.float16, "float16"), 2: (torch.bfloat16, "bfloat16"), 3: (torch.float32, "float32")}


def _fp8_lin(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * 3
    x.view(-1)[:: 97] *= 200  # saturating values
    return x.to(dtype).to(DEV)


def _scales(kind: str, nl: int, nh: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    rng = np.random.default_rng(seed)
    shape = {"scalar": (1,), "head": (nh,), "layer_head": (nl, nh)}[kind]
    return tuple(torch.from_numpy(rng.uniform(0.005, 0.05, size=shape).astype(np.float32)).to(DEV) for _ in range(2))


def _np_scale(s: torch.Tensor, kind: str) -> np.ndarray:
    a = s.cpu().numpy()
    return a.reshape(()) if kind == "scalar" else a


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("code", [1, 2, 3])
def test_fp8_single_layer_entries(fmt, code):
    dtype, name = LIN[code]
    nh, hd, bs, nb, t = 4, 64, 16, 37, 190
    rng = np.random.default_rng(code)
    for entry, kind, mode in (("", "scalar", None), ("_vec4", "scalar", 0), ("_vec4", "head", 1)):
        ks, vs = _scales(kind, 1, nh, code + 7)
        sk, sv_ = _np_scale(ks, kind), _np_scale(vs, kind)
        # quant-store
        dslots = _slots(rng, nb, bs, t, dup=True)
        d_d, dv = _dev(dslots), _inside(dslots, nb, bs)
        kl, vl = _fp8_lin((t, nh, hd), dtype, 70), _fp8_lin((t, nh, hd), dtype, 71)
        kc, vc = _payload((nb, nh, hd, bs), torch.uint8, 72), _payload((nb, nh, hd, bs), torch.uint8, 73)
        wk, wv = bits(kc).copy(), bits(vc).copy()
        args = [P] * 7 + [I64] * 5 + [I32, P] + ([I32] if mode is not None else [])
        fn = _bind(f"musa_aiter_kv_linear_to_paged_fp8{entry}_{fmt}", args)
        call = [kl.data_ptr(), vl.data_ptr(), d_d.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(),
                vs.data_ptr(), t, nb, nh, hd, bs, code, _stream()] + ([mode] if mode is not None else [])
        assert fn(*call) == 0
        ko.linear_to_paged_fp8(ko.from_storage(bits(kl), name), wk, dv, sk, fmt)
        ko.linear_to_paged_fp8(ko.from_storage(bits(vl), name), wv, dv, sv_, fmt)
        assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv), (entry, kind)
        # dequant-gather
        gslots = _slots(rng, nb, bs, t, dup=False)
        g_d, gv = _dev(gslots), _inside(gslots, nb, bs)
        ok, ov = _payload((t, nh, hd), dtype, 74), _payload((t, nh, hd), dtype, 75)
        args = [P] * 7 + [I64] * 5 + [I32, P] + ([I32] if mode is not None else [])
        fn = _bind(f"musa_aiter_kv_paged_fp8_to_linear{entry}_{fmt}", args)
        call = [kc.data_ptr(), vc.data_ptr(), g_d.data_ptr(), ks.data_ptr(), vs.data_ptr(), ok.data_ptr(),
                ov.data_ptr(), t, nb, nh, hd, bs, code, _stream()] + ([mode] if mode is not None else [])
        assert fn(*call) == 0
        assert np.array_equal(bits(ok), ko.paged_fp8_to_linear(bits(kc), gv, sk, fmt, name)), (entry, kind)
        assert np.array_equal(bits(ov), ko.paged_fp8_to_linear(bits(vc), gv, sv_, fmt, name)), (entry, kind)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("kind,mode", [("scalar", 0), ("head", 1), ("layer_head", 2)])
def test_fp8_multi_layer_entries(fmt, kind, mode):
    nl, nh, hd, bs, nb, t, code = 3, 4, 32, 16, 21, 120, 2
    dtype, name = LIN[code]
    rng = np.random.default_rng(mode)
    ks, vs = _scales(kind, nl, nh, mode + 3)
    sk, sv_ = _np_scale(ks, kind), _np_scale(vs, kind)
    dslots = _slots(rng, nb, bs, t, dup=True)
    d_d, dv = _dev(dslots), _inside(dslots, nb, bs)
    kl, vl = _fp8_lin((nl, t, nh, hd), dtype, 80), _fp8_lin((nl, t, nh, hd), dtype, 81)
    kc, vc = _payload((nl, nb, nh, hd, bs), torch.uint8, 82), _payload((nl, nb, nh, hd, bs), torch.uint8, 83)
    wk, wv = bits(kc).copy(), bits(vc).copy()
    fn = _bind(f"musa_aiter_kv_linear_to_paged_fp8_multi_layer_{fmt}", [P] * 7 + [I64] * 6 + [I32, P, I32])
    assert fn(kl.data_ptr(), vl.data_ptr(), d_d.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(),
              vs.data_ptr(), nl, t, nb, nh, hd, bs, code, _stream(), mode) == 0
    for layer in range(nl):
        lay = layer if kind == "layer_head" else None
        ko.linear_to_paged_fp8(ko.from_storage(bits(kl)[layer], name), wk[layer], dv, sk, fmt, lay)
        ko.linear_to_paged_fp8(ko.from_storage(bits(vl)[layer], name), wv[layer], dv, sv_, fmt, lay)
    assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv)
    gslots = _slots(rng, nb, bs, t, dup=False)
    g_d, gv = _dev(gslots), _inside(gslots, nb, bs)
    ok, ov = _payload((nl, t, nh, hd), dtype, 84), _payload((nl, t, nh, hd), dtype, 85)
    fn = _bind(f"musa_aiter_kv_paged_fp8_to_linear_multi_layer_{fmt}", [P] * 7 + [I64] * 6 + [I32, P, I32])
    assert fn(kc.data_ptr(), vc.data_ptr(), g_d.data_ptr(), ks.data_ptr(), vs.data_ptr(), ok.data_ptr(),
              ov.data_ptr(), nl, t, nb, nh, hd, bs, code, _stream(), mode) == 0
    for layer in range(nl):
        lay = layer if kind == "layer_head" else None
        assert np.array_equal(bits(ok)[layer], ko.paged_fp8_to_linear(bits(kc)[layer], gv, sk, fmt, name, lay))
        assert np.array_equal(bits(ov)[layer], ko.paged_fp8_to_linear(bits(vc)[layer], gv, sv_, fmt, name, lay))


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("variant", ["hd64_bs16", "hd128_bs16", "hd128_bs32"])
@pytest.mark.parametrize("code", [1, 2])
def test_fp8_shape_specialised_gathers(fmt, variant, code):
    hd, bs = {"hd64_bs16": (64, 16), "hd128_bs16": (128, 16), "hd128_bs32": (128, 32)}[variant]
    dtype, name = LIN[code]
    nh, nb, t = 8, 19, 140
    rng = np.random.default_rng(hd + bs + code)
    gslots = _slots(rng, nb, bs, t, dup=False)
    g_d, gv = _dev(gslots), _inside(gslots, nb, bs)
    kc, vc = _payload((nb, nh, hd, bs), torch.uint8, 90), _payload((nb, nh, hd, bs), torch.uint8, 91)
    ks, vs = _scales("scalar", 1, nh, 92)
    ok, ov = _payload((t, nh, hd), dtype, 93), _payload((t, nh, hd), dtype, 94)
    fn = _bind(f"musa_aiter_kv_paged_fp8_to_linear_{variant}_{fmt}", [P] * 7 + [I64] * 3 + [I32, P])
    assert fn(kc.data_ptr(), vc.data_ptr(), g_d.data_ptr(), ks.data_ptr(), vs.data_ptr(), ok.data_ptr(),
              ov.data_ptr(), t, nb, nh, code, _stream()) == 0
    assert np.array_equal(bits(ok), ko.paged_fp8_to_linear(bits(kc), gv, _np_scale(ks, "scalar"), fmt, name))
    assert np.array_equal(bits(ov), ko.paged_fp8_to_linear(bits(vc), gv, _np_scale(vs, "scalar"), fmt, name))


# ---- LMCache 6-D and MLA (lmcache_kv_transfer.py:628-696) ---------------------------------------

@pytest.mark.parametrize("suffix,dtype", [("", torch.float32), ("_u16", torch.bfloat16)])
def test_lmcache_six_d_and_mla_entries(suffix, dtype):
    nl, nb, bs, nh, hs, t = 3, 17, 16, 4, 32, 120
    rng = np.random.default_rng(len(suffix))
    gslots, dslots = _slots(rng, nb, bs, t, dup=False), _slots(rng, nb, bs, t, dup=True)
    g_d, d_d = _dev(gslots), _dev(dslots)
    gv, dv = _inside(gslots, nb, bs), _inside(dslots, nb, bs)
    paged = _payload((nl, 2, nb, bs, nh, hs), dtype, 100)
    buf = _payload((2, nl, t, nh * hs), dtype, 101)
    fn = _bind(f"lmcache_paged_to_kv_buffer{suffix}", [P] * 3 + [I64] * 6 + [P])
    assert fn(paged.data_ptr(), buf.data_ptr(), g_d.data_ptr(), nl, t, nb, bs, nh, hs, _stream()) == 0
    want = np.empty_like(bits(buf))
    ko.six_d_to_buffer(bits(paged), want, gv)
    assert np.array_equal(bits(buf), want)
    wp = bits(paged).copy()
    fn = _bind(f"lmcache_kv_buffer_to_paged{suffix}", [P] * 3 + [I64] * 6 + [P])
    assert fn(buf.data_ptr(), paged.data_ptr(), d_d.data_ptr(), nl, t, nb, bs, nh, hs, _stream()) == 0
    ko.buffer_to_six_d(bits(buf), wp, dv)
    assert np.array_equal(bits(paged), wp)
    # MLA [NL, NB, BS, HS] <-> [NL, T, HS]
    mpaged = _payload((nl, nb, bs, 576), dtype, 102)
    mbuf = _payload((nl, t, 576), dtype, 103)
    fn = _bind(f"lmcache_paged_to_kv_buffer_mla{suffix}", [P] * 3 + [I64] * 5 + [P])
    assert fn(mpaged.data_ptr(), mbuf.data_ptr(), g_d.data_ptr(), nl, t, nb, bs, 576, _stream()) == 0
    want = np.empty_like(bits(mbuf))
    ko.mla_to_buffer(bits(mpaged), want, gv)
    assert np.array_equal(bits(mbuf), want)
    wp = bits(mpaged).copy()
    fn = _bind(f"lmcache_kv_buffer_to_paged_mla{suffix}", [P] * 3 + [I64] * 5 + [P])
    assert fn(mbuf.data_ptr(), mpaged.data_ptr(), d_d.data_ptr(), nl, t, nb, bs, 576, _stream()) == 0
    ko.buffer_to_mla(bits(mbuf), wp, dv)
    assert np.array_equal(bits(mpaged), wp)


# ---- LMCache token-row planes: 2 x NL, coalesced, list, list2, MLA list (lmcache_kv_transfer.py:699-993) --

_gather_rows = ko.native_gather_rows
_scatter_rows = ko.native_scatter_rows


@pytest.mark.parametrize("suffix,dtype", [("float", torch.float32), ("u16", torch.float16)])
@pytest.mark.parametrize("skip", [0, 5])
def test_two_x_nl_and_coalesced_entries(suffix, dtype, skip):
    nl, nb, bs, nh, hs, t = 3, 13, 16, 8, 16, 100
    hidden, m = nh * hs, t + skip + 7
    rng = np.random.default_rng(skip)
    gslots, dslots = _slots(rng, nb, bs, t, dup=False), _slots(rng, nb, bs, t, dup=True)
    g_d, d_d = _dev(gslots), _dev(dslots)
    gv, dv = _inside(gslots, nb, bs), _inside(dslots, nb, bs)
    caches = [[_payload((nb, bs, nh, hs), dtype, 110 + 10 * a + layer) for layer in range(nl)] for a in range(2)]
    mem = _payload((2, nl, m, hidden), dtype, 120)
    want = bits(mem).copy()
    fn = _bind(f"lmcache_paged_to_kv_buffer_two_x_nl_{suffix}", [P] * 3 + [I64] * 10 + [P])
    for a in range(2):
        for layer in range(nl):
            assert fn(mem.data_ptr(), caches[a][layer].data_ptr(), g_d.data_ptr(), a, layer, nl, m, t, skip, nb, bs,
                      nh, hs, _stream()) == 0
            _gather_rows(bits(caches[a][layer]).reshape(nb * bs, hidden), gv, want[a, layer], skip)
    assert np.array_equal(bits(mem), want)
    wc = [[bits(c).copy().reshape(nb * bs, hidden) for c in group] for group in caches]
    fn = _bind(f"lmcache_kv_buffer_to_paged_two_x_nl_{suffix}", [P] * 3 + [I64] * 10 + [P])
    for a in range(2):
        for layer in range(nl):
            assert fn(mem.data_ptr(), caches[a][layer].data_ptr(), d_d.data_ptr(), a, layer, nl, m, t, skip, nb, bs,
                      nh, hs, _stream()) == 0
            _scatter_rows(want[a, layer], dv, wc[a][layer], skip)
    for a in range(2):
        for layer in range(nl):
            assert np.array_equal(bits(caches[a][layer]).reshape(nb * bs, hidden), wc[a][layer])
    if suffix != "u16":
        return
    # coalesced: all 2 x NL planes in one launch, K layers then V layers in a host pointer array
    ptrs = (ctypes.c_uint64 * (2 * nl))(*[c.data_ptr() for group in caches for c in group])
    mem = _payload((2, nl, m, hidden), dtype, 121)
    want = bits(mem).copy()
    fn = _bind("lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16",
               [P, ctypes.POINTER(ctypes.c_uint64), P] + [I64] * 7 + [P])
    assert fn(mem.data_ptr(), ptrs, g_d.data_ptr(), nl, m, t, nb, bs, nh, hs, _stream()) == 0
    for a in range(2):
        for layer in range(nl):
            _gather_rows(bits(caches[a][layer]).reshape(nb * bs, hidden), gv, want[a, layer], 0)
    assert np.array_equal(bits(mem), want)
    wc = [[bits(c).copy().reshape(nb * bs, hidden) for c in group] for group in caches]
    fn = _bind("lmcache_kv_buffer_to_paged_two_x_nl_coalesced_u16",
               [P, ctypes.POINTER(ctypes.c_uint64), P] + [I64] * 8 + [P])
    assert fn(mem.data_ptr(), ptrs, d_d.data_ptr(), nl, m, t, skip, nb, bs, nh, hs, _stream()) == 0
    for a in range(2):
        for layer in range(nl):
            _scatter_rows(want[a, layer], dv, wc[a][layer], skip)
            assert np.array_equal(bits(caches[a][layer]).reshape(nb * bs, hidden), wc[a][layer])


@pytest.mark.parametrize("suffix,dtype", [("float", torch.float32), ("u16", torch.bfloat16)])
def test_list_and_list2_entries(suffix, dtype):
    nl, nb, bs, nh, hs, t, skip = 2, 11, 16, 4, 32, 90, 3
    hidden, m = nh * hs, t + skip + 4
    rng = np.random.default_rng(7)
    gslots, dslots = _slots(rng, nb, bs, t, dup=False), _slots(rng, nb, bs, t, dup=True)
    g_d, d_d = _dev(gslots), _dev(dslots)
    gv, dv = _inside(gslots, nb, bs), _inside(dslots, nb, bs)
    kv = [_payload((2, nb, bs, nh, hs), dtype, 130 + layer) for layer in range(nl)]
    mem = _payload((2, nl, m, hidden), dtype, 140)
    want = bits(mem).copy()
    fn = _bind(f"lmcache_paged_to_kv_buffer_list_{suffix}", [P] * 3 + [I64] * 9 + [P])
    for layer in range(nl):
        assert fn(mem.data_ptr(), kv[layer].data_ptr(), g_d.data_ptr(), layer, nl, m, t, skip, nb, bs, nh, hs,
                  _stream()) == 0
        for a in range(2):
            _gather_rows(bits(kv[layer])[a].reshape(nb * bs, hidden), gv, want[a, layer], skip)
    assert np.array_equal(bits(mem), want)
    wkv = [bits(c).copy().reshape(2, nb * bs, hidden) for c in kv]
    fn = _bind(f"lmcache_kv_buffer_to_paged_list_{suffix}", [P] * 3 + [I64] * 9 + [P])
    for layer in range(nl):
        assert fn(mem.data_ptr(), kv[layer].data_ptr(), d_d.data_ptr(), layer, nl, m, t, skip, nb, bs, nh, hs,
                  _stream()) == 0
        for a in range(2):
            _scatter_rows(want[a, layer], dv, wkv[layer][a], skip)
    for layer in range(nl):
        assert np.array_equal(bits(kv[layer]).reshape(2, nb * bs, hidden), wkv[layer])
    if suffix != "u16":
        return
    mem = _payload((2, 2, m, hidden), dtype, 141)
    want = bits(mem).copy()
    fn = _bind("lmcache_paged_to_kv_buffer_list2_u16", [P] * 4 + [I64] * 7 + [P])
    assert fn(mem.data_ptr(), kv[0].data_ptr(), kv[1].data_ptr(), g_d.data_ptr(), m, t, skip, nb, bs, nh, hs,
              _stream()) == 0
    for layer in range(2):
        for a in range(2):
            _gather_rows(bits(kv[layer])[a].reshape(nb * bs, hidden), gv, want[a, layer], skip)
    assert np.array_equal(bits(mem), want)
    wkv = [bits(c).copy().reshape(2, nb * bs, hidden) for c in kv]
    fn = _bind("lmcache_kv_buffer_to_paged_list2_u16", [P] * 4 + [I64] * 7 + [P])
    assert fn(mem.data_ptr(), kv[0].data_ptr(), kv[1].data_ptr(), d_d.data_ptr(), m, t, skip, nb, bs, nh, hs,
              _stream()) == 0
    for layer in range(2):
        for a in range(2):
            _scatter_rows(want[a, layer], dv, wkv[layer][a], skip)
        assert np.array_equal(bits(kv[layer]).reshape(2, nb * bs, hidden), wkv[layer])


@pytest.mark.parametrize("variant", ["coalesced", "contiguous", "contiguous_bulk", "torchmusa_style", "sorted"])
def test_list2_kernel_variant_entries(variant):
    # The reference extension's list2 kernel variants (lmcache_kv_transfer_ext.cpp:42-125), called with its
    # argument orders; the sorted gather also receives the int32 sort order the extension computes.
    nb, bs, nh, hs, t, skip = 11, 16, 4, 32, 90, 3
    hidden, m = nh * hs, t + skip + 4
    rng = np.random.default_rng(9)
    gslots, dslots = _slots(rng, nb, bs, t, dup=False), _slots(rng, nb, bs, t, dup=True)
    g_d, d_d = _dev(gslots), _dev(dslots)
    gv, dv = _inside(gslots, nb, bs), _inside(dslots, nb, bs)
    kv = [_payload((2, nb, bs, nh, hs), torch.bfloat16, 150 + layer) for layer in range(2)]
    mem = _payload((2, 2, m, hidden), torch.bfloat16, 160)
    want = bits(mem).copy()
    name = f"lmcache_paged_to_kv_buffer_list2_u16_{variant}"
    if variant == "sorted":
        order = torch.sort(g_d, stable=False).indices.to(torch.int32)
        fn = _bind(name, [P] * 5 + [I64] * 7 + [P])
        rc = fn(mem.data_ptr(), kv[0].data_ptr(), kv[1].data_ptr(), g_d.data_ptr(), order.data_ptr(), m, t, skip, nb,
                bs, nh, hs, _stream())
    else:
        fn = _bind(name, [P] * 4 + [I64] * 7 + [P])
        rc = fn(mem.data_ptr(), kv[0].data_ptr(), kv[1].data_ptr(), g_d.data_ptr(), m, t, skip, nb, bs, nh, hs,
                _stream())
    assert rc == 0
    for layer in range(2):
        for a in range(2):
            _gather_rows(bits(kv[layer])[a].reshape(nb * bs, hidden), gv, want[a, layer], skip)
    assert np.array_equal(bits(mem), want)
    if variant != "coalesced":
        return
    wkv = [bits(c).copy().reshape(2, nb * bs, hidden) for c in kv]
    fn = _bind("lmcache_kv_buffer_to_paged_list2_u16_coalesced", [P] * 4 + [I64] * 7 + [P])
    assert fn(mem.data_ptr(), kv[0].data_ptr(), kv[1].data_ptr(), d_d.data_ptr(), m, t, skip, nb, bs, nh, hs,
              _stream()) == 0
    for layer in range(2):
        for a in range(2):
            _scatter_rows(want[a, layer], dv, wkv[layer][a], skip)
        assert np.array_equal(bits(kv[layer]).reshape(2, nb * bs, hidden), wkv[layer])


@pytest.mark.parametrize("suffix,dtype", [("float", torch.float32), ("half", torch.float16),
                                          ("bfloat16", torch.bfloat16), ("u16", torch.bfloat16)])
def test_mla_list_entries(suffix, dtype):
    nl, nb, bs, hs, t, skip = 3, 9, 64, 576, 300, 6
    m = t + skip + 2
    rng = np.random.default_rng(11)
    gslots, dslots = _slots(rng, nb, bs, t, dup=False), _slots(rng, nb, bs, t, dup=True)
    g_d, d_d = _dev(gslots), _dev(dslots)
    gv, dv = _inside(gslots, nb, bs), _inside(dslots, nb, bs)
    kv = [_payload((nb, bs, hs), dtype, 150 + layer) for layer in range(nl)]
    mem = _payload((1, nl, m, hs), dtype, 160)
    want = bits(mem).copy()
    fn = _bind(f"lmcache_mla_paged_to_buffer_list_{suffix}", [P] * 3 + [I64] * 6 + [P])
    for layer in range(nl):
        assert fn(mem.data_ptr(), kv[layer].data_ptr(), g_d.data_ptr(), layer, m, t, nb, bs, hs, _stream()) == 0
        _gather_rows(bits(kv[layer]).reshape(nb * bs, hs), gv, want[0, layer], 0)
    assert np.array_equal(bits(mem), want)
    wkv = [bits(c).copy().reshape(nb * bs, hs) for c in kv]
    fn = _bind(f"lmcache_mla_buffer_to_paged_list_{suffix}", [P] * 3 + [I64] * 7 + [P])
    for layer in range(nl):
        assert fn(mem.data_ptr(), kv[layer].data_ptr(), d_d.data_ptr(), layer, m, t, skip, nb, bs, hs,
                  _stream()) == 0
        _scatter_rows(want[0, layer], dv, wkv[layer], skip)
        assert np.array_equal(bits(kv[layer]).reshape(nb * bs, hs), wkv[layer])


# ---- DSV4 byte rows (kv_transfer.py:4209-4406) ---------------------------------------------------

@pytest.mark.parametrize("item", [656, 1152, 37])
def test_byte_row_entries(item):
    nl, src_rows, dst_rows, n = 3, 300, 280, 200
    rng = np.random.default_rng(item)
    sidx = rng.integers(-5, src_rows + 5, size=n).astype(np.int64)
    didx = rng.permutation(dst_rows + 40)[:n].astype(np.int64) - 20  # unique, some outside [0, dst_rows)
    ok_rows = (sidx >= 0) & (sidx < src_rows) & (didx >= 0) & (didx < dst_rows)
    s_d, di_d = _dev(sidx), _dev(didx)
    src = _payload((nl, src_rows, item), torch.uint8, 170)
    dst = _payload((nl, dst_rows, item), torch.uint8, 171)
    sb = bits(src)
    want = bits(dst).copy()
    for layer in range(nl):
        ko.copy_rows(sb[layer], want[layer], sidx[ok_rows], didx[ok_rows])
    fn = _bind("musa_aiter_kv_copy_paged_rows_u8", [P] * 4 + [I64] * 4 + [P])
    got = dst.clone()
    assert fn(src[1].data_ptr(), got[1].data_ptr(), s_d.data_ptr(), di_d.data_ptr(), n, item, src_rows, dst_rows,
              _stream()) == 0
    assert np.array_equal(bits(got)[1], want[1]) and np.array_equal(bits(got)[0], bits(dst)[0])
    got = dst.clone()
    st = _dev(np.array([src[layer].data_ptr() for layer in range(nl)], dtype=np.uint64).view(np.int64))
    dt = _dev(np.array([got[layer].data_ptr() for layer in range(nl)], dtype=np.uint64).view(np.int64))
    fn = _bind("musa_aiter_kv_copy_paged_rows_layer_table_u8", [P] * 4 + [I64] * 5 + [P])
    assert fn(st.data_ptr(), dt.data_ptr(), s_d.data_ptr(), di_d.data_ptr(), n, item, nl, src_rows, dst_rows,
              _stream()) == 0
    assert np.array_equal(bits(got), want)
    got = dst.clone()
    fn = _bind("musa_aiter_kv_copy_paged_rows_contig_layers_u8", [P] * 4 + [I64] * 5 + [P])
    assert fn(src.data_ptr(), got.data_ptr(), s_d.data_ptr(), di_d.data_ptr(), n, item, nl, src_rows, dst_rows,
              _stream()) == 0
    assert np.array_equal(bits(got), want)


# ---- dense preload and block copies: every element suffix (kv_transfer.py:1220-1524, :1962-2032) --

@pytest.mark.parametrize("dtype", DTYPES)
def test_dense_and_block_copy_entries_every_suffix(dtype):
    sfx, nh, hd, bs = SUFFIX[dtype], 4, 32, 16
    rng = np.random.default_rng(13)
    seq_lens = np.array([37, 0, 16, 50], dtype=np.int64)
    nb = 20
    tables = rng.permutation(nb)[:16].reshape(4, 4).astype(np.int64)
    dense_len = 52
    kc, vc = _payload((nb, nh, hd, bs), dtype, 180), _payload((nb, nh, hd, bs), dtype, 181)
    t_d, l_d = _dev(tables), _dev(seq_lens)
    ok, ov = _payload((4, dense_len, nh, hd), dtype, 182), _payload((4, dense_len, nh, hd), dtype, 183)
    fn = _bind(f"musa_aiter_kv_load_and_reshape_flash_{sfx}", [P] * 6 + [I64] * 7 + [P])
    assert fn(kc.data_ptr(), vc.data_ptr(), t_d.data_ptr(), l_d.data_ptr(), ok.data_ptr(), ov.data_ptr(), 4,
              dense_len, 4, nb, nh, hd, bs, _stream()) == 0
    assert np.array_equal(bits(ok), ko.load_and_reshape_flash(bits(kc), tables, seq_lens, dense_len))
    assert np.array_equal(bits(ov), ko.load_and_reshape_flash(bits(vc), tables, seq_lens, dense_len))
    wk, wv = bits(kc).copy(), bits(vc).copy()
    dk, dv = _payload((4, dense_len, nh, hd), dtype, 184), _payload((4, dense_len, nh, hd), dtype, 185)
    fn = _bind(f"musa_aiter_kv_reshape_and_cache_back_flash_{sfx}", [P] * 6 + [I64] * 7 + [P])
    assert fn(dk.data_ptr(), dv.data_ptr(), t_d.data_ptr(), l_d.data_ptr(), kc.data_ptr(), vc.data_ptr(), 4,
              dense_len, 4, nb, nh, hd, bs, _stream()) == 0
    ko.reshape_and_cache_back_flash(bits(dk), wk, tables, seq_lens)
    ko.reshape_and_cache_back_flash(bits(dv), wv, tables, seq_lens)
    assert np.array_equal(bits(kc), wk) and np.array_equal(bits(vc), wv)
    # CSR rows of token-major caches
    ntok = 90
    tk, tv = _payload((ntok, nh, hd), dtype, 186), _payload((ntok, nh, hd), dtype, 187)
    indptr = np.array([0, 10, 10, 40, 75], dtype=np.int64)
    indices = rng.integers(-2, ntok + 3, size=75).astype(np.int64)
    ip_d, ix_d = _dev(indptr), _dev(indices)
    ok, ov = _payload((4, 32, nh, hd), dtype, 188), _payload((4, 32, nh, hd), dtype, 189)
    fn = _bind(f"musa_aiter_kv_triton_indexed_to_dense_{sfx}", [P] * 6 + [I64] * 6 + [P])
    assert fn(tk.data_ptr(), tv.data_ptr(), ip_d.data_ptr(), ix_d.data_ptr(), ok.data_ptr(), ov.data_ptr(), 4, 32,
              75, ntok, nh, hd, _stream()) == 0
    assert np.array_equal(bits(ok), ko.triton_indexed_to_dense(bits(tk), indptr, indices, 32))
    assert np.array_equal(bits(ov), ko.triton_indexed_to_dense(bits(tv), indptr, indices, 32))
    # whole-block copies, multi-layer caches
    pairs = np.array([[3, 0], [7, 2], [1, 5], [2, 2], [0, 9]], dtype=np.int64)
    sk, sv_ = _payload((2, 8, nh, hd, bs), dtype, 190), _payload((2, 8, nh, hd, bs), dtype, 191)
    dk, dv = _payload((2, 10, nh, hd, bs), dtype, 192), _payload((2, 10, nh, hd, bs), dtype, 193)
    wk, wv = bits(dk).copy(), bits(dv).copy()
    m_d = _dev(pairs)
    fn = _bind(f"musa_aiter_kv_copy_paged_blocks_{sfx}", [P] * 5 + [I64] * 7 + [P])
    assert fn(sk.data_ptr(), sv_.data_ptr(), dk.data_ptr(), dv.data_ptr(), m_d.data_ptr(), len(pairs), 2, 8, 10, nh,
              hd, bs, _stream()) == 0
    ko.copy_paged_blocks(bits(sk), wk, pairs, multi_layer=True)
    ko.copy_paged_blocks(bits(sv_), wv, pairs, multi_layer=True)
    assert np.array_equal(bits(dk), wk) and np.array_equal(bits(dv), wv)


# ---- ABI probes (kv_transfer_float.mu:3021-3027, fp8_kv_cache.mu:1529-1531, hicache_transfer.mu:53-55) --

def test_abi_probes():
    lib = _hip.library()
    for name in ("musa_aiter_kv_transfer_abi_version", "native_lmcache_kv_transfer_abi_version",
                 "musa_aiter_fp8_kv_cache_abi_version", "musa_aiter_dsv4_kv_copy_abi_version",
                 "musa_aiter_hicache_transfer_abi_version", "musa_aiter_hip_batch_copy_abi_version"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        assert fn() == 1, name
    fn = lib.musa_aiter_hip_backend_name
    fn.restype = ctypes.c_char_p
    assert fn() == b"rocm-hip"
    fn = lib.musa_aiter_hip_error_string
    fn.argtypes, fn.restype = [ctypes.c_int], ctypes.c_char_p
    assert fn(0) and fn(1)
    rt, drv = ctypes.c_int(0), ctypes.c_int(0)
    fn = lib.musa_aiter_hip_runtime_versions
    fn.restype = ctypes.c_int
    assert fn(ctypes.byref(rt), ctypes.byref(drv)) == 0 and rt.value > 0 and drv.value > 0
