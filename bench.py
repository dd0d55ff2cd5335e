#!/usr/bin/env python3
"""KV-copy throughput on one MI355X: BASELINE.json configs[1] (headline) plus configs 1, 3, 4, 5, the dense preload,
the SGLang HiCache transfers, the LMCache host <-> device copy batches and the CacheGen codec.

Headline workload: 32 layers of Llama-3-8B KV caches
[8192 blocks, 16, 8 kv-heads, 128] bf16 (paged layout [NB, NH, HD, BS]),
64 sequences with lengths uniform in [128, 4096] (redrawn with a fixed seed
until they fit), int64 slot mappings from random block tables, N(0,1) data.
One step = the multi-layer linear->paged scatter followed by the reverse
paged->linear gather, each a single call of the library's C-ABI
(musa_aiter_kv_linear_to_paged_multi_layer_bfloat16 /
musa_aiter_kv_paged_to_linear_multi_layer_bfloat16) on torch's current
stream.  Inputs are resident in HBM before timing; host-side validation runs
once, outside the timed region.

``value`` = algorithmic bytes (payload read + payload written + 8 B per slot)
of K steps / device time of the K steps between HIP events, in GB/s.
``roofline`` is reported for the dominant kernel (the direction with the
larger total time) against the 8 TB/s HBM peak; its ``traffic`` comes from the
committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes.  ``ceilings`` times, on the
same caches and linear buffers, a plain whole-block copy in each kernel's own
visiting order (the gather: cache blocks read in the order the slot mapping
visits them, the linear side written in order; the scatter: cache blocks
written in block order, each block's linear rows read wherever they are; and,
for reference, the scatter's token order): the rate that access pattern allows
a copy with no index work, which the two kernels are measured against.  Each ceiling and
floor is timed with non-temporal and with write-through stores and keeps the
faster.  ``placements``
re-allocates the caches several times in this process and times the step on
each, because where the caches land moves the rate by several percent.
``cpu_baseline`` times the reference's own torch operations
(oracle/torch_cpu_port.py, a port of kv_transfer.py:3047-3112) on this host's
cores: configs[1] on a prefix of its tokens, configs[0] at full shape, and a
vectorised torch line.

The other configs are reported under ``extra`` with the same byte convention
(config 6: the block-table / CSR dense preload for attention and whole-block
copies; config 7: SGLang HiCache layer-first / page-first transfers; config 8:
LMCache host <-> device copy batches, rated against the 64 GB/s PCIe 5.0 x16
link instead of HBM; config 9: the CacheGen-style codec; none is a BASELINE
config).  Their launches are short
(0.01-0.8 ms), so they are timed in batches of back-to-back launches between
two events (host launch overhead hidden behind device work); each is also
checked outside the timed region, by torch indexing, by the reference's FP8
steps restated in torch (tests/torch_ref.py) or by a round trip.  The numpy
oracle runs only in the CPU-baseline leg.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "musa-aiter_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
HOST_LINK_GBS = 64.0  # PCIe 5.0 x16, per direction
METRIC = "KV copy HBM GB/s & % of 8 TB/s peak, paged↔linear/FP8, 1 MI355X"
NL, NB, BS, NH, HD = 32, 8192, 16, 8, 128
ROW = NH * HD  # elements per K or V token row


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_slots(seed: int, num_seqs: int, lo: int, hi: int, num_blocks: int, block_size: int) -> np.ndarray:
    from tests.kvgen import sequence_lengths, sequence_slots

    rng = np.random.default_rng(seed)
    lengths = sequence_lengths(rng, num_seqs, lo, hi, num_blocks=num_blocks, block_size=block_size)
    return sequence_slots(rng, lengths, num_blocks=num_blocks, block_size=block_size)


def make_covering_slots(seed: int, tokens: int, lo: int, hi: int, num_blocks: int, block_size: int) -> np.ndarray:
    """Slots of random sequences (lengths uniform in [lo, hi]) drawn until ``tokens`` are covered, truncated."""
    from tests.kvgen import sequence_slots

    rng = np.random.default_rng(seed)
    lengths, covered = [], 0
    while covered < tokens:
        lengths.append(int(rng.integers(lo, hi + 1)))
        covered += lengths[-1]
    lengths[-1] -= covered - tokens
    return sequence_slots(rng, lengths, num_blocks=num_blocks, block_size=block_size)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "kv_kernels_hbm_traffic.md")


def profiled_traffic(direction: str) -> int | None:
    """HBM bytes per launch of a profiled kernel (cfg 2 scatter/gather, cfg 3 FP8 quant/dequant, cfg 1 gather, one
    cfg 4 chunk gather), from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by the plain-copy calibration); None if absent."""
    try:
        with open(TRAFFIC_PROFILE) as fh:
            text = fh.read()
    except OSError:
        return None
    m = re.search(rf"traffic_bytes_per_launch\.{direction} = (\d+)", text)
    return int(m.group(1)) if m else None


class EventTimer:
    """Accumulates device time between HIP events recorded on torch's current stream."""

    def __init__(self):
        self.pairs: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []

    def start(self) -> torch.cuda.Event:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def stop(self, start: torch.cuda.Event) -> None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self.pairs.append((start, ev))

    def ms(self) -> list[float]:
        return [a.elapsed_time(b) for a, b in self.pairs]


def batched_ms(fn, launches: int = 20, reps: int = 5) -> np.ndarray:
    """Per-launch device ms of ``fn`` from ``reps`` batches of ``launches`` back-to-back calls."""
    per = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(launches):
            fn()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / launches)
    return np.array(per)


def rate(nbytes: int, ms: np.ndarray, tokens: int | None = None) -> dict:
    out = {"p50_ms": float(np.median(ms)), "min_ms": float(ms.min()), "max_ms": float(ms.max()),
           "gbs": nbytes / (np.median(ms) * 1e-3) / 1e9}
    out["pct_of_peak"] = round(100.0 * out["gbs"] / HBM_PEAK_GBS, 2)
    if tokens is not None:
        out["tokens_per_ms"] = tokens / float(np.median(ms))
    return out


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _bind(lib, name: str, nargs_ptr: int, nargs_i64: int):
    fn = getattr(lib, name)
    fn.argtypes = [ctypes.c_void_p] * nargs_ptr + [ctypes.c_int64] * nargs_i64 + [ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{name} returned HIP error {rc}")


def run_blocks(slots_np: np.ndarray, block_size: int) -> np.ndarray:
    """Cache blocks in the order a slot mapping first visits them (skipped tokens ignored)."""
    blk = slots_np[slots_np >= 0] // block_size
    first = np.unique(blk, return_index=True)[1]
    return blk[np.sort(first)].astype(np.int32)


def pattern_copy_fn(src: torch.Tensor, dst: torch.Tensor, *, src_blocks, dst_blocks, num_blocks: int,
                    src_region_blocks: int, dst_region_blocks: int, src_block_bytes: int, dst_block_bytes: int,
                    planes: int, src_plane_stride: int, dst_plane_stride: int, write_through: bool = False):
    """A launcher of the library's block-pattern copy (musa_aiter_hip_block_pattern_copy): whole blocks in the
    given order, no index resolution or transpose, on the caller's own buffers -- the access-pattern ceiling.
    ``write_through`` selects agent-scope stores (through the L2) over plain non-temporal ones."""
    from musa_aiter.ops import _hip

    fn = getattr(_hip.library(), "musa_aiter_hip_block_pattern_copy")
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 8 + [ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    sb = src_blocks.data_ptr() if src_blocks is not None else None
    db = dst_blocks.data_ptr() if dst_blocks is not None else None
    args = (src.data_ptr(), dst.data_ptr(), sb, db, num_blocks, src_region_blocks, dst_region_blocks,
            src_block_bytes, dst_block_bytes, planes, src_plane_stride, dst_plane_stride, int(write_through))
    return lambda: _check(fn(*args, _stream()), "block pattern copy")


ROTATE = 6  # FP8 cache sets rotated through by the configs[2] timings (see bench_config3)


def rotating(call, n: int):
    """A callable that runs ``call(i)`` with i = 0, 1, .., n - 1, 0, .. on successive calls."""
    state = [0]

    def run():
        call(state[0] % n)
        state[0] += 1
    return run


def _run_all(fns):
    """One callable that launches ``fns`` in order."""
    def run():
        for f in fns:
            f()
    return run


def pattern_rate(make, nbytes: int, per_call: int = 1, **timing) -> dict:
    """The faster store policy of a block-pattern copy: ``make(write_through)`` returns the launcher (of
    ``per_call`` copies, each of ``nbytes``).  The ceiling is the better plain copy; both rates are kept."""
    by = {}
    for wt in (False, True):
        f = make(wt)
        f()
        by["write_through" if wt else "non_temporal"] = rate(nbytes, batched_ms(f, **timing) / per_call)
    best = max(by, key=lambda k: by[k]["gbs"])
    return {**by[best], "store_policy": best, "gbs_by_store_policy": {k: v["gbs"] for k, v in by.items()}}


def config2_ceilings(slots_np: np.ndarray, kc: torch.Tensor, vc: torch.Tensor, kl: torch.Tensor,
                     vl: torch.Tensor) -> dict:
    """Access-pattern ceilings of the configs[1] copies, on the same caches and linear buffers: whole 32 KiB
    blocks of all 64 planes, cache blocks in the order the slot mapping visits them (random) and linear
    blocks in order -- read random / write in order (the gather's pattern), the reverse (the scatter's),
    and both in order (a plain copy of the same bytes)."""
    dev = kc.device
    t = int(slots_np.shape[0])
    order_np = run_blocks(slots_np, BS)
    nblk = min(order_np.size, t // BS)
    order = torch.from_numpy(order_np[:nblk].copy()).to(dev)
    # The scatter writes cache blocks in block order (its block-major kernel), reading each block's
    # linear rows wherever they are: sorted destinations, linear blocks in the matching order.
    by_dst = np.argsort(order_np[:nblk], kind="stable")
    dst_sorted = torch.from_numpy(order_np[:nblk][by_dst].astype(np.int32)).to(dev)
    src_by_dst = torch.from_numpy(by_dst.astype(np.int32)).to(dev)
    blk_bytes = ROW * BS * 2
    cache_stride, lin_stride = NB * blk_bytes, t * ROW * 2
    legs = {
        "gather_pattern": dict(src=(kc, vc), dst=(kl, vl), src_blocks=order, dst_blocks=None,
                               src_region_blocks=NB, dst_region_blocks=t // BS, src_plane_stride=cache_stride,
                               dst_plane_stride=lin_stride),
        "scatter_pattern": dict(src=(kl, vl), dst=(kc, vc), src_blocks=src_by_dst, dst_blocks=dst_sorted,
                                src_region_blocks=t // BS, dst_region_blocks=NB, src_plane_stride=lin_stride,
                                dst_plane_stride=cache_stride),
        "scatter_token_order_pattern": dict(src=(kl, vl), dst=(kc, vc), src_blocks=None, dst_blocks=order,
                                            src_region_blocks=t // BS, dst_region_blocks=NB,
                                            src_plane_stride=lin_stride, dst_plane_stride=cache_stride),
        "sequential": dict(src=(kc, vc), dst=(kl, vl), src_blocks=None, dst_blocks=None, src_region_blocks=NB,
                           dst_region_blocks=t // BS, src_plane_stride=cache_stride, dst_plane_stride=lin_stride),
    }
    nbytes = 2 * NL * nblk * blk_bytes * 2
    out = {"blocks_per_plane": nblk, "planes": 2 * NL, "bytes_per_launch_pair": nbytes,
           "shape": "one wave per 1 KiB (16 B per lane), whole 32 KiB blocks, K and V caches one launch each"}
    for name, leg in legs.items():
        def make(wt, leg=leg):
            return _run_all([pattern_copy_fn(src, dst, src_blocks=leg["src_blocks"], dst_blocks=leg["dst_blocks"],
                                             num_blocks=nblk, src_region_blocks=leg["src_region_blocks"],
                                             dst_region_blocks=leg["dst_region_blocks"], src_block_bytes=blk_bytes,
                                             dst_block_bytes=blk_bytes, planes=NL,
                                             src_plane_stride=leg["src_plane_stride"],
                                             dst_plane_stride=leg["dst_plane_stride"], write_through=wt)
                             for src, dst in zip(leg["src"], leg["dst"])])

        out[name] = pattern_rate(make, nbytes, launches=5, reps=5)
    g, sc = out["gather_pattern"]["gbs"], out["scatter_pattern"]["gbs"]
    out["step_ceiling_gbs"] = 2.0 / (1.0 / g + 1.0 / sc)
    log(f"config 2 ceilings: gather pattern {g:.0f}, scatter pattern {sc:.0f} (cache blocks in token order "
        f"{out['scatter_token_order_pattern']['gbs']:.0f}), sequential {out['sequential']['gbs']:.0f}, step "
        f"{out['step_ceiling_gbs']:.0f} GB/s")
    return out


def config2_placements(slots: torch.Tensor, kl: torch.Tensor, vl: torch.Tensor, ok: torch.Tensor,
                       ov: torch.Tensor, placements: int, steps: int) -> dict:
    """The configs[1] step on freshly allocated caches, ``placements`` times in this process, each behind a
    pad allocation of a different size (the caches land at different device addresses), all other buffers
    unchanged: the spread of the step rate with where the caches land."""
    from musa_aiter.ops import _hip

    dev = kl.device
    t = int(slots.shape[0])
    scatter = _bind(_hip.library(), "musa_aiter_kv_linear_to_paged_multi_layer_bfloat16", 5, 6)
    gather = _bind(_hip.library(), "musa_aiter_kv_paged_to_linear_multi_layer_bfloat16", 5, 6)
    per_dir = 2 * (2 * NL * t * ROW * 2) + 8 * t
    runs = []
    for i in range(placements):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        pad = torch.empty(((i * 7 + 1) % 16) * (200 << 20) + (i << 20), dtype=torch.uint8, device=dev)
        kc = torch.empty((NL, NB, NH, HD, BS), device=dev, dtype=torch.bfloat16).normal_()
        vc = torch.empty((NL, NB, NH, HD, BS), device=dev, dtype=torch.bfloat16).normal_()
        sa = (kl.data_ptr(), vl.data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), NL, t, NB, NH, HD, BS)
        ga = (kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), ok.data_ptr(), ov.data_ptr(), NL, t, NB, NH, HD, BS)
        for _ in range(2):
            _check(scatter(*sa, _stream()), "scatter")
            _check(gather(*ga, _stream()), "gather")
        torch.cuda.synchronize()
        ts, tg = EventTimer(), EventTimer()
        for _ in range(steps):
            e = ts.start()
            _check(scatter(*sa, _stream()), "scatter")
            ts.stop(e)
            e = tg.start()
            _check(gather(*ga, _stream()), "gather")
            tg.stop(e)
        torch.cuda.synchronize()
        ms_s, ms_g = float(np.mean(ts.ms())), float(np.mean(tg.ms()))
        runs.append({"pad_bytes": int(pad.numel()), "cache_address": hex(kc.data_ptr()), "scatter_ms": ms_s,
                     "gather_ms": ms_g, "step_gbs": 2 * per_dir / ((ms_s + ms_g) * 1e-3) / 1e9})
        del kc, vc, pad
    torch.cuda.empty_cache()
    vals = np.array([r["step_gbs"] for r in runs])
    out = {"placements": placements, "steps_each": steps, "step_gbs_min": float(vals.min()),
           "step_gbs_median": float(np.median(vals)), "step_gbs_max": float(vals.max()), "runs": runs}
    log(f"config 2 placements: step {out['step_gbs_min']:.0f} / {out['step_gbs_median']:.0f} / "
        f"{out['step_gbs_max']:.0f} GB/s (min / median / max of {placements})")
    return out


def bench_config2(steps: int, warmup: int) -> dict:
    """Multi-layer bf16 paged<->linear scatter + gather."""
    import musa_aiter
    from musa_aiter.ops import _hip

    dev = torch.device("cuda", 0)
    slots_np = make_slots(1002, 64, 128, 4096, NB, BS)
    t = int(slots_np.shape[0])
    log(f"config 2: T={t} tokens, {NL} layers, caches 2 x {NL * NB * ROW * BS * 2 / 2**30:.1f} GiB")
    gen = torch.Generator(device=dev).manual_seed(2)
    slots = torch.from_numpy(slots_np).to(dev)
    kl = torch.randn((NL, t, NH, HD), generator=gen, device=dev, dtype=torch.bfloat16)
    vl = torch.randn((NL, t, NH, HD), generator=gen, device=dev, dtype=torch.bfloat16)
    kc = torch.randn((NL, NB, NH, HD, BS), generator=gen, device=dev, dtype=torch.bfloat16)
    vc = torch.randn((NL, NB, NH, HD, BS), generator=gen, device=dev, dtype=torch.bfloat16)
    ok = torch.empty_like(kl)
    ov = torch.empty_like(vl)

    # Validated public-API pass (not timed): scatter then gather must give the input back.
    musa_aiter.kv_linear_to_paged_multi_layer(kl, vl, kc, vc, slots)
    musa_aiter.kv_paged_to_linear_multi_layer(kc, vc, slots, out_k=ok, out_v=ov)
    torch.cuda.synchronize()
    parity = bool(torch.equal(ok, kl) and torch.equal(ov, vl))
    log(f"config 2 round-trip parity: {parity}")

    lib = _hip.library()
    scatter = _bind(lib, "musa_aiter_kv_linear_to_paged_multi_layer_bfloat16", 5, 6)
    gather = _bind(lib, "musa_aiter_kv_paged_to_linear_multi_layer_bfloat16", 5, 6)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    s_args = (kl.data_ptr(), vl.data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), NL, t, NB, NH, HD, BS,
              stream)
    g_args = (kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), ok.data_ptr(), ov.data_ptr(), NL, t, NB, NH, HD, BS,
              stream)
    for _ in range(warmup):
        _check(scatter(*s_args), "scatter")
        _check(gather(*g_args), "gather")
    torch.cuda.synchronize()
    t_scatter, t_gather, t_total = EventTimer(), EventTimer(), EventTimer()
    total0 = t_total.start()
    for _ in range(steps):
        e0 = t_scatter.start()
        _check(scatter(*s_args), "scatter")
        t_scatter.stop(e0)
        e1 = t_gather.start()
        _check(gather(*g_args), "gather")
        t_gather.stop(e1)
    t_total.stop(total0)
    torch.cuda.synchronize()
    parity = parity and bool(torch.equal(ok, kl) and torch.equal(ov, vl))

    payload = 2 * NL * t * ROW * 2          # K and V rows of every layer, bf16
    per_dir = 2 * payload + 8 * t           # read + write + slots
    ms_s, ms_g = np.array(t_scatter.ms()), np.array(t_gather.ms())
    total_ms = t_total.ms()[0]
    dominant = ("gather", ms_g) if ms_g.sum() >= ms_s.sum() else ("scatter", ms_s)
    avg_dom = float(dominant[1].mean())
    return {
        "tokens": t,
        "bytes_per_direction": per_dir,
        "total_ms": total_ms,
        "ms_per_step": total_ms / steps,
        "value_gbs": 2 * per_dir * steps / (total_ms * 1e-3) / 1e9,
        "scatter": {"avg_ms": float(ms_s.mean()), "p50_ms": float(np.median(ms_s)),
                    "p95_ms": float(np.percentile(ms_s, 95)), "gbs": per_dir / (ms_s.mean() * 1e-3) / 1e9,
                    "tokens_per_ms": t / ms_s.mean()},
        "gather": {"avg_ms": float(ms_g.mean()), "p50_ms": float(np.median(ms_g)),
                   "p95_ms": float(np.percentile(ms_g, 95)), "gbs": per_dir / (ms_g.mean() * 1e-3) / 1e9,
                   "tokens_per_ms": t / ms_g.mean()},
        "dominant": dominant[0],
        "dominant_avg_ms": avg_dom,
        "parity_roundtrip": parity,
        "_tensors": (slots_np, slots, kc, vc, kl, vl, ok, ov),
    }


def bench_config1() -> dict:
    """Single-layer paged->linear K/V gather, fp16, 1024 blocks, 32 seqs len U[1,512]."""
    from musa_aiter.ops import _hip
    from tests.torch_ref import paged_rows

    dev = torch.device("cuda", 0)
    nb = 1024
    slots_np = make_slots(1001, 32, 1, 512, nb, BS)
    t = int(slots_np.shape[0])
    gen = torch.Generator(device=dev).manual_seed(1)
    kc = torch.randn((nb, NH, HD, BS), generator=gen, device=dev, dtype=torch.float16)
    vc = torch.randn((nb, NH, HD, BS), generator=gen, device=dev, dtype=torch.float16)
    slots = torch.from_numpy(slots_np).to(dev)
    ok = torch.empty((t, NH, HD), dtype=torch.float16, device=dev)
    ov = torch.empty_like(ok)
    fn = _bind(_hip.library(), "musa_aiter_kv_paged_to_linear_half", 5, 5)
    args = (kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), ok.data_ptr(), ov.data_ptr(), t, nb, NH, HD, BS)
    _check(fn(*args, _stream()), "cfg1 gather")
    torch.cuda.synchronize()
    parity = bool(torch.equal(ok, paged_rows(kc)[slots]) and torch.equal(ov, paged_rows(vc)[slots]))
    ms = batched_ms(lambda: _check(fn(*args, _stream()), "cfg1 gather"), launches=50)
    nbytes = 2 * (2 * t * ROW * 2) + 8 * t
    floor = short_launch_floor(slots_np, nb, torch.float16)
    return {"tokens": t, "bytes_per_call": nbytes, "gather": rate(nbytes, ms, t), "parity": parity,
            "traffic_per_call": profiled_traffic("cfg1_gather"), "floor": floor,
            "parity_check": "every gathered row equals its slot's cache row (torch indexing)",
            "api": "musa_aiter_kv_paged_to_linear_half"}


def short_launch_floor(slots_np: np.ndarray, nb: int, dtype: torch.dtype) -> dict:
    """What one launch of configs[0]'s size costs with no index work: the gather's bytes as whole cache blocks
    (K and V two planes of one launch), copied by the block-pattern kernel back to back like the gather --
    cache blocks in the order the slots visit them, or both sides in order."""
    dev = torch.device("cuda", 0)
    t = int(slots_np.shape[0])
    nblk = t // BS
    blk_bytes = NH * HD * BS * torch.tensor([], dtype=dtype).element_size()
    src = torch.zeros((2, nb, NH, HD, BS), dtype=dtype, device=dev)
    dst = torch.empty((2, nblk * BS, NH, HD), dtype=dtype, device=dev)
    order = torch.from_numpy(run_blocks(slots_np, BS)[:nblk].copy()).to(dev)
    nbytes = 2 * nblk * blk_bytes * 2
    out = {"bytes_per_launch": nbytes, "blocks_per_plane": nblk, "planes": 2}
    for name, blocks in (("gather_pattern", order), ("sequential", None)):
        def make(wt, blocks=blocks):
            return pattern_copy_fn(src, dst, src_blocks=blocks, dst_blocks=None, num_blocks=nblk,
                                   src_region_blocks=nb, dst_region_blocks=nblk, src_block_bytes=blk_bytes,
                                   dst_block_bytes=blk_bytes, planes=2, src_plane_stride=nb * blk_bytes,
                                   dst_plane_stride=nblk * blk_bytes, write_through=wt)

        out[name] = pattern_rate(make, nbytes, launches=50)
    log(f"config 1 floor: gather pattern {out['gather_pattern']['p50_ms'] * 1e3:.2f} us, sequential "
        f"{out['sequential']['p50_ms'] * 1e3:.2f} us per launch")
    return out


def bench_config3() -> dict:
    """FP8 quant-store into uint8 paged caches and dequant-gather to bf16: E4M3 per-head scales
    (headline), E4M3 scalar scale, E5M2 per-head scales, through the reference-named vec4 C-ABI entries."""
    from musa_aiter.ops import _hip
    from tests import torch_ref

    dev = torch.device("cuda", 0)
    slots_np = make_slots(1003, 64, 128, 4096, NB, BS)
    t = int(slots_np.shape[0])
    gen = torch.Generator(device=dev).manual_seed(3)
    slots = torch.from_numpy(slots_np).to(dev)
    kl = torch.randn((t, NH, HD), generator=gen, device=dev) * 2.0
    vl = torch.randn((t, NH, HD), generator=gen, device=dev) * 2.0
    for x in (kl, vl):
        x.mul_(torch.where(torch.rand(x.shape, generator=gen, device=dev) < 0.01, 50.0, 1.0))
    kl, vl = kl.to(torch.bfloat16), vl.to(torch.bfloat16)
    amax_k = kl.float().abs().amax(dim=(0, 2))
    amax_v = vl.float().abs().amax(dim=(0, 2))
    # ROTATE cache sets (2 x 128 MiB each, 1.5 GiB in all) are written and read in turn, so that a timed call
    # finds its cache in HBM and not in the 256 MB last-level cache left by the call before.
    sets = [(torch.zeros((NB, NH, HD, BS), dtype=torch.uint8, device=dev),
             torch.zeros((NB, NH, HD, BS), dtype=torch.uint8, device=dev)) for _ in range(ROTATE)]
    kc, vc = sets[0]
    ok = torch.empty_like(kl)
    ov = torch.empty_like(vl)
    lib = _hip.library()
    nbytes = 2 * t * ROW * (2 + 1) + 8 * t
    sample = min(t, 2048)
    out = {"tokens": t, "bytes_per_call": nbytes, "cache_sets_rotated": ROTATE}
    variants = (("e4m3_per_head", "e4m3", 1, 448.0), ("e4m3_scalar", "e4m3", 0, 448.0),
                ("e5m2_per_head", "e5m2", 1, 57344.0))
    for name, fmt, mode, fmax in variants:
        if mode == 1:
            ks, vs = (amax_k / fmax).contiguous(), (amax_v / fmax).contiguous()
        else:
            ks, vs = (amax_k.max() / fmax).reshape(1).contiguous(), (amax_v.max() / fmax).reshape(1).contiguous()
        q = _bind(lib, f"musa_aiter_kv_linear_to_paged_fp8_vec4_{fmt}", 7, 5)
        d = _bind(lib, f"musa_aiter_kv_paged_fp8_to_linear_vec4_{fmt}", 7, 5)
        q.argtypes = q.argtypes[:-1] + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        d.argtypes = d.argtypes[:-1] + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        qas = [(kl.data_ptr(), vl.data_ptr(), slots.data_ptr(), a.data_ptr(), b.data_ptr(), ks.data_ptr(),
                vs.data_ptr(), t, NB, NH, HD, BS, 2) for a, b in sets]
        das = [(a.data_ptr(), b.data_ptr(), slots.data_ptr(), ks.data_ptr(), vs.data_ptr(), ok.data_ptr(),
                ov.data_ptr(), t, NB, NH, HD, BS, 2) for a, b in sets]
        for qa in qas:
            _check(q(*qa, _stream(), mode), name)
        _check(d(*das[0], _stream(), mode), name)
        torch.cuda.synchronize()
        # Parity on a sample of tokens, outside the timed region (on the CPU): cache bytes vs the
        # reference encoder's steps in torch, dequantised rows vs its decoder (tests/torch_ref.py).
        got = torch_ref.paged_rows(kc)[slots[:sample]].cpu()      # [sample, NH, HD]
        scale = (ks.reshape(-1, 1) if mode == 1 else ks.reshape(())).cpu()
        want = torch_ref.fp8_quantize(kl[:sample].cpu(), scale, fmt)
        want_deq = torch_ref.fp8_dequantize(want, scale, fmt, torch.bfloat16)
        parity = bool(torch.equal(got, want) and torch.equal(ok[:sample].cpu(), want_deq))
        mq = batched_ms(rotating(lambda i: _check(q(*qas[i], _stream(), mode), name), ROTATE), launches=2 * ROTATE)
        md = batched_ms(rotating(lambda i: _check(d(*das[i], _stream(), mode), name), ROTATE), launches=2 * ROTATE)
        qr, dr = rate(nbytes, mq, t), rate(nbytes, md, t)
        if name == "e4m3_per_head":
            qr["traffic"] = profiled_traffic("fp8_quant")
            dr["traffic"] = profiled_traffic("fp8_dequant")
            # The same dequant-gather on one cache set, called back to back: its 256 MiB of codes stay in the
            # last-level cache between calls (a cache re-read while resident), so this is not an HBM rate.
            dr["one_cache_set_repeated"] = rate(nbytes, batched_ms(lambda: _check(d(*das[0], _stream(), mode),
                                                                                  name)), t)
        out[name] = {"quant_store": qr, "dequant_gather": dr,
                     "scale_rule": f"amax/{fmax:g}" + (" per kv-head" if mode == 1 else " over all heads"),
                     "parity_sample_tokens": sample, "parity": parity,
                     "parity_check": "cache bytes and bf16 rows of the sampled tokens equal the reference's "
                                     "encode/decode steps in torch (tests/torch_ref.py)"}
        log(f"config 3 {name}: quant {out[name]['quant_store']['gbs']:.0f} GB/s, "
            f"dequant {out[name]['dequant_gather']['gbs']:.0f} GB/s, parity {parity}")
    # Access-pattern ceilings on the same buffers: 32 KiB of bf16 rows (16 tokens) per 16 KiB FP8 block; the
    # quant-store writes cache blocks in block order (its block-major form), the dequant-gather reads them in
    # the order the slot mapping visits them.
    order_np = run_blocks(slots_np, BS)
    nblk = min(order_np.size, t // BS)
    order = torch.from_numpy(order_np[:nblk].copy()).to(dev)
    by_dst = np.argsort(order_np[:nblk], kind="stable")
    dst_sorted = torch.from_numpy(order_np[:nblk][by_dst].astype(np.int32)).to(dev)
    src_by_dst = torch.from_numpy(by_dst.astype(np.int32)).to(dev)
    lin_blk, cache_blk = ROW * BS * 2, ROW * BS
    ceil_bytes = 2 * nblk * (lin_blk + cache_blk)
    out["ceilings"] = {"blocks": nblk, "bytes_per_launch_pair": ceil_bytes}
    for name, quant, sbytes, dbytes, sblocks, dblocks, sreg, dreg in (
            ("quant_store_pattern", True, lin_blk, cache_blk, src_by_dst, dst_sorted, t // BS, NB),
            ("quant_store_token_order_pattern", True, lin_blk, cache_blk, None, order, t // BS, NB),
            ("dequant_gather_pattern", False, cache_blk, lin_blk, order, None, NB, t // BS)):
        def make(wt, quant=quant, sbytes=sbytes, dbytes=dbytes, sblocks=sblocks, dblocks=dblocks, sreg=sreg,
                 dreg=dreg):
            per_set = []
            for cache_pair in sets:
                src_pair, dst_pair = ((kl, vl), cache_pair) if quant else (cache_pair, (ok, ov))
                per_set.append(_run_all([pattern_copy_fn(a, b, src_blocks=sblocks, dst_blocks=dblocks,
                                                         num_blocks=nblk, src_region_blocks=sreg,
                                                         dst_region_blocks=dreg, src_block_bytes=sbytes,
                                                         dst_block_bytes=dbytes, planes=1, src_plane_stride=0,
                                                         dst_plane_stride=0, write_through=wt)
                                         for a, b in zip(src_pair, dst_pair)]))
            return rotating(lambda i: per_set[i](), ROTATE)

        out["ceilings"][name] = pattern_rate(make, ceil_bytes, launches=2 * ROTATE)
    log(f"config 3 ceilings: quant pattern {out['ceilings']['quant_store_pattern']['gbs']:.0f}, dequant pattern "
        f"{out['ceilings']['dequant_gather_pattern']['gbs']:.0f} GB/s")
    return out


def bench_config4() -> dict:
    """SGLang-MP [2, 32, 4096, 16, 8, 128] bf16 <-> LMCache [2, 32, 256, 1024], 16 chunks."""
    import musa_aiter

    dev = torch.device("cuda", 0)
    nl, nb, chunk, nchunks = 32, 4096, 256, 16
    gen = torch.Generator(device=dev).manual_seed(4)
    cache = torch.randn((2, nl, nb, BS, NH, HD), generator=gen, device=dev, dtype=torch.bfloat16)
    kvcaches = [list(cache[0].unbind(0)), list(cache[1].unbind(0))]
    slots_np = make_covering_slots(1004, chunk * nchunks, 128, 4096, nb, BS)
    slots = torch.from_numpy(slots_np).to(dev)
    memory = torch.empty((2, nl, chunk * nchunks, ROW), dtype=torch.bfloat16, device=dev)
    chunks = [(slots[i * chunk:(i + 1) * chunk].contiguous(), memory[:, :, i * chunk:(i + 1) * chunk])
              for i in range(nchunks)]
    for s_c, m in chunks:
        musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(kvcaches, m, s_c, BS, NH, HD)
    torch.cuda.synchronize()
    # Parity (outside timing): every row of the buffer equals its slot's row of the cache (torch indexing).
    parity = bool(torch.equal(memory, cache.reshape(2, nl, nb * BS, ROW)[:, :, slots]))
    log(f"config 4: {chunk * nchunks} tokens in {nchunks} chunks, parity {parity}")

    def per_chunk_gather():
        for s_c, m in chunks:
            musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(kvcaches, m, s_c, BS, NH, HD)

    mg = batched_ms(per_chunk_gather, launches=5, reps=5) / nchunks
    # The same per-chunk gathers through the reference-named C entry (host work of a ctypes call only), so
    # consecutive launches are bound by the kernel rather than by the Python API's per-call host time.
    from musa_aiter.ops import _hip

    centry = getattr(_hip.library(), "lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16")
    centry.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64), ctypes.c_void_p] + [ctypes.c_int64] * 7 + \
        [ctypes.c_void_p]
    centry.restype = ctypes.c_int
    cache_ptrs = (ctypes.c_uint64 * (2 * nl))(*[c.data_ptr() for axis in kvcaches for c in axis])
    c_chunks = [(s_c, m.contiguous()) for s_c, m in chunks]

    def per_chunk_gather_c():
        for s_c, m in c_chunks:
            _check(centry(m.data_ptr(), cache_ptrs, s_c.data_ptr(), nl, chunk, chunk, nb, BS, NH, HD, _stream()),
                   "cfg4 chunk")

    per_chunk_gather_c()
    torch.cuda.synchronize()
    flat = cache.reshape(2, nl, nb * BS, ROW)
    parity = parity and all(bool(torch.equal(m, flat[:, :, s_c])) for s_c, m in c_chunks)
    mc = batched_ms(per_chunk_gather_c, launches=5, reps=5) / nchunks
    # The floor of such a launch: each chunk's bytes as whole 32 KiB blocks of all 64 planes (cache blocks in the
    # order the chunk's slots visit them) copied in order into that chunk's own contiguous buffer, the one the
    # C-entry timing above writes, by the block-pattern kernel, same rotation.  (The block-id tensors stay
    # referenced by `orders` while the launchers that read them exist.)
    blk_bytes = BS * ROW * 2
    orders = [torch.from_numpy(run_blocks(slots_np[i * chunk:(i + 1) * chunk], BS)[:chunk // BS].copy()).to(dev)
              for i in range(nchunks)]

    def per_chunk_floor(wt):
        return _run_all([pattern_copy_fn(cache, m, src_blocks=order, dst_blocks=None, num_blocks=int(order.numel()),
                                         src_region_blocks=nb, dst_region_blocks=chunk // BS,
                                         src_block_bytes=blk_bytes, dst_block_bytes=blk_bytes, planes=2 * nl,
                                         src_plane_stride=nb * blk_bytes, dst_plane_stride=chunk * ROW * 2,
                                         write_through=wt)
                         for order, (_, m) in zip(orders, c_chunks)])

    floor_bytes = 2 * nl * (chunk // BS) * blk_bytes * 2
    floor = pattern_rate(per_chunk_floor, floor_bytes, per_call=nchunks, launches=5, reps=5)
    mb = batched_ms(lambda: musa_aiter.lmcache_kv_paged_to_buffer_two_x_nl(kvcaches, memory, slots, BS, NH, HD),
                    launches=10)
    ms = batched_ms(lambda: musa_aiter.lmcache_kv_buffer_to_paged_two_x_nl(memory, kvcaches, slots, 0, BS, NH, HD),
                    launches=10)
    per_chunk = 2 * (2 * nl * chunk * ROW * 2) + 8 * chunk
    return {"chunk_tokens": chunk, "chunks": nchunks, "bytes_per_chunk": per_chunk, "parity": parity,
            "traffic_per_chunk": profiled_traffic("cfg4_chunk_gather"),
            "gather_per_chunk_call": rate(per_chunk, mg, chunk),
            "gather_per_chunk_c_abi": rate(per_chunk, mc, chunk),
            "per_chunk_floor_pattern_copy": floor,
            "gather_batched_16": rate(per_chunk * nchunks, mb, chunk * nchunks),
            "scatter_batched_16": rate(per_chunk * nchunks, ms, chunk * nchunks),
            "note": "per-chunk calls go through the Python API (validation, pointer tables) back to back, or through "
                    "the reference-named C entry (lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16); each of the 16 "
                    "chunks gathers its own rows into its own buffer slice; batched = one call for all 16 chunks"}


def bench_config5() -> dict:
    """MLA flat rows, 61 layers, BS=64, 128 seqs len U[256,8192]: bf16 576-value rows through
    lmcache_{paged_to_kv_buffer,kv_buffer_to_paged}_mla_u16, and 656-byte FP8 rows through
    musa_aiter_kv_copy_paged_rows_contig_layers_u8."""
    from musa_aiter.ops import _hip
    from tests.kvgen import sequence_slots

    dev = torch.device("cuda", 0)
    nl, bs, hs, rowb8 = 61, 64, 576, 656
    rng = np.random.default_rng(1005)
    lengths = [int(x) for x in rng.integers(256, 8193, size=128)]
    nb = sum((n + bs - 1) // bs for n in lengths)
    slots_np = sequence_slots(rng, lengths, num_blocks=nb, block_size=bs)
    t = int(slots_np.shape[0])
    slots = torch.from_numpy(slots_np).to(dev)
    lib = _hip.library()
    out = {"tokens": t, "num_blocks": nb, "layers": nl}
    gen = torch.Generator(device=dev).manual_seed(5)

    paged = torch.randn((nl, nb, bs, hs), generator=gen, device=dev, dtype=torch.bfloat16)
    buf = torch.empty((nl, t, hs), dtype=torch.bfloat16, device=dev)
    g = _bind(lib, "lmcache_paged_to_kv_buffer_mla_u16", 3, 5)
    sct = _bind(lib, "lmcache_kv_buffer_to_paged_mla_u16", 3, 5)
    ga = (paged.data_ptr(), buf.data_ptr(), slots.data_ptr(), nl, t, nb, bs, hs)
    sa = (buf.data_ptr(), paged.data_ptr(), slots.data_ptr(), nl, t, nb, bs, hs)
    before = paged.view(torch.int16).sum(dtype=torch.int64).item()
    _check(g(*ga, _stream()), "cfg5 gather")
    _check(sct(*sa, _stream()), "cfg5 scatter")
    torch.cuda.synchronize()
    pick = rng.integers(0, t, size=256)
    flat = paged.view(nl, nb * bs, hs)
    sample_ok = bool(torch.equal(buf[:, torch.from_numpy(pick).to(dev)],
                                 flat[:, torch.from_numpy(slots_np[pick]).to(dev)]))
    parity = sample_ok and before == paged.view(torch.int16).sum(dtype=torch.int64).item()
    mg = batched_ms(lambda: _check(g(*ga, _stream()), "cfg5 gather"), launches=3, reps=3)
    ms = batched_ms(lambda: _check(sct(*sa, _stream()), "cfg5 scatter"), launches=3, reps=3)
    nbytes = 2 * nl * t * hs * 2 + 8 * t
    out["bf16_576"] = {"bytes_per_call": nbytes, "gather": rate(nbytes, mg, t), "scatter": rate(nbytes, ms, t),
                       "parity": parity, "parity_check": "256 sampled tokens x 61 layers equal to their slot rows; "
                                                          "scatter of the gathered rows leaves the cache checksum unchanged"}
    # Access-pattern ceilings on the same buffers: whole 72 KiB cache blocks (64 rows) in the order the slots visit
    # them against the buffer in order, by the block-pattern kernel.
    blk = bs * hs * 2
    nblk = t // bs
    order = torch.from_numpy(run_blocks(slots_np, bs)[:nblk].copy()).to(dev)
    pbytes = 2 * nl * nblk * blk
    ceil = {"block_bytes": blk, "blocks_per_plane": nblk, "planes": nl}
    for name, src, dst, sblocks, dblocks, sreg, dreg, sps, dps in (
            ("gather_pattern", paged, buf, order, None, nb, nblk, nb * blk, t * hs * 2),
            ("scatter_pattern", buf, paged, None, order, nblk, nb, t * hs * 2, nb * blk)):
        def make(wt, src=src, dst=dst, sblocks=sblocks, dblocks=dblocks, sreg=sreg, dreg=dreg, sps=sps, dps=dps):
            return pattern_copy_fn(src, dst, src_blocks=sblocks, dst_blocks=dblocks, num_blocks=nblk,
                                   src_region_blocks=sreg, dst_region_blocks=dreg, src_block_bytes=blk,
                                   dst_block_bytes=blk, planes=nl, src_plane_stride=sps, dst_plane_stride=dps,
                                   write_through=wt)

        ceil[name] = pattern_rate(make, pbytes, launches=3, reps=3)
    out["bf16_576"]["ceilings"] = ceil
    out["bf16_576"]["gather_frac_of_pattern"] = out["bf16_576"]["gather"]["gbs"] / ceil["gather_pattern"]["gbs"]
    out["bf16_576"]["scatter_frac_of_pattern"] = out["bf16_576"]["scatter"]["gbs"] / ceil["scatter_pattern"]["gbs"]
    log(f"config 5 bf16: gather {out['bf16_576']['gather']['gbs']:.0f} GB/s, "
        f"scatter {out['bf16_576']['scatter']['gbs']:.0f} GB/s, parity {parity}; pattern ceilings "
        f"{ceil['gather_pattern']['gbs']:.0f} / {ceil['scatter_pattern']['gbs']:.0f} GB/s")
    del paged, buf, flat
    torch.cuda.empty_cache()

    src = torch.randint(0, 256, (nl, nb * bs, rowb8), generator=gen, device=dev, dtype=torch.uint8)
    dst = torch.empty((nl, t, rowb8), dtype=torch.uint8, device=dev)
    rows = torch.arange(t, dtype=torch.int64, device=dev)
    cp = _bind(lib, "musa_aiter_kv_copy_paged_rows_contig_layers_u8", 4, 5)
    ca = (src.data_ptr(), dst.data_ptr(), slots.data_ptr(), rows.data_ptr(), t, rowb8, nl, nb * bs, t)
    _check(cp(*ca, _stream()), "cfg5 rows")
    torch.cuda.synchronize()
    parity8 = bool(torch.equal(dst[:, torch.from_numpy(pick).to(dev)], src[:, torch.from_numpy(slots_np[pick]).to(dev)]))
    mr = batched_ms(lambda: _check(cp(*ca, _stream()), "cfg5 rows"), launches=3, reps=3)
    nbytes8 = 2 * nl * t * rowb8 + 2 * 8 * t
    out["fp8_656_rows"] = {"bytes_per_call": nbytes8, "gather": rate(nbytes8, mr, t), "parity": parity8}
    log(f"config 5 fp8 rows: gather {out['fp8_656_rows']['gather']['gbs']:.0f} GB/s, parity {parity8}")
    del src, dst
    torch.cuda.empty_cache()
    return out


def bench_dense() -> dict:
    """Dense preload for attention and whole-block copies (the next row after the BASELINE configs).

    Llama-3-8B single-layer caches [8192, 8, 128, 16] bf16, 64 decode sequences with lengths
    uniform in [128, 4096] and random block tables; dense tensors [64, max_len, 8, 128].
    Bytes per call: cache rows read for valid positions + every dense row written (zeros past
    seq_lens) for the loads, valid rows read + written for the write-back, plus index bytes.
    The block copy moves 1024 random block pairs of a 32-layer cache (disjoint source and
    destination halves).
    """
    from musa_aiter.ops import _hip
    from tests import torch_ref
    from tests.kvgen import sequence_lengths

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(1006)
    lengths = np.array(sequence_lengths(rng, 64, 128, 4096, num_blocks=NB, block_size=BS), dtype=np.int64)
    batch, dense_len = lengths.size, int(lengths.max())
    need = (lengths + BS - 1) // BS
    max_blocks = int(need.max())
    perm = rng.permutation(NB)
    tables_np = np.zeros((batch, max_blocks), dtype=np.int64)
    pos = 0
    for b, k in enumerate(need):
        tables_np[b, :k] = perm[pos:pos + k]
        pos += k
    valid = int(lengths.sum())
    tables = torch.from_numpy(tables_np).to(dev)
    seq_lens = torch.from_numpy(lengths).to(dev)
    gen = torch.Generator(device=dev).manual_seed(6)
    kc = torch.randn((NB, NH, HD, BS), generator=gen, device=dev, dtype=torch.bfloat16)
    vc = torch.randn((NB, NH, HD, BS), generator=gen, device=dev, dtype=torch.bfloat16)
    dk = torch.empty((batch, dense_len, NH, HD), dtype=torch.bfloat16, device=dev)
    dv = torch.empty_like(dk)
    lib = _hip.library()
    out = {"sequences": batch, "dense_len": dense_len, "valid_tokens": valid, "max_blocks": max_blocks}
    row_b = ROW * 2
    idx_bytes = tables_np.size * 8 + batch * 8

    # Slot of every valid dense position, for the parity checks (torch indexing, outside timing).
    j = np.arange(dense_len)
    mask_np = j[None, :] < lengths[:, None]
    slots_np = np.where(mask_np, tables_np[np.arange(batch)[:, None], np.minimum(j // BS, max_blocks - 1)[None, :]]
                        * BS + (j % BS)[None, :], 0)
    flat_slots = torch.from_numpy(slots_np[mask_np]).to(dev)
    mask = torch.from_numpy(mask_np).to(dev)

    rows_of = torch_ref.paged_rows

    load = _bind(lib, "musa_aiter_kv_load_and_reshape_flash_bfloat16", 6, 7)
    la = (kc.data_ptr(), vc.data_ptr(), tables.data_ptr(), seq_lens.data_ptr(), dk.data_ptr(), dv.data_ptr(),
          batch, dense_len, max_blocks, NB, NH, HD, BS)
    _check(load(*la, _stream()), "dense load")
    torch.cuda.synchronize()
    ok = bool(torch.equal(dk[mask], rows_of(kc)[flat_slots]) and torch.equal(dv[mask], rows_of(vc)[flat_slots])
              and not bool(dk[~mask].any()) and not bool(dv[~mask].any()))
    ml = batched_ms(lambda: _check(load(*la, _stream()), "dense load"), launches=5, reps=5)
    nbytes = 2 * valid * row_b + 2 * batch * dense_len * row_b + idx_bytes
    out["load_and_reshape_flash"] = {**rate(nbytes, ml, valid), "bytes_per_call": nbytes, "parity": ok}

    back = _bind(lib, "musa_aiter_kv_reshape_and_cache_back_flash_bfloat16", 6, 7)
    ba = (dk.data_ptr(), dv.data_ptr(), tables.data_ptr(), seq_lens.data_ptr(), kc.data_ptr(), vc.data_ptr(),
          batch, dense_len, max_blocks, NB, NH, HD, BS)
    before = kc.view(torch.int16).sum(dtype=torch.int64).item() + vc.view(torch.int16).sum(dtype=torch.int64).item()
    _check(back(*ba, _stream()), "dense write-back")
    torch.cuda.synchronize()
    after = kc.view(torch.int16).sum(dtype=torch.int64).item() + vc.view(torch.int16).sum(dtype=torch.int64).item()
    mb = batched_ms(lambda: _check(back(*ba, _stream()), "dense write-back"), launches=5, reps=5)
    nbytes = 4 * valid * row_b + idx_bytes
    out["reshape_and_cache_back_flash"] = {**rate(nbytes, mb, valid), "bytes_per_call": nbytes,
                                           "parity": before == after,
                                           "parity_check": "writing the loaded rows back leaves the caches' checksum "
                                                           "unchanged"}

    # FP8 E4M3 per-head dequant-load into bf16, through the generic entry.
    # ROTATE code sets, read in turn (as for configs[2]), so that each timed call reads its codes from HBM.
    sets8 = [torch.randint(0, 256, (NB, NH, HD, BS), generator=gen, device=dev, dtype=torch.uint8)
             for _ in range(ROTATE)]
    sets8 = [(k8, k8.flip(0)) for k8 in sets8]
    k8 = sets8[0][0]
    ks = torch.rand(NH, generator=gen, device=dev) + 0.01
    vs = torch.rand(NH, generator=gen, device=dev) + 0.01
    dq = _hip.fn("musa_aiter_hip_paged_dense_tiles")
    qas = [(0, 1, 1, 2, 2, a.data_ptr(), b.data_ptr(), dk.data_ptr(), dv.data_ptr(), tables.data_ptr(),
            seq_lens.data_ptr(), batch, dense_len, max_blocks, NB, NH, HD, BS, ROW, ks.data_ptr(), vs.data_ptr(), 1,
            1, 0, None) for a, b in sets8]
    _check(dq(*qas[0], _stream()), "fp8 dense load")
    torch.cuda.synchronize()
    want = torch_ref.fp8_dequantize(rows_of(k8)[flat_slots], ks[None, :, None], "e4m3", torch.bfloat16)
    ok8 = bool(torch.equal(dk[mask], want) and not bool(dk[~mask].any()))
    del want
    mq = batched_ms(rotating(lambda i: _check(dq(*qas[i], _stream()), "fp8 dense load"), ROTATE),
                    launches=2 * ROTATE, reps=5)
    nbytes = 2 * valid * ROW + 2 * batch * dense_len * row_b + idx_bytes + 2 * NH * 4
    out["load_and_dequantize_fp8_flash_e4m3"] = {**rate(nbytes, mq, valid), "bytes_per_call": nbytes, "parity": ok8,
                                                 "parity_check": "valid rows equal the reference decoder's value "
                                                                 "x per-head scale rounded to bf16 "
                                                                 "(tests/torch_ref.py)",
                                                 "code_sets_rotated": ROTATE}
    del k8, sets8

    # SGLang Triton-decode CSR indices over token-major caches [NB*BS, NH, HD].
    key_tok, val_tok = rows_of(kc).contiguous(), rows_of(vc).contiguous()
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths)])).to(dev)
    csr = _bind(lib, "musa_aiter_kv_triton_indexed_to_dense_bfloat16", 6, 6)
    ca = (key_tok.data_ptr(), val_tok.data_ptr(), indptr.data_ptr(), flat_slots.data_ptr(), dk.data_ptr(),
          dv.data_ptr(), batch, dense_len, valid, NB * BS, NH, HD)
    _check(csr(*ca, _stream()), "csr dense load")
    torch.cuda.synchronize()
    okc = bool(torch.equal(dk[mask], key_tok[flat_slots]) and torch.equal(dv[mask], val_tok[flat_slots])
               and not bool(dk[~mask].any()))
    mc = batched_ms(lambda: _check(csr(*ca, _stream()), "csr dense load"), launches=5, reps=5)
    nbytes = 2 * valid * row_b + 2 * batch * dense_len * row_b + valid * 8 + (batch + 1) * 8
    out["triton_indexed_to_dense"] = {**rate(nbytes, mc, valid), "bytes_per_call": nbytes, "parity": okc}
    del key_tok, val_tok, dk, dv, kc, vc
    torch.cuda.empty_cache()

    # 1024 block pairs of a 32-layer cache; sources in the first half, destinations in the second.
    nl, nb2, pairs_n = NL, 4096, 1024
    ck = torch.randn((nl, nb2, NH, HD, BS), generator=gen, device=dev, dtype=torch.bfloat16)
    cv = torch.randn((nl, nb2, NH, HD, BS), generator=gen, device=dev, dtype=torch.bfloat16)
    pairs_np = np.stack([rng.permutation(nb2 // 2)[:pairs_n], nb2 // 2 + rng.permutation(nb2 // 2)[:pairs_n]], 1)
    pairs = torch.from_numpy(np.ascontiguousarray(pairs_np)).to(dev)
    cp = _bind(lib, "musa_aiter_kv_copy_paged_blocks_bfloat16", 5, 7)
    pa = (ck.data_ptr(), cv.data_ptr(), ck.data_ptr(), cv.data_ptr(), pairs.data_ptr(), pairs_n, nl, nb2, nb2, NH,
          HD, BS)
    _check(cp(*pa, _stream()), "block copy")
    torch.cuda.synchronize()
    okb = bool(torch.equal(ck[:, pairs[:, 1]], ck[:, pairs[:, 0]]) and torch.equal(cv[:, pairs[:, 1]],
                                                                                 cv[:, pairs[:, 0]]))
    mp = batched_ms(lambda: _check(cp(*pa, _stream()), "block copy"), launches=5, reps=5)
    nbytes = 2 * 2 * nl * pairs_n * ROW * BS * 2 + pairs_n * 16
    out["copy_paged_blocks_32_layers"] = {**rate(nbytes, mp), "bytes_per_call": nbytes, "pairs": pairs_n,
                                          "parity": okb}
    del ck, cv
    torch.cuda.empty_cache()
    log("dense: " + ", ".join(f"{k} {v['gbs']:.0f} GB/s parity {v['parity']}" for k, v in out.items()
                              if isinstance(v, dict)))
    return out


def bench_hicache() -> dict:
    """SGLang HiCache transfers (the next row after the dense preload), Llama-3-8B and DeepSeek shapes.

    Pools of 65536 tokens: the device pool is layer-first [32, tokens, 8*128] bf16 per K and V,
    the second-tier pool page-first [tokens, 32, 8*128] (both resident in HBM: the reference's path
    takes device tensors only).  One transfer moves 512 random pages of 64 tokens (32768 token
    items of 2 KiB) between random page slots of the two pools.  Backup = one all-layer
    layer-first -> page-first call; load = 32 per-layer page-first -> layer-first calls, as SGLang
    loads layer by layer.  Both go through the reference-named C symbol
    musa_aiter_hicache_transfer_bytes.  MLA: 61 layers of 1152-byte latent rows, all-layer
    layer-first -> page-first.  Direct: the public all-layer direct API (page_size 64) end to end,
    host validation of the index tables included.  Bytes = items x layers x planes x (read +
    write) + 16 B of indices per item and launch.
    """
    from musa_aiter.ops import _hip
    import musa_aiter

    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(1007)
    layers, pool, page = NL, 65536, 64
    pages_moved = 512
    n = pages_moved * page
    item = ROW * 2
    j = np.arange(page)
    dev_tok = (rng.permutation(pool // page)[:pages_moved][:, None] * page + j).reshape(-1)
    host_tok = (rng.permutation(pool // page)[:pages_moved][:, None] * page + j).reshape(-1)
    dev_idx = torch.from_numpy(dev_tok.astype(np.int64)).to(dev)
    host_idx = torch.from_numpy(host_tok.astype(np.int64)).to(dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    dk = torch.randn((layers, pool, ROW), generator=gen, device=dev, dtype=torch.bfloat16)
    dv = torch.randn((layers, pool, ROW), generator=gen, device=dev, dtype=torch.bfloat16)
    hk = torch.zeros((pool, layers, ROW), device=dev, dtype=torch.bfloat16)
    hv = torch.zeros_like(hk)
    lib = _hip.library()
    xfer = _bind(lib, "musa_aiter_hicache_transfer_bytes", 6, 8)
    out = {"pool_tokens": pool, "layers": layers, "page_size": page, "items": n, "item_bytes": item}

    lf_stride, lf_layer = item, pool * item          # layer_first [layers, pool, item]
    pf_stride, pf_layer = layers * item, item        # page_first [pool, layers, item]
    backup = (dk.data_ptr(), hk.data_ptr(), dv.data_ptr(), hv.data_ptr(), dev_idx.data_ptr(), host_idx.data_ptr(),
              n, 0, layers, item, lf_stride, lf_layer, pf_stride, pf_layer)
    _check(xfer(*backup, _stream()), "hicache backup")
    torch.cuda.synchronize()
    ok = bool(torch.equal(hk[host_idx].view(torch.int16), dk[:, dev_idx].transpose(0, 1).view(torch.int16))
              and torch.equal(hv[host_idx].view(torch.int16), dv[:, dev_idx].transpose(0, 1).view(torch.int16)))
    mb = batched_ms(lambda: _check(xfer(*backup, _stream()), "hicache backup"), launches=5, reps=5)
    nbytes = 2 * 2 * layers * n * item + 16 * n
    out["all_layer_lf_pf_backup"] = {**rate(nbytes, mb, n), "bytes_per_call": nbytes, "parity": ok}

    dk2, dv2 = torch.zeros_like(dk), torch.zeros_like(dv)

    def load_all_layers():
        for layer in range(layers):
            _check(xfer(hk.data_ptr(), dk2.data_ptr(), hv.data_ptr(), dv2.data_ptr(), host_idx.data_ptr(),
                        dev_idx.data_ptr(), n, layer, 1, item, pf_stride, pf_layer, lf_stride, lf_layer, _stream()),
                   "hicache load")

    load_all_layers()
    torch.cuda.synchronize()
    okl = bool(torch.equal(dk2[:, dev_idx].view(torch.int16), dk[:, dev_idx].view(torch.int16))
               and torch.equal(dv2[:, dev_idx].view(torch.int16), dv[:, dev_idx].view(torch.int16)))
    ml = batched_ms(load_all_layers, launches=2, reps=5)
    nbytes = 2 * 2 * layers * n * item + 16 * n * layers
    out["per_layer_pf_lf_load_x32"] = {**rate(nbytes, ml, n), "bytes_per_call": nbytes, "launches": layers,
                                       "parity": okl, "parity_check": "backup then load restores every moved item"}
    del dk2, dv2

    # Public direct API: all layers, layer-first per-layer tensors -> page-first [pages, layers, 64, item].
    src_layers = [dk[layer] for layer in range(layers)] + [dv[layer] for layer in range(layers)]
    pk = torch.zeros((pool // page, layers, page, ROW), device=dev, dtype=torch.bfloat16)
    pv = torch.zeros_like(pk)

    def direct():
        musa_aiter.hicache_transfer_kv_all_layer_direct_lf_pf(src_layers, [pk, pv], dev_idx, host_idx, page)

    direct()
    torch.cuda.synchronize()
    okd = bool(torch.equal(pk[host_idx // page, :, host_idx % page].view(torch.int16),
                           dk[:, dev_idx].transpose(0, 1).view(torch.int16))
               and torch.equal(pv[host_idx // page, :, host_idx % page].view(torch.int16),
                               dv[:, dev_idx].transpose(0, 1).view(torch.int16)))
    md = batched_ms(direct, launches=5, reps=5)
    nbytes = 2 * 2 * layers * n * item + 16 * n
    out["all_layer_direct_lf_pf_api"] = {**rate(nbytes, md, n), "bytes_per_call": nbytes, "parity": okd,
                                         "timed": "public API incl. host-side index validation"}
    del src_layers, pk, pv, dk, dv, hk, hv
    torch.cuda.empty_cache()

    # MLA: DeepSeek latent rows (512 + 64 bf16), 61 layers, no value plane.
    mla_layers, mla_item = 61, 576 * 2
    mk = torch.randn((mla_layers, pool, 576), generator=gen, device=dev, dtype=torch.bfloat16)
    mh = torch.zeros((pool, mla_layers, 576), device=dev, dtype=torch.bfloat16)
    mla = (mk.data_ptr(), mh.data_ptr(), None, None, dev_idx.data_ptr(), host_idx.data_ptr(), n, 0, mla_layers,
           mla_item, mla_item, pool * mla_item, mla_layers * mla_item, mla_item)
    _check(xfer(*mla, _stream()), "hicache mla backup")
    torch.cuda.synchronize()
    okm = bool(torch.equal(mh[host_idx].view(torch.int16), mk[:, dev_idx].transpose(0, 1).view(torch.int16)))
    mm = batched_ms(lambda: _check(xfer(*mla, _stream()), "hicache mla backup"), launches=5, reps=5)
    nbytes = 2 * mla_layers * n * mla_item + 16 * n
    out["mla_all_layer_lf_pf_backup_61_layers"] = {**rate(nbytes, mm, n), "bytes_per_call": nbytes, "parity": okm}
    del mk, mh
    torch.cuda.empty_cache()
    log("hicache: " + ", ".join(f"{k} {v['gbs']:.0f} GB/s parity {v['parity']}" for k, v in out.items()
                                if isinstance(v, dict)))
    return out


def bench_batch_copy() -> dict:
    """LMCache host <-> device copy batches (the staging step), through the C entry musa_aiter_hip_batch_copy.

    Offload-sized batch: 16 chunks of 256 tokens x 32 layers x K/V, one 512 KiB range (256 x 2 KiB rows)
    per (chunk, layer, K/V): 1024 ranges, 512 MiB, between pinned host memory and HBM.  Small-range
    batch: 4096 ranges of 4 KiB.  Each direction runs through the batch-copy kernel (pinned host
    memory read or written by the GPU over the host link) on at most 64 workgroups and on at most 16
    (the prefer_overlap_with_compute form), and through one hipMemcpyAsync per range;
    a single torch copy of one contiguous pinned buffer of the same total size gives the runtime's
    own rate, and the public lmcache_musa_memcpy_batch_async call (its host planning included) the
    rate a caller sees, with its host time per call.  Bytes = bytes moved across the host link
    (each byte once).
    """
    from musa_aiter.ops import _hip
    from musa_aiter.ops.lmcache_musa_batch_copy import lmcache_musa_memcpy_batch_async

    os.environ["MUSA_AITER_LMCACHE_BATCH_COPY"] = "1"  # the public API's opt-in gate
    dev = torch.device("cuda", 0)
    out = {}
    fn = _hip.fn("musa_aiter_hip_batch_copy")

    def link_rate(total: int, ms: np.ndarray) -> dict:
        r = rate(total, ms)
        r.pop("pct_of_peak")
        r["pct_of_host_link"] = round(100.0 * r["gbs"] / HOST_LINK_GBS, 2)
        return r

    def run(ranges: int, size: int, label: str) -> None:
        total = ranges * size
        ref = torch.randint(0, 256, (total,), dtype=torch.uint8, generator=torch.Generator().manual_seed(8))
        host = torch.empty(total, dtype=torch.uint8).pin_memory()
        gpu = torch.empty(total, dtype=torch.uint8, device=dev)
        # Host range i <-> device range perm[i]: the device side is shuffled.
        perm = np.random.default_rng(1008).permutation(ranges)
        perm_d = torch.from_numpy(perm).to(dev)
        shuffled = torch.empty_like(gpu)
        shuffled.view(ranges, size)[perm_d] = ref.to(dev).view(ranges, size)
        hp = [host.data_ptr() + i * size for i in range(ranges)]
        gp = [gpu.data_ptr() + int(perm[i]) * size for i in range(ranges)]
        sizes = (ctypes.c_uint64 * ranges)(*([size] * ranges))
        arrays = {"h2d": ((ctypes.c_void_p * ranges)(*gp), (ctypes.c_void_p * ranges)(*hp), 0),
                  "d2h": ((ctypes.c_void_p * ranges)(*hp), (ctypes.c_void_p * ranges)(*gp), 1)}
        res = {"ranges": ranges, "range_bytes": size, "bytes": total}
        for direction, (dsts, srcs, code) in arrays.items():
            for path, mode in (("kernel", 0), ("kernel_16_workgroups", 1), ("hip_memcpy_per_range", 2)):
                def call(dsts=dsts, srcs=srcs, code=code, mode=mode):
                    _check(fn(dsts, srcs, sizes, ranges, code, mode, _stream()), "batch copy")

                if direction == "h2d":
                    host.copy_(ref)
                    gpu.zero_()
                else:
                    gpu.copy_(shuffled)
                    host.zero_()
                torch.cuda.synchronize()
                call()
                torch.cuda.synchronize()
                if direction == "h2d":
                    ok = bool(torch.equal(gpu, shuffled))
                else:
                    ok = bool(torch.equal(host, ref))
                ms = batched_ms(call, launches=3, reps=3)
                res[f"{direction}_{path}"] = {**link_rate(total, ms), "parity": ok}
            dst_t, src_t = (gpu, host) if direction == "h2d" else (host, gpu)
            ms = batched_ms(lambda: dst_t.copy_(src_t, non_blocking=True), launches=3, reps=3)
            res[f"{direction}_torch_contiguous_copy"] = link_rate(total, ms)
            # The public API end to end (host planning and checks included): the same ranges as offsets
            # into the two tensors, timed between events like the rest, plus its host time per call.
            g_off = [int(perm[i]) * size for i in range(ranges)]
            h_off = [i * size for i in range(ranges)]
            api_d, api_s = ([gpu] * ranges, [host] * ranges) if direction == "h2d" else ([host] * ranges, [gpu] * ranges)
            d_off, s_off = (g_off, h_off) if direction == "h2d" else (h_off, g_off)

            def api(api_d=api_d, api_s=api_s, d_off=d_off, s_off=s_off):
                if not lmcache_musa_memcpy_batch_async(api_d, api_s, [size] * ranges, destination_offsets=d_off,
                                                       source_offsets=s_off, max_batch_entries=ranges):
                    raise RuntimeError("batch copy API declined the batch")

            (gpu if direction == "h2d" else host).zero_()
            torch.cuda.synchronize()
            api()
            torch.cuda.synchronize()
            api_ok = bool(torch.equal(gpu, shuffled)) if direction == "h2d" else bool(torch.equal(host, ref))
            host_s = []
            for _ in range(5):
                t0 = time.perf_counter()
                api()
                host_s.append(time.perf_counter() - t0)
                torch.cuda.synchronize()
            ms = batched_ms(api, launches=3, reps=3)
            res[f"{direction}_public_api"] = {**link_rate(total, ms), "parity": api_ok,
                                             "host_ms_per_call": round(1e3 * float(np.median(host_s)), 3)}
        out[label] = res
        del host, gpu, shuffled

    run(1024, 512 << 10, "offload_1024_x_512KiB")
    run(4096, 4096, "small_4096_x_4KiB")
    torch.cuda.empty_cache()
    log("batch copy: " + ", ".join(f"{k}.{d} {v[d]['gbs']:.1f} GB/s" for k, v in out.items() for d in v
                                   if isinstance(v[d], dict)))
    return out


def bench_decode() -> dict:
    """Decode-step scatters: T new tokens, one per sequence at a random offset of its own block, into one
    layer's [NB, NH, HD, BS] caches, through the reference-named C entries (the per-layer call of a decode
    step), and the gathers of the same slots back.  Per-call latency (100 back-to-back calls per timing);
    the bf16 copy and the FP8 E4M3 quant-store / dequant-gather with per-head scales.  Calls of at most 256
    tokens resolve repeated slots inside the kernel and gather short runs token by token."""
    from musa_aiter.ops import _hip
    from tests import torch_ref

    dev = torch.device("cuda", 0)
    lib = _hip.library()
    gen = torch.Generator(device=dev).manual_seed(10)
    kc = torch.zeros((NB, NH, HD, BS), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qk = torch.zeros((NB, NH, HD, BS), dtype=torch.uint8, device=dev)
    qv = torch.zeros_like(qk)
    sc = _bind(lib, "musa_aiter_kv_linear_to_paged_bfloat16", 5, 5)
    ga = _bind(lib, "musa_aiter_kv_paged_to_linear_bfloat16", 5, 5)
    q = _bind(lib, "musa_aiter_kv_linear_to_paged_fp8_vec4_e4m3", 7, 5)
    dq = _bind(lib, "musa_aiter_kv_paged_fp8_to_linear_vec4_e4m3", 7, 5)
    for f in (q, dq):
        f.argtypes = f.argtypes[:-1] + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    rng = np.random.default_rng(10)
    out = {"cache": [NB, NH, HD, BS], "pattern": "one token per sequence, random block and offset"}
    parity = True
    for t in (16, 64, 256):
        blocks = rng.choice(NB, size=t, replace=False)
        slots_np = (blocks * BS + rng.integers(0, BS, size=t)).astype(np.int64)
        slots = torch.from_numpy(slots_np).to(dev)
        kl = torch.randn((t, NH, HD), generator=gen, device=dev).to(torch.bfloat16)
        vl = torch.randn((t, NH, HD), generator=gen, device=dev).to(torch.bfloat16)
        ks = (kl.float().abs().amax(dim=(0, 2)) / 448.0).contiguous()
        vs = (vl.float().abs().amax(dim=(0, 2)) / 448.0).contiguous()
        ok, ov = torch.empty_like(kl), torch.empty_like(vl)
        sa = (kl.data_ptr(), vl.data_ptr(), slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), t, NB, NH, HD, BS)
        gargs = (kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), ok.data_ptr(), ov.data_ptr(), t, NB, NH, HD, BS)
        qa = (kl.data_ptr(), vl.data_ptr(), slots.data_ptr(), qk.data_ptr(), qv.data_ptr(), ks.data_ptr(),
              vs.data_ptr(), t, NB, NH, HD, BS, 2)
        da = (qk.data_ptr(), qv.data_ptr(), slots.data_ptr(), ks.data_ptr(), vs.data_ptr(), ok.data_ptr(),
              ov.data_ptr(), t, NB, NH, HD, BS, 2)
        _check(sc(*sa, _stream()), "decode scatter")
        _check(q(*qa, _stream(), 1), "decode quant-store")
        _check(ga(*gargs, _stream()), "decode gather")
        torch.cuda.synchronize()
        parity &= bool(torch.equal(ok, kl) and torch.equal(ov, vl))
        # Parity outside the timed region: the written rows against the inputs (bf16) and against the
        # reference encoder's steps (FP8, tests/torch_ref.py), on the CPU.
        parity &= bool(torch.equal(torch_ref.paged_rows(kc)[slots], kl) and
                       torch.equal(torch_ref.paged_rows(vc)[slots], vl))
        want = torch_ref.fp8_quantize(kl.cpu(), ks.cpu().reshape(-1, 1), "e4m3")
        parity &= bool(torch.equal(torch_ref.paged_rows(qk)[slots].cpu(), want))
        _check(dq(*da, _stream(), 1), "decode dequant-gather")
        torch.cuda.synchronize()
        want_deq = torch_ref.fp8_dequantize(want, ks.cpu().reshape(-1, 1), "e4m3", torch.bfloat16)
        parity &= bool(torch.equal(ok.cpu(), want_deq))
        ms_s = batched_ms(lambda: _check(sc(*sa, _stream()), "decode scatter"), launches=100)
        ms_q = batched_ms(lambda: _check(q(*qa, _stream(), 1), "decode quant-store"), launches=100)
        ms_g = batched_ms(lambda: _check(ga(*gargs, _stream()), "decode gather"), launches=100)
        ms_d = batched_ms(lambda: _check(dq(*da, _stream(), 1), "decode dequant-gather"), launches=100)
        out[f"tokens_{t}"] = {"bf16_scatter_us": float(np.median(ms_s)) * 1e3,
                              "fp8_e4m3_quant_store_us": float(np.median(ms_q)) * 1e3,
                              "bf16_gather_us": float(np.median(ms_g)) * 1e3,
                              "fp8_e4m3_dequant_gather_us": float(np.median(ms_d)) * 1e3}
    out["parity"] = parity
    log("decode (scatter bf16/fp8, gather bf16/fp8): " + ", ".join(
        f"{k} {v['bf16_scatter_us']:.1f}/{v['fp8_e4m3_quant_store_us']:.1f}/{v['bf16_gather_us']:.1f}/"
        f"{v['fp8_e4m3_dequant_gather_us']:.1f} us" for k, v in out.items() if k.startswith("tokens_")))
    return out


def bench_cachegen() -> dict:
    """CacheGen-style codec (kv_cachegen_encode / kv_cachegen_decode, 256 bins) on a 32-layer K/V tensor of
    4096 tokens x 8 heads x 128 ([32, 2, 4096, 8, 128], 268,435,456 elements), in bf16 and float32.

    Bytes: encode reads the input twice (range pass, bin pass) and writes one byte per element; decode reads
    one byte and writes one output element per element (float32 codebook; bf16 output for the bf16 line).
    Parity, outside the timed region: the bins and the codebook against the reference's torch expressions
    (kv_transfer.py:1155-1158) evaluated by torch on this GPU, the CDF against cumsum(bincount) / numel
    within one float32 ulp (torch accumulates and divides differently on the GPU), and decode against
    ``codebook[encoded]``."""
    import musa_aiter

    dev = torch.device("cuda", 0)
    shape = (NL, 2, 4096, NH, HD)
    n = int(np.prod(shape))
    out = {"shape": list(shape), "elements": n, "num_bins": 256}
    g = torch.Generator(device=dev).manual_seed(9)
    base = torch.randn(shape, generator=g, device=dev)
    for dtype, label, dec_dtype in ((torch.bfloat16, "bf16", torch.bfloat16), (torch.float32, "float32", None)):
        x = base.to(dtype)
        enc, book, cdf = musa_aiter.kv_cachegen_encode(x, num_bins=256)
        work = x.float()
        mn, mx = work.min(), work.max()
        ref = torch.round((work - mn) * ((256 - 1) / (mx - mn))).clamp_(0, 255).to(torch.uint8)
        ref_book = torch.linspace(mn.item(), mx.item(), 256, dtype=torch.float32, device=dev)
        counts = torch.bincount(ref.reshape(-1).long(), minlength=256).double()
        ref_cdf = torch.cat([torch.zeros(1, dtype=torch.float64, device=dev), torch.cumsum(counts, 0) / n]).float()
        ulp = torch.finfo(torch.float32).eps
        dec = musa_aiter.kv_cachegen_decode(enc, book, dtype=dec_dtype)
        ref_dec = book[enc.long()] if dec_dtype is None else book.to(dec_dtype)[enc.long()]
        parity = {"bins": bool(torch.equal(enc, ref)), "codebook_vs_torch_linspace": bool(torch.equal(book, ref_book)),
                  "cdf_within_1ulp": bool(((cdf - ref_cdf).abs() <= ulp * ref_cdf.abs()).all()),
                  "decode": bool(torch.equal(dec, ref_dec))}
        del work, ref, ref_dec, dec
        eb = x.element_size()
        enc_ms = batched_ms(lambda: musa_aiter.kv_cachegen_encode(x, num_bins=256), launches=10, reps=5)
        dec_ms = batched_ms(lambda: musa_aiter.kv_cachegen_decode(enc, book, dtype=dec_dtype), launches=10, reps=5)
        ob = 4 if dec_dtype is None else torch.tensor([], dtype=dec_dtype).element_size()
        out[label] = {"encode": {**rate(n * (2 * eb + 1), enc_ms), "bytes": n * (2 * eb + 1)},
                      "decode": {**rate(n * (1 + ob), dec_ms), "bytes": n * (1 + ob),
                                 "output_dtype": "float32" if dec_dtype is None else "bfloat16"},
                      "parity": parity}
        del x, enc, book, cdf
        torch.cuda.empty_cache()
    log("cachegen: " + ", ".join(f"{d} {k} {out[d][k]['gbs']:.0f} GB/s" for d in ("bf16", "float32")
                                 for k in ("encode", "decode")))
    return out


def device_copy(mib: int, reps: int = 5) -> dict:
    """Plain device-to-device copy of a known size (torch ``copy_``): the achievable copy rate of this
    GPU and the calibration kernel for the FETCH_SIZE / WRITE_SIZE traffic counters."""
    dev = torch.device("cuda", 0)
    src = torch.empty(mib << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    timer = EventTimer()
    for _ in range(reps):
        e = timer.start()
        dst.copy_(src)
        timer.stop(e)
    torch.cuda.synchronize()
    ms = np.array(timer.ms())
    nbytes = 2 * (mib << 20)
    return {"bytes_read_plus_written": nbytes, "avg_ms": float(ms.mean()), "gbs": nbytes / (ms.mean() * 1e-3) / 1e9}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, min_s: float) -> tuple[float, int]:
    """Seconds per call of ``fn`` over at least ``min_s`` seconds (one untimed call first)."""
    fn()
    calls, start = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        elapsed = time.perf_counter() - start
        if elapsed >= min_s:
            return elapsed / calls, calls


def cpu_baseline(slots_np: np.ndarray, kc: torch.Tensor, vc: torch.Tensor, sample_tokens: int = 32768,
                 vector_layers: int = 8) -> dict:
    """The reference's CPU algorithm on this host's cores, in the torch operations it uses
    (oracle/torch_cpu_port.py: advanced-index gather + torch.where, kv_transfer.py:3047-3089; per-token
    loop scatter, :3092-3112), with torch's thread count at the host's CPU share.

    value: configs[1]'s step (gather + scatter of K and V in all 32 layers) on its first ``sample_tokens``
    tokens -- the loop scatter of all 128k tokens would take minutes.  Legs: configs[0] at full shape with
    the same ops; configs[1]'s whole token set, first ``vector_layers`` layers, with whole-tensor index ops
    (the vectorised torch-CPU line).  Caches are copied to the host one layer at a time, outside the timed
    regions; algorithmic bytes as for the GPU."""
    from oracle import torch_cpu_port as tp

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        t = int(slots_np.shape[0])
        n = min(sample_tokens, t)
        s_cpu = torch.from_numpy(slots_np)
        s_sample = s_cpu[:n].clone()
        gather_s = scatter_s = 0.0
        for layer in range(NL):
            for cache in (kc, vc):
                host = cache[layer].cpu()
                start = time.perf_counter()
                lin = tp.paged_to_linear_reference_ops(host, s_sample)
                mid = time.perf_counter()
                tp.linear_to_paged_reference_ops(lin, host, s_sample)
                gather_s += mid - start
                scatter_s += time.perf_counter() - mid
        per_dir = 2 * (2 * NL * n * ROW * 2) + 8 * n
        value = 2 * per_dir / (gather_s + scatter_s) / 1e9

        # configs[0] at full shape: fp16 [1024, 8, 128, 16] caches, 32 sequences of 1-512 tokens.
        s1 = torch.from_numpy(make_slots(1001, 32, 1, 512, 1024, BS))
        t1 = int(s1.shape[0])
        gen = torch.Generator().manual_seed(1)
        k1 = torch.randn((1024, NH, HD, BS), generator=gen).to(torch.float16)
        v1 = torch.randn((1024, NH, HD, BS), generator=gen).to(torch.float16)
        b1 = 2 * (2 * t1 * ROW * 2) + 8 * t1
        g1, gcalls = _timed(lambda: (tp.paged_to_linear_reference_ops(k1, s1),
                                     tp.paged_to_linear_reference_ops(v1, s1)), 1.5)
        l1 = (tp.paged_to_linear_reference_ops(k1, s1), tp.paged_to_linear_reference_ops(v1, s1))
        sc1, scalls = _timed(lambda: (tp.linear_to_paged_reference_ops(l1[0], k1, s1),
                                      tp.linear_to_paged_reference_ops(l1[1], v1, s1)), 1.5)

        # Vectorised torch on configs[1]'s whole token set, first layers.
        vec_g = vec_s = 0.0
        for layer in range(min(vector_layers, NL)):
            for cache in (kc, vc):
                host = cache[layer].cpu()
                start = time.perf_counter()
                lin = tp.paged_to_linear_vectorised(host, s_cpu)
                mid = time.perf_counter()
                tp.linear_to_paged_vectorised(lin, host, s_cpu)
                vec_g += mid - start
                vec_s += time.perf_counter() - mid
        vec_dir = 2 * (2 * min(vector_layers, NL) * t * ROW * 2) + 8 * t
    finally:
        torch.set_num_threads(prev_threads)
    return {
        "value": value, "unit": "GB/s", "cores": threads, "kind": "port", "config": "configs[1]",
        "algorithm": "the reference's torch ops: advanced-index gather + torch.where (kv_transfer.py:3047-3089), "
                     "per-token .item()/copy_ loop scatter (:3092-3112); oracle/torch_cpu_port.py",
        "sample": f"configs[1] gather + scatter of K and V in all {NL} layers for the first {n} of {t} tokens "
                  f"({gather_s + scatter_s:.1f} s: gather {gather_s:.2f} s, scatter loop {scatter_s:.1f} s); "
                  f"torch threads {threads} (the scatter loop runs on one); host cpus {os.cpu_count()}",
        "cpu_model": _cpu_model(),
        "legs": {
            "configs[1]_gather_reference_ops": {"gbs": per_dir / gather_s / 1e9, "seconds": gather_s,
                                               "tokens": n},
            "configs[1]_scatter_reference_ops": {"gbs": per_dir / scatter_s / 1e9, "seconds": scatter_s,
                                                "tokens": n},
            "configs[0]_gather_reference_ops": {"gbs": b1 / g1 / 1e9, "ms_per_call": g1 * 1e3, "calls": gcalls,
                                               "tokens": t1, "tokens_per_ms": t1 / (g1 * 1e3),
                                               "shape": "full: fp16 caches [1024, 8, 128, 16], 32 seqs U[1,512]"},
            "configs[0]_scatter_reference_ops": {"gbs": b1 / sc1 / 1e9, "ms_per_call": sc1 * 1e3, "calls": scalls,
                                                "tokens": t1},
            "configs[1]_vectorised_torch": {"gbs_gather": vec_dir / vec_g / 1e9, "gbs_scatter": vec_dir / vec_s / 1e9,
                                            "layers": min(vector_layers, NL), "tokens": t,
                                            "ops": "index on the [NB, BS, NH, HD] view; index_put_ after a "
                                                   "last-writer pass"},
        },
    }


def _pct(gbs: float) -> str:
    return f"{gbs:.0f} GB/s {100.0 * gbs / HBM_PEAK_GBS:.1f}%"


def _of(gbs: float, ceiling: float) -> str:
    return f"{100.0 * gbs / ceiling:.0f}% of pattern {ceiling:.0f}"


def summary_lines(line: dict) -> list[str]:
    """The run's figures for every BASELINE config in a few short lines (under 1.5 KB in all): the end of
    the output, where a log tail keeps them.  GB/s are algorithmic read+write bytes; % is of 8 TB/s;
    'of pattern' is the kernel's fraction of the same-pattern block copy timed in this process."""
    out = []
    d, c, p = line["directions"], line["ceilings"], line.get("placements")
    s2 = (f"cfg2 bf16 32L step {_pct(line['value'])} ({100.0 * line['value'] / c['step_ceiling_gbs']:.0f}% of "
          f"{c['step_ceiling_gbs']:.0f}) | scatter {_pct(d['scatter']['gbs'])} "
          f"{_of(d['scatter']['gbs'], c['scatter_pattern']['gbs'])} | gather {_pct(d['gather']['gbs'])} "
          f"{_of(d['gather']['gbs'], c['gather_pattern']['gbs'])} | seq copy {c['sequential']['gbs']:.0f}")
    if p:
        s2 += f" | placements {p['step_gbs_min']:.0f}/{p['step_gbs_median']:.0f}/{p['step_gbs_max']:.0f}"
    out.append(s2)
    x = line.get("extra", {})
    c1 = x.get("config1_fp16_single_layer_gather")
    if c1:
        us, fl = c1["gather"]["p50_ms"] * 1e3, c1["floor"]["gather_pattern"]["p50_ms"] * 1e3
        out.append(f"cfg1 fp16 gather {us:.1f} us {_pct(c1['gather']['gbs'])} (floor {fl:.1f} us, "
                   f"{100.0 * fl / us:.0f}%)")
    c3 = x.get("config3_fp8")
    if c3:
        qp, dp = c3["ceilings"]["quant_store_pattern"]["gbs"], c3["ceilings"]["dequant_gather_pattern"]["gbs"]
        parts = []
        for name in ("e4m3_per_head", "e4m3_scalar", "e5m2_per_head"):
            v = c3.get(name)
            if v:
                q, g = v["quant_store"]["gbs"], v["dequant_gather"]["gbs"]
                parts.append(f"{name} quant {_pct(q)} ({100.0 * q / qp:.0f}%) dequant {_pct(g)} "
                             f"({100.0 * g / dp:.0f}%)")
        out.append(f"cfg3 fp8 ({c3.get('cache_sets_rotated', 1)} cache sets rotated) [patterns quant {qp:.0f} "
                   f"dequant {dp:.0f}] " + " | ".join(parts))
    c4 = x.get("config4_lmcache_two_x_nl")
    if c4:
        api, ce = c4["gather_per_chunk_call"], c4["gather_per_chunk_c_abi"]
        fl = c4["per_chunk_floor_pattern_copy"]["p50_ms"] * 1e3
        out.append(f"cfg4 2xNL chunk api {api['p50_ms'] * 1e3:.1f} us {_pct(api['gbs'])} | C entry "
                   f"{ce['p50_ms'] * 1e3:.1f} us {_pct(ce['gbs'])} (floor {fl:.1f} us) | batched gather "
                   f"{_pct(c4['gather_batched_16']['gbs'])} scatter {_pct(c4['scatter_batched_16']['gbs'])}")
    c5 = x.get("config5_mla_rows")
    if c5:
        b = c5["bf16_576"]
        out.append(f"cfg5 mla bf16 gather {_pct(b['gather']['gbs'])} "
                   f"{_of(b['gather']['gbs'], b['ceilings']['gather_pattern']['gbs'])} | scatter "
                   f"{_pct(b['scatter']['gbs'])} {_of(b['scatter']['gbs'], b['ceilings']['scatter_pattern']['gbs'])}"
                   f" | fp8 656B rows {_pct(c5['fp8_656_rows']['gather']['gbs'])}")
    dec = x.get("decode_step_scatters")
    if dec:
        ts = [k for k in dec if k.startswith("tokens_")]
        def us(key):
            return "/".join(f"{dec[k][key]:.1f}" for k in ts if key in dec[k])
        out.append("decode us/call T=" + "/".join(k[7:] for k in ts) + ": scatter bf16 " + us("bf16_scatter_us")
                   + ", fp8 e4m3 " + us("fp8_e4m3_quant_store_us") + " | gather bf16 " + us("bf16_gather_us")
                   + ", fp8 e4m3 " + us("fp8_e4m3_dequant_gather_us"))
    nxt = []
    for key, names in (("dense_preload_and_block_copies",
                        (("load_and_reshape_flash", "dense load"), ("reshape_and_cache_back_flash", "write-back"),
                         ("load_and_dequantize_fp8_flash_e4m3", "fp8 dense load"), ("triton_indexed_to_dense", "csr"),
                         ("copy_paged_blocks_32_layers", "block copy"))),
                       ("sglang_hicache_transfers", (("all_layer_lf_pf_backup", "hicache backup"),
                                                     ("per_layer_pf_lf_load_x32", "hicache load")))):
        v = x.get(key) or {}
        nxt += [f"{label} {v[k]['gbs']:.0f}" for k, label in names if isinstance(v.get(k), dict)]
    if nxt:
        out.append("next rows GB/s: " + ", ".join(nxt))
    parity = [bool(line.get("parity_roundtrip"))]
    for v in x.values():
        if isinstance(v, dict):
            parity += [bool(w) for k, w in v.items() if k == "parity" and isinstance(w, bool)]
            parity += [bool(w.get("parity")) for w in v.values() if isinstance(w, dict) and
                       isinstance(w.get("parity"), bool)]
    cpu = line.get("cpu_baseline")
    tail = f"parity {'all ok' if all(parity) else 'FAILED'} ({len(parity)} checks)"
    if cpu:
        tail += f" | cpu baseline {cpu['value']:.2f} GB/s on {cpu['cores']} threads ({cpu['kind']})"
    tail += f" | roofline frac {line['roofline']['frac']:.3f} ({line['roofline']['kernel']})"
    out.append(tail)
    return [f"[summary] {s}" for s in out]


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--configs", default="1,2,3,4,5,6,7,8,9,10",
                        help="comma list of BASELINE configs to run (2, the headline, always runs; 6 = dense "
                             "preload and block copies; 7 = SGLang HiCache transfers; 8 = LMCache host <-> "
                             "device copy batches; 9 = CacheGen codec; 10 = decode-step scatter latency)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--placements", type=int, default=5,
                        help="re-allocate the configs[1] caches this many times and time the step on each "
                             "(0 = skip)")
    parser.add_argument("--copy-mib", type=int, default=1024,
                        help="size of the plain device copy timed first (0 = skip)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported (the path does not shard "
              "across GPUs in this build; see the sharding notes in the docs)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    configs = {int(c) for c in args.configs.split(",") if c}
    extra = {}
    if args.copy_mib > 0:
        extra["device_copy"] = device_copy(args.copy_mib)
        log(f"device copy of {args.copy_mib} MiB: {extra['device_copy']['gbs']:.0f} GB/s (read+write)")
        torch.cuda.empty_cache()
    c2 = bench_config2(args.steps, args.warmup)
    slots_np, slots, kc, vc, kl, vl, ok, ov = c2.pop("_tensors")
    log(f"config 2: scatter {c2['scatter']['gbs']:.0f} GB/s, gather {c2['gather']['gbs']:.0f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(slots_np, kc, vc)
        log(f"cpu baseline {cpu['value']:.2f} GB/s ({cpu['cores']} threads)")
    ceilings = config2_ceilings(slots_np, kc, vc, kl, vl)
    del kc, vc
    placements = None
    if args.placements > 0:
        placements = config2_placements(slots, kl, vl, ok, ov, args.placements, 5)
    del kl, vl, ok, ov, slots
    torch.cuda.empty_cache()
    runners = {1: ("config1_fp16_single_layer_gather", bench_config1), 3: ("config3_fp8", bench_config3),
               4: ("config4_lmcache_two_x_nl", bench_config4), 5: ("config5_mla_rows", bench_config5),
               6: ("dense_preload_and_block_copies", bench_dense), 7: ("sglang_hicache_transfers", bench_hicache),
               8: ("lmcache_host_device_batches", bench_batch_copy), 9: ("cachegen_codec", bench_cachegen),
               10: ("decode_step_scatters", bench_decode)}
    for cfg in sorted(configs - {2}):
        if cfg not in runners:
            continue
        key, fn = runners[cfg]
        extra[key] = fn()
        log(f"config {cfg} done")
        torch.cuda.empty_cache()
    achieved = c2["bytes_per_direction"] / (c2["dominant_avg_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(c2["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) KV rows, random block tables; no checkpoint)",
        "config": {"workload": "configs[1]: 32-layer linear->paged scatter + paged->linear gather, bf16, caches "
                               "[32,8192,8,128,16] (paged [NB,NH,HD,BS]), 64 seqs len U[128,4096]",
                   "tokens": c2["tokens"], "layers": NL, "num_blocks": NB, "block_size": BS, "kv_heads": NH,
                   "head_dim": HD, "step": "scatter + gather (2 launches of the C-ABI)"},
        "pct_of_peak": round(100.0 * c2["value_gbs"] / HBM_PEAK_GBS, 2),
        "tokens_per_ms": {"scatter": round(c2["scatter"]["tokens_per_ms"], 1),
                          "gather": round(c2["gather"]["tokens_per_ms"], 1)},
        "directions": {"scatter": c2["scatter"], "gather": c2["gather"]},
        "parity_roundtrip": c2["parity_roundtrip"],
        "roofline": {"bound": "hbm", "kernel": ("paged_block_scatter_kernel (scatter, 64 planes)"
                                                if c2["dominant"] == "scatter"
                                                else "paged_tile_kernel (gather, 64 planes)"),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(c2["dominant"]),
                     "traffic_source": "rocprofv3 FETCH_SIZE x2.000 + WRITE_SIZE x1.000 per dispatch "
                                       "(profiles/kv_kernels_hbm_traffic.md)",
                     "bytes_per_launch": c2["bytes_per_direction"], "avg_launch_ms": round(c2["dominant_avg_ms"], 4)},
        "cpu_baseline": cpu,
        "ceilings": {**ceilings, "gather_frac_of_pattern": c2["gather"]["gbs"] / ceilings["gather_pattern"]["gbs"],
                     "scatter_frac_of_pattern": c2["scatter"]["gbs"] / ceilings["scatter_pattern"]["gbs"],
                     "step_frac_of_ceiling": c2["value_gbs"] / ceilings["step_ceiling_gbs"]},
        "placements": placements,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    sys.stderr.write("\n".join(summary_lines(line)) + "\n")
    sys.stderr.flush()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
