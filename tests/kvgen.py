"""Seeded input generators shared by the tests and bench.py.

Slot mappings follow the BASELINE workloads: every sequence takes whole blocks
from one random permutation of the cache's blocks, so its tokens fill blocks
in order (``slot = block_table[j // BS] * BS + j % BS``).  Variants add
skipped tokens, duplicates and unstructured slots for edge cases.
"""

from __future__ import annotations

import numpy as np
import torch

BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32, torch.uint8: torch.uint8}
NP_BITS = {torch.bfloat16: np.uint16, torch.float16: np.uint16, torch.float32: np.uint32, torch.uint8: np.uint8}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw storage bits of a tensor as a numpy array (bit-exact comparisons)."""
    return t.detach().contiguous().view(BITS[t.dtype]).cpu().numpy().view(NP_BITS[t.dtype])


def sequence_lengths(rng: np.random.Generator, num_seqs: int, lo: int, hi: int, *, num_blocks: int,
                     block_size: int) -> list[int]:
    """Lengths uniform in [lo, hi], redrawn (same generator) until all sequences fit in the cache."""
    while True:
        lengths = rng.integers(lo, hi + 1, size=num_seqs)
        if int(np.sum((lengths + block_size - 1) // block_size)) <= num_blocks:
            return [int(x) for x in lengths]


def sequence_slots(rng: np.random.Generator, lengths: list[int], *, num_blocks: int, block_size: int) -> np.ndarray:
    perm = rng.permutation(num_blocks)
    need = sum((length + block_size - 1) // block_size for length in lengths)
    if need > num_blocks:
        raise ValueError(f"sequences need {need} blocks, cache has {num_blocks}")
    out, pos = [], 0
    for length in lengths:
        nblk = (length + block_size - 1) // block_size
        table = perm[pos:pos + nblk]
        pos += nblk
        j = np.arange(length)
        out.append(table[j // block_size] * block_size + j % block_size)
    return np.concatenate(out).astype(np.int64) if out else np.zeros(0, np.int64)


def make_slots(kind: str, rng: np.random.Generator, *, block_size: int, tokens: int,
               spare_blocks: int = 7) -> tuple[np.ndarray, int]:
    """(slot_mapping, num_blocks) for a named pattern; num_blocks leaves ``spare_blocks`` unused blocks."""
    bs = block_size
    if kind in ("sequences", "skips"):
        lengths, remaining = [], tokens
        while remaining > 0:
            length = int(min(remaining, rng.integers(1, 3 * bs + 2)))
            lengths.append(length)
            remaining -= length
        nb = sum((length + bs - 1) // bs for length in lengths) + spare_blocks
        slots = sequence_slots(rng, lengths, num_blocks=nb, block_size=bs)
        if kind == "skips":
            slots[rng.random(tokens) < 0.2] = -1
    elif kind == "random":
        nb = 2 * ((tokens + bs - 1) // bs) + spare_blocks
        slots = rng.permutation(nb * bs)[:tokens].astype(np.int64)
    elif kind == "duplicates":
        nb = (tokens + bs - 1) // bs + spare_blocks
        slots = rng.integers(-1, max(2, (nb * bs) // 4), size=tokens).astype(np.int64)
    elif kind == "decode":
        # Decode steps: each sequence appends 1-6 tokens at a random offset of
        # its own blocks (a run may cross into the next block); every eighth
        # appends a longer chunk.  Tiles mix runs of one token with whole blocks.
        lengths, remaining = [], tokens
        while remaining > 0:
            length = int(rng.integers(2 * bs, 3 * bs + 2)) if rng.random() < 0.125 else int(rng.integers(1, 7))
            lengths.append(min(remaining, length))
            remaining -= lengths[-1]
        offsets = rng.integers(0, bs, size=len(lengths))
        need = [(int(o) + n + bs - 1) // bs for o, n in zip(offsets, lengths)]
        nb = sum(need) + spare_blocks
        perm, pos, out = rng.permutation(nb), 0, []
        for o, n, k in zip(offsets, lengths, need):
            table = perm[pos:pos + k]
            pos += k
            j = int(o) + np.arange(n)
            out.append(table[j // bs] * bs + j % bs)
        slots = np.concatenate(out).astype(np.int64)
    elif kind == "identity":
        nb = (tokens + bs - 1) // bs + spare_blocks
        slots = np.arange(tokens, dtype=np.int64)
    else:
        raise ValueError(kind)
    return slots, nb


def random_payload(shape, dtype: torch.dtype, gen: torch.Generator, device="cpu") -> torch.Tensor:
    """Random bit patterns (including NaN/Inf encodings) so copies are checked bit-exactly."""
    if dtype == torch.uint8:
        return torch.randint(0, 256, shape, dtype=torch.uint8, generator=gen).to(device)
    itype = BITS[dtype]
    info = torch.iinfo(itype)
    raw = torch.randint(info.min, info.max, shape, dtype=itype, generator=gen)
    return raw.view(dtype).to(device)
