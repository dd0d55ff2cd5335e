"""torch-CPU restatement of the reference's paged-A copy algorithm -- TEST INFRASTRUCTURE ONLY.

bench.py's CPU-baseline leg times these on the GPU box's host cores; tests/ pins them against
oracle/kv_oracle.py.  Two forms per direction, both on CPU tensors of any dtype:

* ``*_reference_ops``: the reference's own torch operations, step for step:
  ``_kv_paged_to_linear_compute`` (musa_aiter 0.5.0 kv_transfer.py:3047-3089: advanced-index gather
  ``cache[bid, :, :, off]`` and ``torch.where`` on the valid mask) and
  ``_kv_linear_to_paged_scatter`` (:3092-3112: a Python token loop, ``.item()`` per slot, one
  ``copy_`` per K/V row);
* ``*_vectorised``: the same results from whole-tensor index ops (``index_put_`` on the
  block-column view after dropping all but the last writer of a repeated slot), the labelled
  "vectorised torch-CPU" line of the baseline.

Nothing here is part of the product path.
"""

from __future__ import annotations

import torch


def paged_to_linear_reference_ops(cache: torch.Tensor, slots: torch.Tensor) -> torch.Tensor:
    """One cache [NB, NH, HD, BS] -> [T, NH, HD]; skipped tokens (slot < 0) are zeros."""
    bs = cache.shape[3]
    valid = slots >= 0
    safe = torch.where(valid, slots, torch.zeros_like(slots))
    bid = torch.div(safe, bs, rounding_mode="floor")
    off = safe - bid * bs
    gathered = cache[bid, :, :, off]
    mask = valid.view(-1, 1, 1)
    return torch.where(mask, gathered, torch.zeros_like(gathered))


def linear_to_paged_reference_ops(lin: torch.Tensor, cache: torch.Tensor, slots: torch.Tensor) -> None:
    """[T, NH, HD] -> cache [NB, NH, HD, BS] in place, one token at a time (the last writer wins)."""
    nb, _, _, bs = cache.shape
    for t in range(slots.shape[0]):
        s = int(slots[t].item())
        if s < 0:
            continue
        b, off = divmod(s, bs)
        if not (0 <= b < nb):
            raise RuntimeError(f"invalid slot mapping {s} at token {t}")
        cache[b, :, :, off].copy_(lin[t])


def _last_writer(slots: torch.Tensor) -> torch.Tensor:
    """Indices of the tokens that write: valid, and not followed by another token with the same slot."""
    n = slots.shape[0]
    idx = torch.arange(n, dtype=torch.int64)
    valid = slots >= 0
    key = torch.where(valid, slots, torch.full_like(slots, -1))
    # For each slot, the largest token index naming it: scatter_reduce with amax over slots.
    top = int(key.max().item()) + 1 if n else 0
    last = torch.full((max(top, 1),), -1, dtype=torch.int64)
    if top:
        last.scatter_reduce_(0, key.clamp(min=0)[valid], idx[valid], reduce="amax")
    keep = valid.clone()
    keep[valid] = last[key[valid]] == idx[valid]
    return idx[keep]


def paged_to_linear_vectorised(cache: torch.Tensor, slots: torch.Tensor) -> torch.Tensor:
    """The gather with whole-tensor ops on the token-major view [NB, BS, NH, HD] of the cache."""
    nb, nh, hd, bs = cache.shape
    rows = cache.permute(0, 3, 1, 2)                       # [NB, BS, NH, HD] view
    valid = slots >= 0
    out = torch.zeros((slots.shape[0], nh, hd), dtype=cache.dtype)
    s = slots[valid]
    out[valid] = rows[torch.div(s, bs, rounding_mode="floor"), s % bs]
    return out


def linear_to_paged_vectorised(lin: torch.Tensor, cache: torch.Tensor, slots: torch.Tensor) -> None:
    """The scatter with one ``index_put_`` on the token-major view (repeated slots keep the last token)."""
    bs = cache.shape[3]
    keep = _last_writer(slots)
    s = slots[keep]
    rows = cache.permute(0, 3, 1, 2)
    rows.index_put_((torch.div(s, bs, rounding_mode="floor"), s % bs), lin[keep])
