"""CPU oracle for the KV-cache movement path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference PyTorch implementation of
musa_aiter 0.5.0's KV-movement ops (musa_aiter/ops/kv_transfer.py and
musa_aiter/ops/lmcache_kv_transfer.py), one function per reference function,
each citing the file:line it follows.  It exists to check the HIP kernels:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and never as the thing measured or shipped.  The product
package (``musa-aiter_amd/musa_aiter``) does not import it and fails loudly
when its HIP library is missing.

How each part is pinned (checked independently of this restatement):

- copies (paged<->linear, merged, MLA, LMCache, byte rows, strided blocks):
  the reference tests' known-answer scenarios and round trips
  (tests/test_oracle_kats.py), brute-force per-element loops on small inputs
  and torch advanced-indexing equivalents (tests/test_oracle_copies.py);
- FP8 encode/decode: exhaustive comparison over every bf16 and fp16 bit
  pattern and a set of scales against (a) a literal torch restatement of the
  reference steps, (b) torch's own float8_e4m3fn / float8_e5m2 casts on the
  range where the reference encoder is an IEEE round-to-nearest-even cast,
  and (c) special-value known answers (tests/test_oracle_fp8.py);
- bf16 rounding: exhaustive comparison with torch's ``.to(torch.bfloat16)``.

Parity unpinned: torch-version-specific behaviour of ``torch.log2`` inside the
reference encoder (only the current torch is available to compare against).
"""
