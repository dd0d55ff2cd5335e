"""Writes fp8_codec_golden.npz: the reference's FP8 encoder / decoder on exhaustive inputs.

Run once, in the build container only (the reference tree is not present elsewhere):

    python tests/golden/make_fp8_golden.py /root/reference

It imports the two reference functions that no reference test pins byte for byte,
``_fp8_quantize_to_uint8`` and ``_fp8_dequantize_from_uint8`` (musa_aiter 0.5.0,
musa_aiter/ops/kv_transfer.py:2161-2200), runs them on CPU tensors with this container's torch,
and stores inputs and outputs as data.  Nothing else of the reference is used or copied.

Encoder vectors: every bf16 and every fp16 bit pattern, divided by each scale of SCALES, for E4M3
and E5M2 (uint8 codes).  Decoder vectors: all 256 codes times each scale, rounded to bf16, fp16
and float32 (raw bits).
"""

from __future__ import annotations

import os
import sys

import numpy as np

# Scales: unit, powers of two, one ulp either side of 1, and irregular per-head-like values.
SCALES = np.array([1.0, 0.0625, 2.0 ** 8, 1.0 + 2.0 ** -23, 1.0 - 2.0 ** -24, 0.013392857, 0.3, 7.0],
                  dtype=np.float32)


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    import torch
    from musa_aiter.ops.kv_transfer import _fp8_dequantize_from_uint8, _fp8_quantize_to_uint8

    bits16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    inputs = {
        "bf16": torch.from_numpy(bits16.view(np.int16)).view(torch.bfloat16),
        "fp16": torch.from_numpy(bits16.view(np.int16)).view(torch.float16),
    }
    out = {"scales": SCALES, "torch_version": np.array(torch.__version__)}
    for fmt in ("e4m3", "e5m2"):
        for name, x in inputs.items():
            codes = np.stack([_fp8_quantize_to_uint8(x, torch.tensor(float(s), dtype=torch.float32), fmt).numpy()
                              for s in SCALES])
            out[f"encode_{fmt}_{name}"] = codes.astype(np.uint8)      # [scales, 65536]
        codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
        for dname, dtype, view in (("bf16", torch.bfloat16, np.uint16), ("fp16", torch.float16, np.uint16),
                                   ("f32", torch.float32, np.uint32)):
            vals = [_fp8_dequantize_from_uint8(codes, torch.tensor(float(s), dtype=torch.float32), fmt, dtype)
                    for s in SCALES]
            itype = torch.int16 if view is np.uint16 else torch.int32
            out[f"decode_{fmt}_{dname}"] = np.stack([v.view(itype).numpy().view(view) for v in vals])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp8_codec_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes) with torch {torch.__version__}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
