"""Build libmusa_aiter_kv_hip.so for gfx950 with hipcc, and the host helper module, in-tree.

Both are written to ``musa_aiter/_lib/`` next to the Python host layer so that
they travel with the source tree: the HIP kernel library (C ABI) and
``_kv_host``, a small CPython extension built with g++ against torch's headers
that checks lists of cache tensors and packs their addresses.  Usage::

    python musa-aiter_amd/build.py            # build (always recompiles)
    python musa-aiter_amd/build.py --check    # print the hipcc command only
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT_DIR = ROOT / "musa_aiter" / "_lib"
LIB_NAME = "libmusa_aiter_kv_hip.so"
SOURCES = ("kv_paged_tiles.hip", "kv_paged_waves.hip", "kv_rows.hip", "kv_batch_copy.hip", "kv_cachegen.hip",
           "kv_pattern.hip", "kv_abi.hip")
ARCH = os.environ.get("MUSA_AITER_HIP_ARCH", "gfx950")

# Packed fp32 VALU forms are disabled for the whole library; fp32 division
# stays correctly rounded, denormals are preserved (no fast-math) and no
# floating-point contraction is allowed, which the FP8 codec relies on for
# bit-exact parity with the reference's separately rounded torch ops.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-fno-fast-math",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    f"-I{ROOT.parent / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    noise = [ln for ln in proc.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


HOST_SOURCE = "kv_host.cpp"
HOST_MODULE = "_kv_host"


def host_module_path() -> Path:
    return OUT_DIR / (HOST_MODULE + sysconfig.get_config_var("EXT_SUFFIX"))


def _build_host() -> Path:
    """The host helper extension: g++ against the installed torch's headers and libraries."""
    from torch.utils import cpp_extension

    import torch

    out = host_module_path()
    tmp = out.with_name(out.name + ".tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-shared", "-fPIC", "-std=c++17", "-Wall",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={HOST_MODULE}",
           f"-I{sysconfig.get_paths()['include']}", f"-I{ROOT.parent / 'include'}",
           *[f"-I{p}" for p in cpp_extension.include_paths()],
           str(CSRC / HOST_SOURCE), "-o", str(tmp),
           *[f"-L{p}" for p in cpp_extension.library_paths()], "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"host module build failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = ROOT / "_build"
    obj_dir.mkdir(exist_ok=True)
    objs = [obj_dir / (Path(s).stem + ".o") for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as pool:
        host = pool.submit(_build_host)
        futures = [pool.submit(_compile, CSRC / s, o) for s, o in zip(SOURCES, objs)]
        for fut in futures:
            fut.result()
        host_path = host.result()
    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
        print(f"built {host_path}")
    return out


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--check", action="store_true", help="print the compile command and exit")
    args = parser.parse_args()
    if args.check:
        print(" ".join([hipcc(), *HIPCC_FLAGS, "-c", "<src>"]))
        return 0
    build(verbose=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
