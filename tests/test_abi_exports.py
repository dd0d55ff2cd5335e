"""The C-ABI library loads (no GPU needed) and exports every function include/*.h declares.

Declarations are read from the header itself, with its declaration macros
expanded for their dtype / format suffixes, so a symbol added to the header
without an implementation (or renamed on one side) fails here.
"""

from __future__ import annotations

import ctypes
import pathlib
import re

from musa_aiter.ops import _hip

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "musa_aiter_kv_hip.h"


def _declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = text.replace("\\\n", " ")
    macros = {}
    for m in re.finditer(r"#define\s+(\w+)\((\w+)\)\s+(.*)", text):
        macros[m.group(1)] = (m.group(2), m.group(3))
    expanded = []
    for line in text.splitlines():
        m = re.match(r"\s*(\w+)\((\w+)\)\s*$", line)
        if m and m.group(1) in macros:
            param, body = macros[m.group(1)]
            expanded.append(re.sub(rf"\b{param}\b", m.group(2), body.replace(f"##{param}", m.group(2))))
        elif not line.lstrip().startswith("#"):
            expanded.append(line)
    body = "\n".join(expanded)
    return set(re.findall(r"(?:int64_t|int|const char\*)\s+(\w+)\s*\(", body))


def test_header_declares_expected_families():
    names = _declared_symbols()
    assert len(names) == 127
    for required in ("musa_aiter_kv_load_and_reshape_flash_half", "musa_aiter_kv_triton_indexed_to_dense_bfloat16",
                     "musa_aiter_kv_reshape_and_cache_back_flash_float", "musa_aiter_kv_copy_paged_blocks_fp8_vec8",
                     "musa_aiter_hip_paged_dense_tiles","musa_aiter_kv_paged_to_linear_bfloat16", "musa_aiter_kv_linear_to_paged_multi_layer_half",
                     "musa_aiter_kv_paged_fp8_to_linear_vec4_e5m2", "lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16",
                     "lmcache_mla_paged_to_buffer_list_bfloat16", "musa_aiter_kv_copy_paged_rows_layer_table_u8",
                     "lmcache_kv_strided_block_transfer", "musa_aiter_hip_paged_tiles",
                     "musa_aiter_hicache_transfer_bytes", "musa_aiter_hicache_transfer_abi_version",
                     "musa_aiter_hip_copy_rows_paged", "musa_aiter_hip_copy_rows_packed", "musa_aiter_hip_copy_blocks",
                     "musa_aiter_hip_allocated_bytes", "musa_aiter_hip_index_max"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    missing = sorted(name for name in _declared_symbols() if not hasattr(lib, name))
    assert missing == []


def test_probes_callable_without_gpu():
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    for name in ("musa_aiter_kv_transfer_abi_version", "native_lmcache_kv_transfer_abi_version",
                 "musa_aiter_fp8_kv_cache_abi_version", "musa_aiter_dsv4_kv_copy_abi_version",
                 "musa_aiter_hicache_transfer_abi_version"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        assert fn() == 1
    name = lib.musa_aiter_hip_backend_name
    name.restype = ctypes.c_char_p
    assert name() == b"rocm-hip"


def test_noalloc_entry_rejects_caches_beyond_its_scratch_without_a_gpu():
    # The size check runs before any HIP call, so it is observable on the CPU: a deduplicating
    # scatter into more than MUSA_AITER_HIP_NOALLOC_MAX_SLOTS slots returns hipErrorInvalidValue.
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    f = lib.musa_aiter_hip_paged_tiles_noalloc
    f.argtypes = _hip._SIGNATURES["musa_aiter_hip_paged_tiles_noalloc"]
    f.restype = ctypes.c_int
    text = HEADER.read_text()
    max_slots = int(re.search(r"#define MUSA_AITER_HIP_NOALLOC_MAX_SLOTS (\d+)", text).group(1))
    assert max_slots == 1 << 21
    bs = 16
    for nb in (max_slots // bs + 1, 1 << 40):
        rc = f(1, 0, 2, 2, 2, None, None, None, None, None, 1, 10, nb, 8, 128, bs, 1024, 10240,
               None, None, 0, 0, 1, None)
        assert rc == 1, nb


def test_packed_row_copy_call_layout_matches_the_header():
    # The host layer packs musa_aiter_hip_copy_rows_call with struct; its fields, in order, must be the
    # header's (pointers and int64 as 8 bytes, the two flags as int32), 144 bytes in all.
    text = HEADER.read_text()
    body = re.search(r"typedef struct musa_aiter_hip_copy_rows_call \{(.*?)\}", text, re.S).group(1)
    fields = re.findall(r"(const uint64_t\*|const int64_t\*|const musa_aiter_hip_claims\*|int64_t|int32_t)\s+(\w+);",
                        body)
    codes = "".join("i" if kind == "int32_t" else ("q" if kind == "int64_t" else "Q") for kind, _ in fields)
    assert codes == "QQQQqQQqqqqqqqqqiiQ"
    assert _hip._COPY_ROWS_CALL.format == "<4Qq2Q9q2iQ" and _hip._COPY_ROWS_CALL.size == 144
    # Nothing to copy returns success before any HIP call, so the entry is callable without a GPU.
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    f = lib.musa_aiter_hip_copy_rows_packed
    f.argtypes = _hip._SIGNATURES["musa_aiter_hip_copy_rows_packed"]
    f.restype = ctypes.c_int
    empty = _hip._COPY_ROWS_CALL.pack(0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0, 16, 16, 16, 1, 1, 0)
    assert f(empty, None) == 0
    assert f(None, None) != 0
