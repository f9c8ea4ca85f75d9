"""The C ABI: the built library loads and exports every function include/od_mi355x.h declares, the ctypes table in
opendecider_amd/_lib.py matches the header's parameter lists, and the two host-only entry points answer (no GPU
call is made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "od_mi355x.h")


def declarations():
    """name -> number of parameters, for every function prototype in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(od_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def library():
    from opendecider_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from opendecider_amd.build import build
        build()
    return _lib


def test_header_lists_the_entry_points():
    decl = declarations()
    for name in ("od_act_quant", "od_w8a8_gemm", "od_kv_quant_append", "od_branched_attn", "od_wide_attn",
                 "od_strerror", "od_abi_version"):
        assert name in decl, name


def test_ctypes_table_matches_header(library):
    decl = declarations()
    assert set(decl) == set(library.SIGNATURES), (set(decl) ^ set(library.SIGNATURES))
    for name, n in decl.items():
        assert len(library.SIGNATURES[name]) == n, (name, n, len(library.SIGNATURES[name]))


def test_library_exports_every_declared_symbol(library):
    raw = ctypes.CDLL(library.LIB_PATH)
    for name in declarations():
        assert hasattr(raw, name), f"{name} is declared but not exported"


def test_host_only_entry_points(library):
    L = library.lib()
    assert L.od_abi_version() == library.ABI_VERSION
    assert L.od_strerror(0) == b"ok" or b"ok" in L.od_strerror(0).lower()
    for code in (-1, -2, -3, -4, -5):
        assert isinstance(L.od_strerror(code), bytes) and L.od_strerror(code)


def test_bench_work_counters_take_the_abi_arguments():
    """bench.py's timers replace entry points on the loaded library and count each call's work from the raw ABI
    arguments, so every work function must accept exactly that entry point's argument list."""
    import sys
    sys.path.insert(0, ROOT)
    import bench
    from opendecider_amd import _lib
    for name, fn in [("od_w8a8_gemm", bench.gemm_work), ("od_w8a8_gemm_swiglu", bench.swiglu_work),
                     ("od_branched_attn", bench.attn_work), ("od_branched_attn_split", bench.attn_work),
                     ("od_branched_attn_staged", bench.staged_work), ("od_attn_stage", bench.stage_work),
                     ("od_wide_attn", bench.wide_work), ("od_kv_quant_append", bench.append_work),
                     ("od_qk_norm_rope_kv_append", bench.rope_append_work)]:
        n = len(_lib.SIGNATURES[name])
        work = fn(*([1] * n))
        assert len(work) == 2 and all(isinstance(w, (int, float)) for w in work), name
