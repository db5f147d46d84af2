"""C ABI prototype guard (CPU only).

tests/golden/abi_signatures.json holds the expected prototype (return type and
parameter types, in order) of every exported entry point, each citing the
reference header line it must equal (cklxx/kernel-set include/kernel_set/*.h)
or marked as an extension of this build. The table is written by
tests/golden/make_abi_table.py from the reference headers, the pattern of the
reference's bindings/verify/xcheck_signatures.py and scripts/check_abi.py.

Any edit to a prototype in include/kernel_set/*.h (a parameter added, removed,
reordered, or its type changed) fails test_headers_match_table, and the
ctypes declarations of the Python binding must describe the same C types.
"""
import ctypes
import json
import os
import shutil

import pytest

from kernel_set import _lib
from tests.abi_parse import prototypes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include", "kernel_set")
TABLE = os.path.join(ROOT, "tests", "golden", "abi_signatures.json")


def load_table():
    with open(TABLE) as f:
        return json.load(f)


def diff(expected, actual):
    """Human-readable mismatches between two prototype maps."""
    out = []
    for name in sorted(set(expected) | set(actual)):
        if name not in actual:
            out.append(f"{name}: missing from the headers")
        elif name not in expected:
            out.append(f"{name}: not in the expected table")
        else:
            e, a = expected[name], actual[name]
            if (e["ret"], e["params"]) != (a["ret"], a["params"]):
                out.append(f"{name}: expected {e['ret']}({', '.join(e['params'])}) "
                           f"[{e.get('ref')}], header has {a['ret']}({', '.join(a['params'])})")
    return out


def test_table_covers_the_reference_scope():
    table = load_table()
    ref = {n for n, e in table.items() if e["ref"] != "extension"}
    assert len(ref) == 34
    for name in ("ks_gemm_w4a16", "ks_gemm_w8a8", "ks_gemm_fp8", "ks_gemm_fp8_blockwise",
                 "ks_quantize_fp8", "ks_quantize_fp8_group", "ks_quantize_int8",
                 "ks_dequantize_int4", "ks_repack_int4", "ks_moe_compute_permutation",
                 "ks_moe_grouped_gemm"):
        assert name in ref and table[name]["ref"].startswith("include/kernel_set/")
    assert table["ks_gemm_w4a16"]["params"] == [
        "void*", "const void*", "const void*", "const void*", "const void*", "const void*",
        "int64_t", "int64_t", "int64_t", "int", "ks_dtype_t", "ks_stream_t"]


def test_headers_match_table():
    problems = diff(load_table(), prototypes(INC))
    assert not problems, "\n".join(problems)


@pytest.mark.parametrize("edit", [
    ("gemm.h", "int64_t k, int group_size, ks_dtype_t dtype,", "int64_t k, int64_t group_size, ks_dtype_t dtype,"),
    ("gemm.h", "int64_t k, int group_size, ks_dtype_t dtype,", "int64_t k, ks_dtype_t dtype,"),
    ("quant.h", "ks_quantize_fp8_group(", "ks_quantize_fp8_group2("),
])
def test_a_prototype_edit_is_detected(tmp_path, edit):
    """The guard itself: a copy of the headers with one prototype edited no
    longer matches the table."""
    fn, old, new = edit
    inc = tmp_path / "kernel_set"
    shutil.copytree(INC, inc)
    src = (inc / fn).read_text()
    assert old in src
    (inc / fn).write_text(src.replace(old, new, 1))
    assert diff(load_table(), prototypes(str(inc)))


_C_TO_CTYPES = {
    "void*": ctypes.c_void_p, "const void*": ctypes.c_void_p, "ks_stream_t": ctypes.c_void_p,
    "int64_t": ctypes.c_int64, "uint32_t": ctypes.c_uint32, "int": ctypes.c_int, "ks_dtype_t": ctypes.c_int,
    "ks_quant_mode_t": ctypes.c_int, "ks_memcpy_kind_t": ctypes.c_int,
    "ks_status_t": ctypes.c_int, "size_t": ctypes.c_size_t, "float": ctypes.c_float,
    "const char*": ctypes.c_char_p,
    "float*": ctypes.POINTER(ctypes.c_float), "const float*": ctypes.POINTER(ctypes.c_float),
    "int32_t*": ctypes.POINTER(ctypes.c_int32), "const int32_t*": ctypes.POINTER(ctypes.c_int32),
    "int*": ctypes.POINTER(ctypes.c_int), "void**": ctypes.POINTER(ctypes.c_void_p),
    "ks_stream_t*": ctypes.POINTER(ctypes.c_void_p),
    "ks_device_properties_t*": ctypes.POINTER(_lib.ks_device_properties_t),
}


def test_ctypes_declarations_match_the_c_types():
    """Every entry point's ctypes argtypes / restype in kernel_set._lib carry
    the widths of its C prototype (a 64-bit size passed as c_int, or a
    missing argument, would corrupt the call)."""
    problems = []
    for name, e in load_table().items():
        fn = getattr(_lib.lib, name)
        want = [_C_TO_CTYPES[t] for t in e["params"]]
        got = list(fn.argtypes or [])
        if [str(t) for t in got] != [str(t) for t in want]:
            problems.append(f"{name}: argtypes {got} != {want}")
        if str(fn.restype) != str(_C_TO_CTYPES[e["ret"]]):
            problems.append(f"{name}: restype {fn.restype} != {_C_TO_CTYPES[e['ret']]}")
    assert not problems, "\n".join(problems)
