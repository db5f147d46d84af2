"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol the headers declare, keeps the frozen enum values, and validates
arguments (NULL pointers, shapes, dtypes, modes) before touching the device,
with the reference's status codes and message conventions
(kernels/src/common/dispatch.cuh:23-50, each entry point's validation block).
"""
import ctypes
import os
import re

import pytest

import kernel_set as ks
from kernel_set import _lib
from kernel_set.enums import DType, QuantMode, Status

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include", "kernel_set")


def declared_symbols():
    names = set()
    for f in os.listdir(INC):
        if f.endswith(".h"):
            src = open(os.path.join(INC, f)).read()
            names |= set(re.findall(r"KS_API\s+[\w\s\*]+?\b(ks_\w+)\s*\(", src))
    return names


def exported_symbols():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.library_path()],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_exports_every_declared_symbol():
    decl = declared_symbols()
    assert len(decl) >= 28
    missing = decl - exported_symbols()
    assert not missing, missing
    assert not _lib._MISSING, _lib._MISSING


def test_exports_nothing_undeclared():
    extra = {s for s in exported_symbols() if s.startswith("ks_")} - declared_symbols()
    assert not extra, extra


def test_enum_values_match_header():
    src = open(os.path.join(INC, "types.h")).read()
    for enum, py in (("ks_status_t", Status), ("ks_dtype_t", DType),
                     ("ks_quant_mode_t", QuantMode)):
        body = re.search(r"typedef enum %s \{(.*?)\}" % enum, src, re.S).group(1)
        pairs = dict(re.findall(r"(KS_\w+)\s*=\s*(\d+)", body))
        assert len(pairs) == len(py)
        for member in py:
            key = [k for k in pairs if k.endswith("_" + member.name)]
            assert key and int(pairs[key[0]]) == member.value, member


def test_runtime_introspection():
    L = _lib.lib
    assert L.ks_backend_name() == b"hip"
    assert L.ks_version() == b"0.2.1"
    assert L.ks_status_string(0) == b"KS_SUCCESS"
    assert L.ks_status_string(4) == b"KS_ERROR_CUDA"
    assert L.ks_status_string(99) == b"KS_ERROR_UNKNOWN"
    assert [L.ks_dtype_size_bits(d) for d in range(11)] == [32, 16, 16, 8, 8, 64, 64, 32, 8, 8, 4]
    assert L.ks_dtype_name(DType.BF16) == b"bf16" and L.ks_dtype_name(99) == b"unknown"
    assert ctypes.sizeof(_lib.ks_device_properties_t) == 256 + 6 * 4 + 8 + 3 * 4 + 4  # trailing pad to 8


def _status(fn, *args):
    return fn(*args)


P = 16  # a non-null dummy address; validation fails before any dereference


def test_w4a16_validation():
    f = _lib.lib.ks_gemm_w4a16
    st = f(None, P, P, P, None, None, 1, 1, 2, 2, DType.BF16, None)
    assert st == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: c"
    assert f(P, P, P, None, None, None, 1, 1, 2, 2, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: scales"
    assert f(P, P, P, P, None, None, 0, 1, 2, 2, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, P, None, None, 1, 1, 3, 3, DType.BF16, None) == Status.ERROR_UNSUPPORTED_SHAPE
    assert f(P, P, P, P, None, None, 1, 1, 8, 3, DType.BF16, None) == Status.ERROR_UNSUPPORTED_SHAPE
    assert f(P, P, P, P, None, None, 1, 1, 8, 4, DType.F32, None) == Status.ERROR_UNSUPPORTED_DTYPE


def test_w8a8_validation():
    f = _lib.lib.ks_gemm_w8a8
    fp = ctypes.cast(P, _lib._F32P)
    assert f(P, P, P, None, fp, None, 1, 1, 1, 1, 2, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: a_scale"
    assert f(P, P, P, fp, fp, None, 1, 1, 1, QuantMode.PER_CHANNEL, 2, DType.BF16, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, fp, None, 1, 1, 1, 1, QuantMode.PER_TOKEN, DType.BF16, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, fp, None, 1, 1, 1, 1, 2, DType.I8, None) == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, fp, None, 1, -1, 1, 1, 2, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT


def test_fp8_gemm_validation():
    # gemm_fp8.cu:230-275 order: NULL pointers, shape, overflow, modes, dtypes
    f = _lib.lib.ks_gemm_fp8
    fp = ctypes.cast(P, _lib._F32P)
    ok = (QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL, DType.F8E4M3, DType.BF16, None)
    assert f(P, P, P, fp, None, 1, 1, 1, *ok) == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: b_scale"
    assert f(P, P, P, fp, fp, 0, 1, 1, *ok) == Status.ERROR_INVALID_ARGUMENT
    big = 1 << 40
    assert f(P, P, P, fp, fp, big, big, 8, *ok) == Status.ERROR_UNSUPPORTED_SHAPE
    assert f(P, P, P, fp, fp, 1, 1, 1, QuantMode.PER_CHANNEL, QuantMode.PER_CHANNEL,
             DType.F8E4M3, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, fp, 1, 1, 1, QuantMode.PER_TOKEN, QuantMode.PER_TOKEN,
             DType.F8E4M3, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, fp, 1, 1, 1, QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL,
             DType.I8, DType.BF16, None) == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, fp, 1, 1, 1, QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL,
             DType.F8E5M2, DType.I8, None) == Status.ERROR_UNSUPPORTED_DTYPE


def test_fp8_blockwise_fused_quant_validation():
    # extension entry point: pointers, shape, blocks, then the three dtypes
    f = _lib.lib.ks_gemm_fp8_blockwise_fused_quant
    fp = ctypes.cast(P, _lib._F32P)
    ok = (DType.BF16, DType.F8E4M3, DType.BF16, None)
    assert f(P, P, P, None, 1, 1, 1, 128, 128, *ok) == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: b_scale"
    assert f(P, P, P, fp, 1, 0, 1, 128, 128, *ok) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, 1, 1, 1, 128, 0, *ok) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, 1, 1, 1, 128, 128, DType.I8, DType.F8E4M3, DType.BF16, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, 1, 1, 1, 128, 128, DType.BF16, DType.BF16, DType.BF16, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, 1, 1, 1, 128, 128, DType.BF16, DType.F8E5M2, DType.I8, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    big = 1 << 40
    assert f(P, P, P, fp, big, big, 8, 128, 128, *ok) == Status.ERROR_UNSUPPORTED_SHAPE


def test_w8a8_fused_quant_validation():
    # extension entry point: pointers, shape, modes, dtypes, then the K limit
    f = _lib.lib.ks_gemm_w8a8_fused_quant
    fp = ctypes.cast(P, _lib._F32P)
    modes = (QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL)
    ok = (DType.BF16, DType.BF16, None)
    assert f(P, P, P, None, None, 1, 1, 1, *modes, *ok) == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: b_scale"
    assert f(P, P, P, fp, None, 1, 0, 1, *modes, *ok) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, None, 1, 1, 1, QuantMode.PER_CHANNEL, QuantMode.PER_CHANNEL, *ok) \
        == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, None, 1, 1, 1, QuantMode.PER_TOKEN, QuantMode.PER_TOKEN, *ok) \
        == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, None, 1, 1, 1, *modes, DType.I8, DType.BF16, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, None, 1, 1, 1, *modes, DType.BF16, DType.I8, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, None, 1, 16, 300000, *modes, *ok) == Status.ERROR_UNSUPPORTED_SHAPE
    big = 1 << 40
    assert f(P, P, P, fp, None, big, big, 8, *modes, *ok) == Status.ERROR_UNSUPPORTED_SHAPE


def test_fp8_blockwise_validation():
    f = _lib.lib.ks_gemm_fp8_blockwise
    fp = ctypes.cast(P, _lib._F32P)
    assert f(P, P, None, fp, fp, 1, 1, 1, 128, 128, DType.F8E4M3, DType.BF16, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: b_fp8"
    assert f(P, P, P, fp, fp, 1, 1, 1, 0, 128, DType.F8E4M3, DType.BF16, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, fp, fp, 1, 1, 1, 128, 128, DType.BF16, DType.BF16, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, fp, fp, 1, 1, 1, 128, 128, DType.F8E4M3, DType.I8, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    big = 1 << 40
    assert f(P, P, P, fp, fp, big, big, 8, 128, 128, DType.F8E4M3, DType.BF16, None) \
        == Status.ERROR_UNSUPPORTED_SHAPE


def test_quant_validation():
    L = _lib.lib
    fp = ctypes.cast(P, _lib._F32P)
    assert L.ks_quantize_fp8(P, fp, P, 1, 1, DType.BF16, DType.F8E4M3, QuantMode.PER_CHANNEL, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert L.ks_quantize_fp8(P, fp, P, 1, 1, DType.BF16, DType.I8, 1, None) \
        == Status.ERROR_UNSUPPORTED_DTYPE
    assert L.ks_quantize_fp8(P, fp, P, 1, 0, DType.BF16, DType.F8E4M3, 1, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert L.ks_quantize_fp8_group(P, fp, P, 1, 8, 0, DType.BF16, DType.F8E4M3, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert L.ks_quantize_fp8_group(P, None, P, 1, 8, 8, DType.BF16, DType.F8E4M3, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: scale"
    assert L.ks_quantize_int8(P, fp, P, 1, 1, DType.BF16, QuantMode.GROUPWISE, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert L.ks_repack_int4(P, P, None, 16, 4, 8, None) == Status.ERROR_INVALID_ARGUMENT
    assert L.ks_repack_int4(P, P, None, 12, 4, 4, None) == Status.ERROR_UNSUPPORTED_SHAPE
    assert L.ks_dequantize_int4(P, P, P, None, 16, 4, 8, DType.BF16, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert L.ks_dequantize_int4(P, P, P, P, 16, 4, 5, DType.BF16, None) \
        == Status.ERROR_UNSUPPORTED_SHAPE


def test_moe_validation():
    f = _lib.lib.ks_moe_grouped_gemm_w4a16
    ip = ctypes.cast(P, _lib._I32P)
    assert f(P, P, P, P, None, None, 4, 8, 16, 32, 32, DType.BF16, None) \
        == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: expert_offsets"
    assert f(P, P, P, P, None, ip, 0, 8, 16, 32, 32, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert f(P, P, P, P, None, ip, 4, 8, 16, 31, 31, DType.BF16, None) == Status.ERROR_UNSUPPORTED_SHAPE
    assert f(P, P, P, P, None, ip, 4, 8, 16, 32, 32, DType.F32, None) == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, P, None, ip, 4, 0, 16, 32, 32, DType.BF16, None) == Status.SUCCESS


def test_dense_grouped_gemm_validation():
    # moe_grouped_gemm.cu:140-152: NULL pointers and bad shapes are
    # INVALID_ARGUMENT, dtypes outside f32/f16/bf16/fp8 UNSUPPORTED_DTYPE, and
    # total_rows == 0 returns before any launch.
    f = _lib.lib.ks_moe_grouped_gemm
    ip = ctypes.cast(P, _lib._I32P)
    assert f(P, P, P, None, 4, 8, 16, 32, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    assert ks.last_error_string() == "null arg: expert_offsets"
    assert f(None, P, P, ip, 4, 8, 16, 32, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
    for bad in ((0, 8, 16, 32), (4, -1, 16, 32), (4, 8, 0, 32), (4, 8, 16, 0)):
        assert f(P, P, P, ip, *bad, DType.BF16, None) == Status.ERROR_INVALID_ARGUMENT
        assert ks.last_error_string() == "ks_moe_grouped_gemm: bad shape"
    assert f(P, P, P, ip, 4, 8, 16, 32, DType.I8, None) == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, ip, 4, 8, 16, 32, DType.F64, None) == Status.ERROR_UNSUPPORTED_DTYPE
    assert f(P, P, P, ip, 4, 0, 16, 32, DType.F8E5M2, None) == Status.SUCCESS


def test_python_wrappers_raise_kernel_set_error():
    with pytest.raises(ks.KernelSetError) as ei:
        ks.gemm.gemm_w4a16(0, P, P, P, None, 1, 8, 8, 8, dtype=DType.BF16)
    assert ei.value.status == Status.ERROR_INVALID_ARGUMENT
    assert "null arg: c" in str(ei.value)


def test_dispatch_introspection():
    d = ks.dispatch
    assert set(d.ops()) == {"w4a16", "int8_gemm", "fp8_gemm", "fp8_gemm_blockwise",
                            "per_token_group_quant", "moe"}
    for op in d.ops():
        assert d.which(op) == "kernel-set" and d.chain(op) == ["kernel-set"]
    assert d.providers() == ["kernel-set"]
