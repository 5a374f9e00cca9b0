"""The C ABI on the CPU: libpsquant.so loads, exports every entry point include/psquant.h declares,
and rejects bad arguments before touching a device (no kernel is launched here)."""
import ctypes
import os
import re

import pytest

from powershard_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "psquant.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^PSQ_API\s+[\w\s\*]+?\b(psq_\w+)\(", text, flags=re.M)))


def test_header_declares_the_binding_table():
    assert declared() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    missing = [name for name in declared() if not hasattr(lib, name)]
    assert not missing, missing


def test_abi_version_and_empty_error():
    lib = _native.lib()
    assert lib.psq_abi_version() == _native.ABI_VERSION == 1
    assert isinstance(lib.psq_last_error(), bytes)


def _fake(addr=0x10000):
    return ctypes.c_void_p(addr)


@pytest.mark.parametrize("call,code", [
    # null operands
    (lambda L: L.psq_gemm_i8(None, 128, _fake(), _fake(), 128, _fake(), None, 0, _fake(), 0, 16, 16, 16, 128, None), -1),
    # K not a multiple of 128
    (lambda L: L.psq_gemm_i8(_fake(), 96, _fake(), _fake(), 96, _fake(), None, 0, _fake(), 0, 16, 16, 16, 96, None), -2),
    # the 8-wave comparison schedule: whole 256-column tiles and an even stage count only
    (lambda L: L.psq_gemm_i8_8wave(_fake(), 256, _fake(), _fake(), 256, _fake(), None, 0, _fake(), 0, 128, 16, 128, 256,
                                   None), -2),
    (lambda L: L.psq_gemm_i8_8wave(_fake(), 384, _fake(), _fake(), 384, _fake(), None, 0, _fake(), 0, 256, 16, 256, 384,
                                   None), -2),
    # misaligned operand
    (lambda L: L.psq_gemm_i8_i32(_fake(0x10008), 128, _fake(), 128, _fake(), 16, 16, 16, 128, None), -2),
    # bad output dtype
    (lambda L: L.psq_gemm_fp8(_fake(), 128, _fake(), _fake(), 128, _fake(), 0, None, 0, _fake(), 7, 16, 16, 16, 128, None), -1),
    # rotation group not a power of 4
    (lambda L: L.psq_quantize_rows_i8(_fake(), 0, 4, 512, 512, 128, None, _fake(), 512, _fake(), None), -2),
    # K beyond the per-row kernel
    (lambda L: L.psq_quantize_rows_i8(_fake(), 0, 4, 32784, 32784, 0, None, _fake(), 32784, _fake(), None), -2),
    # fp32 activations are not accepted by the quantizer
    (lambda L: L.psq_quantize_rows_fp8(_fake(), 2, 4, 512, 512, 0, None, _fake(), 512, _fake(), None), -1),
    # uint4 group size must be a multiple of 64 for the GEMM
    (lambda L: L.psq_gemm_w4a16(_fake(), 0, 512, _fake(), _fake(), _fake(), 32, None, 0, _fake(), 0, 16, 8, 16, 512,
                                None), -2),
    # negative sizes
    (lambda L: L.psq_dequant_uint4(_fake(), _fake(), _fake(), 128, -1, 512, _fake(), 0, None), -1),
    (lambda L: L.psq_dequant_i8_rows(_fake(), _fake(), 4, 512, 8, _fake(), 0, None), -2),
    # non-finite flag: tickets start at 1; the flag is an aligned 8-byte word
    (lambda L: L.psq_flag_nonfinite(_fake(), 1, 16, _fake(), 0, None), -1),
    (lambda L: L.psq_flag_nonfinite(_fake(), 1, 16, _fake(0x10004), 1, None), -1),
])
def test_argument_errors_are_reported_without_a_device(call, code):
    lib = _native.lib()
    assert call(lib) == code
    assert lib.psq_last_error().decode()


def test_empty_problems_are_no_ops():
    lib = _native.lib()
    assert lib.psq_gemm_i8(_fake(), 128, _fake(), _fake(), 128, _fake(), None, 0, _fake(), 0, 16, 0, 16, 128, None) == 0
    assert lib.psq_quantize_rows_i8(_fake(), 0, 0, 512, 512, 256, None, _fake(), 512, _fake(), None) == 0
    # empty tensors come with null data pointers (torch.empty((0, K)).data_ptr() == 0)
    assert lib.psq_gemm_i8(None, 128, None, _fake(), 128, _fake(), None, 0, None, 0, 16, 0, 16, 128, None) == 0
    assert lib.psq_gemm_i8_act(None, 128, None, _fake(), 128, _fake(), None, 0, 2, None, 0, 64, 0, 128, 128, None) == 0
    assert lib.psq_gemm_fp8(None, 128, None, _fake(), 128, _fake(), 0, None, 0, None, 0, 16, 0, 16, 128, None) == 0
    assert lib.psq_gemm_w4a16(None, 0, 128, _fake(), _fake(), _fake(), 128, None, 0, None, 0, 16, 0, 16, 128, None) == 0
    assert lib.psq_gemm_w8a16(None, 0, 128, _fake(), _fake(), None, 0, None, 0, 16, 0, 16, 128, None) == 0
    assert lib.psq_quantize_rows_i8(None, 0, 0, 512, 512, 256, None, None, 512, None, None) == 0
    assert lib.psq_rotate_rows(None, 0, 0, 512, 512, 256, None, 0, 512, None) == 0
    assert lib.psq_flag_nonfinite(None, 1, 0, _fake(), 1, None) == 0
    # a non-empty problem with a null operand is still an error
    assert lib.psq_gemm_i8(None, 128, _fake(), _fake(), 128, _fake(), None, 0, _fake(), 0, 16, 4, 16, 128, None) == -1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(_native.NativeLibraryError):
        _native.lib()
    assert not _native.available()
    # NativeLibraryError is an ImportError: QuantLinear's warn-and-dequantize fallback does not catch it
    assert not issubclass(_native.NativeLibraryError, (RuntimeError, ValueError, TypeError, NotImplementedError))
