"""ctypes binding of libpsquant.so (the gfx950 HIP kernels behind the C ABI in include/psquant.h).

The library is built in-tree by ``build_lib.py`` into ``lib/libpsquant.so``.  There is no
fallback implementation: if the library is missing, ``lib()`` raises :class:`NativeLibraryError`
(an ``ImportError``, deliberately *not* one of the exception types QuantLinear's native branch
turns into a warn-and-dequantize fallback), so a broken install fails loudly.

The reference loads its own native helper the same way -- a runtime-built ``.so`` with
``extern "C"`` entry points (powershard/ats_memory.py:80-91, ats_allocator.cpp:14-52).
"""
import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("PSQUANT_LIB", Path(__file__).resolve().parent / "lib" / "libpsquant.so"))
ABI_VERSION = 1

BF16, F16, F32 = 0, 1, 2
W_UINT4, W_INT8 = 0, 1   # enum psq_weight_kind

# Every exported entry point: name -> (restype, argtypes).  Mirrors include/psquant.h.
_P, _I64, _I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "psq_abi_version": (_I, []),
    "psq_last_error": (ctypes.c_char_p, []),
    "psq_device_supported": (_I, [_I]),
    "psq_quantize_rows_i8": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _P, _I64, _P, _P]),
    "psq_quantize_rows_fp8": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _P, _I64, _P, _P]),
    "psq_rotate_rows": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _I, _I64, _P]),
    "psq_gemm_i8": (_I, [_P, _I64, _P, _P, _I64, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_i8_act": (_I, [_P, _I64, _P, _P, _I64, _P, _P, _I, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_i8_i32": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_i8_8wave": (_I, [_P, _I64, _P, _P, _I64, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_fp8": (_I, [_P, _I64, _P, _P, _I64, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_fp8_e5m2w": (_I, [_P, _I64, _P, _P, _I64, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_fp8_act": (_I, [_P, _I64, _P, _P, _I64, _P, _I, _P, _I, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_w4a16": (_I, [_P, _I, _I64, _P, _P, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_w8a16": (_I, [_P, _I, _I64, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_gemm_wonly_workspace_bytes": (_I64, [_I, _I64, _I64, _I64, _I64, _I]),
    "psq_gemm_w4a16_ws": (_I, [_P, _I, _I64, _P, _P, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "psq_gemm_w8a16_ws": (_I, [_P, _I, _I64, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "psq_gemm_w4a16_noalloc": (_I, [_P, _I, _I64, _P, _P, _P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _P]),
    "psq_dequant_uint4": (_I, [_P, _P, _P, _I, _I64, _I64, _P, _I, _P]),
    "psq_dequant_i8_rows": (_I, [_P, _P, _I64, _I64, _I, _P, _I, _P]),
    "psq_dequant_fp8": (_I, [_P, _P, _I, _I64, _I64, _P, _I, _P]),
    "psq_dequant_e5m2": (_I, [_P, _P, _I, _I64, _I64, _P, _I, _P]),
    "psq_flag_nonfinite": (_I, [_P, _I, _I64, _P, ctypes.c_uint64, _P]),
}


class NativeLibraryError(ImportError):
    """libpsquant.so is missing or unusable: the native path cannot run."""


_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library (loaded once, thread-safe).  Raises NativeLibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or comfyui-powershard_amd/powershard_amd/build_lib.py")
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as error:
                raise NativeLibraryError(f"cannot load {LIB_PATH}: {error}") from error
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
            if handle.psq_abi_version() != ABI_VERSION:
                raise NativeLibraryError(f"{LIB_PATH}: ABI {handle.psq_abi_version()} != {ABI_VERSION}")
            _lib = handle
    return _lib


def available():
    try:
        lib()
        return True
    except NativeLibraryError:
        return False


def last_error():
    return lib().psq_last_error().decode("utf-8", "replace")


def check(status, what):
    """Turn a non-zero status into RuntimeError (the type QuantLinear's fallback handles)."""
    if status != 0:
        raise RuntimeError(f"psquant {what} failed ({status}): {last_error()}")
