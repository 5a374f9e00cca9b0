"""CPU oracle for the quantized linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only to check or time results, never to produce them.  The product
(``comfyui-powershard_amd/powershard_amd``) never imports it and has no CPU fallback through it.

Two layers:

* ``psq_oracle.c`` (built by ``oracle/Makefile`` into ``oracle/_build/libpsq_oracle.so``): the
  bit-exact restatement of the hot path -- ConvRot fast transform, per-token int8 / fp8
  quantization, int32 GEMM, fused dequant epilogue, uint4 group dequantization, and the scalar
  formats (bf16, fp16, OCP e4m3fn).  Each convention is written at the top of that file.
* this module: ctypes wrappers taking torch CPU tensors, plus numpy/torch restatements of the
  reference's load-time formulas:

  - ``regular_hadamard_kron``  -- powershard/operations.py:72-81 (Kronecker powers of H4)
  - ``dequantize_rows``        -- powershard/operations.py:84-93 (q * s, then ConvRot inverse)
  - ``quantize_weight_int8``   -- tests/test_fp16_safe.py:171-174 (rotate, rowmax/127, round)
  - ``quantize_weight_fp8``    -- scripts/probe_wan_cuda.py:120-125 (absmax/448, cast)
  - ``quantize_weight_uint4``  -- asymmetric group-wise uint4 (the int4 weight convention)
  - ``dequant_then_linear``    -- powershard/quant_linear.py:219-220 (the reference CPU path)

Pinning status of every function is listed in ``PINNING`` below; the tests in
``tests/test_oracle_*.py`` are the pins.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libpsq_oracle.so"

BF16, F16, F32 = 0, 1, 2
_DT = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}

# function -> what pins it (the tests named are in tests/test_oracle_pinning.py)
PINNING = {
    "regular_hadamard": "closed form == Kronecker construction of operations.py:72-81; H @ H.T == I exactly; "
                        "not Sylvester (test_hadamard_*)",
    "rotate_rows": "== dense x @ H in float64 within fp32 rounding; exact on small integers; unit vectors give "
                   "the rows of H (test_rotation_*)",
    "quantize_rows_i8": "known-answer rows (integer multiples of 2^-e), ties to even, rotated unit vector, zero "
                        "row and range invariants, static-scale saturation, NaN-row convention "
                        "(test_quantize_known_rows_without_rotation, test_quantize_ties_round_to_even, "
                        "test_quantize_rotated_unit_vector, test_quantize_zero_row_and_invariants, "
                        "test_quantize_static_scale_saturates, test_quantize_nan_row_convention)",
    "quantize_rows_fp8": "known-answer rows (e4m3 values x 2^-e, absmax element at +-448: codes and scale 2^-e "
                         "exact), ties to even (normal and subnormal), static-scale saturation, zero row, torch "
                         "restatement with torch's own e4m3fn cast (plain and rotated), NaN-row convention "
                         "(test_quantize_fp8_*, test_quantize_nan_row_convention)",
    "gemm_i8_i32": "== numpy int64 matmul, also on selected rows; no overflow at the extremes",
    "epilogue_i32": "within 1 output ulp of float64 acc*a_s*w_s + bias; bf16 output == RNE of the fp32 value",
    "gemm_fp8": "== float64 matmul of torch-decoded e4m3 operands; with e5m2 weights, of torch-decoded "
                "e4m3 activations and e5m2 weights (test_gemm_fp8_e5m2_weights_match_float64_matmul)",
    "e5m2_to_f32 / dequant_fp8(e5m2)": "exhaustive over the 256 codes == torch's float8_e5m2 decode (NaN and inf "
                                       "positions included); x scale then torch's cast "
                                       "(test_e5m2_decode_exhaustive, test_dequant_e5m2_matches_torch_decode)",
    "dequant_fp8": "== torch's float8_e4m3fn decode x scale, then torch's cast (per tensor and per row; "
                   "test_dequant_fp8_matches_torch_decode)",
    "dequant_uint4": "== the nibble/zero/scale formula on torch tensors; quantize error <= s/2",
    "dequant_i8_rows": "== dequantize_rows' dense formula (operations.py:84-93) on the test_convrot recipe",
    "quantize_weight_int8": "round trip through dequantize_rows within half a step per row",
    "gemm_wonly": "== float64 matmul of the dequantized weight",
    "bf16/f16/e4m3 codecs": "exhaustive or dense random vs torch/numpy casts (RNE)",
}


def build():
    """Compile the oracle C library (gcc) into oracle/_build."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.psq_or_regular_hadamard.argtypes = [I, P]
        L.psq_or_rotate_rows.argtypes = [P, I, I64, I64, I64, I, P]
        L.psq_or_quantize_rows_i8.argtypes = [P, I, I64, I64, I64, I, P, P, I64, P]
        L.psq_or_quantize_rows_fp8.argtypes = [P, I, I64, I64, I64, I, P, P, I64, P]
        L.psq_or_gemm_i8_i32.argtypes = [P, I64, P, I64, P, I64, I64, I64, I64, P]
        L.psq_or_epilogue_i32.argtypes = [P, I64, P, P, I, P, I, P, I, I64, I64, I64, P]
        L.psq_or_gemm_fp8.argtypes = [P, I64, P, P, I64, P, I, P, I, P, I, I64, I64, I64, I64, P]
        L.psq_or_gemm_fp8_e5m2w.argtypes = [P, I64, P, P, I64, P, I, P, I, P, I, I64, I64, I64, I64, P]
        L.psq_or_dequant_uint4.argtypes = [P, P, P, I64, I64, I, P, I]
        L.psq_or_dequant_i8_rows.argtypes = [P, P, I64, I64, I, P, I]
        L.psq_or_dequant_fp8.argtypes = [P, P, I, I64, I64, P, I]
        L.psq_or_dequant_e5m2.argtypes = [P, P, I, I64, I64, P, I]
        L.psq_or_gemm_wonly.argtypes = [P, I, I64, P, I, P, P, I, P, I, I64, I64, I64, I64, P]
        L.psq_or_bf16_round.argtypes = [ctypes.c_float]
        L.psq_or_bf16_round.restype = ctypes.c_float
        L.psq_or_f32_to_e4m3.argtypes = [ctypes.c_float]
        L.psq_or_f32_to_e4m3.restype = ctypes.c_uint8
        L.psq_or_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.psq_or_e4m3_to_f32.restype = ctypes.c_float
        L.psq_or_e5m2_to_f32.argtypes = [ctypes.c_uint8]
        L.psq_or_e5m2_to_f32.restype = ctypes.c_float
        L.psq_or_f32_to_f16.argtypes = [ctypes.c_float]
        L.psq_or_f32_to_f16.restype = ctypes.c_uint16
        L.psq_or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.psq_or_f32_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _cpu(t):
    return t.detach().to("cpu").contiguous()


def _rows(row_ids):
    if row_ids is None:
        return None
    return torch.as_tensor(row_ids, dtype=torch.int64).contiguous()


# ----------------------------------------------------------------------- ConvRot
def regular_hadamard(g):
    """Closed form H[i][j] = g^-1/2 (-1)^{#d: i_d + j_d = 3} (fp32 [g, g])."""
    h = torch.empty(g, g, dtype=torch.float32)
    if lib().psq_or_regular_hadamard(g, _ptr(h)) != 0:
        raise ValueError("ConvRot group size must be a power of 4 >= 4")
    return h


def regular_hadamard_kron(g):
    """Kronecker construction, as powershard/operations.py:72-81 builds it (independent path)."""
    if g < 4 or g & (g - 1) or (g.bit_length() - 1) % 2:
        raise ValueError("ConvRot group size must be a power of 4 >= 4")
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = h4
    while h.shape[0] < g:
        h = np.kron(h, h4)
    return h / np.sqrt(g)


def rotate_rows(x, g):
    """fp32 [M, K]: x (bf16/fp16/fp32) rotated per group of g with the fixed-order fast transform."""
    x = _cpu(x)
    M, K = x.shape
    out = torch.empty(M, K, dtype=torch.float32)
    if lib().psq_or_rotate_rows(_ptr(x), _DT[x.dtype], M, K, K, g or 0, _ptr(out)) != 0:
        raise ValueError("bad ConvRot group")
    return out


# ------------------------------------------------------------------ quantization
def quantize_rows_i8(x, g=0, static_scale=None):
    """Per-row (token) int8 quantization of x (optionally ConvRot-rotated): (q int8 [M,K], s fp32 [M])."""
    x = _cpu(x)
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.int8)
    s = torch.empty(M, dtype=torch.float32)
    st = None if static_scale is None else torch.tensor([float(static_scale)], dtype=torch.float32)
    rc = lib().psq_or_quantize_rows_i8(_ptr(x), _DT[x.dtype], M, K, K, g or 0, _ptr(st), _ptr(q), K, _ptr(s))
    if rc != 0:
        raise ValueError(f"oracle quantize_rows_i8 failed ({rc})")
    return q, s


def quantize_rows_fp8(x, g=0, static_scale=None):
    """Per-row fp8 e4m3fn quantization: (q uint8 codes [M,K], s fp32 [M])."""
    x = _cpu(x)
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.uint8)
    s = torch.empty(M, dtype=torch.float32)
    st = None if static_scale is None else torch.tensor([float(static_scale)], dtype=torch.float32)
    rc = lib().psq_or_quantize_rows_fp8(_ptr(x), _DT[x.dtype], M, K, K, g or 0, _ptr(st), _ptr(q), K, _ptr(s))
    if rc != 0:
        raise ValueError(f"oracle quantize_rows_fp8 failed ({rc})")
    return q, s


# -------------------------------------------------------------------------- GEMMs
def gemm_i8_i32(a, w, row_ids=None):
    """int32 [len(rows), N] = a[rows] @ w.T exactly."""
    a, w = _cpu(a), _cpu(w)
    rows = _rows(row_ids)
    M = a.shape[0] if rows is None else rows.numel()
    N, K = w.shape
    c = torch.empty(M, N, dtype=torch.int32)
    lib().psq_or_gemm_i8_i32(_ptr(a), a.shape[1], _ptr(w), K, _ptr(c), N, M, N, K, _ptr(rows))
    return c


def epilogue_i32(c, a_scale, w_scale, bias=None, out_dtype=torch.bfloat16, row_ids=None):
    """y = round_out(fmaf(float(acc), a_s[m] * w_s[n], bias[n])); c holds the selected rows."""
    c, a_scale, w_scale = _cpu(c), _cpu(a_scale).float(), _cpu(w_scale).float().reshape(-1)
    bias = None if bias is None else _cpu(bias)
    rows = _rows(row_ids)
    M, N = c.shape
    y = torch.empty(M, N, dtype=out_dtype)
    lib().psq_or_epilogue_i32(_ptr(c), N, _ptr(a_scale), _ptr(w_scale), int(w_scale.numel() > 1),
                              _ptr(bias), _DT[bias.dtype] if bias is not None else 0, _ptr(y),
                              _DT[out_dtype], N, M, N, _ptr(rows))
    return y


def gemm_fp8(a, a_scale, w, w_scale, bias=None, out_dtype=torch.bfloat16, row_ids=None, w_e5m2=None):
    """fp8 codes a [M,K] (e4m3fn), w [N,K] (e4m3fn, or e5m2 when w_e5m2; default: w's dtype):
    y = round_out(fmaf(float(sum_f64), a_s*w_s, bias))."""
    if w_e5m2 is None:
        w_e5m2 = w.dtype == torch.float8_e5m2
    a, w = _cpu(a).view(torch.uint8), _cpu(w).view(torch.uint8)
    a_scale, w_scale = _cpu(a_scale).float(), _cpu(w_scale).float().reshape(-1)
    bias = None if bias is None else _cpu(bias)
    rows = _rows(row_ids)
    M = a.shape[0] if rows is None else rows.numel()
    N, K = w.shape
    y = torch.empty(M, N, dtype=out_dtype)
    fn = lib().psq_or_gemm_fp8_e5m2w if w_e5m2 else lib().psq_or_gemm_fp8
    fn(_ptr(a), a.shape[1], _ptr(a_scale), _ptr(w), K, _ptr(w_scale), int(w_scale.numel() > 1), _ptr(bias),
       _DT[bias.dtype] if bias is not None else 0, _ptr(y), _DT[out_dtype], N, M, N, K, _ptr(rows))
    return y


def dequant_uint4(wq, scale, zero, group_size, out_dtype=torch.bfloat16):
    wq, scale, zero = _cpu(wq), _cpu(scale).view(torch.int16), _cpu(zero).view(torch.int16)
    N = wq.shape[0]
    K = wq.shape[1] * 2
    out = torch.empty(N, K, dtype=out_dtype)
    if lib().psq_or_dequant_uint4(_ptr(wq), _ptr(scale), _ptr(zero), N, K, group_size, _ptr(out),
                                  _DT[out_dtype]) != 0:
        raise ValueError("bad uint4 layout")
    return out


def dequant_i8_rows(q, scale, rot_group=0, out_dtype=torch.bfloat16):
    """round_out(q * s[n]) with the ConvRot inverse applied by the fixed-order fast transform."""
    q, scale = _cpu(q), _cpu(scale).float().reshape(-1)
    N, K = q.shape
    out = torch.empty(N, K, dtype=out_dtype)
    if lib().psq_or_dequant_i8_rows(_ptr(q), _ptr(scale), N, K, rot_group or 0, _ptr(out), _DT[out_dtype]) != 0:
        raise ValueError("bad ConvRot group")
    return out


def dequant_fp8(q, scale, out_dtype=torch.bfloat16, e5m2=None):
    """round_out(decode(q) * s[n or 0]); q e4m3fn codes, or e5m2 when e5m2 (default: q's dtype)."""
    if e5m2 is None:
        e5m2 = q.dtype == torch.float8_e5m2
    q, scale = _cpu(q).view(torch.uint8), _cpu(scale).float().reshape(-1)
    N, K = q.shape
    out = torch.empty(N, K, dtype=out_dtype)
    fn = lib().psq_or_dequant_e5m2 if e5m2 else lib().psq_or_dequant_fp8
    fn(_ptr(q), _ptr(scale), int(scale.numel() > 1), N, K, _ptr(out), _DT[out_dtype])
    return out


def e5m2_to_f32(codes):
    """The oracle's e5m2 decode of uint8 codes (from the format's definition)."""
    return torch.tensor([lib().psq_or_e5m2_to_f32(int(c)) for c in codes.reshape(-1).tolist()],
                        dtype=torch.float32).reshape(codes.shape)


def gemm_wonly(x, wd, col_scale=None, bias=None, out_dtype=torch.bfloat16, row_ids=None):
    """y = round_out(fmaf(float(sum_f64 x*wd), col_scale[n] or 1, bias[n])) over rows row_ids."""
    x, wd = _cpu(x), _cpu(wd)
    col_scale = None if col_scale is None else _cpu(col_scale).float().reshape(-1)
    bias = None if bias is None else _cpu(bias)
    rows = _rows(row_ids)
    M = x.shape[0] if rows is None else rows.numel()
    N, K = wd.shape
    y = torch.empty(M, N, dtype=out_dtype)
    lib().psq_or_gemm_wonly(_ptr(x), _DT[x.dtype], x.shape[1], _ptr(wd), _DT[wd.dtype], _ptr(col_scale),
                            _ptr(bias), _DT[bias.dtype] if bias is not None else 0, _ptr(y),
                            _DT[out_dtype], N, M, N, K, _ptr(rows))
    return y


# -------------------------------------------------- reference load-time formulas
def dequantize_rows(q, scales, convrot, group_size, dtype=torch.float16):
    """powershard/operations.py:84-93: w = q*s (fp32), ConvRot inverse w @ H.T per group, cast."""
    if q.numel() == 0:
        return q.to(dtype)
    w = q.float() * scales.float()
    if convrot:
        h = torch.from_numpy(regular_hadamard_kron(group_size).astype(np.float32))
        w = (w.reshape(w.shape[0], -1, group_size) @ h.T).reshape_as(w)
    return w.to(dtype)


def quantize_weight_int8(w, convrot, group_size=256):
    """tests/test_fp16_safe.py:171-174: rotated = W @ H per group; s = rowmax|.|/127; q = round."""
    w = w.float()
    if convrot:
        h = torch.from_numpy(regular_hadamard_kron(group_size).astype(np.float32))
        w = (w.reshape(w.shape[0], -1, group_size) @ h).reshape_as(w)
    scale = w.abs().amax(-1, keepdim=True) / 127
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    q = (w / scale).round().clamp(-127, 127).to(torch.int8)
    return q, scale


def quantize_weight_fp8(w):
    """scripts/probe_wan_cuda.py:120-125: s = absmax.clamp(1e-12)/448, q = (w/s).to(e4m3fn)."""
    w = w.float()
    scale = w.abs().max().clamp(min=1e-12) / 448.0
    q = (w / scale).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q, scale.reshape(())


def quantize_weight_e5m2(w):
    """The same per-tensor recipe in e5m2 (max 57344): s = absmax.clamp(1e-12)/57344."""
    w = w.float()
    scale = w.abs().max().clamp(min=1e-12) / 57344.0
    q = (w / scale).clamp(-57344, 57344).to(torch.float8_e5m2)
    return q, scale.reshape(())


def quantize_weight_uint4(w, group_size=128):
    """Asymmetric uint4 per (row, group): s = fp16((max-min)/15) (0 -> 1), z = fp16(-min/s),
    q = clamp(rint(w/s + z), 0, 15); packed two per byte, low nibble = even k."""
    w = w.float()
    N, K = w.shape
    g = w.reshape(N, K // group_size, group_size)
    mn, mx = g.amin(-1), g.amax(-1)
    s = ((mx - mn) / 15.0).to(torch.float16)
    s = torch.where(s == 0, torch.ones_like(s), s)
    z = (-mn / s.float()).to(torch.float16)
    q = torch.round(g / s.float().unsqueeze(-1) + z.float().unsqueeze(-1)).clamp(0, 15).to(torch.uint8)
    q = q.reshape(N, K)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    return packed, s, z


def dequant_then_linear(x, w_deq, bias=None, dtype=torch.bfloat16):
    """powershard/quant_linear.py:219-220: F.linear(rows, qt.dequantize().to(dtype), bias)."""
    return torch.nn.functional.linear(x.to(dtype), w_deq.to(dtype), None if bias is None else bias.to(dtype))


def num_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
