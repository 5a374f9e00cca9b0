"""Torch-facing wrappers of the gfx950 kernels (device tensors in, device tensors out).

Each op checks dtypes, devices and contiguity, allocates its outputs with PyTorch's caching
allocator on the input's device, launches on that device's current stream and raises
``RuntimeError`` (with the library's message) on any failure.  No op has a CPU implementation:
on a tensor that is not on a GPU they raise ``RuntimeError``.
"""
import contextlib
import ctypes

import torch

from . import _native

# Opt-in launch timing: while kernel_timer() is active, every launch is bracketed by a pair of
# HIP events recorded on the stream it runs on (the device's current stream).
_timer = None


@contextlib.contextmanager
def kernel_timer():
    """Collect {op name: [(start event, end event), ...]} for the launches inside the block."""
    global _timer
    prev, _timer = _timer, {}
    try:
        yield _timer
    finally:
        _timer = prev


def kernel_times_ms(events):
    """{op: [milliseconds per launch]} from kernel_timer()'s events (synchronizes)."""
    torch.cuda.synchronize()
    return {k: [a.elapsed_time(b) for a, b in v] for k, v in events.items()}


def _launch(name, fn, *args):
    if _timer is None:
        return _native.check(fn(*args), name)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    status = fn(*args)
    b.record()
    _timer.setdefault(name, []).append((a, b))
    return _native.check(status, name)

_DT = {torch.bfloat16: _native.BF16, torch.float16: _native.F16, torch.float32: _native.F32}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


try:   # the current stream's raw handle without building a torch.cuda.Stream (2.4 -> ~0.3 us a call)
    from torch._C import _cuda_getCurrentRawStream as _raw_stream
except ImportError:
    _raw_stream = None


def _stream(t):
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need_gpu(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"psquant kernels need GPU tensors (got {t.device})")


def _dt(t, what):
    if t.dtype not in _DT:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}")
    return _DT[t.dtype]


def _rows2d(x):
    """[M, K] with unit column stride, rows at least K apart and 16-byte aligned rows: x itself
    when it is so laid out, else a packed copy (torch's contiguous() keeps the strides of size-1
    dimensions and the offset of an aligned-looking view, so the copy is explicit)."""
    if x.dim() != 2:
        raise ValueError("expected a 2-D tensor")
    M, K = x.shape
    if M == 0 or K == 0:
        return x
    if (x.stride(1) != 1 or x.stride(0) < K or (x.stride(0) * x.element_size()) % 16
            or x.data_ptr() % 16):
        x = torch.empty((M, K), dtype=x.dtype, device=x.device).copy_(x)
    return x


def _bias(bias, n, device):
    if bias is None:
        return None, 0
    if bias.numel() != n:
        raise ValueError(f"bias has {bias.numel()} elements, expected {n}")
    bias = bias.to(device).contiguous()
    return bias, _dt(bias, "bias")


# ------------------------------------------------------------------ activations
def quantize_rows(x, fp8=False, rot_group=0, static_scale=None):
    """Fused ConvRot rotation + per-row absmax + int8 (or fp8 e4m3fn) quantization.

    x: [M, K] bf16/f16 on the GPU.  Returns (q [M, K] int8 or float8_e4m3fn, scale [M] fp32).
    static_scale: optional fp32 tensor with one element (the module's input_scale).
    """
    _need_gpu(x, static_scale)
    x = _rows2d(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"quantize_rows: activations must be bf16/f16, got {x.dtype}")
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn if fp8 else torch.int8, device=x.device)
    scale = torch.empty(M, dtype=torch.float32, device=x.device)
    st = None
    if static_scale is not None:
        st = static_scale.to(device=x.device, dtype=torch.float32).reshape(-1)[:1].contiguous()
    fn = _native.lib().psq_quantize_rows_fp8 if fp8 else _native.lib().psq_quantize_rows_i8
    _launch("quantize_rows_fp8" if fp8 else "quantize_rows_i8", fn, _p(x), _DT[x.dtype], M, K, x.stride(0),
            int(rot_group or 0), _p(st), _p(q), K, _p(scale), _stream(x))
    return q, scale


def rotate_rows(x, rot_group, out_dtype=None):
    """x H per group of rot_group elements (the quantizer's fixed-order transform, one rounding to
    out_dtype, default x.dtype).  x: [M, K] bf16/f16 on the GPU; rot_group 0 converts only."""
    _need_gpu(x)
    x = _rows2d(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"rotate_rows: activations must be bf16/f16, got {x.dtype}")
    M, K = x.shape
    y = torch.empty(M, K, dtype=out_dtype or x.dtype, device=x.device)
    _launch("rotate_rows", _native.lib().psq_rotate_rows, _p(x), _DT[x.dtype], M, K, x.stride(0), int(rot_group or 0),
            _p(y), _dt(y, "out"), K, _stream(x))
    return y


# ----------------------------------------------------------------------- GEMMs
# epilogue activations of the W8A8 / FP8 GEMMs (enum psq_activation)
ACTIVATIONS = {None: 0, "none": 0, "gelu_tanh": 1, "silu_gate": 2}


def _act(activation):
    try:
        return ACTIVATIONS[activation]
    except KeyError:
        raise ValueError(f"unknown epilogue activation {activation!r}") from None


def _out_cols(N, act, name):
    """Output columns: N, or N / 2 for the SiLU gate (gate rows, then up rows)."""
    if act != ACTIVATIONS["silu_gate"]:
        return N
    if N % 128:
        raise ValueError(f"{name}: the SiLU gate needs N (gate + up rows) a multiple of 128, got {N}")
    return N // 2


def gemm_i8(a, a_scale, w, w_scale, bias=None, out_dtype=torch.bfloat16, activation=None):
    """y = round(fmaf(a @ w.T (int32), a_scale[m] * w_scale[n], bias[n])): [M, N] out_dtype.

    activation "gelu_tanh": y = round(gelu_tanh(round(...))) -- the GELU of the rounded output,
    rounded again (the Wan FFN's F.gelu(fc1(x).float(), approximate="tanh") then fc2's cast).
    activation "silu_gate": w holds N / 2 gate rows then N / 2 up rows (N a multiple of 128);
    y[m, j] = round(silu(round(g)) * round(u)) is [M, N / 2], g and u the linear outputs of
    columns j and N / 2 + j (the H3 MLP's F.silu(gate.float()) * up.float(), then fc2's cast).
    """
    _need_gpu(a, a_scale, w, w_scale)
    a, w = _rows2d(a), _rows2d(w)
    if a.dtype != torch.int8 or w.dtype != torch.int8:
        raise TypeError("gemm_i8: operands must be int8")
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"gemm_i8: K mismatch {K} vs {w.shape[1]}")
    a_scale = a_scale.to(torch.float32).reshape(-1).contiguous()
    w_scale = w_scale.to(torch.float32).reshape(-1).contiguous()
    if a_scale.numel() != M or w_scale.numel() != N:
        raise ValueError("gemm_i8: scale sizes do not match M / N")
    bias, bdt = _bias(bias, N, a.device)
    act = _act(activation)
    y = torch.empty(M, _out_cols(N, act, "gemm_i8"), dtype=out_dtype, device=a.device)
    if act:
        _launch("gemm_i8", _native.lib().psq_gemm_i8_act, _p(a), a.stride(0), _p(a_scale), _p(w), w.stride(0), _p(w_scale),
                _p(bias), bdt, act, _p(y), _dt(y, "out"), y.shape[1], M, N, K, _stream(a))
    else:
        _launch("gemm_i8", _native.lib().psq_gemm_i8, _p(a), a.stride(0), _p(a_scale), _p(w), w.stride(0), _p(w_scale),
                _p(bias), bdt, _p(y), _dt(y, "out"), N, M, N, K, _stream(a))
    return y


def gemm_i8_i32(a, w):
    """Raw int32 accumulators a @ w.T ([M, N] int32)."""
    _need_gpu(a, w)
    a, w = _rows2d(a), _rows2d(w)
    M, K = a.shape
    N = w.shape[0]
    c = torch.empty(M, N, dtype=torch.int32, device=a.device)
    _launch("gemm_i8_i32", _native.lib().psq_gemm_i8_i32, _p(a), a.stride(0), _p(w), w.stride(0), _p(c), N, M, N, K, _stream(a))
    return c


def gemm_fp8(a, a_scale, w, w_scale, bias=None, out_dtype=torch.bfloat16, activation=None):
    """fp8 GEMM: y = round(fmaf(a @ w.T (fp32), a_scale[m] * w_scale[n or 0], bias[n])).

    a: e4m3fn activation codes.  w: e4m3fn codes, or float8_e5m2 codes (``psq_gemm_fp8_e5m2w``,
    no activation epilogue).  uint8 views are read as e4m3fn.  activation as in gemm_i8.
    """
    _need_gpu(a, a_scale, w, w_scale)
    a, w = _rows2d(a), _rows2d(w)
    if a.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError("gemm_fp8: activations must be float8_e4m3fn")
    e5m2 = w.dtype == torch.float8_e5m2
    if w.dtype not in (torch.float8_e4m3fn, torch.uint8) and not e5m2:
        raise TypeError("gemm_fp8: weights must be float8_e4m3fn or float8_e5m2")
    if e5m2 and activation not in (None, "none"):
        raise ValueError("gemm_fp8: float8_e5m2 weights take no activation epilogue")
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"gemm_fp8: K mismatch {K} vs {w.shape[1]}")
    a_scale = a_scale.to(torch.float32).reshape(-1).contiguous()
    w_scale = w_scale.to(device=a.device, dtype=torch.float32).reshape(-1).contiguous()
    if a_scale.numel() != M or w_scale.numel() not in (1, N):
        raise ValueError("gemm_fp8: scale sizes do not match")
    bias, bdt = _bias(bias, N, a.device)
    act = _act(activation)
    y = torch.empty(M, _out_cols(N, act, "gemm_fp8"), dtype=out_dtype, device=a.device)
    if act:
        _launch("gemm_fp8", _native.lib().psq_gemm_fp8_act, _p(a), a.stride(0), _p(a_scale), _p(w), w.stride(0),
                _p(w_scale), int(w_scale.numel() > 1), _p(bias), bdt, act, _p(y), _dt(y, "out"), y.shape[1], M, N, K,
                _stream(a))
    else:
        fn = _native.lib().psq_gemm_fp8_e5m2w if e5m2 else _native.lib().psq_gemm_fp8
        _launch("gemm_fp8", fn, _p(a), a.stride(0), _p(a_scale), _p(w), w.stride(0),
                _p(w_scale), int(w_scale.numel() > 1), _p(bias), bdt, _p(y), _dt(y, "out"), N, M, N, K, _stream(a))
    return y


# Split-K workspaces of the weight-only GEMMs, one per (device, stream): calls on one stream run in
# order, so they can share it (calls on two streams would race on its counters).  A call that needs
# more gets a larger one (at least twice the size, so a stream is replaced a few times at most), and
# the replaced buffer is kept until the process ends: a launch captured into a graph keeps the
# address it was given, which must not be handed out again.  At most _MAX_WS_STREAMS streams per
# device get one; calls on further streams run without a workspace (the data-parallel tiles: the
# same results, the split of K left out).  For capture and for callers that cannot allocate at all,
# psq_gemm_w4a16_noalloc uses the library's own static scratch instead.
_workspaces = {}
_retired_workspaces = []
_MAX_WS_STREAMS = 16
_WS_MIN_BYTES = 1 << 20


def _workspace(device, stream, nbytes):
    if nbytes <= 0:
        return None, 0
    key = (device.index, stream)
    ws = _workspaces.get(key)
    if ws is None and sum(1 for d, _ in _workspaces if d == device.index) >= _MAX_WS_STREAMS:
        return None, 0
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, _WS_MIN_BYTES, 2 * ws.numel() if ws is not None else 0)
        if ws is not None:
            _retired_workspaces.append(ws)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)   # counter words zero once; calls leave them so
        _workspaces[key] = ws
    return ws, ws.numel()


def gemm_w4a16(x, wq, w_scale, w_zero, group_size, bias=None, out_dtype=None):
    """uint4 asymmetric group weights, in-register dequantized onto bf16/f16 MFMA.

    x [M, K] bf16/f16, wq [N, K/2] uint8 (low nibble = even k), w_scale/w_zero [N, K/group] fp16.
    Shapes that leave CUs idle split K across workgroups through a cached workspace.
    """
    _need_gpu(x, wq, w_scale, w_zero)
    x, wq = _rows2d(x), wq.contiguous()
    M, K = x.shape
    N = wq.shape[0]
    if wq.shape[1] * 2 != K:
        raise ValueError(f"gemm_w4a16: packed weight [{N}, {wq.shape[1]}] does not match K={K}")
    w_scale = w_scale.to(torch.float16).contiguous()
    w_zero = w_zero.to(torch.float16).contiguous()
    bias, bdt = _bias(bias, N, x.device)
    y = torch.empty(M, N, dtype=out_dtype or x.dtype, device=x.device)
    stream = _stream(x)
    ws, nb = _workspace(x.device, stream.value,
                        _native.lib().psq_gemm_wonly_workspace_bytes(_native.W_UINT4, x.stride(0), M, N, K,
                                                                     int(group_size)))
    _launch("gemm_w4a16", _native.lib().psq_gemm_w4a16_ws, _p(x), _dt(x, "x"), x.stride(0), _p(wq), _p(w_scale),
            _p(w_zero), int(group_size), _p(bias), bdt, _p(y), _dt(y, "out"), N, M, N, K, _p(ws), nb, stream)
    return y


def gemm_w8a16(x, wq, w_scale, bias=None, out_dtype=None):
    """int8 weight-only: y = round(fmaf(x @ q.T (fp32), w_scale[n], bias[n]))."""
    _need_gpu(x, wq, w_scale)
    x, wq = _rows2d(x), _rows2d(wq)
    M, K = x.shape
    N = wq.shape[0]
    w_scale = w_scale.to(torch.float32).reshape(-1).contiguous()
    bias, bdt = _bias(bias, N, x.device)
    y = torch.empty(M, N, dtype=out_dtype or x.dtype, device=x.device)
    stream = _stream(x)
    ws, nb = _workspace(x.device, stream.value,
                        _native.lib().psq_gemm_wonly_workspace_bytes(_native.W_INT8, x.stride(0), M, N, K, 0))
    _launch("gemm_w8a16", _native.lib().psq_gemm_w8a16_ws, _p(x), _dt(x, "x"), x.stride(0), _p(wq), _p(w_scale),
            _p(bias), bdt, _p(y), _dt(y, "out"), N, M, N, K, _p(ws), nb, stream)
    return y


# ------------------------------------------------------------------ dequantize
def dequant_uint4(wq, w_scale, w_zero, group_size, out_dtype=torch.bfloat16):
    _need_gpu(wq, w_scale, w_zero)
    wq = wq.contiguous()
    N, K = wq.shape[0], wq.shape[1] * 2
    out = torch.empty(N, K, dtype=out_dtype, device=wq.device)
    _launch("dequant_uint4", _native.lib().psq_dequant_uint4, _p(wq), _p(w_scale.to(torch.float16).contiguous()),
                                                  _p(w_zero.to(torch.float16).contiguous()), int(group_size), N, K,
                                                  _p(out), _dt(out, "out"), _stream(wq))
    return out


def dequant_i8_rows(q, w_scale, rot_group=0, out_dtype=torch.bfloat16):
    _need_gpu(q, w_scale)
    q = q.contiguous()
    N, K = q.shape
    out = torch.empty(N, K, dtype=out_dtype, device=q.device)
    _launch("dequant_i8_rows", _native.lib().psq_dequant_i8_rows, _p(q), _p(w_scale.to(torch.float32).reshape(-1).contiguous()), N, K,
                                                    int(rot_group or 0), _p(out), _dt(out, "out"), _stream(q))
    return out


def dequant_fp8(q, w_scale, out_dtype=torch.bfloat16, e5m2=None):
    """fp8 weight codes [N, K] times the scale (one, or one per row).  e5m2: the codes are
    float8_e5m2 (default: from q's dtype; uint8 views are e4m3fn)."""
    _need_gpu(q)
    if e5m2 is None:
        e5m2 = q.dtype == torch.float8_e5m2
    q = q.contiguous()
    N, K = q.shape
    s = w_scale.to(device=q.device, dtype=torch.float32).reshape(-1).contiguous()
    out = torch.empty(N, K, dtype=out_dtype, device=q.device)
    name, fn = ("dequant_e5m2", _native.lib().psq_dequant_e5m2) if e5m2 else ("dequant_fp8", _native.lib().psq_dequant_fp8)
    _launch(name, fn, _p(q), _p(s), int(s.numel() > 1), N, K, _p(out), _dt(out, "out"), _stream(q))
    return out


# ------------------------------------------------------------------ checks
# Non-finite flags, one per (device, stream), with the last ticket handed out: a call raises the
# flag to its ticket when it finds a NaN or Inf, and the flag is never cleared.
_nonfinite = {}


def any_nonfinite(t):
    """True when the CUDA tensor t (bf16 / f16 / f32) holds a NaN or an Inf: one pass over t and an
    8-byte read back (a synchronization, as `not torch.isfinite(t).all()`, which this replaces where
    it is checked on every call)."""
    _need_gpu(t)
    t = t.contiguous()
    stream = _stream(t)
    key = (t.device.index, stream.value)
    entry = _nonfinite.get(key)
    if entry is None:
        entry = _nonfinite[key] = [torch.zeros(1, dtype=torch.int64, device=t.device), 0]
    entry[1] += 1
    _launch("flag_nonfinite", _native.lib().psq_flag_nonfinite, _p(t), _dt(t, "t"), t.numel(), _p(entry[0]),
            entry[1], stream)
    return int(entry[0].item()) >= entry[1]


def device_supported(device):
    device = torch.device(device)
    if device.type != "cuda":
        return False
    index = device.index if device.index is not None else torch.cuda.current_device()
    return bool(_native.lib().psq_device_supported(index))
