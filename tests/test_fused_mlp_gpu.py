"""GELU(tanh) fused into the W8A8 / FP8 GEMM epilogue, and the chunked Wan MLP built on it.

Reference numerics (powershard/wan_model.py:626, quant_linear.py:197): the hidden activation is
F.gelu(fc1(rows).float(), approximate="tanh"), cast by fc2 to its compute dtype.  The fused
epilogue computes round_out(gelu(round_out(v))), v the linear epilogue value, whose int8 part is
bit-exact with the oracle; the bars isolate the GELU, on the oracle's rounded output (or, for the
fp32-accumulating fp8 path, on the same kernel's output without the activation):

* against the exact function (float64 v sigmoid(2 z), the form without cancellation; its identity
  with torch's tanh form is pinned in test_mlp_cpu -- torch's own float64 evaluation flushes to 0
  for v < -6), then rounded:
  every element within one output ulp (plus 1e-30: below about -9.6, where |gelu| < 1e-37, the
  hardware exp2 overflows or the reciprocal flushes its subnormal result and the kernel returns -0),
  at most 1e-3 of them different at all; fp32 outputs within
  1e-5 relative (the exp2 argument's rounding amplified by ln 2 |w|, |w| <= 126);
* against the reference's own fp32 arithmetic (torch's F.gelu on fp32): every element within one
  output ulp plus 1e-6 absolute.  That evaluation itself cancels in 1 + tanh z for v < -3 (relative
  error up to ~1e-4 there, |gelu| < 1e-2), so it is no bar for the fraction of differing elements;
* the chunked MLP: the fused result is within the 1e-2 rms bar (or one bf16 ulp) of the unfused
  reference sequence on the same modules, and independent of the chunk size (bit-exact).
"""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from conftest import heavy_rows, seeded
from test_quant_linear_gpu import make_layer

pytestmark = pytest.mark.gpu


def _ulp(ref, dtype):
    a = ref.abs().clamp(min=2.0 ** -126)
    bits = 7 if dtype == torch.bfloat16 else 10
    floor = -133 if dtype == torch.bfloat16 else -24   # subnormal spacing
    return torch.pow(2.0, torch.maximum(torch.floor(torch.log2(a)) - bits, torch.full_like(a, floor)))


def exact_gelu(v):
    v = v.double()
    return v * torch.sigmoid(2.0 * math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3))


def assert_gelu_of(y, lin, what, max_frac=1e-3):
    """y: the fused kernel's output; lin: the unactivated output in y's dtype (rounded)."""
    y, lin = y.cpu(), lin.cpu()
    exact = exact_gelu(lin)
    ref32 = F.gelu(lin.float(), approximate="tanh")
    yd = y.double()
    if y.dtype == torch.float32:
        d = (yd - exact).abs()
        bad = d > 1e-5 * exact.abs() + 1e-30
        bad_ref = (yd - ref32.double()).abs() > 1e-4 * exact.abs() + 1e-6
        differ = torch.zeros_like(bad)   # fp32: the relative bar above is the whole check
    else:
        ex = exact.to(y.dtype).double()
        d = (yd - ex).abs()
        bad = d > _ulp(ex, y.dtype) * 1.0000001 + 1e-30
        r = ref32.to(y.dtype).double()
        bad_ref = (yd - r).abs() > _ulp(r, y.dtype) * 1.0000001 + 1e-6
        differ = d > 1e-30
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off the exact GELU, worst {d.max().item():.3e}"
    assert not bad_ref.any(), f"{what}: {int(bad_ref.sum())} elements off torch's fp32 GELU"
    frac = differ.double().mean().item()
    print(f"{what}: {frac:.2e} of {y.numel()} elements differ from the exact GELU (all within one ulp)")
    assert frac <= max_frac, f"{what}: {frac} of the elements differ"
    assert torch.equal(torch.isnan(y.float()), torch.isnan(ref32))


# partial tiles on both edges (element stores), full-width tiles of aligned rows (16-bit outputs:
# the LDS-staged stores; fp32: the register stores), and persistent grids with several tiles per
# workgroup
ACT_CASES = [(300, 200, 640), (1000, 512, 1024), (257, 264, 256), (4100, 4096, 256), (600, 1000, 5120)]


@pytest.mark.parametrize("M,N,K", ACT_CASES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_gemm_i8_gelu(gpu, M, N, K, out_dtype):
    from powershard_amd import ops
    from powershard_amd.quant_tensor import QuantizedWeight
    print(f"gemm_i8 gelu M={M} N={N} K={K} {out_dtype}", flush=True)
    x = heavy_rows(M, K, seed=M + 7 * K)
    qa, sa = oracle.quantize_rows_i8(x, 256 if K % 256 == 0 else 0)
    w = torch.randn(N, K, generator=seeded(N + 2)) * 0.05
    qw = QuantizedWeight.from_float(w, "Int8RowwiseLayout")
    b = (torch.randn(N, generator=seeded(N + 3)) * 0.5).to(torch.bfloat16)
    args = (qa.to(gpu), sa.to(gpu), qw._qdata.to(gpu), qw._params.scale.to(gpu), b.to(gpu))
    y = ops.gemm_i8(*args, out_dtype=out_dtype, activation="gelu_tanh")
    lin = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw._qdata), sa, qw._params.scale, b, out_dtype=out_dtype)
    # the linear part is the kernel's own bit-exact epilogue
    assert torch.equal(ops.gemm_i8(*args, out_dtype=out_dtype).cpu().view(torch.int16 if out_dtype != torch.float32 else torch.int32),
                       lin.view(torch.int16 if out_dtype != torch.float32 else torch.int32))
    assert (lin.float() < -4).any() and (lin.float() > 4).any()   # both tails of the GELU are exercised
    assert_gelu_of(y, lin, "int8 gelu epilogue")


def test_gemm_i8_gelu_unaligned_rows(gpu):
    """ldy with rows not 16-byte aligned: the element-store path of full-width tiles."""
    from powershard_amd import _native
    M, N, K = 300, 512, 256
    g = seeded(91)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 0.02 + 1e-3
    sw = torch.rand(N, generator=g) * 2e-3 + 1e-4
    ldy = N + 3
    y = torch.empty(M, ldy, dtype=torch.bfloat16, device=gpu)
    lib = _native.lib()
    a_d, w_d, sa_d, sw_d = qa.to(gpu), qw.to(gpu), sa.to(gpu), sw.to(gpu)
    _native.check(lib.psq_gemm_i8_act(a_d.data_ptr(), K, sa_d.data_ptr(), w_d.data_ptr(), K, sw_d.data_ptr(), None, 0,
                                      1, y.data_ptr(), 0, ldy, M, N, K, None), "gemm_i8_act")
    torch.cuda.synchronize()
    lin = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw), sa, sw, None, out_dtype=torch.bfloat16)
    assert_gelu_of(y[:, :N].contiguous(), lin, "int8 gelu, unaligned rows")


def test_gemm_act_none_and_bad_activation(gpu):
    """activation 0 through the _act entry point is psq_gemm_i8 itself; an unknown code is an error."""
    from powershard_amd import _native
    M, N, K = 200, 256, 256
    g = seeded(5)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(gpu)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(gpu)
    sa = (torch.rand(M, generator=g) * 0.02).to(gpu)
    sw = (torch.rand(N, generator=g) * 0.002).to(gpu)
    lib = _native.lib()
    y0 = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
    y1 = torch.empty_like(y0)
    common = (qa.data_ptr(), K, sa.data_ptr(), qw.data_ptr(), K, sw.data_ptr(), None, 0)
    _native.check(lib.psq_gemm_i8(*common, y0.data_ptr(), 0, N, M, N, K, None), "gemm_i8")
    _native.check(lib.psq_gemm_i8_act(*common, 0, y1.data_ptr(), 0, N, M, N, K, None), "gemm_i8_act")
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert lib.psq_gemm_i8_act(*common, 7, y1.data_ptr(), 0, N, M, N, K, None) == -1
    assert b"activation" in lib.psq_last_error()


@pytest.mark.parametrize("M,N,K", [(300, 200, 640), (1000, 768, 1024), (4100, 4096, 256)])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_fp8_gelu(gpu, M, N, K, per_row, out_dtype):
    from powershard_amd import ops
    print(f"gemm_fp8 gelu M={M} N={N} K={K} per_row={per_row} {out_dtype}", flush=True)
    x = heavy_rows(M, K, seed=M + 5 * K)
    qa, sa = oracle.quantize_rows_fp8(x)
    w = torch.randn(N, K, generator=seeded(N + K + 1)) * 0.02
    if per_row:
        ws = w.abs().amax(1) / 448.0
        qw = (w / ws[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    else:
        qw, ws = oracle.quantize_weight_fp8(w)
    b = (torch.randn(N, generator=seeded(6)) * 0.5).to(torch.bfloat16)
    args = (qa.view(torch.float8_e4m3fn).to(gpu), sa.to(gpu), qw.to(gpu), ws.to(gpu), b.to(gpu))
    lin = ops.gemm_fp8(*args, out_dtype=out_dtype)
    y = ops.gemm_fp8(*args, out_dtype=out_dtype, activation="gelu_tanh")
    assert_gelu_of(y, lin, "fp8 gelu epilogue")


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}),
                                                ("int8", {"convrot": False}), ("fp8", {})])
def test_chunked_mlp(gpu, weight_format, opts):
    """Wan FFN: fc2(gelu(fc1(x))) with the GELU in fc1's epilogue, against the reference sequence
    F.gelu(fc1(x).float(), approximate="tanh") -> fc2 on the same native modules."""
    from powershard_amd import mlp
    D, H, T = 1024, 2816, 700
    fc1, _, _ = make_layer(D, H, weight_format, opts, torch.bfloat16, True, gpu, seed=21)
    fc2, _, _ = make_layer(H, D, weight_format, opts, torch.bfloat16, True, gpu, seed=22)
    x = heavy_rows(T, D, seed=23).reshape(7, 100, D).to(gpu)
    y = mlp.chunked_mlp(fc1, fc2, x)
    y_chunks = mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=256)
    assert fc1._ps_native and fc2._ps_native
    assert y.shape == (7, 100, D) and y.dtype == torch.float32
    assert torch.equal(y.view(torch.int32), y_chunks.view(torch.int32)), "chunking changed a value"
    hidden_ref = F.gelu(fc1(x).float(), approximate="tanh")
    ref = fc2(hidden_ref).float()
    hidden = fc1.forward_act(x)
    assert hidden.dtype == torch.bfloat16
    assert_gelu_of(hidden.reshape(T, H), fc1(x).reshape(T, H), "fc1 fused hidden")
    # a hidden element one ulp away can move fc2's per-token quantization: the bf16 outputs then
    # differ within the 1e-2 rms bar or by one output ulp (above 2.56 rms one ulp exceeds the bar)
    rms = ref.pow(2).mean().sqrt().item()
    err = (y - ref).abs()
    bound = torch.maximum(torch.full_like(ref, 1e-2 * rms), _ulp(ref.double(), torch.bfloat16).float())
    print(f"chunked mlp {weight_format}: max|d| = {err.max().item():.3e}, rms = {rms:.3e}, "
          f"{(err > 0).double().mean().item():.2e} of the outputs differ")
    assert torch.all(err <= bound)
