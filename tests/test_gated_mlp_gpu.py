"""The SiLU gate fused into the W8A8 / FP8 GEMM epilogue, and the chunked H3 MLP built on it.

Reference numerics (powershard/fp16_safe.py:165-168, quant_linear.py:197): the hidden activation
is F.silu(gate.float()) * up.float() over gate, up = fc1(rows).chunk(2, -1), cast by fc2 to its
compute dtype.  The fused epilogue computes round_out(silu(round_out(g)) round_out(u)), g and u
the linear epilogue values of columns j and N / 2 + j, whose int8 part is bit-exact with the
oracle; the bars isolate the gate, on the oracle's rounded output (or, for the fp32-accumulating
fp8 path, on the same kernel's output without the activation):

* against the exact function (float64 g sigmoid(g) u), then rounded: every element within one
  output ulp (plus 1e-30: below g = -88.7, where |silu| < 1e-36, the hardware exp2 overflows and
  the kernel returns -0), at most 1e-3 of them different at all; fp32 outputs within 1e-5
  relative (the exp2 argument's rounding amplified by |g| <= 88.7 ln 2 is at most 4e-6);
* against the reference's own fp32 arithmetic (torch's F.silu(g) * u on fp32): every element
  within one output ulp plus 1e-30;
* the chunked MLP: the fused result is within the 1e-2 rms bar (or one bf16 ulp) of the unfused
  reference sequence on the same modules, and independent of the chunk size (bit-exact).
"""
import pytest
import torch
import torch.nn.functional as F

import oracle
from conftest import heavy_rows, seeded
from test_fused_mlp_gpu import _ulp
from test_quant_linear_gpu import make_layer

pytestmark = pytest.mark.gpu


def assert_gate_of(y, lin, what, max_frac=1e-3):
    """y: the fused kernel's output [M, H]; lin: the unactivated output [M, 2 H] in y's dtype."""
    y, lin = y.cpu(), lin.cpu()
    H = lin.shape[-1] // 2
    assert y.shape == lin.shape[:-1] + (H,)
    g, u = lin[..., :H], lin[..., H:]
    exact = g.double() * torch.sigmoid(g.double()) * u.double()
    ref32 = F.silu(g.float()) * u.float()
    yd = y.double()
    if y.dtype == torch.float32:
        d = (yd - exact).abs()
        bad = d > 1e-5 * exact.abs() + 1e-30
        bad_ref = (yd - ref32.double()).abs() > 1e-5 * exact.abs() + 1e-30
        differ = torch.zeros_like(bad)   # fp32: the relative bar above is the whole check
    else:
        ex = exact.to(y.dtype).double()
        d = (yd - ex).abs()
        bad = d > _ulp(ex, y.dtype) * 1.0000001 + 1e-30
        r = ref32.to(y.dtype).double()
        bad_ref = (yd - r).abs() > _ulp(r, y.dtype) * 1.0000001 + 1e-30
        differ = d > 1e-30
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off the exact gate, worst {d.max().item():.3e}"
    assert not bad_ref.any(), f"{what}: {int(bad_ref.sum())} elements off torch's fp32 gate"
    frac = differ.double().mean().item()
    print(f"{what}: {frac:.2e} of {y.numel()} elements differ from the exact gate (all within one ulp)")
    assert frac <= max_frac, f"{what}: {frac} of the elements differ"
    assert torch.equal(torch.isnan(y.float()), torch.isnan(ref32))


# N = gate + up rows.  Half tiles at the N edge (the second wave column has no block), partial row
# tiles, full tiles of aligned rows (16-bit outputs: the LDS-staged stores; fp32: element stores),
# persistent grids with several tiles per workgroup, and a long K.
GATE_CASES = [(300, 384, 640), (1000, 1024, 1024), (257, 256, 256), (4100, 4096, 256), (600, 2048, 5120)]


def _i8_case(M, N, K):
    from powershard_amd.quant_tensor import QuantizedWeight
    x = heavy_rows(M, K, seed=M + 7 * K + 1)
    qa, sa = oracle.quantize_rows_i8(x, 256 if K % 256 == 0 else 0)
    w = torch.randn(N, K, generator=seeded(N + 4)) * 0.05
    qw = QuantizedWeight.from_float(w, "Int8RowwiseLayout")
    b = (torch.randn(N, generator=seeded(N + 5)) * 0.5).to(torch.bfloat16)
    return qa, sa, qw._qdata, qw._params.scale, b


@pytest.mark.parametrize("M,N,K", GATE_CASES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_gemm_i8_silu_gate(gpu, M, N, K, out_dtype):
    from powershard_amd import ops
    print(f"gemm_i8 silu_gate M={M} N={N} K={K} {out_dtype}", flush=True)
    qa, sa, qw, sw, b = _i8_case(M, N, K)
    args = (qa.to(gpu), sa.to(gpu), qw.to(gpu), sw.to(gpu), b.to(gpu))
    y = ops.gemm_i8(*args, out_dtype=out_dtype, activation="silu_gate")
    lin = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw), sa, sw, b, out_dtype=out_dtype)
    iv = torch.int16 if out_dtype != torch.float32 else torch.int32
    assert torch.equal(ops.gemm_i8(*args, out_dtype=out_dtype).cpu().view(iv), lin.view(iv))
    g = lin[:, :N // 2].float()
    assert (g < -4).any() and (g > 4).any()   # both tails of the SiLU are exercised
    assert_gate_of(y, lin, "int8 silu gate epilogue")


def test_gemm_i8_silu_gate_unaligned_rows(gpu):
    """ldy with rows not 16-byte aligned: the element-store path."""
    from powershard_amd import _native
    M, N, K = 300, 512, 256
    qa, sa, qw, sw, b = _i8_case(M, N, K)
    ldy = N // 2 + 3
    y = torch.empty(M, ldy, dtype=torch.bfloat16, device=gpu)
    lib = _native.lib()
    a_d, w_d, sa_d, sw_d, b_d = qa.to(gpu), qw.to(gpu), sa.to(gpu), sw.to(gpu), b.to(gpu)
    _native.check(lib.psq_gemm_i8_act(a_d.data_ptr(), K, sa_d.data_ptr(), w_d.data_ptr(), K, sw_d.data_ptr(),
                                      b_d.data_ptr(), 0, 2, y.data_ptr(), 0, ldy, M, N, K, None), "gemm_i8_act")
    torch.cuda.synchronize()
    lin = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw), sa, sw, b, out_dtype=torch.bfloat16)
    assert_gate_of(y[:, :N // 2].contiguous(), lin, "int8 silu gate, unaligned rows")


def test_gemm_silu_gate_shape_errors(gpu):
    from powershard_amd import _native, ops
    M, K = 64, 256
    g = seeded(8)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(gpu)
    sa = (torch.rand(M, generator=g) * 0.02).to(gpu)
    qw = torch.randint(-127, 128, (320, K), generator=g, dtype=torch.int8).to(gpu)
    sw = (torch.rand(320, generator=g) * 0.002).to(gpu)
    with pytest.raises(ValueError, match="multiple of 128"):
        ops.gemm_i8(qa, sa, qw[:200], sw[:200], activation="silu_gate")
    lib = _native.lib()
    y = torch.empty(M, 160, dtype=torch.bfloat16, device=gpu)
    common = (qa.data_ptr(), K, sa.data_ptr(), qw.data_ptr(), K, sw.data_ptr(), None, 0, 2, y.data_ptr(), 0)
    assert lib.psq_gemm_i8_act(*common, 160, M, 320, K, None) == -2          # PSQ_E_SHAPE
    assert b"multiple of 128" in lib.psq_last_error()
    assert lib.psq_gemm_i8_act(*common, 127, M, 256, K, None) == -2
    assert b"ldy < N / 2" in lib.psq_last_error()


@pytest.mark.parametrize("M,N,K", [(300, 384, 640), (1000, 768, 1024), (4100, 4096, 256)])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_fp8_silu_gate(gpu, M, N, K, per_row, out_dtype):
    from powershard_amd import ops
    print(f"gemm_fp8 silu_gate M={M} N={N} K={K} per_row={per_row} {out_dtype}", flush=True)
    x = heavy_rows(M, K, seed=M + 5 * K + 1)
    qa, sa = oracle.quantize_rows_fp8(x)
    w = torch.randn(N, K, generator=seeded(N + K + 2)) * 0.02
    if per_row:
        ws = w.abs().amax(1) / 448.0
        qw = (w / ws[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    else:
        qw, ws = oracle.quantize_weight_fp8(w)
    b = (torch.randn(N, generator=seeded(7)) * 0.5).to(torch.bfloat16)
    args = (qa.view(torch.float8_e4m3fn).to(gpu), sa.to(gpu), qw.to(gpu), ws.to(gpu), b.to(gpu))
    lin = ops.gemm_fp8(*args, out_dtype=out_dtype)
    y = ops.gemm_fp8(*args, out_dtype=out_dtype, activation="silu_gate")
    assert_gate_of(y, lin, "fp8 silu gate epilogue")


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}),
                                                ("int8", {"convrot": False}), ("fp8", {})])
def test_gated_mlp(gpu, weight_format, opts):
    """H3 MLP: fc2(silu(gate) * up) with the gate in fc1's epilogue, against the reference sequence
    gate, up = fc1(x).chunk(2, -1); fc2(F.silu(gate.float()) * up.float()) on the same modules."""
    from powershard_amd import mlp
    D, H, T = 1024, 1536, 700
    fc1, _, _ = make_layer(D, 2 * H, weight_format, opts, torch.bfloat16, True, gpu, seed=31)
    fc2, _, _ = make_layer(H, D, weight_format, opts, torch.bfloat16, True, gpu, seed=32)
    x = heavy_rows(T, D, seed=33).reshape(7, 100, D).to(gpu)
    y = mlp.gated_mlp(fc1, fc2, x)
    y_chunks = mlp.gated_mlp(fc1, fc2, x, chunk_tokens=256)
    assert fc1._ps_native and fc2._ps_native
    assert y.shape == (7, 100, D) and y.dtype == torch.bfloat16
    assert torch.equal(y.view(torch.int16), y_chunks.view(torch.int16)), "chunking changed a value"
    gate, up = fc1(x).chunk(2, -1)
    ref = fc2(F.silu(gate.float()) * up.float())
    hidden = fc1.forward_act(x, "silu_gate")
    assert hidden.dtype == torch.bfloat16 and hidden.shape == (7, 100, H)
    assert_gate_of(hidden.reshape(T, H), fc1(x).reshape(T, 2 * H), "fc1 fused gate")
    ref, yf = ref.float(), y.float()
    rms = ref.pow(2).mean().sqrt().item()
    err = (yf - ref).abs()
    bound = torch.maximum(torch.full_like(ref, 1e-2 * rms), _ulp(ref.double(), torch.bfloat16).float())
    print(f"gated mlp {weight_format}: max|d| = {err.max().item():.3e}, rms = {rms:.3e}, "
          f"{(err > 0).double().mean().item():.2e} of the outputs differ")
    assert torch.all(err <= bound)


def test_forward_act_gate_on_widths_the_epilogue_does_not_pair(gpu):
    """out_features even but not a multiple of 128: the gate runs as the reference's fp32 pass on
    the native linear's output, and the module stays native."""
    D, N = 256, 200
    fc1, _, _ = make_layer(D, N, "int8", {"convrot": True, "convrot_groupsize": 256}, torch.bfloat16, True, gpu, seed=41)
    x = heavy_rows(50, D, seed=42).to(gpu)
    h = fc1.forward_act(x, "silu_gate")
    gate, up = fc1(x).chunk(2, -1)
    assert fc1._ps_native
    assert h.dtype == torch.float32 and torch.equal(h, F.silu(gate.float()) * up.float())
