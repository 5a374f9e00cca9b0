"""GPU parity of every kernel in libpsquant against the CPU oracle, through the C ABI wrappers.

Bars:
* quantized activations, scales, int32 accumulators, the int8 epilogue (bf16/f16/f32 outputs)
  and dequantized weights: bit-exact;
* fp32-accumulating GEMMs (fp8 e4m3 MFMA, bf16/f16 MFMA of the weight-only paths), whose
  in-instruction summation is hardware-defined: the fp32 output is within
  max|y - y_ref| <= 1e-2 * rms(y_ref) of the oracle's exactly-summed value; the bf16 output is
  bit-exactly the round-to-nearest-even of the kernel's own fp32 value; and every bf16 element
  that differs from the oracle's bf16 output differs by one ulp, at a value whose exact sum lies
  within the measured fp32 discrepancy of the rounding midpoint (a rounding tie, not an error).
  Where |y| > 2.56 rms one bf16 ulp alone exceeds 1e-2 rms, so a literal bf16-vs-bf16 bar is only
  meaningful with identical summation order, which int8 has and fp32 MFMA paths cannot.
"""
import pytest
import torch

import oracle
from conftest import heavy_rows, seeded

pytestmark = pytest.mark.gpu

TOL = 1e-2   # max-abs error bar, in units of rms(y_ref)


def _bits(t):
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    return t


def assert_bitexact(got, ref, what):
    got, ref = _bits(got.cpu()), _bits(ref.cpu())
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    bad = (got != ref)
    if bad.any():
        idx = bad.nonzero()[:5].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.numel()} elements differ, first at {idx}")


def assert_close_rms(got, ref, what, tol=TOL):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs().max().item()
    rms = ref.pow(2).mean().sqrt().item()
    print(f"{what}: max|d| = {err:.4e}, rms = {rms:.4e}, ratio = {err / max(rms, 1e-30):.3e}")
    assert err <= tol * rms, f"{what}: max|d| {err} > {tol} * rms {rms}"


def _ulp_bf16(v):
    """bf16 ulp at |v| (float64 tensor)."""
    a = v.abs().clamp(min=2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - 7)


def assert_fp32_path(y32, yb, ref32, what, tol=TOL):
    """Parity of an fp32-accumulating GEMM: y32 / yb are the kernel's fp32 and bf16 outputs of the
    same call pattern, ref32 the oracle's fp32 output (exact sum, then the same epilogue)."""
    y32, yb, ref32 = y32.cpu(), yb.cpu(), ref32.cpu()
    assert_close_rms(y32, ref32, what + " (fp32 output)", tol)
    assert_bitexact(yb, y32.to(torch.bfloat16), what + ": bf16 output == RNE(fp32 output)")
    refb = ref32.to(torch.bfloat16)
    diff = (yb.float() - refb.float()).double().abs()
    bad = diff > tol * ref32.pow(2).mean().sqrt().item()
    if bad.any():
        r = ref32.double()[bad]
        u = _ulp_bf16(r)
        assert torch.all(diff[bad] <= u * 1.0000001), f"{what}: a bf16 difference exceeds one ulp"
        mid = (yb.double()[bad] + refb.double()[bad]) / 2
        slack = (y32.double() - ref32.double()).abs().max().item()
        assert torch.all((r - mid).abs() <= slack), f"{what}: a bf16 flip is not a rounding tie"
    print(f"{what}: {int(bad.sum())} bf16 rounding ties of {yb.numel()} outputs")


# --------------------------------------------------------------------- quantization
QUANT_CASES = [
    # (M, K, group, dtype)
    (64, 5120, 256, torch.bfloat16),
    (37, 512, 16, torch.bfloat16),
    (5, 1024, 1024, torch.bfloat16),
    (9, 13824, 256, torch.bfloat16),
    (4, 9216, 1024, torch.float16),
    (3, 64, 0, torch.bfloat16),
    (17, 256, 64, torch.float16),
    (8, 4096, 4, torch.float16),
    (1, 16, 0, torch.bfloat16),
    (300, 2048, 256, torch.bfloat16),
    # two 16-element chunks per thread (K > 8192): the Wan FFN down K, an odd chunk count with a
    # partial last wave, the Qwen3-VL down_proj K, the maximum, just over 16384
    (9, 8208, 16, torch.bfloat16),
    (7, 25600, 256, torch.bfloat16),
    (3, 32768, 1024, torch.float16),
    (5, 16400, 16, torch.bfloat16),
    # more rows than resident workgroups: each workgroup streams several rows
    (20000, 1024, 256, torch.bfloat16),
    (33000, 256, 64, torch.float16),
]


@pytest.mark.parametrize("M,K,g,dtype", QUANT_CASES)
@pytest.mark.parametrize("fp8", [False, True])
def test_quantize_rows_bitexact(gpu, M, K, g, dtype, fp8):
    from powershard_amd import ops
    print(f"quantize_rows fp8={fp8} M={M} K={K} g={g} {dtype}", flush=True)
    x = heavy_rows(M, K, seed=100 + M + K, dtype=dtype, student_t=(K % 3 == 0))
    x[0, : min(K, 32)] = 0  # partial zero row
    if M > 2:
        x[2] = 0            # all-zero row: scale 1, codes 0
    q, s = ops.quantize_rows(x.to(gpu), fp8=fp8, rot_group=g)
    torch.cuda.synchronize()
    rq, rs = (oracle.quantize_rows_fp8 if fp8 else oracle.quantize_rows_i8)(x, g)
    assert_bitexact(s, rs, "scale")
    assert_bitexact(q.view(torch.uint8) if fp8 else q, rq, "codes")


@pytest.mark.parametrize("fp8", [False, True])
def test_quantize_rows_static_scale(gpu, fp8):
    from powershard_amd import ops
    x = heavy_rows(33, 1024, seed=7)
    st = torch.tensor([0.05], dtype=torch.float32)
    q, s = ops.quantize_rows(x.to(gpu), fp8=fp8, rot_group=256, static_scale=st.to(gpu))
    rq, rs = (oracle.quantize_rows_fp8 if fp8 else oracle.quantize_rows_i8)(x, 256, static_scale=0.05)
    assert_bitexact(s, rs, "scale")
    assert_bitexact(q.view(torch.uint8) if fp8 else q, rq, "codes (saturating)")


def test_quantize_rows_strided_input(gpu):
    from powershard_amd import ops
    big = heavy_rows(20, 1536, seed=9)
    x = big[:, 256:1280]          # row stride 1536, 16-byte aligned rows
    q, s = ops.quantize_rows(x.to(gpu), rot_group=256)
    rq, rs = oracle.quantize_rows_i8(x.contiguous(), 256)
    assert_bitexact(q, rq, "codes")
    assert_bitexact(s, rs, "scale")


def test_launch_stream_is_current_stream(gpu):
    """Every launch takes the handle of torch's current stream on the tensor's device (read raw,
    without a torch.cuda.Stream object): the default stream, then a side stream under
    torch.cuda.stream, then the default stream again; and a quantization on the side stream is
    ordered after the side stream's own writes to its input."""
    from powershard_amd import ops
    x = heavy_rows(64, 1024, seed=12).to(gpu)
    assert ops._stream(x).value == (torch.cuda.current_stream(x.device).cuda_stream or None)
    side = torch.cuda.Stream(device=x.device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert ops._stream(x).value == side.cuda_stream
        y = x.clone()
        y.mul_(3.0)                  # on the side stream, just before the launch reads it
        q, s = ops.quantize_rows(y, rot_group=256)
    torch.cuda.current_stream().wait_stream(side)
    assert ops._stream(x).value == (torch.cuda.current_stream(x.device).cuda_stream or None)
    rq, rs = oracle.quantize_rows_i8((x * 3.0).cpu(), 256)
    assert_bitexact(q, rq, "codes on a side stream")
    assert_bitexact(s, rs, "scale on a side stream")


# --------------------------------------------------------------------------- int8
GEMM_CASES = [
    # (M, N, K)
    (256, 256, 128),
    (300, 200, 640),
    (1, 16, 128),
    (513, 777, 1024),
    (1000, 520, 5120),
    (64, 1024, 13824),
]


@pytest.mark.parametrize("M,N,K", GEMM_CASES)
def test_gemm_i8_i32_bitexact(gpu, M, N, K):
    from powershard_amd import ops
    print(f"gemm_i8_i32 M={M} N={N} K={K}", flush=True)
    g = seeded(M * 7 + N)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    if M > 3:
        a[3] = 127                   # extreme row
        w[0] = -127
    c = ops.gemm_i8_i32(a.to(gpu), w.to(gpu))
    assert_bitexact(c, oracle.gemm_i8_i32(a, w), "int32 acc")


@pytest.mark.parametrize("M,N,K", [(300, 200, 640), (1000, 520, 5120), (257, 264, 256), (130, 777, 384), (70, 100, 256)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("with_bias", [True, False])
def test_gemm_i8_epilogue(gpu, M, N, K, out_dtype, with_bias):
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=M + K)
    qa, sa = oracle.quantize_rows_i8(x, 256 if K % 256 == 0 else 0)
    w = (torch.randn(N, K, generator=seeded(N)) * 0.02)
    from powershard_amd.quant_tensor import QuantizedWeight
    qw = QuantizedWeight.from_float(w, "Int8RowwiseLayout")
    b = (torch.randn(N, generator=seeded(N + 1)) * 0.01).to(torch.bfloat16) if with_bias else None
    y = ops.gemm_i8(qa.to(gpu), sa.to(gpu), qw._qdata.to(gpu), qw._params.scale.to(gpu),
                    None if b is None else b.to(gpu), out_dtype=out_dtype)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw._qdata), sa, qw._params.scale, b, out_dtype=out_dtype)
    assert_bitexact(y, ref, "int8 epilogue output")
    assert_close_rms(y, ref, "int8 epilogue")


# Problems with more 256 x 256 tiles than the GPU has CUs: the persistent GEMM runs several tiles
# per workgroup, its loads cross into the next tile, and the epilogue operands rotate through
# their buffers.  K = 128 is shorter than the load lookahead (one tile per workgroup); K = 256 has
# the lookahead start at the very first stage; the 4100 x 4000 tiles are partial on both edges.
PERSISTENT_CASES = [(4100, 4000, 512), (4352, 4352, 256), (4200, 4100, 128), (8200, 2000, 384)]


@pytest.mark.parametrize("M,N,K", PERSISTENT_CASES)
def test_gemm_i8_i32_persistent_bitexact(gpu, M, N, K):
    from powershard_amd import ops
    print(f"gemm_i8_i32 persistent M={M} N={N} K={K}", flush=True)
    g = seeded(M + 3 * N + K)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    c = ops.gemm_i8_i32(a.to(gpu), w.to(gpu))
    assert_bitexact(c, oracle.gemm_i8_i32(a, w), "int32 acc")


@pytest.mark.parametrize("M,N,K", PERSISTENT_CASES[:2])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_gemm_i8_epilogue_persistent(gpu, M, N, K, out_dtype):
    from powershard_amd import ops
    print(f"gemm_i8 persistent M={M} N={N} K={K} {out_dtype}", flush=True)
    g = seeded(M + N)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 0.05 + 1e-3
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 1e-3 + 1e-5
    b = (torch.randn(N, generator=g) * 0.5).to(out_dtype)
    y = ops.gemm_i8(qa.to(gpu), sa.to(gpu), qw.to(gpu), sw.to(gpu), b.to(gpu), out_dtype=out_dtype)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw), sa, sw, b, out_dtype=out_dtype)
    assert_bitexact(y, ref, "int8 epilogue output")


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_i8_epilogue_subnormal(gpu, out_dtype):
    """Scales whose product is an fp32 subnormal: the epilogue keeps subnormals (no flush to zero)
    and rounds them to bf16 as the oracle does."""
    from powershard_amd import ops
    M, N, K = 300, 512, 256
    g = seeded(77)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.full((M,), 1e-38) * (1 + torch.rand(M, generator=g))
    sw = torch.rand(N, generator=g) * 1e-6
    y = ops.gemm_i8(qa.to(gpu), sa.to(gpu), qw.to(gpu), sw.to(gpu), None, out_dtype=out_dtype)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw), sa, sw, None, out_dtype=out_dtype)
    r = ref.float().abs()
    assert ((r != 0) & (r < 2.0 ** -126)).float().mean() > 0.5   # mostly subnormal outputs, not zeros
    assert_bitexact(y, ref, "subnormal epilogue output")


@pytest.mark.parametrize("M,N,K", [(300, 512, 1024), (4100, 4096, 512), (8200, 2048, 768)])
def test_gemm_i8_8wave_matches_gemm_i8(gpu, M, N, K):
    """psq_gemm_i8_8wave, the 8-wave comparison schedule: bit-identical to psq_gemm_i8 (bf16 with
    a bias) and to the oracle, partial row tiles and several tiles per workgroup included."""
    import ctypes
    from powershard_amd import _native
    print(f"gemm_i8_8wave M={M} N={N} K={K}", flush=True)
    g = seeded(M + 5 * N + K)
    qa = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 0.05 + 1e-3
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 1e-3 + 1e-5
    b = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16)
    lib = _native.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    args = [t.to(gpu) for t in (qa, sa, qw, sw, b)]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ys = []
    for fn in (lib.psq_gemm_i8, lib.psq_gemm_i8_8wave):
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        rc = fn(P(args[0]), K, P(args[1]), P(args[2]), K, P(args[3]), P(args[4]), _native.BF16, P(y), _native.BF16,
                N, M, N, K, st)
        assert rc == 0, _native.last_error()
        ys.append(y)
    torch.cuda.synchronize()
    assert_bitexact(ys[1], ys[0].cpu(), "8-wave against 4-wave output")
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qw), sa, sw, b, out_dtype=torch.bfloat16)
    assert_bitexact(ys[1], ref, "8-wave output against the oracle")


# ---------------------------------------------------------------------------- fp8
@pytest.mark.parametrize("M,N,K", [(300, 200, 640), (1000, 520, 5120), (17, 33, 128), (129, 777, 1024),
                                   (4100, 4000, 512), (4352, 4352, 256)])
@pytest.mark.parametrize("per_row", [False, True])
def test_gemm_fp8(gpu, M, N, K, per_row):
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=M + 3 * K)
    qa, sa = oracle.quantize_rows_fp8(x)
    w = torch.randn(N, K, generator=seeded(N + K)) * 0.02
    if per_row:
        ws = w.abs().amax(1) / 448.0
        qw = (w / ws[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    else:
        qw, ws = oracle.quantize_weight_fp8(w)
    b = (torch.randn(N, generator=seeded(5)) * 0.01).to(torch.bfloat16)
    args = (qa.view(torch.float8_e4m3fn).to(gpu), sa.to(gpu), qw.to(gpu), ws.to(gpu), b.to(gpu))
    y32 = ops.gemm_fp8(*args, out_dtype=torch.float32)
    yb = ops.gemm_fp8(*args, out_dtype=torch.bfloat16)
    ref32 = oracle.gemm_fp8(qa, sa, qw.view(torch.uint8), ws, b, out_dtype=torch.float32)
    assert_fp32_path(y32, yb, ref32, "fp8 gemm")


# ------------------------------------------------------------------- weight-only
# M <= 8 with groups of a multiple of 128 runs a decode kernel: the K-split one for M <= 2 and
# 1024 <= K <= 6144 (1 x 2600 x 5120, 2 x 300 x 1280 with per-item scales, 2 x 20000 x 4608 with
# several units per workgroup, 1 x 25600 x 5120), the item-split one otherwise (5 x 200 x 640,
# 4 x 300 x 7168, 8 x 4000 x 6144, 3 x 1000 x 4608).
# M <= 64 runs a weight-streaming kernel (groups of a multiple of 128 and K of 256: the streaming
# one -- its scale / zero tables whole in LDS when K / g is a multiple of 8 up to 40 and M <= 48, in
# blocks of 8 groups for other multiples of 8, per step otherwise; else, with K % 128 == 0, the
# split-K one), the rest the tiled one.  With the package's workspace, a streaming grid of at most
# half the CUs over K >= 8192 runs the tiled kernel's stream-K instead (12 x 600 x 12288,
# 50 x 256 x 8192, 16 x 5120 x 13824, 64 x 1024 x 25600)
@pytest.mark.parametrize("M,N,K,gs", [(512, 384, 1024, 128), (7, 256, 512, 64), (130, 100, 5120, 128),
                                      (64, 1000, 256, 256), (1, 2600, 5120, 128), (16, 513, 1024, 128),
                                      (33, 64, 2048, 64), (65, 300, 1024, 128), (3, 100, 384, 64),
                                      (600, 512, 2048, 256), (300, 768, 320, 64), (1, 256, 192, 64),
                                      (257, 1280, 1024, 512), (2, 300, 1280, 128), (40, 700, 2560, 256),
                                      (64, 129, 640, 128), (17, 1100, 5120, 128), (48, 256, 1536, 384),
                                      (9, 200, 768, 384), (5, 200, 640, 128), (16, 1024, 5120, 128),
                                      (40, 700, 4096, 128), (24, 1300, 2048, 256), (56, 384, 5120, 128),
                                      (12, 600, 12288, 128), (50, 256, 8192, 256), (60, 200, 3072, 256),
                                      (16, 5120, 13824, 128), (64, 1024, 25600, 128), (4, 300, 7168, 128),
                                      (8, 4000, 6144, 128), (3, 1000, 4608, 256), (2, 20000, 4608, 128),
                                      (1, 25600, 5120, 128)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_gemm_w4a16(gpu, M, N, K, gs, xdt):
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=M + N, outlier_frac=0, dtype=xdt)
    w = torch.randn(N, K, generator=seeded(K)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    b = (torch.randn(N, generator=seeded(6)) * 0.01).to(xdt)
    args = (x.to(gpu), wq.to(gpu), s.to(gpu), z.to(gpu), gs, b.to(gpu))
    y32 = ops.gemm_w4a16(*args, out_dtype=torch.float32)
    yb = ops.gemm_w4a16(*args, out_dtype=torch.bfloat16)
    wd = oracle.dequant_uint4(wq, s, z, gs, out_dtype=xdt)
    ref32 = oracle.gemm_wonly(x, wd, None, b, out_dtype=torch.float32)
    assert_fp32_path(y32, yb, ref32, "w4a16 gemm")


@pytest.mark.parametrize("M,N,K", [(32, 1024, 16384), (64, 640, 8192)])
def test_gemm_w4a16_long_k_small_n_both_routes(gpu, M, N, K):
    """A streaming grid of few workgroups over a long K: with the split-K workspace the tiled
    kernel's stream-K takes it, without one (psq_gemm_w4a16) the weight-streaming kernel.  Both
    meet the bar against the oracle and agree with each other within it."""
    import ctypes
    from powershard_amd import _native, ops
    print(f"w4a16 long-K small-N M={M} N={N} K={K}", flush=True)
    gs = 128
    lib = _native.lib()
    assert lib.psq_gemm_wonly_workspace_bytes(_native.W_UINT4, K, M, N, K, gs) > 0, "the shape must split K"
    x = heavy_rows(M, K, seed=M + K, outlier_frac=0)
    w = torch.randn(N, K, generator=seeded(N + 1)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    b = (torch.randn(N, generator=seeded(9)) * 0.01).to(torch.bfloat16)
    xg, wqg, sg, zg, bg = (t.to(gpu) for t in (x, wq, s, z, b))
    y_split = ops.gemm_w4a16(xg, wqg, sg, zg, gs, bg, out_dtype=torch.float32)
    y_stream = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    rc = lib.psq_gemm_w4a16(P(xg), _native.BF16, K, P(wqg), P(sg), P(zg), gs, P(bg), _native.BF16, P(y_stream),
                            _native.F32, N, M, N, K, st)
    assert rc == 0, _native.last_error()
    torch.cuda.synchronize()
    ref = oracle.gemm_wonly(x, oracle.dequant_uint4(wq, s, z, gs), None, b, out_dtype=torch.float32)
    rms = ref.pow(2).mean().sqrt().item()
    for name, y in (("stream-K", y_split), ("streaming", y_stream)):
        assert (y.cpu() - ref).abs().max().item() <= 1e-2 * rms, name
    assert (y_split - y_stream).abs().max().item() <= 1e-2 * rms


@pytest.mark.parametrize("M,N,K", [(1024, 512, 1024), (5, 40, 256), (200, 300, 5120), (1, 1030, 5120),
                                   (48, 256, 1024), (64, 64, 640), (700, 512, 640), (257, 1024, 192)])
def test_gemm_w8a16(gpu, M, N, K):
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=M, outlier_frac=0)
    w = torch.randn(N, K, generator=seeded(N)) * 0.02
    q, s = oracle.quantize_weight_int8(w, False)
    b = (torch.randn(N, generator=seeded(8)) * 0.01).to(torch.bfloat16)
    args = (x.to(gpu), q.to(gpu), s.to(gpu), b.to(gpu))
    y32 = ops.gemm_w8a16(*args, out_dtype=torch.float32)
    yb = ops.gemm_w8a16(*args, out_dtype=torch.bfloat16)
    ref32 = oracle.gemm_wonly(x, q.to(torch.bfloat16), s, b, out_dtype=torch.float32)
    assert_fp32_path(y32, yb, ref32, "w8a16 gemm")


# ---------------------------------------------------------------------- dequantize
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_uint4_bitexact(gpu, out_dtype):
    from powershard_amd import ops
    w = torch.randn(96, 1024, generator=seeded(3)) * 0.05
    wq, s, z = oracle.quantize_weight_uint4(w, 128)
    got = ops.dequant_uint4(wq.to(gpu), s.to(gpu), z.to(gpu), 128, out_dtype)
    assert_bitexact(got, oracle.dequant_uint4(wq, s, z, 128, out_dtype), "uint4 dequant")


@pytest.mark.parametrize("g", [0, 16, 256, 1024])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_dequant_i8_rows_bitexact(gpu, g, out_dtype):
    from powershard_amd import ops
    gen = seeded(5)
    q = torch.randint(-100, 100, (13, 2048), generator=gen, dtype=torch.int8)
    s = torch.rand(13, 1, generator=gen) * 1e-3
    got = ops.dequant_i8_rows(q.to(gpu), s.to(gpu), g, out_dtype)
    assert_bitexact(got, oracle.dequant_i8_rows(q, s, g, out_dtype), "int8 row dequant")
    if g:
        # against the reference formula (dense fp32 matmul with H): equal up to fp32 summation
        # order, then the output rounding
        ref = oracle.dequantize_rows(q, s, True, g, torch.float32)
        rtol = 1e-3 if out_dtype == torch.float16 else 1e-5
        torch.testing.assert_close(got.float().cpu(), ref, rtol=rtol, atol=1e-6)


def test_dequant_fp8_bitexact(gpu):
    from powershard_amd import ops
    w = torch.randn(64, 512, generator=seeded(11))
    q, s = oracle.quantize_weight_fp8(w)
    got = ops.dequant_fp8(q.to(gpu), s.to(gpu), torch.float32)
    assert_bitexact(got, oracle.dequant_fp8(q, s, torch.float32), "fp8 dequant")


# ----------------------------------------------------------------- rotation only
@pytest.mark.parametrize("M,K,g", [(37, 512, 256), (5, 1024, 1024), (9, 256, 4), (3, 320, 16), (2, 4096, 64),
                                   (4, 20480, 256), (6, 768, 0)])
@pytest.mark.parametrize("xdt,odt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.float16, torch.float32), (torch.bfloat16, torch.float16)])
def test_rotate_rows_bitexact(gpu, M, K, g, xdt, odt):
    """x H per group (the quantizer's transform) rounded once to the output dtype."""
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=K + M, dtype=xdt)
    got = ops.rotate_rows(x.to(gpu), g, out_dtype=odt)
    assert_bitexact(got, oracle.rotate_rows(x, g).to(odt), "rotate_rows")
