"""GPU parity cases beyond the per-kernel suite: the reference's own QuantLinear criterion, the
weight-only kernels at the text-encoder MLP shape 512 x 5120 -> 25600 (their 256-row tile instantiation), the on-disk
int8 ConvRot module through the kernels, NaN rows, and the dequantize kernels at K = 25600.

* ``test_native_matches_dequantize_branch``: the reference checks QuantLinear against
  F.linear(x, qt.dequantize()) (tests/test_quant_formats_torch.py:80-103).  W4A16 quantizes no
  activations, so the native output meets 1e-2 rms of that directly (or differs by one bf16 ulp, a
  rounding tie of two fp32 sums).  W8A8 and FP8 quantize the activations per token, so their
  difference from the dequantize branch is the activation quantization error; it is checked against
  the bound that error allows, computed in float64 per output (no oracle involved):
  sum_k |dx_k| |w_k| with |dx_k| <= s_a / 2 (int8 codes) or 2^-4 |x_k| + 2^-10 s_a (e4m3), plus the
  bf16 rounding of the dequantized weight (2^-8 relative) and of both outputs (half an ulp each).
"""
import json
import os

import pytest
import torch
from torch import nn

import oracle
from conftest import heavy_rows, seeded
from test_gpu_kernels import assert_bitexact, assert_fp32_path

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _layer(K, N, weight_format, opts, dev, seed, compute="native", dtype=torch.bfloat16):
    from powershard_amd.quant_linear import install_quant_linears, quantized_from_float, pack
    net = nn.Sequential(nn.Linear(K, N)).to(dtype)
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    install_quant_linears(net, tensors, weight_format, compute, None, dtype, dev, quant_options=opts)
    layer = net[0]
    g = seeded(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    qt = quantized_from_float(w, layer._ps_qplan.fmt, **opts)
    layer.qbytes = nn.Parameter(pack(qt, layer._ps_qplan, dev), requires_grad=False)
    b = (torch.randn(N, generator=g) * 0.05).to(dtype)
    layer.bias = nn.Parameter(b.to(dev), requires_grad=False)
    return layer, qt, b


def _ulp_bf16(v):
    return torch.pow(2.0, torch.floor(torch.log2(v.abs().clamp(min=2.0 ** -126))) - 7)


# ------------------------------------------------- the reference's QuantLinear criterion
@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}),
                                                ("int8", {"convrot": False}), ("fp8", {}),
                                                ("int4", {"group_size": 128})])
def test_native_matches_dequantize_branch(gpu, weight_format, opts):
    K, N, M = 1024, 512, 300
    layer, qt, b = _layer(K, N, weight_format, opts, gpu, seed=61)
    x = heavy_rows(M, K, seed=62)
    with torch.no_grad():
        y = layer(x.to(gpu)).float().cpu()
        wd = qt.dequantize().to(torch.bfloat16)                              # the dequantize branch's weight
        ref = torch.nn.functional.linear(x.to(gpu), wd.to(gpu), b.to(gpu)).float().cpu()
    assert layer._ps_native
    err = (y - ref).abs()
    rms = ref.pow(2).mean().sqrt().item()
    print(f"{weight_format} {opts}: max|native - dequantize branch| = {err.max().item():.3e}, "
          f"rms err / rms = {(err.pow(2).mean().sqrt() / rms).item():.3e}")
    if weight_format == "int4":
        bound = torch.maximum(torch.full_like(ref, 1e-2 * rms), _ulp_bf16(ref))
    else:
        w64 = qt.dequantize().double().cpu()              # exact dequantized weight (rotated back)
        x64 = x.double()
        if weight_format == "int8":
            g = opts["convrot_groupsize"] if opts.get("convrot") else 0
            _, sa = oracle.quantize_rows_i8(x, g)
            # codes are of u = x H (or x); |du| <= s_a / 2 per element, and with the stored weight
            # q s (= W H) the error of the product is sum_k |du_k| |(q s)_nk|
            ws = (qt._qdata.double() * qt._params.scale.double()).cpu()
            act = sa.double()[:, None] / 2 * ws.abs().sum(1)[None, :]
        else:
            _, sa = oracle.quantize_rows_fp8(x)
            dx = 2.0 ** -4 * x64.abs() + 2.0 ** -10 * sa.double()[:, None]
            act = dx @ w64.abs().T
        wround = 2.0 ** -8 * (x64.abs() @ w64.abs().T)   # bf16 rounding of the dequantized weight
        acc = K * 2.0 ** -22 * (x64.abs() @ w64.abs().T)  # fp32 accumulation, both paths
        bound = act + wround + acc + (_ulp_bf16(y.double()) + _ulp_bf16(ref.double())) / 2
    bad = err.double() > bound
    assert not bad.any(), f"{int(bad.sum())} outputs exceed the bound; worst excess {(err.double() - bound).max():.3e}"


# ------------------------------------------------------- NaN rows (torch's amax convention)
@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("g", [0, 256])
def test_quantize_nan_row(gpu, fp8, g):
    """A NaN makes its row's scale NaN (codes: the lower bound); other rows are unchanged."""
    from powershard_amd import ops
    x = heavy_rows(6, 1024, seed=63)
    x[3, 77] = float("nan")
    q, s = ops.quantize_rows(x.to(gpu), fp8=fp8, rot_group=g)
    rq, rs = (oracle.quantize_rows_fp8 if fp8 else oracle.quantize_rows_i8)(x, g)
    assert_bitexact(q.view(torch.uint8) if fp8 else q, rq, "codes")
    s = s.cpu()
    assert torch.isnan(s[3]) and torch.isnan(rs[3])
    keep = [0, 1, 2, 4, 5]
    assert_bitexact(s[keep], rs[keep], "scales of the other rows")


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}), ("fp8", {})])
def test_quantlinear_nan_row_propagates(gpu, weight_format, opts):
    """The finite tracker sees a NaN input row as a NaN output row, as with F.linear."""
    layer, _, _ = _layer(512, 256, weight_format, opts, gpu, seed=64)
    x = heavy_rows(8, 512, seed=65)
    x[5, 300] = float("nan")
    with torch.no_grad():
        y = layer(x.to(gpu)).float().cpu()
    assert torch.isnan(y[5]).all()
    assert torch.isfinite(y[[0, 1, 2, 3, 4, 6, 7]]).all()


# ------------------- weight-only GEMMs at the text-encoder MLP shape (256-row tiles)
def _wonly_rows(x, wd, b, rows):
    return oracle.gemm_wonly(x, wd, None, b, out_dtype=torch.float32, row_ids=rows)


def _sample_rows(M, n, seed):
    g = torch.Generator().manual_seed(seed)
    mid = torch.randperm(M - 64, generator=g)[: n - 64] + 32
    return torch.cat([torch.arange(32), mid.sort().values, torch.arange(M - 32, M)])


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N", [25600, 25664])
def test_gemm_w4a16_256_row_tiles(gpu, xdt, N):
    """M = 512 with N >= 25600 has more 128-row tiles (4 x 100) than CUs, so the tiled kernel runs its
    256-row instantiation (its own ring depth and LDS layout); N = 25664 adds a partial column tile.
    K = 512 keeps the oracle quick; every row of a 128-row sample is checked."""
    from powershard_amd import ops
    M, K, gs = 512, 512, 128
    x = heavy_rows(M, K, seed=66, outlier_frac=0, dtype=xdt)
    w = torch.randn(N, K, generator=seeded(67)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    b = (torch.randn(N, generator=seeded(68)) * 0.01).to(xdt)
    args = (x.to(gpu), wq.to(gpu), s.to(gpu), z.to(gpu), gs, b.to(gpu))
    rows = _sample_rows(M, 128, 69)
    y32 = ops.gemm_w4a16(*args, out_dtype=torch.float32).cpu()[rows]
    yb = ops.gemm_w4a16(*args, out_dtype=torch.bfloat16).cpu()[rows]
    wd = oracle.dequant_uint4(wq, s, z, gs, out_dtype=xdt)
    assert_fp32_path(y32, yb, _wonly_rows(x, wd, b, rows), f"w4a16 256-row tiles N={N}")


@pytest.mark.parametrize("N", [16640, 16400])
def test_gemm_w8a16_256_row_tiles(gpu, N):
    """W8A16 at M = 512 with 4 x 65 128-row tiles (> 256 CUs): the 256-row instantiation."""
    from powershard_amd import ops
    M, K = 512, 640
    x = heavy_rows(M, K, seed=70, outlier_frac=0)
    w = torch.randn(N, K, generator=seeded(71)) * 0.02
    q, s = oracle.quantize_weight_int8(w, False)
    b = (torch.randn(N, generator=seeded(72)) * 0.01).to(torch.bfloat16)
    args = (x.to(gpu), q.to(gpu), s.to(gpu), b.to(gpu))
    rows = _sample_rows(M, 128, 73)
    y32 = ops.gemm_w8a16(*args, out_dtype=torch.float32).cpu()[rows]
    yb = ops.gemm_w8a16(*args, out_dtype=torch.bfloat16).cpu()[rows]
    ref = oracle.gemm_wonly(x, q.to(torch.bfloat16), s, b, out_dtype=torch.float32, row_ids=rows)
    assert_fp32_path(y32, yb, ref, f"w8a16 256-row tiles N={N}")


def test_int4_text_encoder_mlp_512x5120x25600(gpu):
    """The text-encoder workload itself: uint4 g128 weights 25600 x 5120, M = 512 prompt tokens, through the
    QuantLinear module; 256 sampled rows x all 25600 columns against the oracle."""
    from powershard_amd import ops
    M, K, N = 512, 5120, 25600
    layer, qt, b = _layer(K, N, "int4", {"group_size": 128}, gpu, seed=74)
    x = heavy_rows(M, K, seed=75, outlier_frac=0)
    with torch.no_grad():
        yb = layer(x.to(gpu)).cpu()
        p = qt._params
        y32 = ops.gemm_w4a16(x.to(gpu), qt._qdata.to(gpu), p.scale.to(gpu), p.zero.to(gpu), p.group_size,
                             layer.bias, out_dtype=torch.float32).cpu()
    assert layer._ps_native
    rows = _sample_rows(M, 256, 76)
    wd = oracle.dequant_uint4(qt._qdata, p.scale, p.zero, 128, out_dtype=torch.bfloat16)
    ref = _wonly_rows(x, wd, b, rows)
    assert_fp32_path(y32[rows], yb[rows], ref, "W4A16 512x5120->25600")


# ----------------------------------------------- on-disk int8 ConvRot module (comfy_quant)
def test_file_int8_convrot_module_native_bitexact(gpu, tmp_path):
    """An int8_tensorwise ConvRot module as the reference's checkpoints store it -- I8 [N, K] weight,
    F32 [N, 1] weight_scale and the 72-byte comfy_quant payload of models/convrot_config.json --
    loaded with weight_format="as_file" and compute="native", packed by build_bytes onto the GPU,
    and run through the kernels: bit-exact with the oracle's quantized forward
    (powershard/checkpoint.py:63-82, quant_linear.py:407-444)."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    from powershard_amd import quant_formats as qf
    from powershard_amd import quant_linear as ql
    raw = open(os.path.join(GOLDEN, "convrot_config.json"), "rb").read().strip()
    conf = json.loads(raw)
    N, K = 768, 5376                                       # H3 width (21 ConvRot groups)
    w = torch.randn(N, K, generator=seeded(77)) * 0.02
    q, s = oracle.quantize_weight_int8(w, True, 256)
    bias = (torch.randn(N, generator=seeded(78)) * 0.01).to(torch.bfloat16)
    path = tmp_path / "h3_fc.safetensors"
    save_file({"blk.fc.weight": q, "blk.fc.weight_scale": s.float(), "blk.fc.bias": bias,
               "blk.fc.comfy_quant": torch.frombuffer(bytearray(raw), dtype=torch.uint8)}, str(path))
    code = {torch.float32: "F32", torch.bfloat16: "BF16", torch.int8: "I8", torch.uint8: "U8"}
    with safe_open(str(path), framework="pt") as f:
        table = {k: {"key": k, "dtype": code[f.get_tensor(k).dtype], "shape": list(f.get_tensor(k).shape)}
                 for k in f.keys()}
        qf.annotate_quantized(table, lambda n: json.loads(bytes(f.get_tensor(n).tolist())))
    assert table["blk.fc.weight"]["comfy_quant"] == conf
    net = nn.ModuleDict({"blk": nn.ModuleDict({"fc": nn.Linear(K, N).to(torch.bfloat16)})})
    report = ql.install_quant_linears(net, table, "as_file", "native", None, torch.bfloat16, gpu)
    layer = net["blk"]["fc"]
    assert report["modules"]["int8_tensorwise"]["source"] == {"file": 1}
    with safe_open(str(path), framework="pt") as f:
        full, used = ql.build_bytes(layer, f, gpu)
    assert used == {"blk.fc.weight", "blk.fc.weight_scale", "blk.fc.comfy_quant"}
    assert full.device.type == "cuda"
    layer.qbytes = nn.Parameter(full, requires_grad=False)
    layer.bias = nn.Parameter(bias.to(gpu), requires_grad=False)
    x = heavy_rows(96, K, seed=79)
    with torch.no_grad():
        y = layer(x.to(gpu))
    assert layer._ps_native
    qa, sa = oracle.quantize_rows_i8(x, 256)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, q), sa, s, bias)
    assert_bitexact(y, ref, "as_file int8 ConvRot module")


# ------------------------------------------------------------ dequantize at K = 25600
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_dequant_i8_rows_k25600(gpu, out_dtype):
    """Qwen3-VL down_proj width: two 16-value chunks per thread."""
    from powershard_amd import ops
    gen = seeded(80)
    q = torch.randint(-127, 128, (9, 25600), generator=gen, dtype=torch.int8)
    s = torch.rand(9, 1, generator=gen) * 1e-3
    for g in (0, 256, 1024):
        got = ops.dequant_i8_rows(q.to(gpu), s.to(gpu), g, out_dtype)
        assert_bitexact(got, oracle.dequant_i8_rows(q, s, g, out_dtype), f"int8 row dequant K=25600 g={g}")


def test_quantlinear_dequantize_mode_k25600(gpu):
    """compute="dequantize" at K = 25600 runs the row dequantization kernel (ConvRot inverse)."""
    layer, qt, b = _layer(25600, 64, "int8", {"convrot": True, "convrot_groupsize": 256}, gpu, seed=81,
                          compute="dequantize")
    x = heavy_rows(5, 25600, seed=82)
    with torch.no_grad():
        y = layer(x.to(gpu)).cpu()
    wd = oracle.dequant_i8_rows(qt._qdata, qt._params.scale, 256, torch.bfloat16)
    ref = torch.nn.functional.linear(x.to(gpu), wd.to(gpu), b.to(gpu)).cpu()
    assert_bitexact(y, ref, "dequantize mode at K=25600")


# ------------------------------------------------------ Int8Linear with coherent activations
def test_int8linear_coherent_activations_stay_finite(gpu):
    """Activations aligned with a row of H make |x H| = sqrt(g) max|x| (80000 here), beyond fp16: the
    kernel path's rotation overflows, the layer recomputes the call on the row tiles, and the output
    equals the reference tile path's (finite, as the reference's is)."""
    from powershard_amd.operations import Int8Linear
    K, N, g = 512, 64, 256
    gen = seeded(83)

    def make():
        lin = Int8Linear(torch.nn.Linear(K, N), dict(convrot=True, group_size=g), rows=32).to_empty(device=gpu)
        w = torch.randn(N, K, generator=seeded(84)) * 0.02
        q, s = oracle.quantize_weight_int8(w, True, g)
        lin.weight.data.copy_(q)
        lin.weight_scale.data.copy_(s)
        lin.bias = torch.nn.Parameter(torch.zeros(N, dtype=torch.float16, device=gpu), requires_grad=False)
        return lin
    h = oracle.regular_hadamard(g)
    x = torch.randn(4, K, generator=gen).half()
    x[1, :g] = (5000 * 16 * h[7]).half()          # entries +-5000: x H = 80000 e_7 in that group
    kern, tiles = make(), make()
    tiles._ps_native = False
    with torch.no_grad():
        y = kern(x.to(gpu))
        ref = tiles(x.to(gpu))
    assert torch.isfinite(y).all()
    assert_bitexact(y, ref, "Int8Linear recomputed on the tiles")


# ------------------------------------------------------------ split-K of the tiled kernel
def _split_plan(M, N, K, gs, kind=0):
    """Workspace bytes the library asks for (0: no split)."""
    from powershard_amd import _native
    return _native.lib().psq_gemm_wonly_workspace_bytes(kind, K, M, N, K, gs)


@pytest.mark.parametrize("M,N,K,xdt", [(128, 25600, 5120, torch.bfloat16), (100, 2048, 2048, torch.bfloat16),
                                       (77, 1280, 1024, torch.float16), (200, 520, 4096, torch.bfloat16),
                                       (1024, 5120, 5120, torch.bfloat16), (100, 40960, 4096, torch.bfloat16)])
def test_gemm_w4a16_split_k(gpu, M, N, K, xdt):
    """Shapes whose tiles leave CUs idle split K across workgroups (stream-K): each tile's K range
    in a few parts, or equal runs of (tile, K stage) units that cross tile boundaries (1024 x 5120
    x 5120, and 100 x 40960 x 4096 with its one partial row tile); the last workgroup of a tile to
    finish adds the fp32 partials in K order.  Same bar as the unsplit kernel, and repeated calls
    are bit-identical (the order does not depend on which workgroup finishes last)."""
    from powershard_amd import ops
    gs = 128
    assert _split_plan(M, N, K, gs) > 0, "shape expected to split"
    x = heavy_rows(M, K, seed=90 + M, outlier_frac=0, dtype=xdt)
    w = torch.randn(N, K, generator=seeded(91)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    b = (torch.randn(N, generator=seeded(92)) * 0.01).to(xdt)
    args = (x.to(gpu), wq.to(gpu), s.to(gpu), z.to(gpu), gs, b.to(gpu))
    y32 = ops.gemm_w4a16(*args, out_dtype=torch.float32)
    again = [ops.gemm_w4a16(*args, out_dtype=torch.float32) for _ in range(3)]
    for a in again:
        assert torch.equal(a.view(torch.int32), y32.view(torch.int32)), "split-K result changed between calls"
    yb = ops.gemm_w4a16(*args, out_dtype=torch.bfloat16)
    rows = _sample_rows(M, 64, 93) if M > 64 else torch.arange(M)
    wd = oracle.dequant_uint4(wq, s, z, gs, out_dtype=xdt)
    assert_fp32_path(y32.cpu()[rows], yb.cpu()[rows], _wonly_rows(x, wd, b, rows), f"w4a16 split-K {M}x{N}x{K}")


@pytest.mark.parametrize("kind,M,N,K", [("w4", 128, 25600, 5120), ("w4", 1024, 5120, 5120), ("w8", 1024, 5120, 5120),
                                         ("w4", 1, 25600, 5120), ("w4", 5, 25600, 5120)])
def test_gemm_wonly_repeat_bit_identical(gpu, kind, M, N, K):
    """100 calls in a row give bit-identical fp32 outputs: the stream-K shapes of the tiled kernel
    (whose partial tiles once came back stale now and then, 2-20 elements per 48-80 calls, until
    the ordering of their stores and reads was fixed) and the decode kernels (K-split at M = 1,
    item-split at M = 5), whose cross-wave sums are in a fixed order."""
    from powershard_amd import ops
    print(f"repeat {kind} {M}x{N}x{K}", flush=True)
    x = heavy_rows(M, K, seed=98 + M, outlier_frac=0).to(gpu)
    w = torch.randn(N, K, generator=seeded(99)) * 0.02
    b = (torch.randn(N, generator=seeded(100)) * 0.01).to(torch.bfloat16).to(gpu)
    if kind == "w4":
        wq, s, z = oracle.quantize_weight_uint4(w, 128)
        args = (x, wq.to(gpu), s.to(gpu), z.to(gpu), 128, b)
        call = lambda: ops.gemm_w4a16(*args, out_dtype=torch.float32)
    else:
        q, s = oracle.quantize_weight_int8(w, False)
        args = (x, q.to(gpu), s.to(gpu), b)
        call = lambda: ops.gemm_w8a16(*args, out_dtype=torch.float32)
    y0 = call()
    diffs = [int((call().view(torch.int32) != y0.view(torch.int32)).sum()) for _ in range(100)]
    assert sum(diffs) == 0, f"calls differing from the first: {[(i, d) for i, d in enumerate(diffs) if d][:5]}"


@pytest.mark.parametrize("M,N,K", [(200, 1024, 2048), (1024, 5120, 5120), (100, 40960, 4096)])
def test_gemm_w8a16_split_k(gpu, M, N, K):
    """K split across workgroups for the int8 weights: 128-row tiles in K parts (200 x 1024 x 2048)
    and runs of (tile, K stage) units that cross tiles (1024 x 5120 x 5120 and 100 x 40960 x 4096:
    160 tiles each, too many to split in whole parts on 256 CUs)."""
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=94, outlier_frac=0)
    w = torch.randn(N, K, generator=seeded(95)) * 0.02
    q, s = oracle.quantize_weight_int8(w, False)
    b = (torch.randn(N, generator=seeded(96)) * 0.01).to(torch.bfloat16)
    args = (x.to(gpu), q.to(gpu), s.to(gpu), b.to(gpu))
    y32 = ops.gemm_w8a16(*args, out_dtype=torch.float32)
    yb = ops.gemm_w8a16(*args, out_dtype=torch.bfloat16)
    rows = _sample_rows(M, 64, 97)
    ref = oracle.gemm_wonly(x, q.to(torch.bfloat16), s, b, out_dtype=torch.float32, row_ids=rows)
    assert_fp32_path(y32.cpu()[rows], yb.cpu()[rows], ref, f"w8a16 split-K {M}x{N}x{K}")


def _fma_form_weights(wq, s, z, gs, cols, dtype):
    """round_16(fmaf(q, s, -z s)) of weight columns `cols`, as float32 [N, len(cols)]: the per-weight
    arithmetic of the decode, streaming and tiled uint4 kernels.  fmaf is exact in float64 here (q s
    has at most 15 significant bits, -z s is the fp32 product rounded once), then rounded once to
    fp32 and once to the 16-bit type."""
    k = cols.long()
    q = ((wq[:, k // 2].int() >> (4 * (k % 2)).int()) & 15).double()
    sg, zg = s[:, k // gs].float(), z[:, k // gs].float()
    c = -(zg * sg)                                        # fp32 product, rounded once
    return (q * sg.double() + c.double()).float().to(dtype).float()


def _one_hot_case(M, K, xdt, seed=110):
    N, gs = 640, 128
    w = torch.randn(N, K, generator=seeded(seed)) * 0.02
    w[:, :128] *= 1e-3                                    # tiny scales (fp16 subnormal range) in group 0
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    cols = (torch.arange(M) * 37 + 5) % K                 # spread over every group and nibble position
    x = torch.zeros(M, K, dtype=xdt)
    x[torch.arange(M), cols] = 1
    return x, wq, s, z, gs, cols


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(2, 1024), (4, 7168), (4, 1024), (48, 1024), (160, 1024)])
# decode: K-split (M <= 2, 1024 <= K <= 6144) and item-split (the rest); streaming; tiled
def test_w4a16_dequantized_weights_exact(gpu, M, K, xdt):
    """One-hot activation rows make every output one dequantized weight (the MFMA adds zeros to a
    single product), so each kernel's uint4 dequantization -- the nibble as an fp16 subnormal into
    v_fma_mix_f32 -- is checked bit for bit against round_16(fmaf(q, s, -z s))."""
    from powershard_amd import ops
    x, wq, s, z, gs, cols = _one_hot_case(M, K, xdt)
    y = ops.gemm_w4a16(x.to(gpu), wq.to(gpu), s.to(gpu), z.to(gpu), gs, None, out_dtype=torch.float32).cpu()
    want = _fma_form_weights(wq, s, z, gs, cols, xdt).T
    bad = (y != want).sum().item()
    assert bad == 0, f"{bad} of {y.numel()} dequantized weights differ"


def test_w4a16_decode_inf_propagates(gpu):
    """An infinite activation in a decode row (the K-split kernel: M = 2, K = 2048) gives what x @ W^T
    gives with the 16-bit dequantized weights: +-inf where the weight at that k is nonzero (its sign
    times the activation's), NaN where it is zero; the other row stays within the bar."""
    from powershard_amd import ops
    M, N, K, gs = 2, 640, 2048, 128
    x = heavy_rows(M, K, seed=77, outlier_frac=0)
    w = torch.randn(N, K, generator=seeded(78)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    x[1, 700] = float("-inf")
    y = ops.gemm_w4a16(x.to(gpu), wq.to(gpu), s.to(gpu), z.to(gpu), gs, None, out_dtype=torch.float32).cpu()
    wd = oracle.dequant_uint4(wq, s, z, gs, out_dtype=torch.bfloat16).double()
    col = wd[:, 700]
    want = torch.where(col == 0, torch.tensor(float("nan"), dtype=torch.float64),
                       torch.where(col > 0, torch.tensor(float("-inf"), dtype=torch.float64),
                                   torch.tensor(float("inf"), dtype=torch.float64)))
    got = y[1].double()
    assert torch.equal(torch.isnan(got), torch.isnan(want)), "NaN pattern"
    fin = ~torch.isnan(want)
    assert torch.equal(got[fin], want[fin]), "infinities and their signs"
    ref0 = oracle.gemm_wonly(x[:1], oracle.dequant_uint4(wq, s, z, gs, out_dtype=torch.bfloat16), None, None,
                             out_dtype=torch.float32)
    rms = ref0.pow(2).mean().sqrt().item()
    assert (y[:1] - ref0).abs().max().item() <= 1e-2 * rms


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(48, 640, 1024), (160, 640, 1024), (1024, 5120, 5120)])   # skinny; tiled, K in
def test_w8a16_dequantized_weights_exact(gpu, M, N, K, xdt):                                     # parts; stream-K runs
    """One-hot activation rows make every W8A16 output one weight times its row scale, fmaf(q, s, 0)
    rounded once in fp32: pins the int8 -> bf16 conversion and the f16 one (a byte under the
    exponent of 1024, then a packed f16 subtraction of 1152) for every code, -128 included."""
    from powershard_amd import ops
    g = seeded(120)
    q = torch.randint(-128, 128, (N, K), dtype=torch.int16, generator=g).to(torch.int8)
    q[0, :256] = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8)   # every code in row 0
    sc = torch.rand(N, generator=g) * 0.01 + 1e-3
    cols = (torch.arange(M) * 37 + 5) % K
    cols[:min(M, 256)] = torch.arange(min(M, 256))        # row 0's codes reach the outputs
    x = torch.zeros(M, K, dtype=xdt)
    x[torch.arange(M), cols] = 1
    y = ops.gemm_w8a16(x.to(gpu), q.to(gpu), sc.to(gpu), None, out_dtype=torch.float32).cpu()
    want = (q[:, cols].float() * sc[:, None]).T           # one fp32 product each
    bad = (y != want).sum().item()
    assert bad == 0, f"{bad} of {y.numel()} int8 weights differ"


@pytest.mark.parametrize("out_dt,bias_dt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                            (torch.float32, torch.float32)])
def test_gemm_w4a16_split_k_output_layouts(gpu, out_dt, bias_dt):
    """The workgroup that adds up a split tile runs the tiled kernel's epilogue: 16-byte row stores
    when the tile is whole and the rows are aligned, element stores otherwise (the last, partial
    column tile; odd row strides).  Every layout gives the same bits: padded rows (aligned, N not
    a multiple of 4), odd row strides, a bias that starts at an odd element."""
    import ctypes
    from powershard_amd import _native
    M, N, K, gs = 128, 2050, 2048, 128
    assert _split_plan(M, N, K, gs) > 0, "shape expected to split"
    x = heavy_rows(M, K, seed=100, outlier_frac=0).to(gpu)
    w = torch.randn(N, K, generator=seeded(101)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    wq, s, z = wq.to(gpu), s.to(gpu), z.to(gpu)
    bias_store = (torch.randn(N + 1, generator=seeded(102)) * 0.01).to(bias_dt).to(gpu)
    lib = _native.lib()
    nb = lib.psq_gemm_wonly_workspace_bytes(_native.W_UINT4, K, M, N, K, gs)
    ws = torch.zeros(nb, dtype=torch.uint8, device=gpu)   # the counter words zero at first use
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    code = {torch.bfloat16: _native.BF16, torch.float16: _native.F16, torch.float32: _native.F32}

    def run(ldy, bias):
        y = torch.full((M, ldy), float("nan"), dtype=out_dt, device=gpu)
        rc = lib.psq_gemm_w4a16_ws(P(x), _native.BF16, K, P(wq), P(s), P(z), gs, P(bias), code[bias_dt], P(y),
                                   code[out_dt], ldy, M, N, K, P(ws), nb, st)
        assert rc == 0, _native.last_error()
        torch.cuda.synchronize()
        return y[:, :N].cpu()

    bits = lambda t: t.view(torch.uint8)
    aligned = run(N + 2, bias_store[:N])           # padded rows: whole-quad stores, scalar last quad
    for ldy in (N, N + 1):                         # rows not aligned for whole-quad stores
        assert torch.equal(bits(aligned), bits(run(ldy, bias_store[:N]))), f"ldy={ldy}: outputs differ"
    shifted = bias_store[1:]                       # starts at an odd element: read element by element
    assert torch.equal(bits(run(N + 2, shifted)), bits(run(N + 2, shifted.clone()))), "odd bias offset"
    assert torch.count_nonzero(ws[:65536]).item() == 0, "a call left a tile's arrival counter nonzero"
    wd = oracle.dequant_uint4(wq.cpu(), s.cpu(), z.cpu(), gs)
    rows = _sample_rows(M, 32, 103)
    ref = _wonly_rows(x.cpu(), wd, bias_store[:N].cpu(), rows).float()
    err = (aligned[rows].float() - ref).abs()
    bar = torch.maximum(torch.full_like(ref, 1e-2 * ref.pow(2).mean().sqrt().item()), ref.abs() * 2.0 ** -7)
    assert torch.all(err <= bar), f"max err {err.max().item()}"


def test_gemm_w4a16_unsplit_entry_point(gpu):
    """psq_gemm_w4a16 (no workspace) keeps the unsplit kernel; its output meets the same bar."""
    import ctypes
    from powershard_amd import _native
    M, N, K, gs = 128, 2048, 2048, 128
    x = heavy_rows(M, K, seed=98, outlier_frac=0).to(gpu)
    w = torch.randn(N, K, generator=seeded(99)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    wq, s, z = wq.to(gpu), s.to(gpu), z.to(gpu)
    y = torch.empty(M, N, dtype=torch.float32, device=gpu)
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _native.lib().psq_gemm_w4a16(P(x), _native.BF16, K, P(wq), P(s), P(z), gs, None, 0, P(y), _native.F32,
                                      N, M, N, K, st)
    assert rc == 0, _native.last_error()
    ref = oracle.gemm_wonly(x.cpu(), oracle.dequant_uint4(wq.cpu(), s.cpu(), z.cpu(), gs), None, None,
                            out_dtype=torch.float32)
    rms = ref.pow(2).mean().sqrt().item()
    assert (y.cpu() - ref).abs().max().item() <= 1e-2 * rms


# ------------------------------------------------------------ W4A16 decode kernel (M <= 8)
@pytest.mark.parametrize("M,N,K,gs", [(1, 25600, 5120, 128), (2, 2600, 5120, 128), (3, 389, 1024, 256),
                                      (4, 1000, 3072, 128), (1, 130, 25600, 128), (4, 256, 512, 512),
                                      (5, 777, 5120, 128), (8, 25600, 5120, 128), (6, 300, 12800, 256),
                                      (7, 129, 1024, 128), (3, 25600, 6144, 128)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
def test_gemm_w4a16_decode(gpu, M, N, K, gs, xdt):
    """M <= 8 with K % 512 == 0 (the activations fitting in LDS) runs the barrier-free decode kernel
    (activations in LDS, a private weight ring per wave); same bar as the other weight-only paths.
    Each CU takes a range of 16-column units whose items its 8 waves split evenly, and a unit split
    between waves is added up through LDS in a fixed order: N = 25600 (7 units on some CUs), 2600
    (one unit per CU over 8 waves), 389 x 1024 and 129 x 1024 (fewer items than waves: empty runs),
    with the scale / zero tables in LDS or, at K = 6144 (G = 48 > 40) and K = 12800, per-block scale
    loads.  Repeated calls are bit-identical."""
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=110 + M, outlier_frac=0, dtype=xdt)
    w = torch.randn(N, K, generator=seeded(111)) * 0.02
    wq, s, z = oracle.quantize_weight_uint4(w, gs)
    b = (torch.randn(N, generator=seeded(112)) * 0.01).to(xdt)
    args = (x.to(gpu), wq.to(gpu), s.to(gpu), z.to(gpu), gs, b.to(gpu))
    y32 = ops.gemm_w4a16(*args, out_dtype=torch.float32)
    for _ in range(3):
        again = ops.gemm_w4a16(*args, out_dtype=torch.float32)
        assert torch.equal(again.view(torch.int32), y32.view(torch.int32)), "decode result changed between calls"
    yb = ops.gemm_w4a16(*args, out_dtype=torch.bfloat16)
    wd = oracle.dequant_uint4(wq, s, z, gs, out_dtype=xdt)
    assert_fp32_path(y32, yb, oracle.gemm_wonly(x, wd, None, b, out_dtype=torch.float32), f"w4a16 decode {M}x{N}x{K}")

