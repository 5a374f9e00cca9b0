"""QuantLinear end to end on the GPU: install, pack, forward through the native gfx950 kernels,
checked against the CPU oracle (the module-level counterpart of test_quant_formats_torch.py:80-103
in the reference, which compares QuantLinear with F.linear on the dequantized weight).

* W8A8 (ConvRot and plain): bit-exact with the oracle for bf16 and f16 compute.
* fp8 and int4: the fp32-accumulating bar of test_gpu_kernels (1e-2 rms or one output ulp).
* The dequantize compute mode: equal to F.linear on the oracle-dequantized weight.
* A shape the native kernels do not take warns once, switches the module to dequantize and still
  returns the dequantize result (quant_linear.py:207-215 policy).
"""
import warnings

import pytest
import torch
from torch import nn

import oracle
from conftest import heavy_rows, seeded

pytestmark = pytest.mark.gpu


def make_layer(K, N, weight_format, opts, compute_dtype, native, dev, seed, bias=True, follow_input=False):
    from powershard_amd.quant_linear import install_quant_linears, quantized_from_float, pack
    net = nn.Sequential(nn.Linear(K, N, bias=bias)).to(compute_dtype)
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    install_quant_linears(net, tensors, weight_format, "native" if native else "dequantize", None, compute_dtype,
                          dev, quant_options=opts, follow_input=follow_input)
    layer = net[0]
    g = seeded(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    qt = quantized_from_float(w, layer._ps_qplan.fmt, **opts)
    layer.qbytes = nn.Parameter(pack(qt, layer._ps_qplan, dev), requires_grad=False)
    b = (torch.randn(N, generator=g) * 0.05).to(compute_dtype) if bias else None
    layer.bias = None if b is None else nn.Parameter(b.to(dev), requires_grad=False)
    return layer, qt, b


def within_fp32_bar(y, ref):
    y, ref = y.float().cpu(), ref.float().cpu()
    rms = ref.pow(2).mean().sqrt().item()
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7)
    bound = torch.maximum(torch.full_like(ref, 1e-2 * rms), ulp)
    err = (y - ref).abs()
    assert torch.all(err <= bound), f"max err {err.max().item():.3e} vs rms {rms:.3e}"


@pytest.mark.parametrize("convrot", [True, False])
@pytest.mark.parametrize("compute_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [True, False])
def test_w8a8_quantlinear_bitexact(gpu, convrot, compute_dtype, bias):
    K, N = 1024, 768
    opts = {"convrot": convrot, "convrot_groupsize": 256} if convrot else {"convrot": False}
    layer, qt, b = make_layer(K, N, "int8", opts, compute_dtype, True, gpu, seed=11, bias=bias)
    x = heavy_rows(2 * 77, K, seed=12, dtype=compute_dtype).reshape(2, 77, K)   # leading dims flatten
    with warnings.catch_warnings():
        warnings.simplefilter("error")      # the native path must not fall back
        y = layer(x.to(gpu))
    assert layer._ps_native and y.shape == (2, 77, N) and y.dtype == compute_dtype
    qa, sa = oracle.quantize_rows_i8(x.reshape(-1, K), 256 if convrot else 0)
    p = qt._params
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qt._qdata), sa, p.scale, b, out_dtype=compute_dtype)
    assert torch.equal(y.reshape(-1, N).cpu().view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("weight_format,opts", [("fp8", {}), ("int4", {"group_size": 128})])
@pytest.mark.parametrize("M", [1, 40, 300])
def test_fp8_int4_quantlinear(gpu, weight_format, opts, M):
    K, N = 1024, 640
    layer, qt, b = make_layer(K, N, weight_format, opts, torch.bfloat16, True, gpu, seed=21 + M)
    x = heavy_rows(M, K, seed=22 + M, dtype=torch.bfloat16, outlier_frac=0 if weight_format == "int4" else 0.01)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = layer(x.to(gpu))
    assert layer._ps_native
    p = qt._params
    if weight_format == "fp8":
        qa, sa = oracle.quantize_rows_fp8(x)
        ref = oracle.gemm_fp8(qa, sa, qt._qdata.view(torch.uint8), p.scale, b)
    else:
        wd = oracle.dequant_uint4(qt._qdata, p.scale, p.zero, p.group_size)
        ref = oracle.gemm_wonly(x, wd, None, b)
    within_fp32_bar(y, ref)


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}),
                                                ("fp8", {}), ("int4", {"group_size": 128})])
def test_dequantize_mode_matches_dequantized_linear(gpu, weight_format, opts):
    """compute='dequantize': F.linear(rows, qt.dequantize().to(dtype), bias) (quant_linear.py:219-220),
    with the GPU decoders bit-identical to the oracle's, so the torch GEMM sees the same weight."""
    K, N, M = 512, 384, 70
    layer, qt, b = make_layer(K, N, weight_format, opts, torch.bfloat16, False, gpu, seed=31)
    x = heavy_rows(M, K, seed=32, dtype=torch.bfloat16)
    y = layer(x.to(gpu))
    assert not layer._ps_native
    p = qt._params
    if weight_format == "int8":
        wd = oracle.dequant_i8_rows(qt._qdata, p.scale, 256, out_dtype=torch.bfloat16)
    elif weight_format == "fp8":
        wd = oracle.dequant_fp8(qt._qdata.view(torch.uint8), p.scale, out_dtype=torch.bfloat16)
    else:
        wd = oracle.dequant_uint4(qt._qdata, p.scale, p.zero, p.group_size, out_dtype=torch.bfloat16)
    ref = torch.nn.functional.linear(x.to(gpu), wd.to(gpu), b.to(gpu))
    assert torch.equal(y, ref)


def test_unsupported_shape_warns_and_dequantizes(gpu):
    """K = 960 quantizes but is not a whole number of 128-byte GEMM stages: the native GEMM reports
    PSQ_E_SHAPE -> RuntimeError -> one warning, the module switches to dequantize for good."""
    K, N, M = 960, 256, 33
    layer, qt, b = make_layer(K, N, "int8", {"convrot": False}, torch.bfloat16, True, gpu, seed=41)
    x = heavy_rows(M, K, seed=42, dtype=torch.bfloat16)
    with pytest.warns(UserWarning, match="switches to dequantize"):
        y = layer(x.to(gpu))
    assert not layer._ps_native
    wd = oracle.dequant_i8_rows(qt._qdata, qt._params.scale, 0, out_dtype=torch.bfloat16)
    ref = torch.nn.functional.linear(x.to(gpu), wd.to(gpu), b.to(gpu))
    assert torch.equal(y, ref)
    with warnings.catch_warnings():
        warnings.simplefilter("error")      # no second warning
        layer(x.to(gpu))


def test_follow_input_returns_input_dtype(gpu):
    """Text-encoder install (follow_input=True, native_te.py:370-372): an fp32 graph gets fp32 back,
    computed by the bf16 native path (quant_linear.py:221-223)."""
    K, N, M = 512, 256, 9
    layer, qt, b = make_layer(K, N, "int8", {"convrot": True, "convrot_groupsize": 256}, torch.bfloat16, True, gpu,
                              seed=51, follow_input=True)
    x = heavy_rows(M, K, seed=52).float()
    y = layer(x.to(gpu))
    assert y.dtype == torch.float32 and layer._ps_native
    qa, sa = oracle.quantize_rows_i8(x.to(torch.bfloat16), 256)
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qt._qdata), sa, qt._params.scale, b)
    assert torch.equal(y.cpu(), ref.float())


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}), ("fp8", {})])
def test_reuse_quantized_inputs(gpu, weight_format, opts):
    """q, k, v on one input inside reuse_quantized_inputs(): one quantize launch, outputs identical
    to the uncached calls; an in-place change of the input, another tensor or another stream
    quantizes again."""
    from powershard_amd import ops
    from powershard_amd.quant_linear import reuse_quantized_inputs
    K = 1024
    layers = [make_layer(K, 512, weight_format, opts, torch.bfloat16, True, gpu, seed=40 + i)[0] for i in range(3)]
    x = heavy_rows(300, K, seed=44).to(gpu)
    ref = [l(x) for l in layers]
    name = "quantize_rows_fp8" if weight_format == "fp8" else "quantize_rows_i8"
    with ops.kernel_timer() as ev, reuse_quantized_inputs():
        got = [l(x) for l in layers]
        launches = len(ev.get(name, []))
        x2 = x.clone()
        got2 = layers[0](x2)                 # another tensor with equal values
        x.mul_(2.0)                          # in place: version bump
        got3 = layers[0](x)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            got4 = layers[1](x)
        torch.cuda.current_stream().wait_stream(side)
        total = len(ev.get(name, []))
    assert launches == 1, launches
    assert total == 4, total
    for a, b in zip(got, ref):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(got2.view(torch.int16), ref[0].view(torch.int16))
    # under inference_mode (no version counter) the three calls still share one quantization
    with torch.inference_mode():
        xi = heavy_rows(300, K, seed=45).to(gpu)
        refi = [l(xi) for l in layers]
        with ops.kernel_timer() as ev, reuse_quantized_inputs():
            goti = [l(xi) for l in layers]
        assert len(ev.get(name, [])) == 1
        for a, b in zip(goti, refi):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with torch.no_grad():
        assert torch.equal(got3.view(torch.int16), layers[0](x).view(torch.int16))
        assert torch.equal(got4.view(torch.int16), layers[1](x).view(torch.int16))


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}),
                                                ("fp8", {}), ("int4", {"group_size": 128})])
def test_empty_batch_stays_native(gpu, weight_format, opts):
    """An empty token batch (empty tensors have null data pointers) is a no-op for every kernel:
    the module returns [0, N] (and [0, N / 2] for the gate) and keeps its native path."""
    layer, _, _ = make_layer(256, 256, weight_format, opts, torch.bfloat16, True, gpu, seed=81)
    x = torch.empty(0, 256, dtype=torch.bfloat16, device=gpu)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = layer(x)
        assert y.shape == (0, 256) and layer._ps_native
        if weight_format != "int4":
            assert layer.forward_act(x, "gelu_tanh").shape == (0, 256)
            assert layer.forward_act(x, "silu_gate").shape == (0, 128)
        y3 = layer(torch.empty(2, 0, 256, dtype=torch.bfloat16, device=gpu))
        assert y3.shape == (2, 0, 256) and layer._ps_native
    torch.cuda.synchronize()


def test_empty_batch_int8linear_stays_on_the_kernels(gpu):
    from powershard_amd.operations import Int8Linear
    src = torch.nn.Linear(512, 256)
    layer = Int8Linear(src, dict(convrot=True, group_size=256), rows=64).to_empty(device=gpu)
    layer.weight.data.copy_(torch.randint(-127, 128, (256, 512), generator=seeded(82), dtype=torch.int8))
    layer.weight_scale.data.copy_(torch.rand(256, 1, generator=seeded(83)) * 1e-3 + 1e-4)
    layer.bias = torch.nn.Parameter(torch.zeros(256, dtype=torch.float16, device=gpu), requires_grad=False)
    y = layer(torch.empty(0, 512, dtype=torch.float16, device=gpu))
    torch.cuda.synchronize()
    assert y.shape == (0, 256) and getattr(layer, "_ps_native", True)


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 256}),
                                                ("fp8", {}), ("int4", {"group_size": 128})])
def test_strided_inputs_stay_native(gpu, weight_format, opts):
    """Row slices, offset views and broadcast rows reach the kernels as packed copies: the same
    output as the contiguous input, bit for bit, and the module keeps its native path."""
    layer, _, _ = make_layer(256, 384, weight_format, opts, torch.bfloat16, True, gpu, seed=91)
    wide = heavy_rows(64, 300, seed=92).to(gpu)
    flat = wide.reshape(-1)
    inputs = [wide[:, :256], flat[1:1 + 48 * 256].view(48, 256), wide[0, :256].expand(7, 256)]
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        for x in inputs:
            y = layer(x)
            ref = layer(x.contiguous().clone())
            assert layer._ps_native
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
