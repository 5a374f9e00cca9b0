"""The benchmark workloads at their own full shapes, through the QuantLinear module, checked against
the oracle on sampled rows.

At M = 32760 a persistent workgroup of the int8 / fp8 GEMM walks ~27 output tiles of 40 K stages
each, streaming its LDS ring across the tile boundaries, and the last row tile is partial (32760 =
127 x 256 + 248).  Smaller shapes give every workgroup one tile, so these cases are the only ones
that exercise that regime.  Rows checked: the first 64, 128 spread over the middle, the last 64 (in
the partial tile).

* Wan-14B FFN up projection, W8A8 + ConvRot, 5120 -> 13824, N(0,1) activations with 1% of
  channels x20: int8 codes, scales and the bf16 output bit-exact (the reference's criterion for
  QuantLinear is tests/test_quant_formats_torch.py:80-103; the int8 path is held to exactness).
* Wan-14B fused QKV, fp8 e4m3 weights with a per-tensor scale and per-token e4m3 activations,
  5120 -> 15360: codes and scales bit-exact, the fp32 output within 1e-2 rms of the oracle's exact
  sum, the bf16 output the RNE of the kernel's fp32 output, differences from the oracle's bf16 only
  rounding ties.
* The 40-block Wan stack's heavy-tailed inputs (Student-t df=3, 1% of channels x50): the FFN down
  projection 13824 -> 5120 and the up projection 5120 -> 13824, bit-exact.
"""
import pytest
import torch
from torch import nn

import oracle
from test_gpu_kernels import assert_bitexact, assert_fp32_path

pytestmark = pytest.mark.gpu

M_FULL = 32760


def _sample_rows(M, n, seed):
    """n row indices: the first and last n/4 rows (the edge tiles) and n/2 spread between."""
    e = n // 4
    g = torch.Generator().manual_seed(seed)
    mid = torch.randperm(M - 2 * e, generator=g)[: n - 2 * e] + e
    return torch.cat([torch.arange(e), mid.sort().values, torch.arange(M - e, M)])


def _rows_on_gpu(M, K, seed, dev, outlier_scale, student_t=False):
    """bf16 [M, K] drawn on the GPU: N(0,1) or Student-t (df=3, one normal over the root of a
    chi-square of three), with 1% of the channels (a seeded pick) scaled by outlier_scale."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev)
    if student_t:
        chi = torch.zeros_like(x)
        for _ in range(3):
            chi += torch.randn(M, K, generator=g, device=dev) ** 2
        x /= (chi / 3).sqrt()
        del chi
    idx = torch.randperm(K, generator=torch.Generator().manual_seed(seed + 1))[: int(0.01 * K)].to(dev)
    x[:, idx] *= outlier_scale
    return x.to(torch.bfloat16)


def _layer(K, N, weight_format, opts, dev, seed):
    """A QuantLinear installed and filled through the package's install / pack path."""
    from powershard_amd.quant_linear import install_quant_linears, quantized_from_float, pack
    with torch.device("meta"):
        net = nn.Sequential(nn.Linear(K, N, dtype=torch.bfloat16))
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    install_quant_linears(net, tensors, weight_format, "native", None, torch.bfloat16, dev, quant_options=opts)
    layer = net[0]
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    qt = quantized_from_float(w, layer._ps_qplan.fmt, **opts)
    del w
    layer.qbytes = nn.Parameter(pack(qt, layer._ps_qplan, dev), requires_grad=False)
    b = (torch.randn(N, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    layer.bias = nn.Parameter(b, requires_grad=False)
    return layer, qt, b.cpu()


def _int8_case(gpu, K, N, seed, outlier_scale, student_t, what):
    from powershard_amd import ops
    print(f"{what}: M={M_FULL} K={K} N={N}", flush=True)
    opts = {"convrot": True, "convrot_groupsize": 256}
    layer, qt, b = _layer(K, N, "int8", opts, gpu, seed)
    x = _rows_on_gpu(M_FULL, K, seed + 10, gpu, outlier_scale, student_t)
    with torch.no_grad():
        y = layer(x)
    assert layer._ps_native, f"{what}: the native path fell back"
    rows = _sample_rows(M_FULL, 256, seed + 20)
    x_rows = x[rows.to(gpu)].cpu()
    # the module's own quantizer pass at the full shape, on the sampled rows
    qx, sx = ops.quantize_rows(x, rot_group=256)
    qa, sa = oracle.quantize_rows_i8(x_rows, 256)
    assert_bitexact(qx[rows.to(gpu)], qa, f"{what}: int8 codes")
    assert_bitexact(sx[rows.to(gpu)], sa, f"{what}: row scales")
    ref = oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qt._qdata.cpu()), sa, qt._params.scale.cpu(), b)
    assert_bitexact(y[rows.to(gpu)], ref, f"{what}: bf16 output")


def test_c1_wan_ffn_up_w8a8_convrot_full_m(gpu):
    _int8_case(gpu, 5120, 13824, 7100, 20.0, False, "c1 W8A8+ConvRot 5120->13824")


def test_c4_wan_ffn_down_heavy_tailed_full_m(gpu):
    _int8_case(gpu, 13824, 5120, 7200, 50.0, True, "c4 down 13824->5120 (Student-t, x50)")


def test_c4_wan_ffn_up_heavy_tailed_full_m(gpu):
    _int8_case(gpu, 5120, 13824, 7300, 50.0, True, "c4 up 5120->13824 (Student-t, x50)")


def test_c3_wan_qkv_fp8_full_m(gpu):
    from powershard_amd import ops
    K, N = 5120, 15360
    print(f"c3 fp8 QKV: M={M_FULL} K={K} N={N}", flush=True)
    layer, qt, b = _layer(K, N, "fp8", {}, gpu, 7400)
    x = _rows_on_gpu(M_FULL, K, 7410, gpu, 1.0)
    with torch.no_grad():
        y = layer(x)
    assert layer._ps_native, "c3: the native path fell back"
    rows = _sample_rows(M_FULL, 128, 7420)
    rg = rows.to(gpu)
    qa, sa = oracle.quantize_rows_fp8(x[rg].cpu())
    qx, sx = ops.quantize_rows(x, fp8=True)
    assert_bitexact(qx[rg].view(torch.uint8), qa.view(torch.uint8), "c3: e4m3 codes")
    assert_bitexact(sx[rg], sa, "c3: row scales")
    w_codes, w_scale = qt._qdata, qt._params.scale
    assert w_scale.numel() == 1, "c3 is a per-tensor weight scale"
    y32 = ops.gemm_fp8(qx, sx, w_codes, w_scale, b.to(gpu), out_dtype=torch.float32)
    ref32 = oracle.gemm_fp8(qa, sa, w_codes.cpu().view(torch.uint8), w_scale.cpu(), b, out_dtype=torch.float32)
    assert_fp32_path(y32[rg], y[rg], ref32, "c3 fp8 5120->15360")
