"""One Wan-14B-shaped block of W8A8 + ConvRot QuantLinears on the heavy-tailed activations of the
40-block benchmark (Student-t df=3, 1% of channels x50): q, k and v on one input (sharing its
quantization, reuse_quantized_inputs), o, then the FFN as the block runs it -- up with the GELU in
its epilogue, down on up's bf16 output -- and a down projection on its own heavy-tailed hidden
input.  Every layer's output is bit-exact with the oracle on sampled rows (int8 codes, int32
accumulators and the epilogue are exact, so any difference is an error)."""
import pytest
import torch
from torch import nn

import oracle
from conftest import heavy_rows, seeded

pytestmark = pytest.mark.gpu

D, F = 5120, 13824
OPTS = {"convrot": True, "convrot_groupsize": 256}


def _layer(K, N, dev, seed):
    from powershard_amd.quant_linear import install_quant_linears, quantized_from_float, pack
    net = nn.Sequential(nn.Linear(K, N)).to(torch.bfloat16)
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    install_quant_linears(net, tensors, "int8", "native", None, torch.bfloat16, dev, quant_options=OPTS)
    layer = net[0]
    g = seeded(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    qt = quantized_from_float(w, "int8_tensorwise", **OPTS)
    layer.qbytes = nn.Parameter(pack(qt, layer._ps_qplan, dev), requires_grad=False)
    b = (torch.randn(N, generator=g) * 0.05).to(torch.bfloat16)
    layer.bias = nn.Parameter(b.to(dev), requires_grad=False)
    return layer, qt, b


def _oracle_rows(x_rows, qt, b):
    qa, sa = oracle.quantize_rows_i8(x_rows, 256)
    return oracle.epilogue_i32(oracle.gemm_i8_i32(qa, qt._qdata.cpu()), sa, qt._params.scale.cpu(), b)


def _check(y, x, qt, b, rows, what):
    ref = _oracle_rows(x[rows], qt, b)
    got = y.cpu()[rows]
    bad = got.view(torch.int16) != ref.view(torch.int16)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} outputs differ"


def test_wan_block_heavy_tailed(gpu):
    from powershard_amd.quant_linear import reuse_quantized_inputs
    M = 384
    x = heavy_rows(M, D, seed=120, outlier_scale=50.0, student_t=True)
    h = heavy_rows(M, F, seed=121, outlier_scale=50.0, student_t=True)
    assert x.float().abs().max() > 200        # the tails and outliers are there
    layers = {name: _layer(K, N, gpu, seed) for name, K, N, seed in
              [("q", D, D, 130), ("k", D, D, 131), ("v", D, D, 132), ("o", D, D, 133), ("up", D, F, 134),
               ("down", F, D, 135)]}
    rows = torch.randperm(M, generator=seeded(136))[:24].sort().values
    xg, hg = x.to(gpu), h.to(gpu)
    with torch.no_grad():
        with reuse_quantized_inputs():
            ys = {name: layers[name][0](xg) for name in ("q", "k", "v")}
        ys["o"] = layers["o"][0](xg)
        hidden = layers["up"][0].forward_act(xg, "gelu_tanh")      # the block's FFN: up + GELU ...
        ys["down_ffn"] = layers["down"][0](hidden)                  # ... then down on its output
        ys["down"] = layers["down"][0](hg)
        ys["up"] = layers["up"][0](xg)
    for name in ("q", "k", "v", "o", "up"):
        _, qt, b = layers[name]
        _check(ys[name], x, qt, b, rows, f"block {name}")
    _, qt, b = layers["down"]
    _check(ys["down"], h, qt, b, rows, "block down (heavy-tailed hidden)")
    _check(ys["down_ffn"], hidden.cpu(), qt, b, rows, "block down on up's GELU output")
    # up's fused epilogue: round(gelu(round(y))) of the plain up output, elementwise
    up_y = ys["up"].cpu()[rows].float()
    ref_gelu = torch.nn.functional.gelu(up_y, approximate="tanh").to(torch.bfloat16).float()
    got_gelu = hidden.cpu()[rows].float()
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref_gelu.abs().clamp(min=2.0 ** -126))) - 7)
    # one output ulp plus 1e-6 absolute: torch's fp32 tanh form cancels in 1 + tanh z below v = -3
    assert torch.all((got_gelu - ref_gelu).abs() <= ulp * 1.0000001 + 1e-6), \
        "fused GELU beyond one bf16 ulp of torch's fp32 form"
