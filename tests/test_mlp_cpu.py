"""The GELU of the fused epilogue and the chunked MLP's host logic, on the CPU.

The GEMM epilogue evaluates gelu_tanh(v) = v / (1 + 2^(v (k0 + k1 v^2))), k0 = -2 sqrt(2/pi) log2 e,
k1 = 0.044715 k0, in fp32 with those two constants rounded to fp32.  That this is the function
torch's F.gelu(approximate="tanh") computes (the reference's call, powershard/wan_model.py:626) is
pinned here against torch itself, in float64 and at the kernel's fp32 constants.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from conftest import seeded
from powershard_amd import mlp
from powershard_amd import quant_linear as ql

K0 = -2.0 * math.sqrt(2.0 / math.pi) * math.log2(math.e)
K1 = K0 * 0.044715


def logistic_form(x, k0, k1):
    return x / (1.0 + np.exp2(x * (k0 + k1 * x * x)))


def test_gelu_logistic_form_is_torch_gelu_tanh():
    x = np.linspace(-6.0, 6.0, 24001)
    ours = logistic_form(x, K0, K1)
    ref = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.max(np.abs(ours - ref)) < 1e-14
    # sign and scale of each constant matter: a flipped sign or a dropped cubic term is far off
    assert np.max(np.abs(logistic_form(x, -K0, K1) - ref)) > 1.0
    assert np.max(np.abs(logistic_form(x, K0, 0.0) - ref)) > 1e-2
    assert np.max(np.abs(F.gelu(torch.from_numpy(x)).numpy() - ref)) > 1e-4   # not the erf GELU


def test_gelu_fp32_constants():
    """The formula at fp32 constants and fp32 arithmetic stays within 2e-6 relative of the exact
    function (the exp2 argument's rounding, amplified by ln 2 |w| <= 16 at v = -4) wherever torch's
    fp32 tanh form is itself accurate."""
    x = np.linspace(-4.0, 8.0, 48001).astype(np.float32)
    k0, k1 = np.float32(K0), np.float32(K1)
    w = (x * ((x * x) * k1 + k0)).astype(np.float32)
    ours = (x / (np.float32(1.0) + np.exp2(w).astype(np.float32))).astype(np.float32)
    exact = F.gelu(torch.from_numpy(x.astype(np.float64)), approximate="tanh").numpy()
    big = np.abs(exact) > 1e-3
    rel = np.abs(ours.astype(np.float64) - exact)[big] / np.abs(exact[big])
    assert rel.max() < 2e-6
    # rounded to bf16 the two agree with torch's own fp32 result except at rare rounding ties
    ours_b = torch.from_numpy(ours).to(torch.bfloat16)
    ref_b = F.gelu(torch.from_numpy(x), approximate="tanh").to(torch.bfloat16)
    assert (ours_b != ref_b).double().mean().item() < 2e-3


def _layer(K, N, weight_format, opts, seed):
    net = nn.Sequential(nn.Linear(K, N)).to(torch.bfloat16)
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    ql.install_quant_linears(net, tensors, weight_format, "dequantize", None, torch.bfloat16, torch.device("cpu"),
                             quant_options=opts)
    layer = net[0]
    g = seeded(seed)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    qt = ql.quantized_from_float(w, layer._ps_qplan.fmt, **opts)
    layer.qbytes = nn.Parameter(ql.pack(qt, layer._ps_qplan, torch.device("cpu")), requires_grad=False)
    layer.bias = nn.Parameter((torch.randn(N, generator=g) * 0.1).to(torch.bfloat16), requires_grad=False)
    return layer


@pytest.mark.parametrize("weight_format,opts", [("int8", {"convrot": True, "convrot_groupsize": 64}),
                                                ("fp8", {}), ("int4", {"group_size": 64})])
def test_forward_act_off_the_native_path_is_the_reference_sequence(weight_format, opts):
    layer = _layer(128, 96, weight_format, opts, seed=3)
    x = torch.randn(2, 5, 128, generator=seeded(4)).to(torch.bfloat16)
    h = layer.forward_act(x)
    assert h.dtype == torch.float32 and h.shape == (2, 5, 96)
    assert torch.equal(h, F.gelu(layer(x).float(), approximate="tanh"))
    with pytest.raises(ValueError):
        layer.forward_act(x, "relu")


def test_chunked_mlp_matches_the_reference_loop():
    """Plain linears: F.gelu(fc1(rows).float()) -> fc2 -> fp32, per chunk (wan_model.py:621-628)."""
    torch.manual_seed(0)
    fc1, fc2 = nn.Linear(64, 160), nn.Linear(160, 48)
    x = torch.randn(3, 41, 64)
    ref = fc2(F.gelu(fc1(x.reshape(-1, 64)).float(), approximate="tanh")).float().reshape(3, 41, 48)
    for chunk in (None, 1, 7, 123, 1000):
        assert torch.allclose(mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=chunk), ref, rtol=0, atol=1e-6)
    assert mlp.chunked_mlp(fc1, fc2, x[:0]).shape == (0, 41, 48)
    with pytest.raises(ValueError):
        mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=-2)


def test_chunked_mlp_with_quant_linears_on_cpu():
    fc1 = _layer(128, 256, "int8", {"convrot": True, "convrot_groupsize": 64}, seed=8)
    fc2 = _layer(256, 128, "int8", {"convrot": True, "convrot_groupsize": 64}, seed=9)
    x = torch.randn(37, 128, generator=seeded(10)).to(torch.bfloat16)
    ref = fc2(F.gelu(fc1(x).float(), approximate="tanh")).float()
    assert torch.equal(mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=16), ref)


def test_silu_logistic_form_is_torch_silu():
    """The epilogue's silu(g) = g / (1 + 2^(-g log2 e)) is torch's F.silu (fp16_safe.py:167)."""
    x = np.linspace(-80.0, 80.0, 32001)
    ours = x / (1.0 + np.exp2(-x * math.log2(math.e)))
    ref = F.silu(torch.from_numpy(x)).numpy()
    assert np.max(np.abs(ours - ref) / np.maximum(np.abs(ref), 1e-300)) < 1e-14
    assert np.max(np.abs(x / (1.0 + np.exp2(x * math.log2(math.e))) - ref)) > 1.0   # sign of the exponent


def test_gated_mlp_matches_the_reference_loop():
    """Plain linears: gate, up = fc1(rows).chunk(2, -1); fc2(F.silu(gate.float()) * up.float())
    per chunk, in x's dtype (fp16_safe.py:126-172)."""
    torch.manual_seed(1)
    fc1, fc2 = nn.Linear(64, 2 * 80), nn.Linear(80, 48)
    x = torch.randn(3, 41, 64)
    gate, up = fc1(x.reshape(-1, 64)).chunk(2, -1)
    ref = fc2(F.silu(gate.float()) * up.float()).reshape(3, 41, 48)
    for chunk in (None, 1, 7, 123, 1000):
        assert torch.allclose(mlp.gated_mlp(fc1, fc2, x, chunk_tokens=chunk), ref, rtol=0, atol=1e-6)
    assert mlp.gated_mlp(fc1, fc2, x[:0]).shape == (0, 41, 48)
    with pytest.raises(ValueError):
        mlp.gated_mlp(fc1, fc2, x, chunk_tokens=0)


def test_gated_mlp_with_quant_linears_on_cpu():
    fc1 = _layer(128, 256, "int8", {"convrot": True, "convrot_groupsize": 64}, seed=11)
    fc2 = _layer(128, 128, "int8", {"convrot": True, "convrot_groupsize": 64}, seed=12)
    x = torch.randn(37, 128, generator=seeded(13)).to(torch.bfloat16)
    h = fc1.forward_act(x, "silu_gate")
    gate, up = fc1(x).chunk(2, -1)
    assert h.dtype == torch.float32 and torch.equal(h, F.silu(gate.float()) * up.float())
    ref = fc2(F.silu(gate.float()) * up.float())
    out = mlp.gated_mlp(fc1, fc2, x, chunk_tokens=16)
    assert out.dtype == torch.bfloat16 and torch.equal(out, ref)
    odd = _layer(128, 95, "int8", {"convrot": True, "convrot_groupsize": 64}, seed=14)
    with pytest.raises(ValueError):
        odd.forward_act(x, "silu_gate")
