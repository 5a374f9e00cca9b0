"""float8_e5m2 weights on the GPU: the decode kernel (psq_dequant_e5m2) bit-exact with the oracle
over all 256 codes, the fp8 GEMM with e5m2 weight codes (psq_gemm_fp8_e5m2w) against the oracle's
exact sum, and an F8_E5M2 comfy_quant module loaded as_file and run natively (its activations
quantized per token to e4m3fn) against the oracle's quantized forward."""
import json

import pytest
import torch
from torch import nn

import oracle
from conftest import heavy_rows, seeded
from test_gpu_kernels import assert_bitexact, assert_fp32_path

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_e5m2_all_codes(gpu, per_row, out_dtype):
    from powershard_amd import ops
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).repeat(24, 2)        # [24, 512], every code
    codes = codes[:, torch.randperm(512, generator=seeded(101))].contiguous()
    s = torch.rand(24, generator=seeded(102)) * 1e-2 + 1e-4 if per_row else torch.tensor(3.3e-3)
    got = ops.dequant_fp8(codes.view(torch.float8_e5m2).to(gpu), s.to(gpu), out_dtype).cpu()
    ref = oracle.dequant_fp8(codes.view(torch.float8_e5m2), s, out_dtype)
    # NaN codes (S.11111.mm, mm != 0) give NaN; their payload bits are not part of the contract
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan) and int(nan.sum()) == 24 * 12
    assert_bitexact(got[~nan], ref[~nan], "e5m2 dequant")


@pytest.mark.parametrize("M,N,K", [(300, 200, 640), (1000, 520, 5120), (17, 33, 128), (129, 777, 1024)])
@pytest.mark.parametrize("per_row", [False, True])
def test_gemm_fp8_e5m2_weights(gpu, M, N, K, per_row):
    from powershard_amd import ops
    x = heavy_rows(M, K, seed=M + 5 * K)
    qa, sa = oracle.quantize_rows_fp8(x)
    w = torch.randn(N, K, generator=seeded(N + 3 * K)) * 0.02
    if per_row:
        ws = w.abs().amax(1) / 57344.0
        qw = (w / ws[:, None]).clamp(-57344, 57344).to(torch.float8_e5m2)
    else:
        qw, ws = oracle.quantize_weight_e5m2(w)
    b = (torch.randn(N, generator=seeded(7)) * 0.01).to(torch.bfloat16)
    args = (qa.view(torch.float8_e4m3fn).to(gpu), sa.to(gpu), qw.to(gpu), ws.to(gpu), b.to(gpu))
    y32 = ops.gemm_fp8(*args, out_dtype=torch.float32)
    yb = ops.gemm_fp8(*args, out_dtype=torch.bfloat16)
    ref32 = oracle.gemm_fp8(qa, sa, qw, ws, b, out_dtype=torch.float32)
    assert_fp32_path(y32, yb, ref32, "fp8 gemm, e5m2 weights")


def test_file_e5m2_module_native(gpu, tmp_path):
    """as_file + native: the module's qbytes hold the file's e5m2 codes; the forward quantizes the
    activations to e4m3fn per token and runs psq_gemm_fp8_e5m2w."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    from powershard_amd import quant_formats as qf
    from powershard_amd import quant_linear as ql
    N, K, M = 384, 1024, 77
    w = torch.randn(N, K, generator=seeded(103)) * 0.02
    q, s = oracle.quantize_weight_e5m2(w)
    bias = (torch.randn(N, generator=seeded(104)) * 0.01).to(torch.bfloat16)
    payload = json.dumps({"format": "float8_e5m2"}).encode()
    path = tmp_path / "e5m2.safetensors"
    save_file({"m.weight": q, "m.weight_scale": s.float(), "m.bias": bias,
               "m.comfy_quant": torch.frombuffer(bytearray(payload), dtype=torch.uint8)}, str(path))
    code = {torch.float32: "F32", torch.bfloat16: "BF16", torch.uint8: "U8", torch.float8_e5m2: "F8_E5M2"}
    with safe_open(str(path), framework="pt") as f:
        table = {k: {"key": k, "dtype": code[f.get_tensor(k).dtype], "shape": list(f.get_tensor(k).shape)}
                 for k in f.keys()}
        qf.annotate_quantized(table, lambda n: json.loads(bytes(f.get_tensor(n).tolist())))
    net = nn.ModuleDict({"m": nn.Linear(K, N).to(torch.bfloat16)})
    report = ql.install_quant_linears(net, table, "as_file", "native", None, torch.bfloat16, gpu)
    layer = net["m"]
    assert report["modules"]["float8_e5m2"]["source"] == {"file": 1}
    with safe_open(str(path), framework="pt") as f:
        full, _ = ql.build_bytes(layer, f, gpu)
    layer.qbytes = nn.Parameter(full, requires_grad=False)
    layer.bias = nn.Parameter(bias.to(gpu), requires_grad=False)
    x = heavy_rows(M, K, seed=105)
    with torch.no_grad():
        y = layer(x.to(gpu))
    assert layer._ps_native
    from powershard_amd import ops
    qa, sa = oracle.quantize_rows_fp8(x)
    ref32 = oracle.gemm_fp8(qa, sa, q, s, bias, out_dtype=torch.float32)
    qx, sx = ops.quantize_rows(x.to(gpu), fp8=True)
    assert_bitexact(qx.view(torch.uint8), qa, "e4m3 activation codes")
    y32 = ops.gemm_fp8(qx, sx, q.to(gpu), s.to(gpu), bias.to(gpu), out_dtype=torch.float32)
    assert_fp32_path(y32, y, ref32, "as_file e5m2 module")
