"""Inputs at the edges of what F.linear accepts, on the native gfx950 path of every format: empty
batches (whose tensors come with null data pointers), rows that are strided, offset from an aligned
base or broadcast (row stride 0), and 3-D inputs.  The kernels take them (the rows are packed first
where they must be), the module stays native, and the outputs equal those of the same rows passed
contiguous."""
import pytest
import torch

from conftest import heavy_rows
from test_gpu_kernels import assert_bitexact
from test_parity_gpu import _layer

pytestmark = pytest.mark.gpu

FORMATS = [("int8", {"convrot": True, "convrot_groupsize": 256}), ("int8", {"convrot": False}), ("fp8", {}),
           ("int4", {"group_size": 128})]


@pytest.mark.parametrize("weight_format,opts", FORMATS)
def test_empty_batches(gpu, weight_format, opts):
    K, N = 512, 384
    layer, _, _ = _layer(K, N, weight_format, opts, gpu, seed=140)
    with torch.no_grad():
        for shape in [(0, K), (2, 0, K), (0, 3, K)]:
            y = layer(torch.empty(shape, dtype=torch.bfloat16, device=gpu))
            assert y.shape == shape[:-1] + (N,) and y.dtype == torch.bfloat16
    assert layer._ps_native


@pytest.mark.parametrize("weight_format,opts", FORMATS)
def test_strided_offset_and_broadcast_rows(gpu, weight_format, opts):
    K, N, M = 1024, 320, 37
    layer, _, _ = _layer(K, N, weight_format, opts, gpu, seed=141)
    x = heavy_rows(M, K, seed=142).to(gpu)
    with torch.no_grad():
        ref = layer(x)
        big = torch.zeros(M, K + 512, dtype=torch.bfloat16, device=gpu)
        big[:, 256:256 + K] = x
        assert_bitexact(layer(big[:, 256:256 + K]), ref, "strided rows")
        flat = torch.zeros(M * K + 3, dtype=torch.bfloat16, device=gpu)
        flat[3:] = x.reshape(-1)
        off = flat[3:].view(M, K)                      # 6 bytes past an aligned base
        assert off.data_ptr() % 16 != 0
        assert_bitexact(layer(off), ref, "rows offset from an aligned base")
        one = x[5:6].expand(M, K)                      # row stride 0
        assert_bitexact(layer(one), ref[5:6].expand(M, N), "broadcast row")
        y3 = layer(x.reshape(1, M, K))
        assert y3.shape == (1, M, N)
        assert_bitexact(y3[0], ref, "3-D input")
    assert layer._ps_native
