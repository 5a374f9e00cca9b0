"""Int8Linear (the ``precision=int8_fp16`` storage, powershard/operations.py:96-132) on the gfx950
kernels: the activation rotation and the int8 weight-only GEMM instead of per-tile dequantization.

The reference pins this layer against F.linear on the dequantized weight: within 1e-3
(tests/test_portable.py:61-67) and a relative RMS below 2e-3 under scaled fp16
(tests/test_fp16_safe.py:71-85).  The kernel path rounds x H to fp16 where the tile path rounds
(q s) H^T, so the two differ by fp16 rounding only; the test holds both reference bars and the
1e-2 rms max-abs bar against the tile path computed on the same GPU.
"""
import pytest
import torch

from conftest import seeded
from powershard_amd.operations import Int8Linear

pytestmark = pytest.mark.gpu


def make(K, N, convrot, gs, dev, seed, bias=True):
    g = seeded(seed)
    src = torch.nn.Linear(K, N, bias=bias)
    layer = Int8Linear(src, dict(convrot=convrot, group_size=gs), rows=64).to_empty(device=dev)
    layer.weight.data.copy_(torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8))
    layer.weight_scale.data.copy_(torch.rand(N, 1, generator=g) * 1e-3 + 1e-4)
    if bias:
        layer.bias = torch.nn.Parameter((torch.randn(N, generator=g) * 0.01).half().to(dev), requires_grad=False)
    return layer


@pytest.mark.parametrize("convrot,gs", [(True, 256), (False, 256), (True, 64)])
@pytest.mark.parametrize("K,N,lead", [(512, 384, (2, 37)), (1024, 200, (5,)), (5120, 640, (1,))])
def test_int8linear_kernel_path_matches_tile_path(gpu, convrot, gs, K, N, lead):
    layer = make(K, N, convrot, gs, gpu, seed=K + N)
    x = (torch.randn(*lead, K, generator=seeded(7)) * 2).half().to(gpu)
    y = layer(x)
    assert getattr(layer, "_ps_native", True), "the kernel path fell back to tiles"
    assert y.dtype == torch.float16 and y.shape == (*lead, N)
    tiles = make(K, N, convrot, gs, gpu, seed=K + N)
    tiles._ps_native = False
    ref = tiles(x)
    d, r = (y.float() - ref.float()), ref.float()
    rel_rms = (d.pow(2).mean().sqrt() / r.pow(2).mean().sqrt()).item()
    assert rel_rms < 2e-3, rel_rms
    assert d.abs().max().item() <= 1e-2 * r.pow(2).mean().sqrt().item()
    torch.testing.assert_close(y, ref, atol=1e-3 * r.abs().max().item(), rtol=1e-3)


def test_int8linear_range_bound_falls_back(gpu):
    """A weight whose dequantized fp16 range is not provably safe takes the tile path, which raises
    the reference's overflow error (tests/test_portable.py:70-72)."""
    layer = make(256, 64, True, 256, gpu, seed=3)
    layer.weight_scale.data.fill_(1000.0)
    with pytest.raises(FloatingPointError):
        layer(torch.randn(4, 256).half().to(gpu))
    assert layer._ps_native is False


def test_int8linear_unsupported_shape_uses_tiles(gpu):
    """K = 336 is not a whole number of 64-element GEMM stages: the kernel reports a shape error and
    the layer keeps the tile path."""
    layer = make(336, 48, False, 16, gpu, seed=4)
    x = torch.randn(3, 336).half().to(gpu)
    y = layer(x)
    assert layer._ps_native is False
    tiles = make(336, 48, False, 16, gpu, seed=4)
    tiles._ps_native = False
    torch.testing.assert_close(y, tiles(x))


@pytest.mark.parametrize("safe", [False, True])
def test_prepared_linears_on_the_gpu_tile_path(gpu, safe):
    """operations.py:158-191 on the GPU: Int8Linear on its tile path (the fp32 island, or the kernels
    switched off) dequantizes its tiles once per MLP through the dequant kernel; the outputs equal
    the per-call tiles' bit for bit, and the cache is dropped on exit.  On the kernel path nothing is
    prepared."""
    from powershard_amd import mlp
    from powershard_amd.operations import prepared_linears
    fc1, fc2 = make(512, 256, True, 256, gpu, seed=71), make(256, 128, True, 256, gpu, seed=72)
    for m in (fc1, fc2):
        if safe:
            m._ps_safe, m._ps_fp32 = True, False
        else:
            m._ps_native = False
    x = (torch.randn(300, 512, generator=seeded(73))).half().to(gpu)
    ref = mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=64)
    with prepared_linears((fc1, fc2), budget=1 << 30) as info:
        assert info["prepared_weight_bytes"] == (512 * 256 + 256 * 128) * (4 if safe else 2)
        assert fc1._ps_prepared[0].device.type == "cuda"
    out = mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=64, prepare_budget=1 << 30)
    assert torch.equal(out, ref) and not hasattr(fc1, "_ps_prepared")
    native = make(512, 256, True, 256, gpu, seed=74)
    with prepared_linears((native,), budget=1 << 30) as info:
        assert info["prepared_weight_bytes"] == 0 and not hasattr(native, "_ps_prepared")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,offset", [(1, 0), (7, 1), (8, 0), (9, 3), (1000, 5), ((1 << 20) + 3, 2)])
def test_any_nonfinite_matches_torch(gpu, dtype, n, offset):
    """ops.any_nonfinite (psq_flag_nonfinite: raw-bit test, flag raised to a per-call ticket) against
    `not torch.isfinite(t).all()`: all-finite tensors with the type's largest finite values and its
    subnormals, then one NaN, +Inf or -Inf at the first element, the middle one or the last, with a
    finite call after each (the flag is never cleared; the ticket tells the calls apart), on views
    that start off a 16-byte boundary."""
    from powershard_amd import ops
    g = seeded(n + offset)
    base = (torch.randn(n + offset, generator=g) * 10).to(dtype).to(gpu)
    t = base[offset:]
    fi = torch.finfo(dtype)
    t[0] = fi.max
    t[-1] = -fi.max
    if n > 2:
        t[n // 2] = fi.tiny / 4 if dtype != torch.float32 else fi.tiny / 8   # subnormal
    assert not ops.any_nonfinite(t) and bool(torch.isfinite(t).all())
    for pos in sorted({0, n // 2, n - 1}):
        for bad in (float("nan"), float("inf"), float("-inf")):
            keep = t[pos].item()
            t[pos] = bad
            assert ops.any_nonfinite(t), (pos, bad)
            t[pos] = keep
            assert not ops.any_nonfinite(t), (pos, bad, "after")
