"""psq_gemm_w4a16_noalloc (the entry point that allocates nothing) against psq_gemm_w4a16_ws, the
entry point whose kernels use the same split-K buffer as a caller workspace: two calls in a row
through the C ABI, the second with a smaller problem, each bit-identical to the workspace entry
point's output (same split plan, same summation order) and within the fp32-accumulation bar of
the oracle."""
import ctypes

import pytest
import torch

import oracle
from conftest import heavy_rows, seeded

pytestmark = pytest.mark.gpu


def _call(fn, args, ws=None):
    from powershard_amd import _native
    x, wq, s, z, gs, b, y, M, N, K, st = args
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    head = (P(x), _native.BF16, K, P(wq), P(s), P(z), gs, P(b), _native.BF16, P(y), _native.F32, N, M, N, K)
    rc = fn(*head, st) if ws is None else fn(*head, P(ws), ws.numel(), st)
    assert rc == 0, _native.last_error()


@pytest.mark.parametrize("shapes", [[(128, 25600, 5120), (100, 2048, 2048)]])
def test_noalloc_matches_workspace_entry_point(gpu, shapes):
    from powershard_amd import _native
    lib = _native.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    for M, N, K in shapes:            # second call: a smaller problem than the first
        gs = 128
        need = lib.psq_gemm_wonly_workspace_bytes(_native.W_UINT4, K, M, N, K, gs)
        assert need > 0, "the shape must use the split-K buffer"
        x = heavy_rows(M, K, seed=M + N, outlier_frac=0).to(gpu)
        w = torch.randn(N, K, generator=seeded(N)) * 0.02
        wq, s, z = oracle.quantize_weight_uint4(w, gs)
        wq, s, z = wq.to(gpu), s.to(gpu), z.to(gpu)
        b = (torch.randn(N, generator=seeded(K)) * 0.01).to(torch.bfloat16).to(gpu)
        y_ws = torch.empty(M, N, dtype=torch.float32, device=gpu)
        y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
        ws = torch.zeros(need, dtype=torch.uint8, device=gpu)   # the counter words zero at first use
        _call(lib.psq_gemm_w4a16_ws, (x, wq, s, z, gs, b, y_ws, M, N, K, st), ws)
        _call(lib.psq_gemm_w4a16_noalloc, (x, wq, s, z, gs, b, y_na, M, N, K, st))
        torch.cuda.synchronize()
        assert torch.equal(y_na.view(torch.int32), y_ws.view(torch.int32)), f"{M}x{N}x{K}: outputs differ"
        rows = torch.arange(0, M, max(1, M // 32))
        ref = oracle.gemm_wonly(x.cpu(), oracle.dequant_uint4(wq.cpu(), s.cpu(), z.cpu(), gs), None, b.cpu(),
                                out_dtype=torch.float32, row_ids=rows)
        rms = ref.pow(2).mean().sqrt().item()
        assert (y_na.cpu()[rows] - ref).abs().max().item() <= 1e-2 * rms
