import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "comfyui-powershard_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libpsquant.so")


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 with the native library loaded (fails loudly if the library is missing)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from powershard_amd import _native, ops
    _native.lib()
    dev = torch.device("cuda:0")
    assert ops.device_supported(dev), f"{torch.cuda.get_device_name(dev)} is not gfx950"
    return dev


def seeded(seed):
    import torch
    return torch.Generator().manual_seed(seed)


def heavy_rows(M, K, seed, outlier_frac=0.01, outlier_scale=20.0, dtype=None, student_t=False):
    """Activations: N(0,1) (or Student-t df=3) with a fraction of channels scaled (outliers)."""
    import torch
    dtype = dtype or torch.bfloat16
    g = seeded(seed)
    x = torch.randn(M, K, generator=g)
    if student_t:
        chi = sum(torch.randn(M, K, generator=g) ** 2 for _ in range(3)) / 3.0
        x = x / chi.sqrt()
    n_out = int(outlier_frac * K)
    if n_out:
        idx = torch.randperm(K, generator=g)[:n_out]
        x[:, idx] *= outlier_scale
    return x.to(dtype)
