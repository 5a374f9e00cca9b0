"""ConvRot int8 helpers and the row-tiled Int8Linear (the ``precision=int8_fp16`` storage).

Mirrors powershard/operations.py:72-155: ``regular_hadamard`` (72-81), ``dequantize_rows``
(84-93), ``Int8Linear`` (96-132) and ``install_int8`` (135-155).  On a GPU the row dequantization
runs the gfx950 kernel (``psq_dequant_i8_rows``: q * s, then the ConvRot inverse by the fast
transform); on the CPU it is the reference's torch formula.
"""
from functools import lru_cache

import torch
from torch import nn
from torch.nn import functional as F

from .quant_tensor import regular_hadamard as _hadamard


@lru_cache(maxsize=8)
def regular_hadamard(size, device):
    """ConvRot's regular (non-Sylvester) Hadamard of size 4^k, normalized."""
    return _hadamard(size, device)


def dequantize_rows(q, scales, convrot, group_size, dtype=torch.float16, check=True):
    """w = q * s per row, then (ConvRot) w @ H^T per group; overflow-checked against dtype."""
    if q.numel() == 0:
        return q.to(dtype)  # empty trailing FSDP shard: reshape(0, -1, gs) is invalid
    if q.device.type == "cuda":
        from . import ops
        w = ops.dequant_i8_rows(q, scales, group_size if convrot else 0, out_dtype=torch.float32)
    else:
        w = q.float() * scales.float()
        if convrot:
            h = regular_hadamard(group_size, q.device)
            w = (w.reshape(w.shape[0], -1, group_size) @ h.T).reshape_as(w)
    if check and w.numel() and (not torch.isfinite(w).all() or w.abs().max() > torch.finfo(dtype).max):
        raise FloatingPointError(f"INT8 dequantization exceeds the {dtype} range")
    return w.to(dtype)


class Int8Linear(nn.Module):
    """Linear with int8 weight [N, K] and fp32 row scale [N, 1]; forward dequantizes `rows` output
    rows at a time (``dequant_rows``) and runs F.linear in fp16 (fp32 when ``_ps_safe``)."""

    def __init__(self, src, quant, rows):
        super().__init__()
        self.in_features, self.out_features = src.in_features, src.out_features
        self.weight = nn.Parameter(torch.empty(src.weight.shape, dtype=torch.int8, device="meta"), requires_grad=False)
        self.weight_scale = nn.Parameter(torch.empty((src.out_features, 1), dtype=torch.float32, device="meta"),
                                         requires_grad=False)
        self.bias = src.bias
        self._ps_original_compute_dtype = src.weight.dtype
        self.convrot, self.group_size, self.rows = quant["convrot"], quant["group_size"], rows

    def forward(self, x):
        safe = getattr(self, "_ps_safe", False)
        tracker = getattr(self, "_ps_tracker", None)
        x = x.float() if safe else x.half()
        out = torch.empty(x.shape[:-1] + (self.out_features,), dtype=x.dtype, device=x.device)
        for a in range(0, self.out_features, self.rows):
            b = min(a + self.rows, self.out_features)
            w = dequantize_rows(self.weight[a:b], self.weight_scale[a:b], self.convrot, self.group_size,
                                dtype=torch.float32 if safe else torch.float16, check=tracker is None)
            bias = None if self.bias is None else self.bias[a:b].to(x.dtype)
            out[..., a:b] = F.linear(x, w, bias)
            del w
        if tracker is not None:
            tracker.observe(self._ps_finite_slot, out)
        elif not torch.isfinite(out).all():
            raise FloatingPointError("NaN/Inf after the INT8 -> FP16 Linear")
        return out


def install_int8(model, quant, rows):
    """Replace the Linears named in `quant` ({name: {convrot, group_size}}) by Int8Linear; quantized
    embeddings are left in place and returned."""
    skipped = {}
    for name, conf in quant.items():
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name)
        old = getattr(parent, leaf)
        if isinstance(old, nn.Embedding):
            skipped[name] = conf
            continue
        if not isinstance(old, nn.Linear) or not hasattr(old, "in_features"):
            raise ValueError(f"INT8 expects a Linear/Embedding (got {type(old).__name__}): {name}")
        setattr(parent, leaf, Int8Linear(old, conf, rows))
    return skipped
