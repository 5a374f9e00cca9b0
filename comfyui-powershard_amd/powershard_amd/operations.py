"""ConvRot int8 helpers and Int8Linear (the ``precision=int8_fp16`` storage).

Mirrors powershard/operations.py:72-191: ``regular_hadamard`` (72-81), ``dequantize_rows``
(84-93), ``Int8Linear`` (96-132), ``install_int8`` (135-155) and ``prepared_linears`` (158-191).  On a GPU the row dequantization
runs the gfx950 kernel (``psq_dequant_i8_rows``: q * s, then the ConvRot inverse by the fast
transform); on the CPU it is the reference's torch formula.

On a gfx950 GPU Int8Linear does not dequantize at all: since the stored weight is W H per ConvRot
group (H symmetric, H H^T = I), x W^T = (x H)(q s)^T, so the forward is the activation rotation
(``psq_rotate_rows``) and the int8 weight-only GEMM (``psq_gemm_w8a16``, q exact in fp16, s in the
epilogue).  The reference's per-tile dequantize + F.linear remains the path on the CPU, in the fp32
island and for shapes the kernels do not take.
"""
from contextlib import contextmanager
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
        from . import ops
        safe = getattr(self, "_ps_safe", False)
        tracker = getattr(self, "_ps_tracker", None)
        x = x.float() if safe else x.half()
        out = None
        finite = False   # out known to be finite
        if not safe and x.device.type == "cuda" and getattr(self, "_ps_native", True):
            out = self._native_forward(x, check=tracker is None)
            # The kernel path rounds x H to fp16, and |x H| reaches sqrt(g) max|x| where coherent
            # activations line up with a row of H; the tile path never forms x H.  A non-finite
            # kernel output is therefore recomputed on the tiles before it is reported or raised.
            # That decision reads the output's flag back (an 8-byte read, a synchronization) on
            # every call, also with a finite tracker attached, whose own checks the reference
            # defers to one read per forward (fp16_safe.py FiniteTracker.finish): the tracker must
            # not see an overflow the tile path would not have produced.
            if out is not None:
                finite = not ops.any_nonfinite(out)
                if not finite:
                    out = None
        if out is None:
            out = torch.empty(x.shape[:-1] + (self.out_features,), dtype=x.dtype, device=x.device)
            prepared = getattr(self, "_ps_prepared", None)
            for a in range(0, self.out_features, self.rows):
                b = min(a + self.rows, self.out_features)
                if prepared is not None and prepared[a // self.rows].dtype == x.dtype:
                    w = prepared[a // self.rows]
                else:
                    w = dequantize_rows(self.weight[a:b], self.weight_scale[a:b], self.convrot, self.group_size,
                                        dtype=torch.float32 if safe else torch.float16, check=tracker is None)
                bias = None if self.bias is None else self.bias[a:b].to(x.dtype)
                out[..., a:b] = F.linear(x, w, bias)
                del w
        if tracker is not None:
            tracker.observe(self._ps_finite_slot, out)
        elif not finite and (ops.any_nonfinite(out) if out.is_cuda else not torch.isfinite(out).all()):
            raise FloatingPointError("NaN/Inf after the INT8 -> FP16 Linear")
        return out


    def _tiled(self):
        """True when the forward dequantizes row tiles (CPU, the fp32 island, the kernels refused)."""
        return getattr(self, "_ps_safe", False) or self.weight.device.type != "cuda" or not getattr(self, "_ps_native", True)

    def _native_forward(self, x, check):
        """fp16 x [..., K] -> fp16 [..., N] on the gfx950 kernels, or None (and the tile path from
        then on) when the kernels do not take the shape.  A missing library raises (as on the tile
        path, whose GPU dequantization is a kernel too).  The dequantized weight's fp16 range check
        of the tile path (dequantize_rows) is kept as a bound, once: every element of (q s) H^T is
        at most sqrt(g) max|q s| in magnitude."""
        from . import ops
        if check and not getattr(self, "_ps_range_ok", False):
            bound = (self.weight.abs().amax(dim=1, keepdim=True).float() * self.weight_scale.float().abs()).max()
            if self.convrot:
                bound = bound * self.group_size ** 0.5
            if not torch.isfinite(bound) or bound > torch.finfo(torch.float16).max:
                self._ps_native = False
                return None
            self._ps_range_ok = True
        rows = x.reshape(-1, self.in_features).contiguous()
        bias = None if self.bias is None else self.bias.to(torch.float16)
        try:
            xr = ops.rotate_rows(rows, self.group_size) if self.convrot else rows
            y = ops.gemm_w8a16(xr, self.weight, self.weight_scale, bias, out_dtype=torch.float16)
        except RuntimeError:
            self._ps_native = False
            return None
        return y.reshape(x.shape[:-1] + (self.out_features,))


def install_int8(model, quant, rows):
    """Replace the Linears named in `quant` ({name: {convrot, group_size}}) by Int8Linear; quantized
    embeddings are left in place and returned ({name: conf}).  Every name is resolved and checked
    before any module is replaced, so a bad entry leaves the model untouched (ValueError)."""
    found = {name: model.get_submodule(name) for name in quant}
    for name, module in found.items():
        if not isinstance(module, (nn.Linear, nn.Embedding)):
            raise ValueError(f"INT8 expects a Linear/Embedding (got {type(module).__name__}): {name}")
    for name, module in found.items():
        if isinstance(module, nn.Linear):
            owner, _, leaf = name.rpartition(".")
            setattr(model.get_submodule(owner) if owner else model, leaf, Int8Linear(module, quant[name], rows))
    return {name: quant[name] for name, module in found.items() if isinstance(module, nn.Embedding)}


@contextmanager
def prepared_linears(modules, budget, enabled=True):
    """Bounded cache of an active MLP's dequantized weight tiles, dropped when the block exits
    (powershard/operations.py:158-191: the reference keeps it for one MLP over its token chunks).

    Only an Int8Linear on the tile path (the CPU, the fp32 island, shapes the kernels refuse) has
    tiles to prepare; on the gfx950 kernel path nothing is dequantized, and other modules are left
    alone.  When ``enabled`` and the tiles' bytes fit ``budget``, each such module's row tiles are
    dequantized once, in the dtype its forward uses, and reused by every forward inside the block:
    the values are those of the per-call tiles.  Yields the reference's report keys.
    """
    tiled = [m for m in modules if isinstance(m, Int8Linear) and m._tiled()]
    elem = {id(m): 4 if getattr(m, "_ps_safe", False) else 2 for m in tiled}
    size = sum(m.in_features * m.out_features * elem[id(m)] for m in tiled)
    staging = max((4 * m.in_features * min(m.rows, m.out_features) for m in tiled), default=0)
    use = bool(enabled and tiled and size + staging <= budget)
    info = dict(prepared_weight_bytes=size if use else 0, preparation_peak_estimate=size + staging if use else 0,
                preparation="active MLP, reused across token chunks" if use else
                "per-call tiles; nothing to prepare, preparation budget insufficient or one chunk")
    try:
        if use:
            for m in tiled:
                dtype = torch.float32 if elem[id(m)] == 4 else torch.float16
                m._ps_prepared = [dequantize_rows(m.weight[a:a + m.rows], m.weight_scale[a:a + m.rows], m.convrot,
                                                  m.group_size, dtype=dtype, check=getattr(m, "_ps_tracker", None) is None)
                                  for a in range(0, m.out_features, m.rows)]
        yield info
    finally:
        for m in modules:
            if hasattr(m, "_ps_prepared"):
                del m._ps_prepared
