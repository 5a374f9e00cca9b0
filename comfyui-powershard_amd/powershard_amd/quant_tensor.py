"""Quantized weight container and the three weight layouts of the quantized linear path.

The reference stores weights as ComfyUI ``comfy.quant_ops.QuantizedTensor`` objects -- packed
``_qdata`` plus a ``Params`` dataclass -- and leaves their arithmetic to comfy-kitchen
(powershard/quant_linear.py:53-62, 107-122, 147-152).  This module is that container for this
package: the same ``_qdata`` / ``_layout_cls`` / ``_params`` shape, so QuantPlan / pack / unpack
(powershard/quant_linear.py:38-122) work unchanged, with the layouts defined here:

``int8_tensorwise`` (Int8RowwiseLayout)
    int8 [N, K], fp32 per-row scale [N, 1] (the on-disk ``comfy_quant`` int8 format,
    models/convrot_config.json).  Optional ConvRot: stored q = round(W H / s) per group
    (tests/test_fp16_safe.py:171-174); dequantize = (q s) H^T (powershard/operations.py:84-93).
``float8_e4m3fn`` (Float8ScaledLayout)
    OCP e4m3fn [N, K] with a per-tensor (or per-row) fp32 scale; s = absmax / 448 at
    quantization ("recalculate", powershard/quant_linear.py:147-152; scripts/probe_wan_cuda.py:120-125).
``int4_asym_group`` (UInt4GroupLayout)
    uint4 two per byte [N, K/2] (low nibble = even k), fp16 scale and zero per (row, group of
    ``group_size`` along K): w = (q - z) s.  The reference's int4 target, comfy-kitchen's
    ``convrot_w4a4``, keeps its layout inside comfy-kitchen; this asymmetric group format is
    the one the int4 path here defines and documents.

Weight quantization (``from_float``) is load-time work and runs with torch ops on whatever
device holds the weight.  ``dequantize()`` runs the gfx950 kernels for GPU tensors and torch ops
for CPU tensors (the dequantize compute mode of the reference works on any device).
"""
import dataclasses
import functools

import torch


@functools.lru_cache(maxsize=16)
def _hadamard_cpu(size):
    if size < 4 or size & (size - 1) or (size.bit_length() - 1) % 2:
        raise ValueError("ConvRot group_size must be a power of 4")
    k = (size.bit_length() - 1) // 2
    idx = torch.arange(size)
    sign = torch.zeros(size, size, dtype=torch.int64)
    a, b = idx[:, None].clone(), idx[None, :].clone()
    for _ in range(k):
        sign ^= ((a & 3) + (b & 3) == 3).long()
        a, b = a >> 2, b >> 2
    return (1 - 2 * sign).float() / (2.0 ** k)


def regular_hadamard(size, device="cpu"):
    """ConvRot's regular Hadamard H4^{(x)k} / sqrt(4^k), H4[a][b] = -1 iff a + b == 3
    (powershard/operations.py:72-81), from its closed form over base-4 digits."""
    return _hadamard_cpu(int(size)).to(device)


# ----------------------------------------------------------------------------- params
@dataclasses.dataclass
class Int8RowwiseParams:
    scale: torch.Tensor                  # fp32 [N, 1]
    orig_dtype: torch.dtype = torch.bfloat16
    convrot: bool = False
    convrot_groupsize: int = 256


@dataclasses.dataclass
class Float8ScaledParams:
    scale: torch.Tensor                  # fp32 [] (per tensor) or [N] / [N, 1] (per row)
    orig_dtype: torch.dtype = torch.bfloat16


@dataclasses.dataclass
class UInt4GroupParams:
    scale: torch.Tensor                  # fp16 [N, K / group_size]
    zero: torch.Tensor                   # fp16 [N, K / group_size]
    orig_dtype: torch.dtype = torch.bfloat16
    group_size: int = 128


class Int8RowwiseLayout:
    name = "Int8RowwiseLayout"
    params_cls = Int8RowwiseParams


class Float8ScaledLayout:
    name = "Float8ScaledLayout"
    params_cls = Float8ScaledParams


class UInt4GroupLayout:
    name = "UInt4GroupLayout"
    params_cls = UInt4GroupParams


LAYOUTS = {cls.name: cls for cls in (Int8RowwiseLayout, Float8ScaledLayout, UInt4GroupLayout)}

# format -> layout and whether the activations are quantized too (W8A8 / FP8) or the GEMM
# is weight-only (W4A16); same keys as ComfyUI's QUANT_ALGOS (powershard/quant_linear.py:58-62, 233).
QUANT_ALGOS = {
    "int8_tensorwise": {"comfy_tensor_layout": "Int8RowwiseLayout", "quantize_input": True},
    "float8_e4m3fn": {"comfy_tensor_layout": "Float8ScaledLayout", "quantize_input": True},
    "float8_e5m2": {"comfy_tensor_layout": "Float8ScaledLayout", "quantize_input": True},
    "int4_asym_group": {"comfy_tensor_layout": "UInt4GroupLayout", "quantize_input": False},
}


def layout_name(fmt):
    if fmt not in QUANT_ALGOS:
        raise ValueError(f"Format {fmt} is not supported by powershard_amd: {sorted(QUANT_ALGOS)}")
    return QUANT_ALGOS[fmt]["comfy_tensor_layout"]


# ------------------------------------------------------------------------ container
class QuantizedWeight:
    """Packed quantized weight: ``_qdata`` + layout class + params (cf. QuantizedTensor)."""

    def __init__(self, qdata, layout, params):
        self._qdata = qdata
        self._layout_cls = LAYOUTS[layout] if isinstance(layout, str) else layout
        self._params = params

    @property
    def shape(self):
        return self.logical_shape()

    def logical_shape(self):
        n, k = self._qdata.shape
        return (n, k * 2) if self._layout_cls is UInt4GroupLayout else (n, k)

    @property
    def device(self):
        return self._qdata.device

    # ---------------------------------------------------------------- dequantize
    def dequantize(self):
        """Full-precision weight [N, K] in params.orig_dtype."""
        p, q = self._params, self._qdata
        dtype = p.orig_dtype
        gpu = q.device.type == "cuda"
        if self._layout_cls is Int8RowwiseLayout:
            group = p.convrot_groupsize if p.convrot else 0
            if gpu:
                from . import ops
                return ops.dequant_i8_rows(q, p.scale, group, out_dtype=dtype)
            w = q.float() * p.scale.float().reshape(-1, 1)
            if group:
                h = regular_hadamard(group, q.device)
                w = (w.reshape(w.shape[0], -1, group) @ h.T).reshape_as(w)
            return w.to(dtype)
        if self._layout_cls is Float8ScaledLayout:
            if gpu:
                from . import ops
                return ops.dequant_fp8(q.view(torch.uint8), p.scale, out_dtype=dtype,
                                       e5m2=q.dtype == torch.float8_e5m2)
            s = p.scale.float()
            w = q.float() * (s.reshape(-1, 1) if s.numel() > 1 else s.reshape(()))
            return w.to(dtype)
        if self._layout_cls is UInt4GroupLayout:
            if gpu:
                from . import ops
                return ops.dequant_uint4(q, p.scale, p.zero, p.group_size, out_dtype=dtype)
            n, k2 = q.shape
            lo, hi = (q & 15).float(), (q >> 4).float()
            qq = torch.stack([lo, hi], -1).reshape(n, k2 * 2)
            g = p.group_size
            s = p.scale.float().repeat_interleave(g, dim=1)
            z = p.zero.float().repeat_interleave(g, dim=1)
            return ((qq - z) * s).to(dtype)
        raise ValueError(f"unknown layout {self._layout_cls}")

    # ---------------------------------------------------------------- quantize
    @classmethod
    def from_float(cls, weight, layout, scale=None, **kw):
        """Quantize a float weight [N, K] into `layout` (load-time, torch ops on weight.device).

        scale: None or "recalculate" re-derive the scale from the weight (the only mode used
        for weights, powershard/quant_linear.py:147-152).  Keyword options: convrot /
        convrot_groupsize (int8), group_size (uint4), fp8_dtype (float8_e4m3fn, the default, or
        float8_e5m2).
        """
        layout = LAYOUTS[layout] if isinstance(layout, str) else layout
        dtype = weight.dtype if weight.is_floating_point() else torch.bfloat16
        w = weight.detach().float()
        if w.dim() != 2:
            raise ValueError("weights must be 2-D [out_features, in_features]")
        n, k = w.shape
        if layout is Int8RowwiseLayout:
            convrot = bool(kw.get("convrot", False))
            group = int(kw.get("convrot_groupsize", 256))
            if convrot:
                if k % group:
                    raise ValueError(f"ConvRot group {group} does not divide in_features {k}")
                h = regular_hadamard(group, w.device)
                w = (w.reshape(n, -1, group) @ h).reshape(n, k)
            s = w.abs().amax(-1, keepdim=True) / 127.0
            s = torch.where(s == 0, torch.ones_like(s), s)
            q = torch.round(w / s).clamp(-127, 127).to(torch.int8)
            return cls(q, layout, Int8RowwiseParams(s.contiguous(), dtype, convrot, group))
        if layout is Float8ScaledLayout:
            code = kw.get("fp8_dtype", torch.float8_e4m3fn)
            if code not in (torch.float8_e4m3fn, torch.float8_e5m2):
                raise ValueError(f"fp8 weights are float8_e4m3fn or float8_e5m2, not {code}")
            top = torch.finfo(code).max            # 448 / 57344
            s = w.abs().amax().clamp(min=1e-12) / top
            q = (w / s).clamp(-top, top).to(code)
            return cls(q, layout, Float8ScaledParams(s.reshape(()).contiguous(), dtype))
        if layout is UInt4GroupLayout:
            group = int(kw.get("group_size", 128))
            if k % group or k % 2:
                raise ValueError(f"uint4 group {group} does not divide in_features {k}")
            g = w.reshape(n, k // group, group)
            mn, mx = g.amin(-1), g.amax(-1)
            s = ((mx - mn) / 15.0).to(torch.float16)
            s = torch.where(s == 0, torch.ones_like(s), s)
            z = (-mn / s.float()).to(torch.float16)
            qv = torch.round(g / s.float().unsqueeze(-1) + z.float().unsqueeze(-1)).clamp(0, 15).to(torch.uint8)
            qv = qv.reshape(n, k)
            packed = (qv[:, 0::2] | (qv[:, 1::2] << 4)).contiguous()
            return cls(packed, layout, UInt4GroupParams(s.contiguous(), z.contiguous(), dtype, group))
        raise ValueError(f"unknown layout {layout}")

    def requantize_from_float(self, weight, scale="recalculate"):
        """Re-quantize a new float weight with this tensor's layout options (LoRA merge,
        powershard/quant_linear.py:155-159)."""
        p = self._params
        if self._layout_cls is Int8RowwiseLayout:
            return QuantizedWeight.from_float(weight, self._layout_cls, scale, convrot=p.convrot,
                                              convrot_groupsize=p.convrot_groupsize)
        if self._layout_cls is UInt4GroupLayout:
            return QuantizedWeight.from_float(weight, self._layout_cls, scale, group_size=p.group_size)
        return QuantizedWeight.from_float(weight, self._layout_cls, scale, fp8_dtype=self._qdata.dtype)

    def __repr__(self):
        return f"QuantizedWeight({self._layout_cls.name}, shape={tuple(self.logical_shape())}, device={self.device})"
