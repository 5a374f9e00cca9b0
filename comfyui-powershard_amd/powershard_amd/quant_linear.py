"""QuantLinear: quantized Linear layers stored as one aligned byte vector, computed by the gfx950
kernels of libpsquant (native) or by dequantize + F.linear.

Drop-in for powershard/quant_linear.py (ComfyUI-PowerShard 0.6.0).  What a caller or a state dict
binds to is kept:

* the module and its state dict -- ``QuantLinear(src, plan, compute_dtype, native,
  follow_input, full_precision)`` with a 1-D ``uint8`` parameter ``qbytes`` and ``bias``
  (quant_linear.py:163-189);
* the byte layout of ``QuantPlan`` -- components 16-byte aligned, ``_qdata`` first, then the
  tensor fields of the params dataclass in order, then ``x:<extra>`` (quant_linear.py:27, 38-49,
  65-122), so FSDP can shard and gather ``qbytes`` as plain bytes;
* the compute modes ``native`` / ``dequantize`` / ``auto`` and the fallback convention: a
  native failure of type NotImplementedError / RuntimeError / TypeError / ValueError warns and
  switches the module to dequantize for good; out-of-memory propagates (quant_linear.py:207-215);
* ``install_quant_linears`` / ``build_bytes`` / ``float_weight`` (quant_linear.py:285-444).

Below the module, ComfyUI's QuantizedTensor is replaced by
:class:`~powershard_amd.quant_tensor.QuantizedWeight`, and comfy-kitchen's int8_linear /
torch._scaled_mm / w4a8 ops by the HIP kernels (``native_linear``):

* int8_tensorwise: fused ConvRot + per-token int8 quantize, then the int8 MFMA GEMM with the
  dequant epilogue;
* float8_e4m3fn: per-token e4m3 quantize, then the fp8 MFMA GEMM;
* int4_asym_group: weight-only GEMM with in-register uint4 dequantization (W4A16).
"""
import contextlib
import dataclasses
import itertools
import json
import threading
import warnings
from typing import NamedTuple

import torch
from torch import nn
from torch.nn import functional as F

from . import quant_formats as qf
from . import quant_tensor as qtm

ALIGN = 16
# Extra per-module tensors of ModelOpt/AWQ files: pre_quant_scale multiplies the input,
# input_scale is a static activation scale.  Stored in the same byte vector as "x:<name>".
EXTRAS = ("pre_quant_scale", "input_scale")
# Formats with a native kernel here and the library op that runs them.
NATIVE = {"int8_tensorwise": "gemm_i8", "float8_e4m3fn": "gemm_fp8", "float8_e5m2": "gemm_fp8",
          "int4_asym_group": "gemm_w4a16"}
# The exceptions of a native attempt that switch a module to dequantize (quant_linear.py:207-215).
NATIVE_FAILURES = (NotImplementedError, RuntimeError, TypeError, ValueError)


# ------------------------------------------------------------------- the byte plan
class _Slot(NamedTuple):
    """One component's place in the byte vector (a plain tuple to the plan's readers)."""
    name: str
    dtype: torch.dtype
    shape: tuple
    offset: int
    nbytes: int


def _padded(nbytes):
    return -(-nbytes // ALIGN) * ALIGN


def _byte_view(tensor):
    """The tensor's bytes as a 1-D uint8 view (a contiguous copy first when it is strided)."""
    return tensor.detach().contiguous().view(-1).view(torch.uint8)


@dataclasses.dataclass
class QuantPlan:
    fmt: str
    layout: object
    params_cls: type
    fields: dict         # the params' non-tensor fields (ConvRot, group size, ...)
    specs: list          # [(name, dtype, shape, offset, nbytes)], "_qdata" first
    total: int
    source: dict         # kind=file|quantize, module, key, table, conf

    def signature(self):
        return [(n, str(d), list(s), o, b) for n, d, s, o, b in self.specs]

    @classmethod
    def of(cls, qt, fmt, source, extras=None):
        tensors, fields = components(qt, extras)
        sizes = [t.numel() * t.element_size() for _, t in tensors]
        offsets = itertools.accumulate((_padded(n) for n in sizes), initial=0)
        specs = [_Slot(name, t.dtype, tuple(t.shape), off, n) for (name, t), off, n in zip(tensors, offsets, sizes)]
        end = specs[-1].offset + _padded(specs[-1].nbytes)
        return cls(fmt, qt._layout_cls, type(qt._params), fields, specs, max(end, ALIGN), source)

    def check(self, tensors, fields):
        """RuntimeError when a weight's components or parameters differ from the planned ones."""
        layout = [(name, t.dtype, tuple(t.shape)) for name, t in tensors]
        if layout != [(n, d, tuple(s)) for n, d, s, _, _ in self.specs]:
            raise RuntimeError(f"Layout of {self.fmt} differs from the template: {layout}")
        differ = {k: (fields.get(k), self.fields.get(k)) for k in fields.keys() | self.fields.keys()
                  if not _same_param(fields.get(k), self.fields.get(k))}
        if differ or fields.keys() != self.fields.keys():
            raise RuntimeError(f"Parameters of {self.fmt} differ from the template (the data would decode "
                               f"wrongly): {differ}")

    def to_bytes(self, tensors, device):
        """The byte vector: every component at its offset, zero padding between and after."""
        pieces = []
        for (_, tensor), slot in zip(tensors, self.specs):
            pieces.append(_byte_view(tensor).to(device))
            gap = _padded(slot.nbytes) - slot.nbytes
            if gap:
                pieces.append(torch.zeros(gap, dtype=torch.uint8, device=device))
        out = torch.cat(pieces)
        if out.numel() < self.total:
            out = torch.cat([out, torch.zeros(self.total - out.numel(), dtype=torch.uint8, device=device)])
        return out

    def views(self, full):
        """{name: zero-copy view of its component in `full`}."""
        return {n: full.narrow(0, o, b).view(d).view(s) for n, d, s, o, b in self.specs}


def _same_param(a, b):
    """Equal parameter values; the dtype field (orig_dtype) is set at unpack and never compared."""
    if isinstance(a, torch.dtype) or isinstance(b, torch.dtype):
        return True
    if isinstance(a, (tuple, list)) and isinstance(b, (tuple, list)):
        return list(a) == list(b)
    return a == b


def comfy_quant():
    """The module holding QuantizedWeight / QUANT_ALGOS (ComfyUI's comfy.quant_ops in the reference)."""
    return qtm


def layout_name(fmt):
    return qtm.layout_name(fmt)


def components(qt, extras=None):
    """(tensors in byte-vector order, non-tensor fields): _qdata, the params' tensor fields in
    declaration order, then the extras by name as "x:<name>"."""
    values = {f.name: getattr(qt._params, f.name) for f in dataclasses.fields(qt._params)}
    tensors = [("_qdata", qt._qdata)]
    tensors += [(k, v) for k, v in values.items() if isinstance(v, torch.Tensor)]
    tensors += [("x:" + k, (extras or {})[k]) for k in sorted(extras or {})]
    return tensors, {k: v for k, v in values.items() if not isinstance(v, torch.Tensor)}


def plan_from_quantized(qt, fmt, source, extras=None):
    return QuantPlan.of(qt, fmt, source, extras)


def pack(qt, plan, device, extras=None):
    """One uint8 vector [plan.total] holding every component at its aligned offset."""
    tensors, fields = components(qt, extras)
    plan.check(tensors, fields)
    return plan.to_bytes(tensors, device)


def unpack(full, plan, dtype=None, with_extras=False):
    """Gathered byte vector -> QuantizedWeight of zero-copy views [+ extras]."""
    views = plan.views(full)
    extras = {name[2:]: v for name, v in views.items() if name.startswith("x:")}
    tensor_fields = {name: v for name, v in views.items() if name != "_qdata" and not name.startswith("x:")}
    fields = dict(plan.fields)
    if dtype is not None and "orig_dtype" in fields:
        fields["orig_dtype"] = dtype
    qt = qtm.QuantizedWeight(views["_qdata"], plan.layout, plan.params_cls(**tensor_fields, **fields))
    return (qt, extras) if with_extras else qt


# ------------------------------------------------------------------- file formats
def quantized_from_file(handle, entries, module, conf, shape, device, dtype, meta=False):
    """QuantizedWeight from a module's file tensors.

    entries: name -> file key (or, with meta=True, name -> (torch dtype, shape): a template
    without reading data).  conf: the module's ``comfy_quant`` JSON.  Layouts on disk:
    int8_tensorwise = weight I8 [N, K] + weight_scale F32 [N, 1] (+ convrot,
    convrot_groupsize); float8_e4m3fn / float8_e5m2 = weight F8_E4M3 / F8_E5M2 + weight_scale /
    scale_weight F32 ([] or [N]); int4_asym_group = weight U8 [N, K/2] + weight_scale / weight_zero F16 [N, K/g] (+ group_size).
    """
    prefix = module + "."
    fmt = conf.get("format")
    if meta:
        state = {n: torch.empty(d[1], dtype=d[0], device="meta") for n, d in entries.items()}
    else:
        state = {n: handle.get_tensor(k) for n, k in entries.items()}
    weight = state.get(prefix + "weight")
    if weight is None:
        raise ValueError(f"{module}: no weight in the file entries")
    n, k = int(shape[0]), int(shape[1])
    dev = torch.device("meta") if meta else device
    if fmt == "int8_tensorwise":
        scale = state.get(prefix + "weight_scale")
        if weight.dtype != torch.int8 or scale is None or scale.numel() != n:
            raise ValueError(f"{module}: int8_tensorwise expects I8 [N, K] weight and F32 [N, 1] weight_scale")
        rot = qf.convrot_config(conf, k, module)
        params = qtm.Int8RowwiseParams(scale.to(dev, torch.float32).reshape(n, 1), dtype, rot["convrot"],
                                       rot["group_size"])
        return qtm.QuantizedWeight(weight.to(dev), qtm.Int8RowwiseLayout, params)
    if fmt in ("float8_e4m3fn", "float8_e5m2"):
        code = torch.float8_e4m3fn if fmt == "float8_e4m3fn" else torch.float8_e5m2
        scale = state.get(prefix + "weight_scale", state.get(prefix + "scale_weight"))
        if weight.dtype != code or scale is None:
            raise ValueError(f"{module}: {fmt} expects {'F8_E4M3' if fmt == 'float8_e4m3fn' else 'F8_E5M2'} "
                             "weight and a weight_scale")
        scale = scale.to(dev, torch.float32)
        scale = scale.reshape(()) if scale.numel() == 1 else scale.reshape(n)
        return qtm.QuantizedWeight(weight.to(dev), qtm.Float8ScaledLayout, qtm.Float8ScaledParams(scale, dtype))
    if fmt == "int4_asym_group":
        scale, zero = state.get(prefix + "weight_scale"), state.get(prefix + "weight_zero")
        group = int(qf.conf_value(conf, "group_size", 128))
        if (weight.dtype != torch.uint8 or tuple(weight.shape) != (n, k // 2) or scale is None or zero is None
                or k % group or tuple(scale.shape) != (n, k // group) or tuple(zero.shape) != (n, k // group)):
            raise ValueError(f"{module}: int4_asym_group expects U8 [N, K/2] weight and F16 [N, K/g] scale/zero")
        params = qtm.UInt4GroupParams(scale.to(dev, torch.float16), zero.to(dev, torch.float16), dtype, group)
        return qtm.QuantizedWeight(weight.to(dev), qtm.UInt4GroupLayout, params)
    raise ValueError(f"{module}: format {fmt} is not supported by powershard_amd: {sorted(qtm.QUANT_ALGOS)}")


def quantized_from_float(weight, fmt, **options):
    """Quantize a float weight into `fmt` (scale recomputed from the data, as ComfyUI set_weight)."""
    if fmt == "float8_e5m2":
        options = dict(options, fp8_dtype=torch.float8_e5m2)
    return qtm.QuantizedWeight.from_float(weight, layout_name(fmt), scale="recalculate", **options)


def requantize_like(template, weight, fmt):
    """A new weight (after LoRA) in the template's layout: its ConvRot / group options carry over."""
    again = getattr(template, "requantize_from_float", None)
    return quantized_from_float(weight, fmt) if again is None else again(weight, scale="recalculate")


# ------------------------------------------------------------------------- module
class QuantLinear(nn.Module):
    """Linear whose weight is one QuantizedWeight byte vector (FSDP Shard(0) over bytes)."""

    # attributes the FP16-safe / finite-tracking machinery set on the Linear it replaces
    CARRIED = ("_ps_tracker", "_ps_finite_slot", "_ps_safe", "_ps_fp32")

    def __init__(self, src, plan, compute_dtype, native, follow_input=False, full_precision=False):
        super().__init__()
        self.in_features, self.out_features = src.in_features, src.out_features
        self.qbytes = nn.Parameter(torch.empty(plan.total, dtype=torch.uint8, device="meta"), requires_grad=False)
        self.bias = src.bias
        self._ps_qplan = plan
        self._ps_compute_dtype = compute_dtype
        self._ps_native = native
        self._ps_follow_input = follow_input
        self._ps_full_precision = full_precision  # comfy_quant full_precision_matrix_mult: dequantize only
        for attr in self.CARRIED:
            if hasattr(src, attr):
                setattr(self, attr, getattr(src, attr))

    # ComfyUI model code calls comfy.ops.linear_input_act(linear, x, act); weight=None and
    # comfy_force_forward route it into this forward without reading the packed weight.
    comfy_force_forward = True

    @property
    def weight(self):
        return None

    def extra_repr(self):
        return f"{self.in_features}, {self.out_features}, format={self._ps_qplan.fmt}, native={self._ps_native}"

    def forward(self, x):
        return self._forward(x, None)

    def forward_act(self, x, activation="gelu_tanh"):
        """act(self(x)) with the activation fused into the native GEMM's epilogue.

        "gelu_tanh": the reference applies it outside the linear, F.gelu(fc1(rows).float(),
        approximate="tanh") (powershard/wan_model.py:626).  "silu_gate": gate, up =
        fc1(rows).chunk(2, -1); F.silu(gate.float()) * up.float() (powershard/fp16_safe.py:165-167),
        [..., out_features / 2].  The next QuantLinear casts the fp32 result to its compute dtype
        first (quant_linear.py:197).  On the native W8A8 / FP8 path the result comes back in the
        compute dtype: the values that cast gives, without the fp32 intermediate (the gate fused for
        out_features a multiple of 128).  Elsewhere it is the reference's fp32 expression on the
        forward's output.
        """
        if activation not in ("gelu_tanh", "silu_gate"):
            raise ValueError(f"unsupported activation {activation!r}")
        if activation == "silu_gate" and self.out_features % 2:
            raise ValueError(f"silu_gate needs an even number of output features, got {self.out_features}")
        return self._forward(x, activation)

    # -- the forward in four steps: compute dtype, the native attempt, the dequantize branch, delivery
    def _dtype_for(self, x):
        """The compute dtype; a dequantizing text-encoder module follows a floating input instead."""
        if self._ps_follow_input and not self._ps_native and x.is_floating_point():
            return x.dtype
        return self._ps_compute_dtype

    def _native_attempt(self, rows, qt, bias, extras, activation):
        """(output, activation applied) from the native kernels, or (None, False) to dequantize:
        the FP16-safe mode and full-precision files never go native, and a native failure switches
        the module to dequantize for good with one warning."""
        safe = getattr(self, "_ps_safe", False) and rows.dtype == torch.float16
        if not self._ps_native or safe or self._ps_full_precision:
            return None, False
        # the fused gate pairs 64-column blocks: other widths take the gate as a separate pass
        act = None if activation == "silu_gate" and self.out_features % 128 else activation
        try:
            return native_linear(rows, qt, bias, self._ps_qplan.fmt, extras.get("input_scale"), act), act is not None
        except torch.cuda.OutOfMemoryError:
            raise
        except NATIVE_FAILURES as error:
            warnings.warn(f"PowerShard: native {self._ps_qplan.fmt} GEMM unavailable ({error}); the module "
                          f"switches to dequantize")
            self._ps_native = False
            return None, False

    def _dequantized(self, rows, qt, bias):
        """F.linear on the dequantized weight; the V100 "FP16 safe" mode computes it in fp32."""
        if getattr(self, "_ps_safe", False) and rows.dtype == torch.float16:
            return F.linear(rows.float(), qt.dequantize().float(), None if bias is None else bias.float())
        return F.linear(rows, qt.dequantize().to(rows.dtype), bias)

    def _deliver(self, out, x):
        out = out.reshape(*x.shape[:-1], out.shape[-1])
        if self._ps_follow_input and x.is_floating_point() and out.dtype != x.dtype:
            out = out.to(x.dtype)  # text encoder: the FP32 graph is not narrowed to bf16 by the native kernel
        tracker = getattr(self, "_ps_tracker", None)
        if tracker is not None:
            tracker.observe(self._ps_finite_slot, out)
        return out

    def _forward(self, x, activation):
        dtype = self._dtype_for(x)
        qt, extras = unpack(self.qbytes, self._ps_qplan, dtype, with_extras=True)
        rows = x.reshape(-1, x.shape[-1]).to(dtype)
        pre = extras.get("pre_quant_scale")
        if pre is not None:  # ModelOpt AWQ smoothing
            rows = rows * pre.to(rows.dtype)
        bias = None if self.bias is None else self.bias.to(dtype)
        out, applied = self._native_attempt(rows, qt, bias, extras, activation)
        if out is None:
            out = self._dequantized(rows, qt, bias)
        if activation is not None and not applied:
            out = apply_activation(out, activation)
        return self._deliver(out, x)


# ------------------------------------------------------------------ shared activation quantization
_shared = threading.local()


@contextlib.contextmanager
def reuse_quantized_inputs():
    """Within the block, native W8A8 / FP8 modules that receive the same activation tensor quantize
    it once: the q, k and v projections of one attention input (three QuantLinear calls on the same
    x in the reference's Wan block, each quantizing x itself) share one rotate + quantize pass.

    A quantized input is reused only for the same storage, offset, shape, strides, dtype and
    in-place version of the rows tensor, the same rotation group / format / static scale, and the
    same stream; the cache holds a reference to the rows, so their memory cannot be reused while it
    lives, and it is dropped when the block exits.  Values are those of the uncached path.
    Inference tensors (torch.inference_mode, as ComfyUI runs) have no version counter, so there an
    in-place change of the input between two calls inside the block goes unnoticed: wrap only
    consecutive uses of one unchanged input, as the q, k, v projections are.
    """
    prev = getattr(_shared, "cache", None)
    _shared.cache = {}
    try:
        yield
    finally:
        _shared.cache = prev


def _quantize_input(rows, fp8, group, input_scale):
    from . import ops
    cache = getattr(_shared, "cache", None)
    if cache is None:
        return ops.quantize_rows(rows, fp8=fp8, rot_group=group, static_scale=input_scale)
    try:
        version = rows._version
    except RuntimeError:   # inference tensors (torch.inference_mode) carry no version counter
        version = None
    key = (rows.data_ptr(), tuple(rows.shape), tuple(rows.stride()), rows.dtype, version, bool(fp8),
           int(group or 0), None if input_scale is None else (input_scale.data_ptr(), input_scale._version),
           torch.cuda.current_stream(rows.device).cuda_stream)
    hit = cache.get(key)
    if hit is not None:
        return hit[1], hit[2]
    qx, sx = ops.quantize_rows(rows, fp8=fp8, rot_group=group, static_scale=input_scale)
    cache[key] = (rows, qx, sx, input_scale)   # the references keep the keyed memory alive
    return qx, sx


def apply_activation(out, activation):
    """The reference's fp32 activation of a linear output: F.gelu(out.float(), approximate="tanh")
    (wan_model.py:626), or for "silu_gate" F.silu(gate.float()) * up.float() over
    out.chunk(2, -1) (fp16_safe.py:165-167)."""
    if activation == "gelu_tanh":
        return F.gelu(out.float(), approximate="tanh")
    if activation == "silu_gate":
        gate, up = out.chunk(2, -1)
        return F.silu(gate.float()) * up.float()
    raise ValueError(f"unsupported activation {activation!r}")


def native_linear(rows, qt, bias, fmt, input_scale=None, activation=None):
    """The native GEMM of one format on the gfx950 kernels (replaces F.linear(QuantizedTensor)).

    rows [M, K] in the compute dtype on the GPU; returns [M, N] in rows.dtype.  activation
    "gelu_tanh" returns gelu(y) rounded to rows.dtype, "silu_gate" silu(gate) * up over the two
    halves of y ([M, N / 2], N a multiple of 128), fused into the W8A8 / FP8 epilogues.
    """
    from . import ops
    if rows.device.type != "cuda":
        raise RuntimeError("native quantized GEMM needs a GPU tensor")
    layout, p = qt._layout_cls, qt._params
    if layout is qtm.Int8RowwiseLayout:
        group = p.convrot_groupsize if p.convrot else 0
        qx, a_scale = _quantize_input(rows, False, group, input_scale)
        return ops.gemm_i8(qx, a_scale, qt._qdata, p.scale, bias, out_dtype=rows.dtype, activation=activation)
    if layout is qtm.Float8ScaledLayout:
        qx, a_scale = _quantize_input(rows, True, 0, input_scale)
        if qt._qdata.dtype == torch.float8_e5m2 and activation is not None:
            # e5m2 weights have no fused epilogue: the linear output, rounded, then the activation
            out = ops.gemm_fp8(qx, a_scale, qt._qdata, p.scale, bias, out_dtype=rows.dtype)
            return apply_activation(out, activation).to(rows.dtype)
        return ops.gemm_fp8(qx, a_scale, qt._qdata, p.scale, bias, out_dtype=rows.dtype, activation=activation)
    if layout is qtm.UInt4GroupLayout:
        out = ops.gemm_w4a16(rows, qt._qdata, p.scale, p.zero, p.group_size, bias, out_dtype=rows.dtype)
        if activation is not None:   # weight-only GEMM: the activation stays a separate pass
            out = apply_activation(out, activation).to(rows.dtype)
        return out
    raise NotImplementedError(f"no native kernel for {fmt}")


def native_support(fmt, device):
    """(bool, reason): whether a native kernel runs this format on this device."""
    from . import ops, _native
    device = torch.device(device)
    if device.type != "cuda":
        return False, "not a GPU"
    op = NATIVE.get(fmt)
    if op is None:
        return False, f"no native kernel for {fmt}"
    if not _native.available():
        return False, f"{_native.LIB_PATH.name} is not built"
    if not ops.device_supported(device):
        return False, f"{torch.cuda.get_device_name(device)} is not gfx950"
    return True, f"psquant {op} (gfx950)"


# ------------------------------------------------------------------ installation
# weight_format -> stored format (quant_linear.py:269; int4 is this package's asymmetric group format)
TARGETS = {"int8": "int8_tensorwise", "fp8": "float8_e4m3fn", "int4": "int4_asym_group"}
# formats of the reference this package does not implement (Blackwell-only block formats)
UNSUPPORTED_TARGETS = ("mxfp8", "nvfp4")


def is_linear(module):
    """nn.Linear, or a Linear-like module (in_features and a 2-D weight Parameter)."""
    if isinstance(module, nn.Linear):
        return True
    weight = getattr(module, "weight", None)
    return hasattr(module, "in_features") and isinstance(weight, nn.Parameter) and weight.ndim == 2


def fits_blocks(module, fmt):
    """Whether the format's blocks fit the layer: 16 output features at least, and for the uint4
    groups an input width that holds whole 128-element groups."""
    if module.out_features < 16:
        return False
    return fmt != "int4_asym_group" or module.in_features % 128 == 0


class _Installer:
    """One install_quant_linears pass: picks the eligible Linears, decides their stored format and
    source, shares one weight template per layout signature and one native decision per format,
    swaps in the QuantLinear modules and builds the report."""

    def __init__(self, tensors, weight_format, compute, scope, compute_dtype, device, name_map, follow_input,
                 quant_options, open_file=None):
        self.tensors, self.weight_format, self.compute = tensors, weight_format, compute
        self.scope, self.compute_dtype, self.device = scope, compute_dtype, device
        self.name_map, self.follow_input, self.options = name_map, follow_input, quant_options or {}
        self.open_file = open_file
        self.templates, self.natives = {}, {}
        self.report = dict(weight_format=weight_format, compute=compute, modules={}, skipped=0, stored_bytes=0)

    def eligible(self, name, module):
        if not is_linear(module) or isinstance(module, QuantLinear) or getattr(module, "_ps_fp32", False):
            return False
        weight = getattr(module, "weight", None)
        if weight is not None and weight.dtype == torch.float32:
            return False   # FP32 islands (AdaLN / timestep / caption) stay unquantized
        return not self.scope or name.startswith(tuple(self.scope))

    def locate(self, name):
        """(table, weight key, its description) of a module's weight, or None without one."""
        table, key = self.name_map(name + ".weight") if self.name_map else (self.tensors, name + ".weight")
        desc = table.get(key) if table is not None else None
        return None if desc is None else (table, key, desc)

    def stored_format(self, desc):
        """(format, "file" | "quantize") or None when the module stays as it is."""
        record = desc.get("comfy_quant")
        if self.weight_format == "as_file":
            return None if record is None else (record["format"], "file")
        fmt = TARGETS[self.weight_format]
        return fmt, "file" if record is not None and record.get("format") == fmt else "quantize"

    def file_template(self, table, key, desc, fmt, shape):
        module = key[:-len(".weight")]
        own = {n: (getattr(torch, SAFETENSORS_DTYPES[d["dtype"]]), d.get("stored_shape", d["shape"]))
               for n, d in _module_tensors(table, module).items()}
        extras = {x: torch.empty(own[module + "." + x][1], dtype=own[module + "." + x][0], device="meta")
                  for x in EXTRAS if module + "." + x in own}
        signature = ("file", fmt, json_key(desc["comfy_quant"]), tuple(shape),
                     tuple((n[len(module):], str(dt), tuple(sh)) for n, (dt, sh) in sorted(own.items())))
        if signature not in self.templates:
            # powershard/quant_linear.py:329-337: a template that cannot be built from shapes alone is
            # built from the module's real tensors, read on the CPU through open_file(table, key)
            try:
                qt = quantized_from_file(None, own, module, desc["comfy_quant"], shape, self.device,
                                         self.compute_dtype, meta=True)
            except Exception:
                if self.open_file is None:
                    raise
                handle = self.open_file(table, key)
                real = {n: d["key"] for n, d in _module_tensors(table, module).items()}
                qt = quantized_from_file(handle, real, module, desc["comfy_quant"], shape, torch.device("cpu"),
                                         self.compute_dtype)
            self.templates[signature] = qt
        source = dict(kind="file", table=table, module=module, conf=desc["comfy_quant"], key=key)
        return self.templates[signature], source, extras

    def quantize_template(self, table, key, fmt, shape):
        signature = ("quantize", fmt, tuple(shape))
        if signature not in self.templates:
            self.templates[signature] = _template_from_shape(
                torch.empty(shape, dtype=self.compute_dtype, device="meta"), fmt, self.options)
        return self.templates[signature], dict(kind="quantize", table=table, module=key[:-len(".weight")], key=key)

    def native(self, fmt):
        if fmt not in self.natives:
            self.natives[fmt] = {"native": (True, "native selected"),
                                 "dequantize": (False, "dequantize selected")}.get(self.compute) \
                or native_support(fmt, torch.device(self.device))
        return self.natives[fmt]

    def install(self, net, name, module):
        found = self.locate(name)
        if found is None:
            return
        table, key, desc = found
        chosen = self.stored_format(desc)
        if chosen is None:
            return
        fmt, kind = chosen
        if not fits_blocks(module, fmt):
            self.report["skipped"] += 1
            return
        shape = [module.out_features, module.in_features]
        if kind == "file":
            qt, source, extras = self.file_template(table, key, desc, fmt, shape)
        else:
            (qt, source), extras = self.quantize_template(table, key, fmt, shape), None
        plan = plan_from_quantized(qt, fmt, source, extras)
        native, reason = self.native(fmt)
        full_precision = kind == "file" and bool(desc["comfy_quant"].get("full_precision_matrix_mult"))
        parent, _, leaf = name.rpartition(".")
        owner = net.get_submodule(parent) if parent else net
        setattr(owner, leaf, QuantLinear(module, plan, self.compute_dtype, native, self.follow_input, full_precision))
        entry = self.report["modules"].setdefault(fmt, dict(count=0, native=native, reason=reason, source={}))
        entry["count"] += 1
        entry["source"][kind] = entry["source"].get(kind, 0) + 1
        self.report["stored_bytes"] += plan.total


def install_quant_linears(net, tensors, weight_format, compute, scope, compute_dtype, device, open_file=None,
                          name_map=None, follow_input=False, quant_options=None):
    """Replace the Linears in scope by QuantLinear.  tensors: model name -> desc (key, dtype, shape,
    stored_shape, comfy_quant).  weight_format: dequantize | as_file | int8 | fp8 | int4.
    name_map: parameter name -> (table, name in table) for multi-file models.
    quant_options (this package's addition): layout options of quantize-at-load weights, e.g.
    {"convrot": True, "convrot_groupsize": 256} for int8 or {"group_size": 128} for int4.
    open_file(table, key) -> a handle with get_tensor(name): used, as in the reference, only when a
    file module's template cannot be built from its shapes; the template then comes from the
    module's real tensors on the CPU.
    Returns a report.
    """
    if weight_format in UNSUPPORTED_TARGETS:
        raise ValueError(f"weight_format {weight_format} is a Blackwell block format, not supported on MI355X")
    installer = _Installer(tensors, weight_format, compute, scope, compute_dtype, device, name_map, follow_input,
                           quant_options, open_file)
    if weight_format != "dequantize":
        for name, module in list(net.named_modules()):
            if installer.eligible(name, module):
                installer.install(net, name, module)
    return installer.report


def _convrot_options(options, k):
    rot = qf.convrot_config({"convrot": options.get("convrot", False),
                             "convrot_groupsize": options.get("convrot_groupsize", 256)}, k, "in_features")
    return rot["convrot"], rot["group_size"]


def _template_from_shape(weight_meta, fmt, options):
    """Shapes/dtypes of `fmt` for a weight of weight_meta's shape, without data (meta tensors)."""
    n, k = weight_meta.shape
    dtype = weight_meta.dtype
    meta = torch.device("meta")
    if fmt == "int8_tensorwise":
        convrot, group = _convrot_options(options, k)
        params = qtm.Int8RowwiseParams(torch.empty(n, 1, dtype=torch.float32, device=meta), dtype, convrot, group)
        return qtm.QuantizedWeight(torch.empty(n, k, dtype=torch.int8, device=meta), qtm.Int8RowwiseLayout, params)
    if fmt in ("float8_e4m3fn", "float8_e5m2"):
        code = torch.float8_e4m3fn if fmt == "float8_e4m3fn" else torch.float8_e5m2
        params = qtm.Float8ScaledParams(torch.empty((), dtype=torch.float32, device=meta), dtype)
        return qtm.QuantizedWeight(torch.empty(n, k, dtype=code, device=meta), qtm.Float8ScaledLayout, params)
    if fmt == "int4_asym_group":
        g = int(options.get("group_size", 128))
        if k % g:
            raise ValueError(f"uint4 group {g} does not divide in_features {k}")
        params = qtm.UInt4GroupParams(torch.empty(n, k // g, dtype=torch.float16, device=meta),
                                      torch.empty(n, k // g, dtype=torch.float16, device=meta), dtype, g)
        return qtm.QuantizedWeight(torch.empty(n, k // 2, dtype=torch.uint8, device=meta), qtm.UInt4GroupLayout, params)
    raise ValueError(f"Format {fmt} is not supported by powershard_amd")


def json_key(conf):
    return json.dumps(conf, sort_keys=True)


def _module_tensors(table, module):
    """A module's own file tensors (weight, scales, zero, extras): no bias, no comfy_quant record."""
    return qf.QuantHeader(table).own(module, with_record=False)


# safetensors dtype code -> torch dtype attribute name
SAFETENSORS_DTYPES = {"F64": "float64", "F32": "float32", "F16": "float16", "BF16": "bfloat16", "I64": "int64",
                      "I32": "int32", "I16": "int16", "I8": "int8", "U8": "uint8", "BOOL": "bool",
                      "F8_E4M3": "float8_e4m3fn", "F8_E5M2": "float8_e5m2"}


def _torch_dtype(code):
    return SAFETENSORS_DTYPES[code]


# ------------------------------------------------------------------------ loading
# the scale tensors that accompany a plain fp8 weight, in the order they are looked up
_FP8_SCALE_SUFFIXES = (".scale_weight", ".weight_scale")


def _fp8_scale(handle, table, module, device):
    """The first float scale beside a plain fp8 weight (per tensor, or per row as [N, 1]); None if
    there is none."""
    for suffix in _FP8_SCALE_SUFFIXES:
        desc = table.get(module + suffix)
        if desc is not None and desc["dtype"] in ("F32", "F16", "BF16"):
            value = handle.get_tensor(desc["key"]).float().to(device)
            return value.reshape(-1, 1) if value.numel() > 1 else value.reshape(())
    return None


def float_weight(handle, table, key, device, dtype=torch.float32):
    """A module's full weight as float: plain / fp8 (+scale) / comfy_quant (dequantized here)."""
    desc = table[key]
    module = key[:-len(".weight")]
    if desc.get("comfy_quant") is not None:
        return qf.dequantize_module(handle, qf.module_entries(table, module), module, desc["comfy_quant"],
                                    desc["shape"], device, dtype)
    weight = handle.get_tensor(desc["key"]).to(device)
    if desc["dtype"] in ("F8_E4M3", "F8_E5M2"):
        weight = weight.float()
        scale = _fp8_scale(handle, table, module, device)
        if scale is not None:
            weight = weight * scale
    return weight.to(dtype)


def _used_names(table, module, key, kind):
    """The table entries a module's bytes are built from."""
    used = set(_module_tensors(table, module)) | {key}
    if module + qf.QUANT_SUFFIX in table:
        used.add(module + qf.QUANT_SUFFIX)
    if kind != "file":
        used |= {module + s for s in _FP8_SCALE_SUFFIXES if module + s in table}
    return used


def _checked_finite(weight, key, when):
    if not torch.isfinite(weight).all():
        raise FloatingPointError(f"{key}: non-finite weights {when}")
    return weight


def _file_weight(handle, plan, shape, device, dtype, delta):
    """(QuantizedWeight, extras) of a file module; a LoRA delta is added to the true weight
    W = Wq * pre_quant_scale (per input), i.e. delta / s in Wq space, and the sum requantized in the
    file's layout."""
    src = plan.source
    table, module = src["table"], src["module"]
    files = {n: d["key"] for n, d in _module_tensors(table, module).items()}
    qt = quantized_from_file(handle, files, module, src["conf"], shape, device, dtype)
    extras = {x: handle.get_tensor(table[module + "." + x]["key"]).to(device) for x in EXTRAS
              if module + "." + x in table}
    if delta is not None:
        pre = extras.get("pre_quant_scale")
        step = delta.float() if pre is None else delta.float() / pre.float().reshape(1, -1)
        weight = _checked_finite(qt.dequantize().float() + step, src["key"], "after LoRA")
        qt = requantize_like(qt, weight.to(dtype), plan.fmt)
    return qt, extras


def _quantized_at_load(handle, plan, device, dtype, delta):
    """QuantizedWeight of a float (or fp8-scaled) file weight quantized into the planned layout."""
    src = plan.source
    weight = float_weight(handle, src["table"], src["key"], device)
    if delta is not None:
        weight = weight + delta
    weight = _checked_finite(weight, src["key"], "before quantization")
    return quantized_from_float(weight.to(dtype), plan.fmt, **_quantize_options(plan))


def build_bytes(module, handle, device, lora_delta=None):
    """The full QuantLinear byte vector on device; returns (bytes, table names used)."""
    plan = module._ps_qplan
    src = plan.source
    shape = [module.out_features, module.in_features]
    delta = lora_delta(src["key"], shape, device) if lora_delta else None
    dtype = module._ps_compute_dtype
    if src["kind"] == "file":
        qt, extras = _file_weight(handle, plan, shape, device, dtype, delta)
    else:
        qt, extras = _quantized_at_load(handle, plan, device, dtype, delta), None
    return pack(qt, plan, device, extras), _used_names(src["table"], src["module"], src["key"], src["kind"])


def _quantize_options(plan):
    """Layout options of the template, so quantize-at-load reproduces the planned layout."""
    f = plan.fields
    if plan.layout is qtm.Int8RowwiseLayout:
        return dict(convrot=f.get("convrot", False), convrot_groupsize=f.get("convrot_groupsize", 256))
    if plan.layout is qtm.UInt4GroupLayout:
        return dict(group_size=f.get("group_size", 128))
    return {}
