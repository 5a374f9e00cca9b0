"""QuantLinear: quantized Linear layers stored as one aligned byte vector, computed by the gfx950
kernels of libpsquant (native) or by dequantize + F.linear.

Drop-in for powershard/quant_linear.py (ComfyUI-PowerShard 0.6.0):

* the module / state-dict contract -- ``QuantLinear(src, plan, compute_dtype, native,
  follow_input, full_precision)`` with a 1-D ``uint8`` parameter ``qbytes`` and ``bias``
  (quant_linear.py:163-189);
* the byte layout discipline of ``QuantPlan`` -- components 16-byte aligned, ``_qdata`` first,
  then the tensor fields of the params dataclass in order, then ``x:<extra>`` (quant_linear.py:27,
  38-49, 65-122), so FSDP can shard and gather ``qbytes`` as plain bytes;
* the compute modes ``native`` / ``dequantize`` / ``auto`` and the fallback convention: a
  native failure of type NotImplementedError / RuntimeError / TypeError / ValueError warns and
  switches the module to dequantize for good; out-of-memory propagates (quant_linear.py:207-215);
* ``install_quant_linears`` / ``build_bytes`` / ``float_weight`` (quant_linear.py:285-444).

What differs is below the module: ComfyUI's QuantizedTensor is replaced by
:class:`~powershard_amd.quant_tensor.QuantizedWeight`, and comfy-kitchen's int8_linear /
torch._scaled_mm / w4a8 ops by the HIP kernels (``native_linear``):

* int8_tensorwise: fused ConvRot + per-token int8 quantize, then the int8 MFMA GEMM with the
  dequant epilogue;
* float8_e4m3fn: per-token e4m3 quantize, then the fp8 MFMA GEMM;
* int4_asym_group: weight-only GEMM with in-register uint4 dequantization (W4A16).
"""
import contextlib
import dataclasses
import json
import math
import threading
import warnings

import torch
from torch import nn
from torch.nn import functional as F

from . import quant_tensor as qtm

ALIGN = 16
# Extra per-module tensors of ModelOpt/AWQ files: pre_quant_scale multiplies the input,
# input_scale is a static activation scale.  Stored in the same byte vector as "x:<name>".
EXTRAS = ("pre_quant_scale", "input_scale")
# Formats with a native kernel here and the library op that runs them.
NATIVE = {"int8_tensorwise": "gemm_i8", "float8_e4m3fn": "gemm_fp8", "int4_asym_group": "gemm_w4a16"}


@dataclasses.dataclass
class QuantPlan:
    fmt: str
    layout: object
    params_cls: type
    fields: dict
    specs: list          # [(name, dtype, shape, offset, nbytes)], "_qdata" first
    total: int
    source: dict         # kind=file|quantize, module, key, table, conf

    def signature(self):
        return [(n, str(d), list(s), o, b) for n, d, s, o, b in self.specs]


# ------------------------------------------------------------ QuantizedWeight <-> bytes
def comfy_quant():
    """The module holding QuantizedWeight / QUANT_ALGOS (ComfyUI's comfy.quant_ops in the reference)."""
    return qtm


def layout_name(fmt):
    return qtm.layout_name(fmt)


def components(qt, extras=None):
    """(tensors in byte-vector order, non-tensor fields)."""
    tensors, fields = [("_qdata", qt._qdata)], {}
    for field in dataclasses.fields(qt._params):
        value = getattr(qt._params, field.name)
        if isinstance(value, torch.Tensor):
            tensors.append((field.name, value))
        else:
            fields[field.name] = value
    for name, value in sorted((extras or {}).items()):
        tensors.append(("x:" + name, value))
    return tensors, fields


def _same_field(a, b):
    if isinstance(a, torch.dtype) or isinstance(b, torch.dtype):
        return True  # orig_dtype is set by unpack
    if isinstance(a, (tuple, list)) or isinstance(b, (tuple, list)):
        return tuple(a) == tuple(b)
    return a == b


def plan_from_quantized(qt, fmt, source, extras=None):
    tensors, fields = components(qt, extras)
    specs, offset = [], 0
    for name, tensor in tensors:
        nbytes = tensor.numel() * tensor.element_size()
        specs.append((name, tensor.dtype, tuple(tensor.shape), offset, nbytes))
        offset += math.ceil(nbytes / ALIGN) * ALIGN
    return QuantPlan(fmt, qt._layout_cls, type(qt._params), fields, specs, max(offset, ALIGN), source)


def pack(qt, plan, device, extras=None):
    """One uint8 vector [plan.total] holding every component at its aligned offset."""
    tensors, fields = components(qt, extras)
    got = [(n, t.dtype, tuple(t.shape)) for n, t in tensors]
    if got != [(n, d, s) for n, d, s, _, _ in plan.specs]:
        raise RuntimeError(f"Layout of {plan.fmt} differs from the template: {got}")
    differ = {k: (v, plan.fields.get(k)) for k, v in fields.items() if not _same_field(v, plan.fields.get(k))}
    if differ or fields.keys() != plan.fields.keys():
        raise RuntimeError(f"Parameters of {plan.fmt} differ from the template (the data would decode wrongly): {differ}")
    out = torch.zeros(plan.total, dtype=torch.uint8, device=device)
    for (name, tensor), (_, _, _, offset, nbytes) in zip(tensors, plan.specs):
        out[offset:offset + nbytes].copy_(tensor.detach().contiguous().reshape(-1).view(torch.uint8).to(device))
    return out


def unpack(full, plan, dtype=None, with_extras=False):
    """Gathered byte vector -> QuantizedWeight of zero-copy views [+ extras]."""
    values, extras = {}, {}
    for name, tensor_dtype, shape, offset, nbytes in plan.specs:
        view = full[offset:offset + nbytes].view(tensor_dtype).reshape(shape)
        if name.startswith("x:"):
            extras[name[2:]] = view
        else:
            values[name] = view
    fields = dict(plan.fields)
    if dtype is not None and "orig_dtype" in fields:
        fields["orig_dtype"] = dtype
    params = plan.params_cls(**fields, **{k: v for k, v in values.items() if k != "_qdata"})
    qt = qtm.QuantizedWeight(values["_qdata"], plan.layout, params)
    return (qt, extras) if with_extras else qt


# ------------------------------------------------------------------- file formats
def _conf_param(conf, name, default):
    params = conf.get("params") if isinstance(conf.get("params"), dict) else {}
    return conf.get(name, params.get(name, default))


def quantized_from_file(handle, entries, module, conf, shape, device, dtype, meta=False):
    """QuantizedWeight from a module's file tensors.

    entries: name -> file key (or, with meta=True, name -> (torch dtype, shape): a template
    without reading data).  conf: the module's ``comfy_quant`` JSON.  Layouts on disk:
    int8_tensorwise = weight I8 [N, K] + weight_scale F32 [N, 1] (+ convrot,
    convrot_groupsize); float8_e4m3fn = weight F8_E4M3 + weight_scale / scale_weight F32 ([] or
    [N]); int4_asym_group = weight U8 [N, K/2] + weight_scale / weight_zero F16 [N, K/g] (+ group_size).
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
        convrot = bool(_conf_param(conf, "convrot", False))
        group = int(_conf_param(conf, "convrot_groupsize", 256))
        if convrot and (group < 4 or group & (group - 1) or (group.bit_length() - 1) % 2 or k % group):
            raise ValueError(f"{module}: invalid ConvRot group {group}")
        params = qtm.Int8RowwiseParams(scale.to(dev, torch.float32).reshape(n, 1), dtype, convrot, group)
        return qtm.QuantizedWeight(weight.to(dev), qtm.Int8RowwiseLayout, params)
    if fmt == "float8_e4m3fn":
        scale = state.get(prefix + "weight_scale", state.get(prefix + "scale_weight"))
        if weight.dtype != torch.float8_e4m3fn or scale is None:
            raise ValueError(f"{module}: float8_e4m3fn expects F8_E4M3 weight and a weight_scale")
        scale = scale.to(dev, torch.float32)
        scale = scale.reshape(()) if scale.numel() == 1 else scale.reshape(n)
        return qtm.QuantizedWeight(weight.to(dev), qtm.Float8ScaledLayout, qtm.Float8ScaledParams(scale, dtype))
    if fmt == "int4_asym_group":
        scale, zero = state.get(prefix + "weight_scale"), state.get(prefix + "weight_zero")
        group = int(_conf_param(conf, "group_size", 128))
        if (weight.dtype != torch.uint8 or tuple(weight.shape) != (n, k // 2) or scale is None or zero is None
                or k % group or tuple(scale.shape) != (n, k // group) or tuple(zero.shape) != (n, k // group)):
            raise ValueError(f"{module}: int4_asym_group expects U8 [N, K/2] weight and F16 [N, K/g] scale/zero")
        params = qtm.UInt4GroupParams(scale.to(dev, torch.float16), zero.to(dev, torch.float16), dtype, group)
        return qtm.QuantizedWeight(weight.to(dev), qtm.UInt4GroupLayout, params)
    raise ValueError(f"{module}: format {fmt} is not supported by powershard_amd: {sorted(qtm.QUANT_ALGOS)}")


def quantized_from_float(weight, fmt, **options):
    """Quantize a float weight into `fmt` (scale recomputed from the data, as ComfyUI set_weight)."""
    return qtm.QuantizedWeight.from_float(weight, layout_name(fmt), scale="recalculate", **options)


def requantize_like(template, weight, fmt):
    """New weight (after LoRA) in the template's layout; ConvRot / group options are kept."""
    if hasattr(template, "requantize_from_float"):
        return template.requantize_from_float(weight, scale="recalculate")
    return quantized_from_float(weight, fmt)


# ------------------------------------------------------------------------- module
class QuantLinear(nn.Module):
    """Linear whose weight is one QuantizedWeight byte vector (FSDP Shard(0) over bytes)."""

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
        for attr in ("_ps_tracker", "_ps_finite_slot", "_ps_safe", "_ps_fp32"):
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

    def _forward(self, x, activation):
        plan = self._ps_qplan
        shape = x.shape
        if self._ps_follow_input and not self._ps_native:
            dtype = x.dtype if x.is_floating_point() else self._ps_compute_dtype
        else:
            dtype = self._ps_compute_dtype
        rows = x.reshape(-1, shape[-1]).to(dtype)
        bias = None if self.bias is None else self.bias.to(dtype)
        qt, extras = unpack(self.qbytes, plan, dtype, with_extras=True)
        pre = extras.get("pre_quant_scale")
        if pre is not None:  # ModelOpt AWQ smoothing
            rows = rows * pre.to(rows.dtype)
        # The reference's V100 "FP16 safe" mode computes the dequantized GEMM with an FP32 result.
        safe = getattr(self, "_ps_safe", False) and dtype == torch.float16
        out = None
        fused = False   # activation applied by native_linear
        if self._ps_native and not safe and not self._ps_full_precision:
            # the fused gate pairs 64-column blocks: other widths take the gate as a separate pass
            native_act = None if activation == "silu_gate" and self.out_features % 128 else activation
            try:
                out = native_linear(rows, qt, bias, plan.fmt, extras.get("input_scale"), native_act)
                fused = native_act is not None
            except torch.cuda.OutOfMemoryError:
                raise
            except (NotImplementedError, RuntimeError, TypeError, ValueError) as error:
                warnings.warn(f"PowerShard: native {plan.fmt} GEMM unavailable ({error}); the module switches to dequantize")
                self._ps_native = False
                out = None
        if out is None and safe:
            out = F.linear(rows.float(), qt.dequantize().float(), None if bias is None else bias.float())
        elif out is None:
            out = F.linear(rows, qt.dequantize().to(dtype), bias)
        if activation is not None and not fused:
            out = apply_activation(out, activation)
        out = out.reshape(shape[:-1] + (out.shape[-1],))
        if self._ps_follow_input and x.is_floating_point() and out.dtype != x.dtype:
            out = out.to(x.dtype)  # text encoder: the FP32 graph is not narrowed to bf16 by the native kernel
        tracker = getattr(self, "_ps_tracker", None)
        if tracker is not None:
            tracker.observe(self._ps_finite_slot, out)
        return out


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
    weight = getattr(module, "weight", None)
    return isinstance(module, nn.Linear) or (hasattr(module, "in_features") and isinstance(weight, nn.Parameter)
                                             and weight.ndim == 2)


def fits_blocks(module, fmt):
    k, n = module.in_features, module.out_features
    if fmt == "int4_asym_group":
        return k % 128 == 0 and n >= 16
    return n >= 16


def install_quant_linears(net, tensors, weight_format, compute, scope, compute_dtype, device, open_file=None,
                          name_map=None, follow_input=False, quant_options=None):
    """Replace the Linears in scope by QuantLinear.  tensors: model name -> desc (key, dtype, shape,
    stored_shape, comfy_quant).  weight_format: dequantize | as_file | int8 | fp8 | int4.
    name_map: parameter name -> (table, name in table) for multi-file models.
    quant_options (this package's addition): layout options of quantize-at-load weights, e.g.
    {"convrot": True, "convrot_groupsize": 256} for int8 or {"group_size": 128} for int4.
    Returns a report.
    """
    report = dict(weight_format=weight_format, compute=compute, modules={}, skipped=0, stored_bytes=0)
    if weight_format == "dequantize":
        return report
    if weight_format in UNSUPPORTED_TARGETS:
        raise ValueError(f"weight_format {weight_format} is a Blackwell block format, not supported on MI355X")
    templates, natives = {}, {}
    for name, module in list(net.named_modules()):
        if not is_linear(module) or getattr(module, "_ps_fp32", False) or isinstance(module, QuantLinear):
            continue
        if getattr(module, "weight", None) is not None and module.weight.dtype == torch.float32:
            continue  # FP32 islands (AdaLN / timestep / caption) stay unquantized
        if scope and not any(name.startswith(s) for s in scope):
            continue
        table, key = (name_map(name + ".weight") if name_map else (tensors, name + ".weight"))
        desc = table.get(key) if table is not None else None
        if desc is None:
            continue
        file_conf = desc.get("comfy_quant")
        if weight_format == "as_file":
            if file_conf is None:
                continue
            fmt, kind = file_conf["format"], "file"
        else:
            fmt = TARGETS[weight_format]
            kind = "file" if file_conf is not None and file_conf.get("format") == fmt else "quantize"
        if not fits_blocks(module, fmt):
            report["skipped"] += 1
            continue
        module_key = key[:-len(".weight")]
        shape = [module.out_features, module.in_features]
        extras = None
        if kind == "file":
            entries = {n: (getattr(torch, _torch_dtype(d["dtype"])), d.get("stored_shape", d["shape"]))
                       for n, d in _entries(table, module_key).items()}
            extras = {x: torch.empty(entries[module_key + "." + x][1], dtype=entries[module_key + "." + x][0],
                                     device="meta") for x in EXTRAS if module_key + "." + x in entries}
            signature = ("file", fmt, json_key(file_conf), tuple(shape),
                         tuple((n[len(module_key):], str(v[0]), tuple(v[1])) for n, v in sorted(entries.items())))
            if signature not in templates:
                templates[signature] = quantized_from_file(None, entries, module_key, file_conf, shape, device,
                                                           compute_dtype, meta=True)
            qt = templates[signature]
            source = dict(kind="file", table=table, module=module_key, conf=file_conf, key=key)
        else:
            signature = ("quantize", fmt, tuple(shape))
            if signature not in templates:
                dummy = torch.ones(shape, dtype=compute_dtype, device="meta")
                templates[signature] = _template_from_shape(dummy, fmt, quant_options or {})
            qt = templates[signature]
            source = dict(kind="quantize", table=table, module=module_key, key=key)
        plan = plan_from_quantized(qt, fmt, source, extras)
        if fmt not in natives:
            if compute == "native":
                natives[fmt] = (True, "native selected")
            elif compute == "dequantize":
                natives[fmt] = (False, "dequantize selected")
            else:
                natives[fmt] = native_support(fmt, torch.device(device))
        parent_name, _, leaf = name.rpartition(".")
        parent = net.get_submodule(parent_name) if parent_name else net
        full_precision = bool(kind == "file" and file_conf.get("full_precision_matrix_mult"))
        setattr(parent, leaf, QuantLinear(module, plan, compute_dtype, natives[fmt][0], follow_input, full_precision))
        entry = report["modules"].setdefault(fmt, dict(count=0, native=natives[fmt][0], reason=natives[fmt][1],
                                                      source={}))
        entry["count"] += 1
        entry["source"][kind] = entry["source"].get(kind, 0) + 1
        report["stored_bytes"] += plan.total
    return report


def _template_from_shape(weight_meta, fmt, options):
    """Shapes/dtypes of `fmt` for a weight of weight_meta's shape, without data (meta tensors)."""
    n, k = weight_meta.shape
    dtype = weight_meta.dtype
    meta = torch.device("meta")
    if fmt == "int8_tensorwise":
        convrot = bool(options.get("convrot", False))
        group = int(options.get("convrot_groupsize", 256))
        if convrot and (group < 4 or group & (group - 1) or (group.bit_length() - 1) % 2 or k % group):
            raise ValueError(f"invalid ConvRot group {group} for in_features {k}")
        params = qtm.Int8RowwiseParams(torch.empty(n, 1, dtype=torch.float32, device=meta), dtype, convrot, group)
        return qtm.QuantizedWeight(torch.empty(n, k, dtype=torch.int8, device=meta), qtm.Int8RowwiseLayout, params)
    if fmt == "float8_e4m3fn":
        params = qtm.Float8ScaledParams(torch.empty((), dtype=torch.float32, device=meta), dtype)
        return qtm.QuantizedWeight(torch.empty(n, k, dtype=torch.float8_e4m3fn, device=meta), qtm.Float8ScaledLayout,
                                   params)
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


def _entries(table, module):
    prefix = module + "."
    return {n: d for n, d in table.items()
            if n.startswith(prefix) and "." not in n[len(prefix):] and not n.endswith(".bias")
            and not n.endswith(".comfy_quant")}


# safetensors dtype code -> torch dtype attribute name
SAFETENSORS_DTYPES = {"F64": "float64", "F32": "float32", "F16": "float16", "BF16": "bfloat16", "I64": "int64",
                      "I32": "int32", "I16": "int16", "I8": "int8", "U8": "uint8", "BOOL": "bool",
                      "F8_E4M3": "float8_e4m3fn", "F8_E5M2": "float8_e5m2"}


def _torch_dtype(code):
    return SAFETENSORS_DTYPES[code]


# ------------------------------------------------------------------------ loading
def float_weight(handle, table, key, device, dtype=torch.float32):
    """A module's full weight as float: plain / fp8 (+scale) / comfy_quant (dequantized here)."""
    from .quant_formats import dequantize_module, module_entries
    desc = table[key]
    module = key[:-len(".weight")]
    if desc.get("comfy_quant") is not None:
        return dequantize_module(handle, module_entries(table, module), module, desc["comfy_quant"], desc["shape"],
                                 device, dtype)
    weight = handle.get_tensor(desc["key"]).to(device)
    if desc["dtype"] in ("F8_E4M3", "F8_E5M2"):
        weight = weight.float()
        for suffix in (".scale_weight", ".weight_scale"):
            scale = table.get(module + suffix)
            if scale is not None and scale["dtype"] in ("F32", "F16", "BF16"):
                value = handle.get_tensor(scale["key"]).float().to(device)
                weight = weight * (value.reshape(-1, 1) if value.numel() > 1 else value.reshape(()))
                break
    return weight.to(dtype)


def build_bytes(module, handle, device, lora_delta=None):
    """The full QuantLinear byte vector on device; returns (bytes, table names used)."""
    plan = module._ps_qplan
    source = plan.source
    table, key, name = source["table"], source["key"], source["module"]
    used = set(_entries(table, name)) | {key}
    if name + ".comfy_quant" in table:
        used.add(name + ".comfy_quant")
    dtype = module._ps_compute_dtype
    shape = [module.out_features, module.in_features]
    delta = lora_delta(key, shape, device) if lora_delta else None
    extras = None
    if source["kind"] == "file":
        entries = {n: d["key"] for n, d in _entries(table, name).items()}
        qt = quantized_from_file(handle, entries, name, source["conf"], shape, device, dtype)
        extras = {x: handle.get_tensor(table[name + "." + x]["key"]).to(device) for x in EXTRAS
                  if name + "." + x in table}
        if delta is not None:
            # LoRA on the true weight W = Wq * pre_quant_scale (per input): delta / s in Wq space.
            weight = qt.dequantize().float()
            pre = extras.get("pre_quant_scale")
            weight = weight + (delta.float() / pre.float().reshape(1, -1) if pre is not None else delta.float())
            if not torch.isfinite(weight).all():
                raise FloatingPointError(f"{key}: non-finite weights after LoRA")
            qt = requantize_like(qt, weight.to(dtype), plan.fmt)
            del weight
    else:
        weight = float_weight(handle, table, key, device)
        for suffix in (".scale_weight", ".weight_scale"):
            if name + suffix in table:
                used.add(name + suffix)
        if delta is not None:
            weight = weight + delta
        if not torch.isfinite(weight).all():
            raise FloatingPointError(f"{key}: non-finite weights before quantization")
        qt = quantized_from_float(weight.to(dtype), plan.fmt, **_quantize_options(plan))
        del weight
    return pack(qt, plan, device, extras), used


def _quantize_options(plan):
    """Layout options of the template, so quantize-at-load reproduces the planned layout."""
    f = plan.fields
    if plan.layout is qtm.Int8RowwiseLayout:
        return dict(convrot=f.get("convrot", False), convrot_groupsize=f.get("convrot_groupsize", 256))
    if plan.layout is qtm.UInt4GroupLayout:
        return dict(group_size=f.get("group_size", 128))
    return {}
