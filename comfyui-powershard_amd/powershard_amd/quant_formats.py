"""Weight-format metadata of the quantized linear path: ``comfy_quant`` JSON, packed vs logical
shapes, the user vocabulary, and full-weight dequantization of a file module.

Interface of powershard/quant_formats.py (PACKED_BITS, packed_bits, logical_shape,
read_quant_json, annotate_quantized, module_entries, formats_summary, dequantize_module,
WEIGHT_FORMATS, COMPUTE_MODES, validate_quant_choice, resolve_weight_dtype) and the int8
``comfy_quant`` checks of powershard/checkpoint.py:63-82 / powershard/wan_config.py:132-162.

A checkpoint's tensor table (name -> {"key", "dtype", "shape", ...}) is read through
:class:`QuantHeader`, which groups a module's tensors, decodes its ``comfy_quant`` record and
validates the int8 layouts; the module-level functions are that class's entry points under the
reference's names.  Everything above ``dequantize_module`` imports only json, so node and config
code can use it before torch is loaded.
"""
import json

QUANT_SUFFIX = ".comfy_quant"
# Storage bits per element of the packed formats (a [N, K] weight is stored as [N, K * bits / 8]).
PACKED_BITS = {"nvfp4": 4, "asym_w4a8_int8": 4, "w6a8_int8": 6, "int4_asym_group": 4}
# Largest comfy_quant JSON payload accepted from a file header (its real size is 72 bytes).
MAX_QUANT_JSON = 1 << 20


def conf_value(conf, name, default):
    """A comfy_quant option, given at the top level of the record or under its "params"."""
    nested = conf.get("params")
    if isinstance(nested, dict) and name in nested and name not in conf:
        return nested[name]
    return conf.get(name, default)


def packed_bits(conf):
    """Bits per weight element in the file: convrot_w4a4 packs int4 unless its linear dtype is int8."""
    fmt = conf.get("format")
    if fmt == "convrot_w4a4":
        return 8 if conf_value(conf, "linear_dtype", "int4") != "int4" else 4
    return PACKED_BITS.get(fmt, 8)


def logical_shape(stored_shape, conf):
    """The dequantized weight's shape from its stored shape (2-D packed widths are unpacked)."""
    shape = list(stored_shape)
    bits = packed_bits(conf)
    if bits == 8 or len(shape) != 2:
        return shape
    width, rest = divmod(shape[1] * 8, bits)
    if rest:
        raise ValueError(f"{conf.get('format')}: width {shape[1]} does not match {bits}-bit packing")
    return [shape[0], width]


def read_quant_json(path, data_start, desc):
    """The comfy_quant record of one U8 header entry, read from the file's data section."""
    start, end = desc["data_offsets"]
    if desc["dtype"] != "U8" or not 0 <= end - start <= MAX_QUANT_JSON:
        raise ValueError("Invalid comfy_quant metadata")
    with open(path, "rb") as f:
        f.seek(data_start + start)
        payload = f.read(end - start)
    return json.loads(payload)


def _is_power_of_4(n):
    return n >= 4 and n & (n - 1) == 0 and (n.bit_length() - 1) % 2 == 0


def convrot_config(conf, in_features, module="?"):
    """{convrot, group_size} of an int8_tensorwise comfy_quant config (powershard/checkpoint.py:63-82):
    the group is a power of 4 dividing in_features; ``convrot_groupsize`` defaults to 256 and may
    also sit under ``params``."""
    group = int(conf_value(conf, "convrot_groupsize", 256))
    enabled = bool(conf_value(conf, "convrot", False))
    if enabled and not (_is_power_of_4(group) and in_features % group == 0):
        raise ValueError(f"Invalid ConvRot group: {module}")
    return {"convrot": enabled, "group_size": group}


class QuantHeader:
    """A checkpoint tensor table seen per module: its own tensors, its comfy_quant record and the
    layout checks of the int8 storage.  ``read_json(name)`` returns the decoded record of a
    ``<module>.comfy_quant`` entry."""

    def __init__(self, tensors, read_json=None):
        self.tensors = tensors
        self.read_json = read_json

    @staticmethod
    def owns(module, name, with_record=True):
        """True for `module`'s direct tensors (weight, scales, zero, extras and, unless with_record
        is False, its comfy_quant record), never its bias nor the tensors of its submodules."""
        head, dot, leaf = name.rpartition(".")
        if dot != "." or head != module or leaf == "bias":
            return False
        return with_record or leaf != QUANT_SUFFIX[1:]

    def own(self, module, with_record=True):
        return {name: desc for name, desc in self.tensors.items() if self.owns(module, name, with_record)}

    def quantized_modules(self):
        return [name[:-len(QUANT_SUFFIX)] for name in self.tensors if name.endswith(QUANT_SUFFIX)]

    def record(self, module):
        conf = self.read_json(module + QUANT_SUFFIX)
        if not isinstance(conf, dict) or not conf.get("format"):
            raise ValueError(f"comfy_quant without a format: {module + QUANT_SUFFIX}")
        return conf

    def annotate(self):
        """Give every quantized weight its logical shape ("shape"), its stored shape
        ("stored_shape") and its record ("comfy_quant"); returns {module: record}."""
        configs = {}
        for module in self.quantized_modules():
            conf = configs[module] = self.record(module)
            desc = self.tensors.get(module + ".weight")
            if desc is not None:
                stored = list(desc["shape"])
                desc.update(stored_shape=stored, shape=logical_shape(stored, conf), comfy_quant=conf)
        return configs

    def int8_layout(self, name, desc):
        """{convrot, group_size} of the I8 tensor `name`, after the checks of the native int8 storage:
        a Linear weight with a comfy_quant int8_tensorwise record and an F32 [N, 1] row scale."""
        if not name.endswith(".weight") or len(desc["shape"]) != 2:
            raise ValueError(f"INT8 outside a Linear: {name}")
        module = name[:-len(".weight")]
        if module + QUANT_SUFFIX not in self.tensors:
            raise ValueError(f"INT8 without comfy_quant metadata: {module}")
        conf = self.read_json(module + QUANT_SUFFIX)
        if conf.get("format") != "int8_tensorwise":
            raise ValueError(f"Unsupported quantization of {module}: {conf}")
        n, k = desc["shape"]
        scale = self.tensors.get(module + ".weight_scale") or {}
        if scale.get("dtype") != "F32" or scale.get("shape") != [n, 1]:
            raise ValueError(f"Expected a row-wise FP32 scale: {module}")
        return convrot_config(conf, k, module)

    def int8_map(self):
        return {name[:-len(".weight")]: self.int8_layout(name, desc)
                for name, desc in self.tensors.items() if desc["dtype"] == "I8"}


def annotate_quantized(tensors, read_json):
    """tensors: name -> desc.  Weights with comfy_quant get their logical shape ("shape"), their
    on-disk shape ("stored_shape") and their record ("comfy_quant").  Returns {module: record}."""
    return QuantHeader(tensors, read_json).annotate()


def int8_quantization(tensors, read_json):
    """Native int8 storage map of a checkpoint header: {module: {convrot, group_size}} for every I8
    Linear weight, with the row-wise F32 [N, 1] scale checked (powershard/checkpoint.py:63-82)."""
    return QuantHeader(tensors, read_json).int8_map()


def module_entries(tensors, module):
    """A module's own tensors (weight + scales / zero / extras), bias excluded: name -> file key."""
    return {name: desc["key"] for name, desc in QuantHeader(tensors).own(module).items()}


def formats_summary(configs):
    """{format: number of modules} of annotate_quantized's result."""
    counts = {}
    for conf in configs.values():
        counts[conf["format"]] = counts.get(conf["format"], 0) + 1
    return counts


# ------------------------------------------------------------------ torch side
def dequantize_module(handle, entries, module, conf, shape, device, dtype):
    """A file module's full dequantized weight.  entries: name -> file key."""
    import torch
    from .quant_linear import quantized_from_file
    names = {n: k for n, k in entries.items() if not n.endswith(QUANT_SUFFIX)}
    full = quantized_from_file(handle, names, module, conf, shape, device, dtype).dequantize()
    pre_key = names.get(module + ".pre_quant_scale")
    if pre_key is not None:
        # ModelOpt AWQ: y = (x * s) Wq^T = x (Wq * s)^T -- the input scale folds into the weight.
        full = full.float() * handle.get_tensor(pre_key).to(device).float().reshape(1, -1)
    full = full.to(device=device, dtype=dtype)
    if tuple(full.shape) != tuple(shape):
        raise ValueError(f"{module}: dequantized shape {tuple(full.shape)} != {tuple(shape)} ({conf.get('format')})")
    if not torch.isfinite(full).all():
        raise FloatingPointError(f"{module}: non-finite values after dequantization ({conf.get('format')})")
    return full


WEIGHT_FORMATS = ("dequantize", "as_file", "int8", "fp8", "mxfp8", "nvfp4", "int4")
COMPUTE_MODES = ("auto", "native", "dequantize")


def validate_quant_choice(weight_format, compute):
    """The node's two choices, checked against the vocabulary (ValueError names the options)."""
    for value, options, what in ((weight_format, WEIGHT_FORMATS, "weight_format"), (compute, COMPUTE_MODES, "compute")):
        if value not in options:
            raise ValueError(f"{what}: {' / '.join(options)}")


_BF16_ARCHS = ("gfx90a", "gfx94", "gfx95", "gfx11", "gfx12")


def _native_bf16(device):
    arch = str(device.get("arch") or "")
    if arch:
        return arch.startswith(_BF16_ARCHS)
    return tuple(device.get("capability") or (0, 0)) >= (8, 0)


def resolve_weight_dtype(choice, selected):
    """auto: bf16 when every selected GPU has native bf16 (CUDA sm80+, or a gfx90a+/RDNA3+ AMD GPU,
    MI355X included), else fp16.  selected: dicts with "capability" (CUDA) or "arch" (gcnArchName)."""
    if choice in ("fp16", "bf16"):
        return choice
    if choice != "auto":
        raise ValueError("weight_dtype: auto / fp16 / bf16")
    return "bf16" if selected and all(_native_bf16(d) for d in selected) else "fp16"
