"""Weight-format metadata of the quantized linear path: ``comfy_quant`` JSON, packed vs logical
shapes, the user vocabulary, and full-weight dequantization of a file module.

Mirrors powershard/quant_formats.py (PACKED_BITS / packed_bits / logical_shape / annotate_quantized /
module_entries / dequantize_module / WEIGHT_FORMATS / COMPUTE_MODES / validate_quant_choice /
resolve_weight_dtype) and the ``comfy_quant`` checks of powershard/checkpoint.py:63-82 and
powershard/wan_config.py:132-162.  The torch-free part (everything above ``dequantize_module``)
imports nothing but json, as in the reference, so node/config code can use it before any worker.
"""
import json

# Bits per element of packed storage (on disk [N, K * bits / 8]).
PACKED_BITS = {"nvfp4": 4, "asym_w4a8_int8": 4, "w6a8_int8": 6, "int4_asym_group": 4}
QUANT_SUFFIX = ".comfy_quant"


def packed_bits(conf):
    fmt = conf.get("format")
    if fmt == "convrot_w4a4":
        params = conf.get("params") if isinstance(conf.get("params"), dict) else {}
        return 4 if conf.get("linear_dtype", params.get("linear_dtype", "int4")) == "int4" else 8
    return PACKED_BITS.get(fmt, 8)


def logical_shape(stored_shape, conf):
    """Shape of the original (dequantized) weight from the stored shape and the format."""
    shape = list(stored_shape)
    bits = packed_bits(conf)
    if len(shape) == 2 and bits != 8:
        if (shape[1] * 8) % bits:
            raise ValueError(f"{conf.get('format')}: width {shape[1]} does not match {bits}-bit packing")
        shape[1] = shape[1] * 8 // bits
    return shape


def read_quant_json(path, data_start, desc):
    a, b = desc["data_offsets"]
    if desc["dtype"] != "U8" or b - a > 1 << 20:
        raise ValueError("Invalid comfy_quant metadata")
    with open(path, "rb") as f:
        f.seek(data_start + a)
        return json.loads(f.read(b - a))


def annotate_quantized(tensors, read_json):
    """tensors: name -> desc.  Weights with comfy_quant get their logical shape.

    desc["shape"] becomes the logical shape, desc["stored_shape"] the on-disk one and
    desc["comfy_quant"] the format config.  Returns {module: config}.
    """
    configs = {}
    for name in [n for n in tensors if n.endswith(QUANT_SUFFIX)]:
        module = name[:-len(QUANT_SUFFIX)]
        conf = read_json(name)
        if not isinstance(conf, dict) or not conf.get("format"):
            raise ValueError(f"comfy_quant without a format: {name}")
        configs[module] = conf
        weight = tensors.get(module + ".weight")
        if weight is not None:
            weight["stored_shape"] = list(weight["shape"])
            weight["shape"] = logical_shape(weight["shape"], conf)
            weight["comfy_quant"] = conf
    return configs


def convrot_config(conf, in_features, module="?"):
    """{convrot, group_size} of an int8_tensorwise comfy_quant config (powershard/checkpoint.py:63-82):
    the group is a power of 4 dividing in_features; ``convrot_groupsize`` defaults to 256 and may
    also sit under ``params``."""
    params = conf.get("params") if isinstance(conf.get("params"), dict) else {}
    gs = int(conf.get("convrot_groupsize", params.get("convrot_groupsize", 256)))
    convrot = bool(conf.get("convrot", params.get("convrot", False)))
    if convrot and (gs < 4 or gs & (gs - 1) or (gs.bit_length() - 1) % 2 or in_features % gs):
        raise ValueError(f"Invalid ConvRot group: {module}")
    return {"convrot": convrot, "group_size": gs}


def int8_quantization(tensors, read_json):
    """Native int8 storage map of a checkpoint header: {module: {convrot, group_size}} for every I8
    Linear weight, with the row-wise F32 [N, 1] scale checked (powershard/checkpoint.py:63-82)."""
    configs = {}
    for name, d in tensors.items():
        if d["dtype"] != "I8":
            continue
        if not name.endswith(".weight") or len(d["shape"]) != 2:
            raise ValueError(f"INT8 outside a Linear: {name}")
        module = name[:-len(".weight")]
        if module + QUANT_SUFFIX not in tensors:
            raise ValueError(f"INT8 without comfy_quant metadata: {module}")
        conf = read_json(module + QUANT_SUFFIX)
        if conf.get("format") != "int8_tensorwise":
            raise ValueError(f"Unsupported quantization of {module}: {conf}")
        scale = tensors.get(module + ".weight_scale")
        if scale is None or scale["shape"] != [d["shape"][0], 1] or scale["dtype"] != "F32":
            raise ValueError(f"Expected a row-wise FP32 scale: {module}")
        configs[module] = convrot_config(conf, d["shape"][1], module)
    return configs


def module_entries(tensors, module):
    """A module's own tensors (weight + scales / zero / extras), bias excluded: name -> file key."""
    prefix = module + "."
    return {name: desc["key"] for name, desc in tensors.items()
            if name.startswith(prefix) and "." not in name[len(prefix):] and not name.endswith(".bias")}


def formats_summary(configs):
    out = {}
    for conf in configs.values():
        out[conf["format"]] = out.get(conf["format"], 0) + 1
    return out


# ------------------------------------------------------------------ torch side
def dequantize_module(handle, entries, module, conf, shape, device, dtype):
    """A file module's full dequantized weight.  entries: name -> file key."""
    import torch
    from .quant_linear import quantized_from_file
    prefix = module + "."
    names = {n: k for n, k in entries.items() if not n.endswith(QUANT_SUFFIX)}
    qt = quantized_from_file(handle, names, module, conf, shape, device, dtype)
    full = qt.dequantize()
    pre_key = names.get(prefix + "pre_quant_scale")
    if pre_key is not None:
        # ModelOpt AWQ: y = (x * s) Wq^T = x (Wq * s)^T -- the input scale folds into the weight.
        pre = handle.get_tensor(pre_key).to(device).float()
        full = full.float() * pre.reshape(1, -1)
    full = full.to(device=device, dtype=dtype)
    if tuple(full.shape) != tuple(shape):
        raise ValueError(f"{module}: dequantized shape {tuple(full.shape)} != {tuple(shape)} ({conf.get('format')})")
    if not torch.isfinite(full).all():
        raise FloatingPointError(f"{module}: non-finite values after dequantization ({conf.get('format')})")
    return full


WEIGHT_FORMATS = ("dequantize", "as_file", "int8", "fp8", "mxfp8", "nvfp4", "int4")
COMPUTE_MODES = ("auto", "native", "dequantize")


def validate_quant_choice(weight_format, compute):
    if weight_format not in WEIGHT_FORMATS:
        raise ValueError(f"weight_format: {' / '.join(WEIGHT_FORMATS)}")
    if compute not in COMPUTE_MODES:
        raise ValueError(f"compute: {' / '.join(COMPUTE_MODES)}")


_BF16_ARCHS = ("gfx90a", "gfx94", "gfx95", "gfx11", "gfx12")


def resolve_weight_dtype(choice, selected):
    """auto: bf16 when every selected GPU has native bf16 (CUDA sm80+, or a gfx90a+/RDNA3+ AMD GPU,
    MI355X included), else fp16.  selected: dicts with "capability" (CUDA) or "arch" (gcnArchName)."""
    if choice in ("fp16", "bf16"):
        return choice
    if choice != "auto":
        raise ValueError("weight_dtype: auto / fp16 / bf16")

    def bf16(d):
        arch = str(d.get("arch") or "")
        if arch:
            return arch.startswith(_BF16_ARCHS)
        return tuple(d.get("capability") or (0, 0)) >= (8, 0)
    return "bf16" if selected and all(bf16(d) for d in selected) else "fp16"
