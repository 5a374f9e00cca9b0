"""Host logic of the drop-in boundary on the CPU (no GPU): QuantPlan / pack / unpack, QuantLinear in the
dequantize compute mode, the native-failure fallback convention, installation, file loading and the
format vocabulary.  Mirrors the reference's tests/test_quant_formats_torch.py (which needed ComfyUI),
tests/test_portable.py:50-72 and tests/test_fp16_safe.py:71-85.
"""
import json
import os
import warnings

import pytest
import torch
from torch import nn

import oracle
from powershard_amd import quant_formats as qf
from powershard_amd import quant_linear as ql
from powershard_amd import quant_tensor as qtm
from powershard_amd.operations import Int8Linear, dequantize_rows, install_int8, regular_hadamard

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FORMATS = {"int8": "int8_tensorwise", "fp8": "float8_e4m3fn", "int4": "int4_asym_group"}


def make_layer(weight_format, compute="dequantize", K=128, N=64, opts=None, dtype=torch.bfloat16):
    torch.manual_seed(0)
    net = nn.Sequential(nn.Linear(K, N)).to(dtype)
    tensors = {"0.weight": {"key": "0.weight", "dtype": "BF16", "shape": [N, K]}}
    report = ql.install_quant_linears(net, tensors, weight_format, compute, None, dtype, torch.device("cpu"),
                                      quant_options=opts)
    return net, report


@pytest.mark.parametrize("weight_format", ["int8", "fp8", "int4"])
def test_quant_linear_pack_unpack_dequantize(weight_format):
    """Byte vector (as after an FSDP all-gather) -> QuantizedWeight -> GEMM == dequant reference
    (tests/test_quant_formats_torch.py:79-103)."""
    fmt = FORMATS[weight_format]
    net, report = make_layer(weight_format)
    layer = net[0]
    assert isinstance(layer, ql.QuantLinear) and report["modules"][fmt]["count"] == 1
    assert layer.weight is None and layer.comfy_force_forward
    weight = torch.randn(64, 128, dtype=torch.bfloat16)
    qt = ql.quantized_from_float(weight, fmt)
    layer.qbytes = nn.Parameter(ql.pack(qt, layer._ps_qplan, "cpu"), requires_grad=False)
    layer.bias = nn.Parameter(torch.zeros(64, dtype=torch.bfloat16), requires_grad=False)
    x = torch.randn(2, 3, 128, dtype=torch.bfloat16)
    out = layer(x)
    ref = torch.nn.functional.linear(x, qt.dequantize().to(torch.bfloat16))
    assert out.shape == (2, 3, 64)
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)
    # the dequantized weight is close to the float weight (quantization error only)
    rel = (qt.dequantize().float() - weight.float()).norm() / weight.float().norm()
    assert rel < {"int8": 0.02, "fp8": 0.05, "int4": 0.15}[weight_format]


def test_plan_layout_is_aligned_and_qdata_first():
    net, _ = make_layer("int4")
    plan = net[0]._ps_qplan
    names = [s[0] for s in plan.specs]
    assert names == ["_qdata", "scale", "zero"]
    assert all(off % ql.ALIGN == 0 for _, _, _, off, _ in plan.specs)
    assert plan.total == sum(-(-nb // 16) * 16 for *_, nb in plan.specs)
    assert net[0].qbytes.dtype == torch.uint8 and net[0].qbytes.shape == (plan.total,)
    assert list(plan.signature()[0]) == ["_qdata", "torch.uint8", [64, 64], 0, 64 * 64]


def test_unpack_is_zero_copy():
    net, _ = make_layer("int8")
    layer = net[0]
    qt = ql.quantized_from_float(torch.randn(64, 128), "int8_tensorwise")
    full = ql.pack(qt, layer._ps_qplan, "cpu")
    back = ql.unpack(full, layer._ps_qplan, torch.bfloat16)
    assert back._qdata.data_ptr() == full.data_ptr()
    assert torch.equal(back._qdata, qt._qdata) and torch.equal(back._params.scale, qt._params.scale)
    assert back._params.orig_dtype == torch.bfloat16


def test_pack_rejects_layout_mismatch():
    net, _ = make_layer("int8")
    plan = net[0]._ps_qplan
    other = ql.quantized_from_float(torch.randn(64, 256), "int8_tensorwise")
    with pytest.raises(RuntimeError):
        ql.pack(other, plan, "cpu")
    rot = ql.quantized_from_float(torch.randn(64, 128), "int8_tensorwise", convrot=True, convrot_groupsize=16)
    with pytest.raises(RuntimeError):   # same tensors, different ConvRot parameters
        ql.pack(rot, plan, "cpu")


def test_extras_are_stored_after_params():
    qt = ql.quantized_from_float(torch.randn(32, 64), "int8_tensorwise")
    extras = {"pre_quant_scale": torch.rand(64), "input_scale": torch.tensor([0.1])}
    plan = ql.plan_from_quantized(qt, "int8_tensorwise", {}, extras)
    assert [s[0] for s in plan.specs] == ["_qdata", "scale", "x:input_scale", "x:pre_quant_scale"]
    full = ql.pack(qt, plan, "cpu", extras)
    _, ex = ql.unpack(full, plan, with_extras=True)
    assert torch.equal(ex["pre_quant_scale"], extras["pre_quant_scale"])


def test_native_failure_warns_and_falls_back():
    """The reference's convention (quant_linear.py:207-215): a native failure warns once and the
    module stays on dequantize.  On the CPU the native kernels refuse to run."""
    net, _ = make_layer("int8", compute="native")
    layer = net[0]
    assert layer._ps_native
    qt = ql.quantized_from_float(torch.randn(64, 128), "int8_tensorwise")
    layer.qbytes = nn.Parameter(ql.pack(qt, layer._ps_qplan, "cpu"), requires_grad=False)
    x = torch.randn(4, 128, dtype=torch.bfloat16)
    with pytest.warns(UserWarning, match="switches to dequantize"):
        out = layer(x)
    assert not layer._ps_native and out.shape == (4, 64)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        layer(x)   # no second warning


def test_follow_input_keeps_fp32_graph():
    net, _ = make_layer("int8")
    layer = net[0]
    layer._ps_follow_input = True
    layer.qbytes = nn.Parameter(ql.pack(ql.quantized_from_float(torch.randn(64, 128), "int8_tensorwise"),
                                        layer._ps_qplan, "cpu"), requires_grad=False)
    out = layer(torch.randn(3, 128))
    assert out.dtype == torch.float32


def test_install_scope_fp32_islands_and_report():
    net = nn.ModuleDict({"blocks": nn.ModuleList([nn.Linear(128, 64).to(torch.bfloat16) for _ in range(2)]),
                         "head": nn.Linear(128, 64).to(torch.bfloat16),
                         "island": nn.Linear(128, 64)})
    tensors = {f"{n}.weight": {"key": f"{n}.weight", "dtype": "BF16", "shape": [64, 128]}
               for n in ("blocks.0", "blocks.1", "head", "island")}
    report = ql.install_quant_linears(net, tensors, "int8", "dequantize", ("blocks.",), torch.bfloat16, "cpu")
    assert isinstance(net["blocks"][0], ql.QuantLinear) and isinstance(net["blocks"][1], ql.QuantLinear)
    assert not isinstance(net["head"], ql.QuantLinear) and not isinstance(net["island"], ql.QuantLinear)
    assert report["modules"]["int8_tensorwise"]["count"] == 2
    assert report["modules"]["int8_tensorwise"]["native"] is False
    assert report["stored_bytes"] == 2 * net["blocks"][0]._ps_qplan.total
    assert ql.install_quant_linears(net, tensors, "dequantize", "auto", None, torch.bfloat16, "cpu")["modules"] == {}


def test_auto_compute_on_cpu_is_dequantize():
    _, report = make_layer("int8", compute="auto")
    assert report["modules"]["int8_tensorwise"]["native"] is False
    assert report["modules"]["int8_tensorwise"]["reason"] == "not a GPU"


def test_blackwell_formats_are_refused():
    with pytest.raises(ValueError):
        make_layer("nvfp4")


def test_fits_blocks():
    assert not ql.fits_blocks(nn.Linear(64, 8), "int8_tensorwise")
    assert ql.fits_blocks(nn.Linear(128, 16), "int8_tensorwise")
    assert not ql.fits_blocks(nn.Linear(96, 64), "int4_asym_group")


# ------------------------------------------------------------------- file loading
def _save(tmp_path, tensors, conf=None, name="m"):
    from safetensors.torch import save_file
    tensors = dict(tensors)
    if conf is not None:
        tensors[f"{name}.comfy_quant"] = torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)
    path = tmp_path / "w.safetensors"
    save_file(tensors, str(path))
    return path


def _table(path):
    from safetensors import safe_open
    code = {torch.float32: "F32", torch.float16: "F16", torch.bfloat16: "BF16", torch.int8: "I8",
            torch.uint8: "U8", torch.float8_e4m3fn: "F8_E4M3", torch.float8_e5m2: "F8_E5M2"}
    with safe_open(str(path), framework="pt") as f:
        table = {k: {"key": k, "dtype": code[f.get_tensor(k).dtype], "shape": list(f.get_tensor(k).shape)}
                 for k in f.keys()}
        confs = qf.annotate_quantized(table, lambda n: json.loads(bytes(f.get_tensor(n).tolist())))
    return table, confs


def test_int8_rowwise_file_dequantizes_to_q_times_scale(tmp_path):
    """tests/test_quant_formats_torch.py:38-44."""
    from safetensors import safe_open
    g = torch.Generator().manual_seed(0)
    q = torch.randint(-127, 128, (8, 16), generator=g, dtype=torch.int8)
    scale = torch.rand((8, 1), generator=g) * .01
    conf = {"format": "int8_tensorwise"}
    path = _save(tmp_path, {"m.weight": q, "m.weight_scale": scale}, conf)
    table, _ = _table(path)
    with safe_open(str(path), framework="pt") as f:
        out = qf.dequantize_module(f, qf.module_entries(table, "m"), "m", conf, [8, 16], torch.device("cpu"),
                                   torch.float32)
    torch.testing.assert_close(out, q.float() * scale)


def test_fp8_scaled_file(tmp_path):
    """tests/test_quant_formats_torch.py:47-53."""
    from safetensors import safe_open
    w = torch.randn(8, 16)
    scale = w.abs().max() / 448.
    q = (w / scale).to(torch.float8_e4m3fn)
    conf = {"format": "float8_e4m3fn"}
    path = _save(tmp_path, {"m.weight": q, "m.weight_scale": scale.reshape(())}, conf)
    table, _ = _table(path)
    with safe_open(str(path), framework="pt") as f:
        out = qf.dequantize_module(f, qf.module_entries(table, "m"), "m", conf, [8, 16], torch.device("cpu"),
                                   torch.float32)
        plain = ql.float_weight(f, {"m.weight": {"key": "m.weight", "dtype": "F8_E4M3", "shape": [8, 16]},
                                    "m.weight_scale": {"key": "m.weight_scale", "dtype": "F32", "shape": []}},
                                "m.weight", "cpu")
    torch.testing.assert_close(out, q.float() * scale)
    torch.testing.assert_close(plain, q.float() * scale)


def test_e5m2_scaled_file_module_as_file(tmp_path):
    """A float8_e5m2 comfy_quant module (F8_E5M2 weight, F32 per-tensor weight_scale) loads as_file:
    its qbytes keep the e5m2 codes, unpack rebuilds them, and the dequantize branch equals the
    reference's decode q * s (the plain formula of powershard/quant_formats.py:95-103)."""
    from safetensors import safe_open
    g = torch.Generator().manual_seed(3)
    w = torch.randn(32, 256, generator=g)
    scale = w.abs().max() / 57344.0
    q = (w / scale).to(torch.float8_e5m2)
    conf = {"format": "float8_e5m2"}
    path = _save(tmp_path, {"m.weight": q, "m.weight_scale": scale.reshape(()), "m.bias": torch.zeros(32)}, conf)
    table, confs = _table(path)
    assert confs == {"m": conf}
    with safe_open(str(path), framework="pt") as f:
        out = qf.dequantize_module(f, qf.module_entries(table, "m"), "m", conf, [32, 256], torch.device("cpu"),
                                   torch.float32)
    torch.testing.assert_close(out, q.float() * scale)
    net = nn.ModuleDict({"m": nn.Linear(256, 32).to(torch.bfloat16)})
    report = ql.install_quant_linears(net, table, "as_file", "dequantize", None, torch.bfloat16, "cpu")
    layer = net["m"]
    assert report["modules"]["float8_e5m2"]["source"] == {"file": 1}
    with safe_open(str(path), framework="pt") as f:
        full, used = ql.build_bytes(layer, f, "cpu")
    assert used == {"m.weight", "m.weight_scale", "m.comfy_quant"}
    qt = ql.unpack(full, layer._ps_qplan, torch.bfloat16)
    assert qt._qdata.dtype == torch.float8_e5m2 and torch.equal(qt._qdata.view(torch.uint8), q.view(torch.uint8))
    layer.qbytes = nn.Parameter(full, requires_grad=False)
    layer.bias = None
    x = torch.randn(5, 256, dtype=torch.bfloat16)
    ref = torch.nn.functional.linear(x, (q.float() * scale).to(torch.bfloat16))
    torch.testing.assert_close(layer(x), ref, atol=0, rtol=0)


def test_e5m2_requantize_keeps_the_format():
    """A LoRA merge re-quantizes an e5m2 weight into e5m2 (scale absmax / 57344), as the template."""
    g = torch.Generator().manual_seed(4)
    w = torch.randn(16, 128, generator=g)
    qt = ql.quantized_from_float(w, "float8_e5m2")
    assert qt._qdata.dtype == torch.float8_e5m2
    assert torch.equal(qt._params.scale, w.abs().max() / 57344.0)
    again = ql.requantize_like(qt, w * 2, "float8_e5m2")
    assert again._qdata.dtype == torch.float8_e5m2
    torch.testing.assert_close(again.dequantize().float(), (w * 2).to(torch.bfloat16).float(), rtol=0.13, atol=1e-6)


def test_convrot_file_module_loads_as_file_and_matches_dequantize_rows(tmp_path):
    """as_file: an int8 ConvRot comfy_quant module keeps its file layout in qbytes; the forward
    equals F.linear with dequantize_rows (powershard/operations.py:84-93)."""
    from safetensors import safe_open
    conf = json.load(open(os.path.join(GOLDEN, "convrot_config.json")))
    w = torch.randn(32, 512)
    q, s = oracle.quantize_weight_int8(w, True, 256)
    path = _save(tmp_path, {"m.weight": q, "m.weight_scale": s, "m.bias": torch.zeros(32)}, conf)
    table, confs = _table(path)
    assert confs == {"m": conf} and table["m.weight"]["comfy_quant"] == conf
    net = nn.ModuleDict({"m": nn.Linear(512, 32).to(torch.bfloat16)})
    report = ql.install_quant_linears(net, table, "as_file", "dequantize", None, torch.bfloat16, "cpu")
    layer = net["m"]
    assert report["modules"]["int8_tensorwise"]["source"] == {"file": 1}
    with safe_open(str(path), framework="pt") as f:
        full, used = ql.build_bytes(layer, f, "cpu")
    assert used == {"m.weight", "m.weight_scale", "m.comfy_quant"}
    layer.qbytes = nn.Parameter(full, requires_grad=False)
    layer.bias = None
    x = torch.randn(5, 512, dtype=torch.bfloat16)
    ref = torch.nn.functional.linear(x, dequantize_rows(q, s, True, 256, torch.bfloat16))
    torch.testing.assert_close(layer(x).float(), ref.float(), atol=2e-2, rtol=2e-2)


def test_open_file_builds_the_template_when_shapes_are_not_enough(tmp_path, monkeypatch):
    """powershard/quant_linear.py:329-337: when a file template cannot be built from shapes (meta
    tensors), install_quant_linears opens the file through open_file(table, key) and builds it from
    the real tensors; without open_file the error propagates.  Forced here by a decoder that refuses
    meta tensors, as a format whose layout depends on the data would."""
    from safetensors import safe_open
    conf = json.load(open(os.path.join(GOLDEN, "convrot_config.json")))
    w = torch.randn(32, 512)
    q, s = oracle.quantize_weight_int8(w, True, 256)
    path = _save(tmp_path, {"m.weight": q, "m.weight_scale": s, "m.bias": torch.zeros(32)}, conf)
    table, _ = _table(path)
    real_from_file = ql.quantized_from_file

    def needs_data(handle, entries, module, conf, shape, device, dtype, meta=False):
        if meta:
            raise RuntimeError("this layout needs the data")
        return real_from_file(handle, entries, module, conf, shape, device, dtype, meta)
    monkeypatch.setattr(ql, "quantized_from_file", needs_data)
    with pytest.raises(RuntimeError, match="needs the data"):
        ql.install_quant_linears(nn.ModuleDict({"m": nn.Linear(512, 32).to(torch.bfloat16)}), table, "as_file",
                                 "dequantize", None, torch.bfloat16, "cpu")
    opened = []
    with safe_open(str(path), framework="pt") as f:
        def open_file(tab, key):
            opened.append(key)
            return f
        net = nn.ModuleDict({"m": nn.Linear(512, 32).to(torch.bfloat16), "n": nn.Linear(512, 32).to(torch.bfloat16)})
        table2 = dict(table)
        for k in [k for k in table if k.startswith("m.")]:   # a second module of the same layout
            table2["n." + k[2:]] = dict(table[k], key=k)
        report = ql.install_quant_linears(net, table2, "as_file", "dequantize", None, torch.bfloat16, "cpu",
                                          open_file=open_file)
        assert opened == ["m.weight"], "one template per layout signature, opened once"
        assert report["modules"]["int8_tensorwise"]["count"] == 2
        monkeypatch.setattr(ql, "quantized_from_file", real_from_file)
        layer = net["m"]
        full, _ = ql.build_bytes(layer, f, "cpu")
    layer.qbytes = nn.Parameter(full, requires_grad=False)
    layer.bias = None
    x = torch.randn(5, 512, dtype=torch.bfloat16)
    ref = torch.nn.functional.linear(x, dequantize_rows(q, s, True, 256, torch.bfloat16))
    torch.testing.assert_close(layer(x).float(), ref.float(), atol=2e-2, rtol=2e-2)


def test_quantize_at_load_from_bf16_file(tmp_path):
    from safetensors import safe_open
    w = torch.randn(64, 256, dtype=torch.bfloat16)
    path = _save(tmp_path, {"0.weight": w})
    table, _ = _table(path)
    for weight_format, opts in (("int8", {"convrot": True, "convrot_groupsize": 256}), ("fp8", None),
                                ("int4", {"group_size": 128})):
        net = nn.Sequential(nn.Linear(256, 64).to(torch.bfloat16))
        ql.install_quant_linears(net, table, weight_format, "dequantize", None, torch.bfloat16, "cpu",
                                 quant_options=opts)
        layer = net[0]
        with safe_open(str(path), framework="pt") as f:
            full, used = ql.build_bytes(layer, f, "cpu")
        assert used == {"0.weight"} and full.numel() == layer._ps_qplan.total
        qt = ql.unpack(full, layer._ps_qplan, torch.float32)
        rel = (qt.dequantize() - w.float()).norm() / w.float().norm()
        assert rel < 0.15, (weight_format, rel)


def test_lora_delta_requantizes_like_template(tmp_path):
    from safetensors import safe_open
    conf = {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 16}
    w = torch.randn(16, 64)
    q, s = oracle.quantize_weight_int8(w, True, 16)
    path = _save(tmp_path, {"m.weight": q, "m.weight_scale": s}, conf)
    table, _ = _table(path)
    net = nn.ModuleDict({"m": nn.Linear(64, 16, bias=False).to(torch.bfloat16)})
    ql.install_quant_linears(net, table, "as_file", "dequantize", None, torch.bfloat16, "cpu")
    delta = torch.randn(16, 64) * 0.1
    with safe_open(str(path), framework="pt") as f:
        full, _ = ql.build_bytes(net["m"], f, "cpu", lambda key, shape, dev: delta)
    qt = ql.unpack(full, net["m"]._ps_qplan, torch.float32)
    assert qt._params.convrot and qt._params.convrot_groupsize == 16
    target = dequantize_rows(q, s, True, 16, torch.float32) + delta
    assert (qt.dequantize() - target).norm() / target.norm() < 0.02


def test_non_finite_weights_are_refused(tmp_path):
    from safetensors import safe_open
    w = torch.randn(16, 128)
    w[3, 5] = float("nan")
    path = _save(tmp_path, {"0.weight": w})
    table, _ = _table(path)
    net = nn.Sequential(nn.Linear(128, 16).to(torch.bfloat16))
    ql.install_quant_linears(net, table, "int8", "dequantize", None, torch.bfloat16, "cpu")
    with safe_open(str(path), framework="pt") as f, pytest.raises(FloatingPointError):
        ql.build_bytes(net[0], f, "cpu")


# ------------------------------------------------------------------ metadata
def test_convrot_config_fixture_is_the_72_byte_payload():
    """models/convrot_config.json: the exact comfy_quant U8[72] payload of the int8 ConvRot files."""
    raw = open(os.path.join(GOLDEN, "convrot_config.json"), "rb").read().strip()
    assert len(raw) == 72
    conf = json.loads(raw)
    assert qf.convrot_config(conf, 5376) == {"convrot": True, "group_size": 256}
    with pytest.raises(ValueError):
        qf.convrot_config(dict(conf, convrot_groupsize=128), 5376)
    with pytest.raises(ValueError):
        qf.convrot_config(conf, 5000)
    assert qf.convrot_config({"format": "int8_tensorwise", "params": {"convrot": True, "convrot_groupsize": 64}},
                             128) == {"convrot": True, "group_size": 64}


def test_real_header_int8_quantization_map():
    """Real int8-ConvRot checkpoint header entries (models/*_int8_convrot.safetensors.header.json)."""
    header = json.load(open(os.path.join(GOLDEN, "int8_convrot_header_subset.json")))
    conf = json.load(open(os.path.join(GOLDEN, "convrot_config.json")))
    configs = qf.int8_quantization(header, lambda name: conf)
    assert configs["blocks.0.mlp.fc1"] == {"convrot": True, "group_size": 256}
    assert header["blocks.0.mlp.fc1.weight"]["shape"] == [28672, 5376]
    bad = dict(header)
    bad["blocks.0.mlp.fc1.weight_scale"] = dict(bad["blocks.0.mlp.fc1.weight_scale"], shape=[28672])
    with pytest.raises(ValueError):
        qf.int8_quantization(bad, lambda name: conf)


def test_packed_and_logical_shapes():
    assert qf.logical_shape([25600, 2560], {"format": "int4_asym_group"}) == [25600, 5120]
    assert qf.logical_shape([64, 32], {"format": "nvfp4"}) == [64, 64]
    assert qf.logical_shape([64, 48], {"format": "w6a8_int8"}) == [64, 64]
    assert qf.logical_shape([64, 64], {"format": "convrot_w4a4", "linear_dtype": "int8"}) == [64, 64]
    assert qf.logical_shape([13824, 5120], {"format": "int8_tensorwise"}) == [13824, 5120]
    with pytest.raises(ValueError):
        qf.logical_shape([64, 34], {"format": "w6a8_int8"})


def test_vocabulary():
    qf.validate_quant_choice("int8", "native")
    with pytest.raises(ValueError):
        qf.validate_quant_choice("int3", "auto")
    with pytest.raises(ValueError):
        qf.validate_quant_choice("int8", "fast")
    assert qf.resolve_weight_dtype("auto", [{"arch": "gfx950"}]) == "bf16"
    assert qf.resolve_weight_dtype("auto", [{"capability": (7, 0)}]) == "fp16"
    assert qf.resolve_weight_dtype("fp16", []) == "fp16"


# --------------------------------------------------------------- operations
def test_regular_hadamard_matches_oracle_and_is_orthonormal():
    for g in (4, 16, 64, 256):
        h = regular_hadamard(g, "cpu")
        assert torch.equal(h, oracle.regular_hadamard(g))
    with pytest.raises(ValueError):
        regular_hadamard(32, "cpu")


def test_convrot_int8linear():
    """tests/test_portable.py:50-67 (without the comfy-kitchen cross-check, which is absent here)."""
    h = regular_hadamard(256, "cpu")
    torch.testing.assert_close(h @ h.T, torch.eye(256), rtol=0, atol=0)
    g = torch.Generator().manual_seed(5)
    q = torch.randint(-100, 100, (13, 512), generator=g, dtype=torch.int8)
    scale = torch.rand((13, 1), generator=g) * .001
    actual = dequantize_rows(q, scale, True, 256)
    expected = oracle.dequantize_rows(q, scale, True, 256, torch.float16)
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)
    src = nn.Linear(512, 13, bias=False, device="meta", dtype=torch.float16)
    layer = Int8Linear(src, dict(convrot=True, group_size=256), rows=4).to_empty(device="cpu")
    layer.weight.data.copy_(q)
    layer.weight_scale.data.copy_(scale)
    x = torch.randn(3, 512, generator=g).half()
    torch.testing.assert_close(layer(x), torch.nn.functional.linear(x, expected), atol=1e-3, rtol=1e-3)
    assert layer.weight.dtype == torch.int8 and not layer.weight.requires_grad
    assert not any(p.dtype == torch.float16 and p.shape == q.shape for p in layer.parameters())
    # parameter bytes: int8 weight + fp32 row scale only (tests/test_fp16_safe.py:85)
    assert sum(p.numel() * p.element_size() for p in layer.parameters()) == 13 * 512 + 13 * 4


def test_dequantize_rows_overflow_guard():
    """tests/test_portable.py:70-72."""
    q = torch.full((4, 256), 127, dtype=torch.int8)
    with pytest.raises(FloatingPointError):
        dequantize_rows(q, torch.full((4, 1), 1e8), False, 256)
    assert dequantize_rows(torch.empty(0, 256, dtype=torch.int8), torch.empty(0, 1), True, 256).numel() == 0


def test_install_int8():
    model = nn.Sequential(nn.Linear(256, 32).half(), nn.Embedding(10, 4))
    skipped = install_int8(model, {"0": {"convrot": True, "group_size": 256}, "1": {"convrot": False,
                                                                                    "group_size": 256}}, 8)
    assert isinstance(model[0], Int8Linear) and "1" in skipped
    with pytest.raises(ValueError):
        install_int8(nn.Sequential(nn.Conv1d(2, 2, 1)), {"0": {"convrot": False, "group_size": 256}}, 8)


def test_reuse_quantized_inputs_nests_and_restores():
    from powershard_amd.quant_linear import _shared, reuse_quantized_inputs
    assert getattr(_shared, "cache", None) is None
    with reuse_quantized_inputs():
        outer = _shared.cache
        outer["k"] = 1
        with reuse_quantized_inputs():
            assert _shared.cache == {}
        assert _shared.cache is outer
    assert _shared.cache is None


def _int8linear(K, N, rows, seed, safe=False, group=256):
    g = torch.Generator().manual_seed(seed)
    src = nn.Linear(K, N, bias=True, device="meta", dtype=torch.float16)
    layer = Int8Linear(src, dict(convrot=True, group_size=group), rows=rows).to_empty(device="cpu")
    layer.weight.data.copy_(torch.randint(-100, 100, (N, K), generator=g, dtype=torch.int8))
    layer.weight_scale.data.copy_(torch.rand((N, 1), generator=g) * .001)
    layer.bias.data.copy_((torch.randn(N, generator=g) * 0.1).half())
    if safe:
        layer._ps_safe, layer._ps_fp32 = True, False
    return layer


@pytest.mark.parametrize("safe", [False, True])
def test_prepared_linears_reuse_the_per_call_tiles(safe):
    """operations.py:158-191: inside the block the tile path reuses tiles dequantized once; the
    outputs are those of the per-call tiles; the cache is gone after the block, also on an error."""
    from powershard_amd.operations import prepared_linears
    fc1, fc2 = _int8linear(512, 40, 16, 1, safe), _int8linear(256, 24, 8, 2, safe)
    other = nn.Linear(4, 4)
    x = torch.randn(5, 512).half()
    h = torch.randn(5, 256).half()
    ref1, ref2 = fc1(x), fc2(h)
    with prepared_linears((fc1, fc2, other), budget=1 << 30) as info:
        assert info["prepared_weight_bytes"] == (512 * 40 + 256 * 24) * (4 if safe else 2)
        assert len(fc1._ps_prepared) == 3 and len(fc2._ps_prepared) == 3
        assert torch.equal(fc1(x), ref1) and torch.equal(fc2(h), ref2)
    assert not hasattr(fc1, "_ps_prepared") and not hasattr(fc2, "_ps_prepared")
    with prepared_linears((fc1,), budget=100) as info:      # too small: per-call tiles
        assert info["prepared_weight_bytes"] == 0 and not hasattr(fc1, "_ps_prepared")
        assert torch.equal(fc1(x), ref1)
    with pytest.raises(KeyError):
        with prepared_linears((fc1,), budget=1 << 30, enabled=True):
            raise KeyError("inside")
    assert not hasattr(fc1, "_ps_prepared")
    with prepared_linears((fc1,), budget=1 << 30, enabled=False) as info:
        assert info["prepared_weight_bytes"] == 0 and not hasattr(fc1, "_ps_prepared")


def test_chunked_mlp_prepares_tiles_once_per_mlp(monkeypatch):
    """tests/test_mlp_policy.py:49-60: over 9 token chunks the row tiles are dequantized once per
    MLP (8 + 2 tiles), not once per chunk; the values are those of the unprepared loop."""
    import powershard_amd.operations as ops
    from powershard_amd import mlp
    fc1, fc2 = _int8linear(256, 64, 8, 5), _int8linear(64, 16, 8, 6, group=64)
    x = torch.randn(17, 256)
    ref = mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=2)
    count = 0
    original = ops.dequantize_rows

    def counted(*a, **kw):
        nonlocal count
        count += 1
        return original(*a, **kw)
    monkeypatch.setattr(ops, "dequantize_rows", counted)
    out = mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=2, prepare_budget=1 << 30)
    assert count == 64 // 8 + 16 // 8
    assert torch.equal(out, ref) and not hasattr(fc1, "_ps_prepared")
    count = 0
    mlp.chunked_mlp(fc1, fc2, x, chunk_tokens=2)
    assert count == 9 * (64 // 8 + 16 // 8)
    count = 0
    mlp.chunked_mlp(fc1, fc2, x, prepare_budget=1 << 30)         # one chunk: nothing prepared
    assert count == 64 // 8 + 16 // 8


def test_rows2d_packs_what_the_kernels_cannot_address():
    """The kernels address rows as base + m * ld with ld >= K, a multiple of 16 bytes, and a
    16-byte aligned base; every other layout is copied, the values unchanged."""
    from powershard_amd.ops import _rows2d
    base = torch.randn(8, 300)
    cases = {
        "packed": base[:, :256].contiguous(),
        "row slice": base[:, :256],                                   # ld 300: 1200 B, not 16-aligned
        "offset view": base.reshape(-1)[1:1 + 4 * 256].view(4, 256),  # base 4 B past an aligned one
        "broadcast rows": base[0, :256].expand(5, 256),               # ld 0
        "one column-major row": torch.randn(256, 1).t(),              # [1, 256] with ld 1
        "transposed": base[:, :8].t(),
    }
    for name, x in cases.items():
        y = _rows2d(x)
        assert torch.equal(y, x), name
        assert y.stride(1) == 1 and y.stride(0) >= y.shape[1], name
        assert (y.stride(0) * y.element_size()) % 16 == 0 and y.data_ptr() % 16 == 0, name
    packed = cases["packed"]
    assert _rows2d(packed).data_ptr() == packed.data_ptr()          # no copy when not needed
    assert _rows2d(torch.empty(0, 256)).shape == (0, 256)
