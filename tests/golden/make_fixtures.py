"""Writes the data fixtures of tests/golden from the reference's model metadata (data only).

    python tests/golden/make_fixtures.py [/root/reference]

* convrot_config.json -- models/convrot_config.json: the exact 72-byte ``comfy_quant`` payload
  stored (as U8[72]) beside every int8 ConvRot weight of the reference's checkpoints.
* int8_convrot_header_subset.json -- the block-0 attention/MLP entries (I8 weights, F32 [N, 1]
  scales, U8[72] comfy_quant) of models/minimax_h3_fl2va_pruned_int8_convrot.safetensors.header.json
  and the Qwen3-VL-32B MLP entries of models/qwen3vl_32b_minimax_h3_int8_convrot.safetensors.header.json:
  real layouts that the loader checks are run against.
"""
import json
import os
import shutil
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
out = os.path.dirname(os.path.abspath(__file__))
shutil.copyfile(os.path.join(ref, "models", "convrot_config.json"), os.path.join(out, "convrot_config.json"))
subset = {}
h3 = json.load(open(os.path.join(ref, "models", "minimax_h3_fl2va_pruned_int8_convrot.safetensors.header.json")))
for k, v in h3.items():
    if k.startswith(("blocks.0.attn.qkv_proj.", "blocks.0.attn.out_proj.", "blocks.0.mlp.fc1.", "blocks.0.mlp.fc2.")):
        subset[k] = {"dtype": v["dtype"], "shape": v["shape"]}
qw = json.load(open(os.path.join(ref, "models", "qwen3vl_32b_minimax_h3_int8_convrot.safetensors.header.json")))
for k, v in qw.items():
    if isinstance(v, dict) and ".layers.0.mlp." in k:
        subset[k] = {"dtype": v["dtype"], "shape": v["shape"]}
json.dump(dict(sorted(subset.items())), open(os.path.join(out, "int8_convrot_header_subset.json"), "w"), indent=1)
print(f"wrote {len(subset)} header entries")
