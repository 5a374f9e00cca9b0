"""ComfyUI custom-node entry of comfyui-powershard_amd.

The package proper is ``powershard_amd`` (the MI355X quantized linear path); this file only makes it
importable when ComfyUI loads the directory as a custom node.  The quantized path adds no nodes of
its own: the reference's weight-format node vocabulary (``weight_format`` / ``compute``) is kept
by ``powershard_amd.quant_formats``.
"""
import os
import sys

_here = os.path.dirname(os.path.abspath(__file__))
if _here not in sys.path:
    sys.path.insert(0, _here)

NODE_CLASS_MAPPINGS = {}
NODE_DISPLAY_NAME_MAPPINGS = {}
