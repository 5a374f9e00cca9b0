"""powershard_amd -- MI355X (gfx950) native quantized linear path of ComfyUI-PowerShard.

Modules (each mirrors the reference module of the same name):
  quant_linear   QuantLinear / QuantPlan / pack / unpack / install_quant_linears / build_bytes
  quant_formats  comfy_quant metadata, packed shapes, vocabulary, dequantize_module
  operations     regular_hadamard / dequantize_rows / Int8Linear / install_int8
  quant_tensor   QuantizedWeight and its three layouts (int8 rows + ConvRot, fp8 e4m3fn, uint4 groups)
  mlp            chunked Linear -> GELU(tanh) -> Linear (the Wan FFN) with the GELU in the GEMM epilogue
  ops            torch-facing wrappers of the HIP kernels in libpsquant.so
"""
__version__ = "0.1.0"
