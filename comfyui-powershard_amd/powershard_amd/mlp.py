"""Linear -> GELU(tanh) / SiLU gate -> Linear over token chunks, the activation fused into the
up-projection.

Host side of the Wan FFN (powershard/wan_model.py:584-630, ``ffn_forward`` / ``chunked_mlp``).
Per chunk of token rows the reference computes

    hidden = F.gelu(fc1(rows).float(), approximate="tanh")     # fp32 [rows, hidden]
    result[a:b] = fc2(hidden).float()                          # fc2 first casts hidden to bf16

and so moves the hidden activation through HBM four times (fc1's bf16 output, its fp32 copy, the
fp32 GELU, fc2's bf16 cast).  Here fc1's W8A8 / FP8 GEMM applies the GELU to its rounded output in
the epilogue and writes the bf16 values fc2's cast would produce, once (QuantLinear.forward_act).
The reference's memory planner (``mlp_plan`` / ``mlp_budget``, chunk sizing from an allocator
budget) is not part of this package: ``chunk_tokens`` fixes the chunk size, None = one chunk.
The H3 MLP (powershard/fp16_safe.py:126-172, ``chunked_mlp_forward``) gates instead:
``gate, up = fc1(rows).chunk(2, -1); fc2(F.silu(gate.float()) * up.float())``; fc1's epilogue
computes silu(gate) * up from the two halves of its output and writes half the columns.
With ``prepare_budget`` and more than one chunk, Int8Linear layers on their row-tile path
dequantize their tiles once for all chunks (operations.prepared_linears, as the reference's H3
chunked MLP does, powershard/fp16_safe.py:126-172).
"""
import contextlib

import torch
import torch.nn.functional as F

from .operations import prepared_linears
from .quant_linear import QuantLinear

__all__ = ["gelu_linear", "silu_gate_linear", "chunked_mlp", "gated_mlp"]


def gelu_linear(linear, rows):
    """gelu_tanh(linear(rows)): fused for a QuantLinear (compute dtype), else the reference's fp32."""
    if isinstance(linear, QuantLinear):
        return linear.forward_act(rows, "gelu_tanh")
    return F.gelu(linear(rows).float(), approximate="tanh")


def silu_gate_linear(linear, rows):
    """silu(gate) * up over the halves of linear(rows): fused for a QuantLinear (compute dtype),
    else the reference's fp32 (fp16_safe.py:165-167)."""
    if isinstance(linear, QuantLinear):
        return linear.forward_act(rows, "silu_gate")
    gate, up = linear(rows).chunk(2, -1)
    return F.silu(gate.float()) * up.float()


def _chunk_step(n, chunk_tokens):
    if chunk_tokens is not None and int(chunk_tokens) <= 0:
        raise ValueError("chunk_tokens must be positive")
    return max(n, 1) if chunk_tokens is None else int(chunk_tokens)


def gated_mlp(fc1, fc2, x, chunk_tokens=None, prepare_budget=None):
    """fc2(silu(gate) * up), gate, up = fc1(x).chunk(2, -1), over chunks of ``chunk_tokens`` rows.

    Follows fp16_safe.py:126-172: the result has x's dtype (fp32 for modules in the fp32 safe
    mode) and shape [..., fc2.out_features]; the chunk size and ``prepare_budget`` (bytes, the
    bound of ``prepared_linears`` over more than one chunk) change no value.
    """
    shape = x.shape
    rows = x.reshape(-1, shape[-1])
    n = rows.shape[0]
    step = _chunk_step(n, chunk_tokens)
    dtype = torch.float32 if getattr(fc1, "_ps_safe", False) else x.dtype
    result = torch.empty((n, fc2.out_features), dtype=dtype, device=x.device)
    prepare = prepare_budget is not None and n > step
    with prepared_linears((fc1, fc2), prepare_budget) if prepare else contextlib.nullcontext():
        for a in range(0, n, step):
            b = min(a + step, n)
            activation = silu_gate_linear(fc1, rows[a:b])
            result[a:b] = fc2(activation)
            del activation
    return result.reshape(shape[:-1] + (fc2.out_features,))


def chunked_mlp(fc1, fc2, x, chunk_tokens=None, prepare_budget=None):
    """fc2(gelu_tanh(fc1(x))) in fp32, computed over chunks of ``chunk_tokens`` token rows.

    Follows wan_model.py:589-630: the result is fp32 [..., fc2.out_features]; each chunk's rows
    are independent, so the chunk size does not change any value.  ``prepare_budget`` (bytes)
    bounds the tile cache of ``prepared_linears``; it does not change any value either.
    """
    shape = x.shape
    rows = x.reshape(-1, shape[-1])
    n = rows.shape[0]
    step = _chunk_step(n, chunk_tokens)
    result = torch.empty((n, fc2.out_features), dtype=torch.float32, device=x.device)
    prepare = prepare_budget is not None and n > step
    with prepared_linears((fc1, fc2), prepare_budget) if prepare else contextlib.nullcontext():
        for a in range(0, n, step):
            b = min(a + step, n)
            hidden = gelu_linear(fc1, rows[a:b])
            result[a:b] = fc2(hidden).float()
            del hidden
    return result.reshape(shape[:-1] + (fc2.out_features,))
