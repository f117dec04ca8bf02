"""Fused projection kernels for the Qwen3 engine, MI355X-native.

Same import surface as the reference's ``src/kernels/__init__.py:3-14``, plus
the int8 weight-only variants, the plain ``down``/``o`` projection and the
RMSNorm prologue fused into the projections.
"""

from .fused_ffn import TritonFFN, fused_gate_up_silu, fused_gate_up_silu_w8, triton_fused_gate_up_silu
from .fused_qkv import TritonAttention, fused_qkv, fused_qkv_w8, triton_fused_qkv
from .fused_norm import (fused_rmsnorm_gate_up_silu, fused_rmsnorm_gate_up_silu_w8,
                         fused_rmsnorm_qkv, fused_rmsnorm_qkv_w8)
from .linear import FusedLinear, fused_linear, fused_linear_w8
from .quant import dequantize_w8, quantize_w8_per_row
from .swap import apply_triton_kernels, prewarm_triton_kernels

__all__ = [
    "FusedLinear",
    "fused_rmsnorm_qkv",
    "fused_rmsnorm_gate_up_silu",
    "fused_rmsnorm_qkv_w8",
    "fused_rmsnorm_gate_up_silu_w8",
    "fused_linear",
    "fused_linear_w8",
    "TritonAttention",
    "TritonFFN",
    "apply_triton_kernels",
    "prewarm_triton_kernels",
    "triton_fused_gate_up_silu",
    "triton_fused_qkv",
    "fused_qkv",
    "fused_gate_up_silu",
    "fused_qkv_w8",
    "fused_gate_up_silu_w8",
    "quantize_w8_per_row",
    "dequantize_w8",
]
