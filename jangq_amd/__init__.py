"""jangq_amd — MI355X (gfx950) quantized-weight matmul path of the JANG format.

Operators (``jangq_amd.ops``) mirror MLX's affine ``quantize`` / ``dequantize`` /
``quantized_matmul`` / ``gather_qmm``; modules (``jangq_amd.nn``) mirror the reference's
quantized linear, switch-linear and SwitchGLU layers. All compute runs in the hand-written
HIP kernels of ``libjangq_amd.so`` (C ABI: ``include/jangq_amd.h``).
"""
from .ops import (  # noqa: F401
    dequantize,
    dequantize_tensor,
    expand_packed_1bit_to_2bit,
    gather_qmm,
    moe_block,
    moe_combine,
    moe_experts,
    moe_route,
    quantize,
    quantized_matmul,
    quantized_matmul_multi,
    quantized_swiglu,
    switch_glu,
    switch_glu_combine,
    swiglu,
    unpack,
)
from ._lib import JangqError  # noqa: F401
from .shapes import bit_inference, infer_bits_group_size  # noqa: F401

__all__ = [
    "dequantize", "dequantize_tensor", "expand_packed_1bit_to_2bit", "gather_qmm", "moe_block", "moe_combine", "moe_experts", "moe_route", "quantize", "quantized_matmul",
    "quantized_matmul_multi", "quantized_swiglu", "switch_glu", "switch_glu_combine", "swiglu", "unpack", "bit_inference", "infer_bits_group_size",
    "JangqError",
]
