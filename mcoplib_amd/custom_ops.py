"""``mcoplib.custom_ops`` wrappers of the fused norm/quant path (reference
mcoplib/custom_ops.py:7-45): allocate the outputs the way the reference does, then call the
``op`` entry point."""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import op as ops


def fused_add_rms_norm_dynamic_per_token_quant_padding_output(
        input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, pad_size: int,
        epsilon: float):
    """Allocates the padded output as bf16 [..., pad_size] (2*pad_size bytes per row, viewed as
    int8 for the kernel), output_rms like input, the unpacked int8 codes and scales [T, 1], and
    returns (output, residual, output_rms, output_quant_int8, scales); ``residual`` is updated
    in place (reference mcoplib/custom_ops.py:7-27)."""
    assert input.is_contiguous()
    shape = list(input.shape)
    shape[-1] = pad_size
    output = torch.empty(shape, dtype=torch.bfloat16, device=input.device)
    assert weight.is_contiguous()
    output_rms = torch.empty_like(input)
    output_quant_int8 = torch.empty_like(input, dtype=torch.int8)
    scales = torch.empty((input.numel() // input.shape[-1], 1), device=input.device,
                         dtype=torch.float32)
    ops.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
        output.view(dtype=torch.int8), output_rms, output_quant_int8, scales, input, residual,
        weight, pad_size, epsilon)
    return output, residual, output_rms, output_quant_int8, scales


def rms_norm_dynamic_per_token_quant(input: torch.Tensor, weight: torch.Tensor, epsilon: float,
                                     quant_dtype: torch.dtype,
                                     scale_ub: Optional[torch.Tensor] = None,
                                     residual: Optional[torch.Tensor] = None
                                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Returns (codes like input in quant_dtype, scales [T, 1] fp32); updates ``residual`` in
    place when given.  ``quant_dtype`` must be int8, as for the reference custom op."""
    output = torch.empty_like(input, dtype=quant_dtype)
    scales = torch.empty((input.numel() // input.shape[-1], 1), device=input.device,
                         dtype=torch.float32)
    ops.rms_norm_dynamic_per_token_quant_custom(output, input, weight, scales, epsilon, scale_ub,
                                                residual)
    return output, scales
