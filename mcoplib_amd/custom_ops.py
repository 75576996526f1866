"""``mcoplib.custom_ops`` wrappers of the fused norm/quant path (reference
mcoplib/custom_ops.py:29-45): allocate the outputs the way the reference does, then call the
``op`` entry point."""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import op as ops


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
