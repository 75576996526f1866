"""``mcoplib.op`` surface of the fused norm/quant path: the C++ functions of the _torch_ops
extension (csrc/torch_ops.cpp) over libmcop_norm.so (gfx950).

Functions keep the reference pybind signatures (op/pybind.cpp:42-44, 51, 54, 55; declarations
in include/fused_rms_norm_dq.h:3-24, include/rms_norm_dynamic_per_token_quant.h:2-8,
include/scale_dynamic_quant.h:6-10,
include/fused_add_layernorm_per_token_quant_padding_output.h:3-11), their positional argument
order, in-place outputs and error behaviour (the reference's TORCH_CHECK conditions; keyword
names are accepted as well).  Every call enqueues one kernel on torch's current stream of the
tensors' device and returns without synchronizing.
"""

from __future__ import annotations

from . import _lib  # noqa: F401  (loads libmcop_norm.so first; raises ImportError if missing)
from ._torch_ops import (fused_add_rms_norm_dynamic_per_token_quant_padding_output,
                         head_rms_norm, rms_norm, rms_norm_dynamic_per_token_quant,
                         rms_norm_dynamic_per_token_quant_custom, scale_dynamic_quant)

__all__ = [
    "rms_norm_dynamic_per_token_quant",
    "rms_norm_dynamic_per_token_quant_custom",
    "scale_dynamic_quant",
    "fused_add_rms_norm_dynamic_per_token_quant_padding_output",
    "rms_norm",
    "head_rms_norm",
]
