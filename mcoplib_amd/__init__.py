"""mcoplib_amd -- MI355X (gfx950) implementation of MetaX-MACA/mcoplib's fused RMSNorm +
per-token quantization path.

Surfaces (same names, argument order and in-place conventions as the reference):
  mcoplib_amd.op          -- mcoplib.op: rms_norm_dynamic_per_token_quant (fused_rms_norm_dq),
                             rms_norm_dynamic_per_token_quant_custom, scale_dynamic_quant,
                             fused_add_rms_norm_dynamic_per_token_quant_padding_output,
                             rms_norm, head_rms_norm
  mcoplib_amd.custom_ops  -- mcoplib.custom_ops.rms_norm_dynamic_per_token_quant and
                             fused_add_rms_norm_dynamic_per_token_quant_padding_output
  mcoplib_amd._C          -- registers torch.ops._C.rms_norm, torch.ops._C.fused_add_rms_norm,
                             torch.ops._C.rms_norm_dynamic_per_token_quant,
                             torch.ops._C.rms_norm_per_block_quant,
                             torch.ops._C.dynamic_scaled_int8_quant and
                             torch.ops._C.dynamic_per_token_scaled_fp8_quant

op and _C are C++ (csrc/torch_ops.cpp, built into _torch_ops.so) and custom_ops is Python, as
in the reference; all of them call libmcop_norm.so (hand-written HIP kernels, C ABI in
include/mcop_norm.h).  Importing the package fails if either library is not built: there is no
other implementation.
"""

from . import _lib  # noqa: F401  (loads libmcop_norm.so; raises ImportError if missing)
from . import op, custom_ops  # noqa: F401

__version__ = "0.1.0"
LIBRARY_PATH = str(_lib.LIB_PATH)
