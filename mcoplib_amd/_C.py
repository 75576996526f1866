"""``torch.ops._C`` surface (the vLLM operator library that mcoplib builds as ``mcoplib._C``).

Importing this module registers, in the ``_C`` torch.library namespace, the schemas of
op/vllm/torch_bindings.cpp:155-158 (``rms_norm``), :161-164 (``fused_add_rms_norm``), :216-221
(``rms_norm_dynamic_per_token_quant``), :224-229 (``rms_norm_per_block_quant``), :359-364
(``dynamic_per_token_scaled_fp8_quant``) and :374-379 (``dynamic_scaled_int8_quant``) with
implementations for the CUDA (HIP) dispatch key in the C++ extension _torch_ops
(csrc/torch_ops.cpp) that call libmcop_norm.so, and a no-op Meta kernel.  If another library
(vLLM's own ``_C``) already defined a schema, only the CUDA implementation is registered over
it.  There is no CPU implementation: calling these ops on CPU tensors raises, as the reference
does.  The same implementations are exported here as plain functions.
"""

from __future__ import annotations

from . import _lib  # noqa: F401  (loads libmcop_norm.so first; raises ImportError if missing)
from . import _torch_ops

_torch_ops.register_vllm_ops()

rms_norm = _torch_ops.c_rms_norm
fused_add_rms_norm = _torch_ops.c_fused_add_rms_norm
rms_norm_dynamic_per_token_quant = _torch_ops.c_rms_norm_dynamic_per_token_quant
rms_norm_per_block_quant = _torch_ops.c_rms_norm_per_block_quant
dynamic_scaled_int8_quant = _torch_ops.c_dynamic_scaled_int8_quant
dynamic_per_token_scaled_fp8_quant = _torch_ops.c_dynamic_per_token_scaled_fp8_quant
