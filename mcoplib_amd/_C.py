"""``torch.ops._C`` surface (the vLLM operator library that mcoplib builds as ``mcoplib._C``).

Importing this module registers, in the ``_C`` torch.library namespace, the schemas of
op/vllm/torch_bindings.cpp:155-158 (``rms_norm``), :161-164 (``fused_add_rms_norm``), :216-221
(``rms_norm_dynamic_per_token_quant``), :224-229 (``rms_norm_per_block_quant``), :359-364
(``dynamic_per_token_scaled_fp8_quant``) and :374-379 (``dynamic_scaled_int8_quant``) with
implementations for the CUDA (HIP) dispatch key that call libmcop_norm.so.  If another library (vLLM's own ``_C``) already defined a schema, only the
CUDA implementation is registered over it.  There is no CPU implementation: calling these ops on
CPU tensors raises, as the reference does.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._checks import (contiguous_check, dispatch_check, numel_check, on_cuda, rows_of,
                      torch_check)
from .op import _norm_quant

SCHEMAS = {
    "rms_norm": "rms_norm(Tensor! result, Tensor input, Tensor weight, float epsilon) -> ()",
    "fused_add_rms_norm":
        "fused_add_rms_norm(Tensor! input, Tensor! residual, Tensor weight, float epsilon) -> ()",
    "rms_norm_dynamic_per_token_quant":
        "rms_norm_dynamic_per_token_quant(Tensor! result, Tensor input, Tensor weight, "
        "Tensor! scale, float epsilon, Tensor? scale_ub, Tensor!? residual) -> ()",
    "rms_norm_per_block_quant":
        "rms_norm_per_block_quant(Tensor! result, Tensor input, Tensor weight, Tensor! scale, "
        "float epsilon, Tensor? scale_ub, Tensor!? residual, int group_size, "
        "bool is_scale_transposed) -> ()",
    "dynamic_scaled_int8_quant":
        "dynamic_scaled_int8_quant(Tensor! result, Tensor input, Tensor! scale, "
        "Tensor!? azp) -> ()",
    "dynamic_per_token_scaled_fp8_quant":
        "dynamic_per_token_scaled_fp8_quant(Tensor! result, Tensor input, Tensor! scale, "
        "Tensor? scale_ub) -> ()",
}


def rms_norm(result: torch.Tensor, input: torch.Tensor, weight: torch.Tensor,
             epsilon: float) -> None:
    """result <- RMSNorm(input) * weight for every row of a 2-D, 3-D or 4-D input whose rows may
    be strided (reference host function op/vllm/layernorm_kernels.cu:186-231)."""
    name = "rms_norm"
    torch_check(result.is_contiguous(), "out.is_contiguous()")
    if input.stride(-1) != 1:
        input = input.contiguous()
    torch_check(weight.is_contiguous(), "weight.is_contiguous()")
    dispatch_check(input.dtype, "rms_norm_kernel")
    if input.dim() not in (2, 3, 4):
        raise RuntimeError(f"Expects rank 2, 3 or 4 tensors but got {input.dim()}")
    if weight.dtype != input.dtype or result.dtype != input.dtype:
        raise RuntimeError(f"{name}: result, input and weight must share one dtype")
    on_cuda(name, result, input, weight)
    T, H = rows_of(input)
    numel_check(name, "result", result, T * H)
    numel_check(name, "weight", weight, H)
    nd = input.dim()
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_vllm_rms_norm(
            result.data_ptr(), input.data_ptr(), weight.data_ptr(), T, H, nd, input.stride(-2),
            input.stride(-3) if nd >= 3 else 0, input.stride(-4) if nd >= 4 else 0,
            input.size(-2) if nd >= 3 else 0, input.size(-3) if nd >= 4 else 0,
            _lib.DTYPE_CODE[input.dtype], float(epsilon), _lib.stream_of(input)))


def fused_add_rms_norm(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                       epsilon: float) -> None:
    """In place: residual <- input + residual; input <- RMSNorm(residual) * weight
    (reference host function op/vllm/layernorm_kernels.cu:243-292)."""
    name = "fused_add_rms_norm"
    torch_check(weight.dtype == input.dtype, "weight.scalar_type() == input.scalar_type()")
    torch_check(input.dtype == residual.dtype, "input.scalar_type() == residual.scalar_type()")
    torch_check(residual.is_contiguous(), "residual.is_contiguous()")
    torch_check(weight.is_contiguous(), "weight.is_contiguous()")
    dispatch_check(input.dtype, "fused_add_rms_norm_kernel")
    on_cuda(name, input, residual, weight)
    T, H = rows_of(input)
    numel_check(name, "residual", residual, T * H)
    numel_check(name, "weight", weight, H)
    # Rows of `input` are addressed as row * stride(-2) (the reference's input_stride), which
    # needs a unit last-dimension stride and uniformly strided rows.
    if input.dim() >= 2 and T > 1:
        if input.stride(-1) != 1:
            raise RuntimeError(f"{name}: input must be contiguous in its last dimension")
        for d in range(input.dim() - 2):
            if input.size(d) > 1 and input.stride(d) != input.stride(d + 1) * input.size(d + 1):
                raise RuntimeError(f"{name}: input rows must be uniformly strided")
        row_stride = input.stride(-2)
    else:
        row_stride = H
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_fused_add_rms_norm(
            input.data_ptr(), row_stride, residual.data_ptr(), weight.data_ptr(), T, H,
            _lib.DTYPE_CODE[input.dtype], float(epsilon), _lib.stream_of(input)))


def rms_norm_dynamic_per_token_quant(result: torch.Tensor, input: torch.Tensor,
                                     weight: torch.Tensor, scale: torch.Tensor, epsilon: float,
                                     scale_ub: Optional[torch.Tensor] = None,
                                     residual: Optional[torch.Tensor] = None) -> None:
    """(Residual add +) RMSNorm + dynamic per-token int8 / fp8-e4m3fn quantization (reference
    host function
    op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:163-192)."""
    fp8 = torch.float8_e4m3fn
    torch_check(result.dtype in (fp8, torch.int8),
                "out.dtype() == kFp8Type || out.dtype() == torch::kInt8")
    torch_check(result.is_contiguous() and input.is_contiguous(),
                "out.is_contiguous() && input.is_contiguous()")
    if scale_ub is not None:
        torch_check(result.dtype == fp8, "out.dtype() == kFp8Type")
    torch_check(weight.dtype == input.dtype, "weight.dtype() == input.dtype()")
    torch_check(scale.dtype == torch.float32, "scales.dtype() == torch::kFloat32")
    if residual is not None:
        torch_check(residual.dtype == input.dtype,
                    "residual->scalar_type() == input.scalar_type()")
    dispatch_check(input.dtype, "rms_norm_dynamic_per_token_quant_dispatch")
    _norm_quant("rms_norm_dynamic_per_token_quant", result, input, weight, scale, epsilon,
                scale_ub, residual)


def rms_norm_per_block_quant(result: torch.Tensor, input: torch.Tensor, weight: torch.Tensor,
                             scale: torch.Tensor, epsilon: float,
                             scale_ub: Optional[torch.Tensor], residual: Optional[torch.Tensor],
                             group_size: int, is_scale_transposed: bool) -> None:
    """(Residual add +) RMSNorm + dynamic per-group int8 / fp8-e4m3fn quantization, one scale
    per group of 64 or 128 elements (reference host function
    op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:238-270)."""
    name = "rms_norm_per_block_quant"
    fp8 = torch.float8_e4m3fn
    torch_check(result.dtype in (fp8, torch.int8),
                "out.dtype() == kFp8Type || out.dtype() == torch::kInt8")
    torch_check(result.is_contiguous() and input.is_contiguous(),
                "out.is_contiguous() && input.is_contiguous()")
    if scale_ub is not None:
        torch_check(result.dtype == fp8, "out.dtype() == kFp8Type")
    torch_check(weight.dtype == input.dtype, "weight.dtype() == input.dtype()")
    torch_check(scale.dtype == torch.float32, "scales.dtype() == torch::kFloat32")
    if residual is not None:
        torch_check(residual.dtype == input.dtype,
                    "residual->scalar_type() == input.scalar_type()")
    if group_size not in (64, 128):
        raise RuntimeError(f"Unsupported group size: {group_size}")
    dispatch_check(input.dtype, "rms_norm_per_block_quant_fp_dispatch")
    on_cuda(name, result, input, weight, scale, scale_ub, residual)
    T, H = rows_of(input)
    if H % group_size != 0:
        raise RuntimeError(f"{name}: hidden_size {H} is not a multiple of group_size "
                           f"{group_size}")
    numel_check(name, "result", result, T * H)
    numel_check(name, "weight", weight, H)
    numel_check(name, "scale", scale, T * (H // group_size))
    contiguous_check(name, "weight", weight)
    contiguous_check(name, "scale", scale)
    if residual is not None:
        contiguous_check(name, "residual", residual)
        numel_check(name, "residual", residual, T * H)
    if scale_ub is not None and (scale_ub.dtype != torch.float32 or scale_ub.numel() < 1):
        raise RuntimeError(f"{name}: scale_ub must be a float32 tensor with one element")
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_rms_norm_per_block_quant(
            result.data_ptr(), _lib.DTYPE_CODE[result.dtype], scale.data_ptr(),
            input.data_ptr(), weight.data_ptr(),
            None if scale_ub is None else scale_ub.data_ptr(),
            None if residual is None else residual.data_ptr(), T, H,
            _lib.DTYPE_CODE[input.dtype], float(epsilon), int(group_size),
            1 if is_scale_transposed else 0, _lib.stream_of(input)))


def dynamic_scaled_int8_quant(result: torch.Tensor, input: torch.Tensor, scale: torch.Tensor,
                              azp: Optional[torch.Tensor] = None) -> None:
    """Per-token int8 quantization, symmetric or with a per-token zero point (reference host
    function op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:459-527)."""
    name = "dynamic_scaled_int8_quant"
    torch_check(input.is_contiguous(), "input.is_contiguous()")
    torch_check(result.is_contiguous(), "out.is_contiguous()")
    torch_check(scale.is_contiguous(), "scales.is_contiguous()")
    torch_check(azp is None or azp.is_contiguous(), "!azp || azp->is_contiguous()")
    dispatch_check(input.dtype, "dynamic_scaled_int8_quant_kernel")
    if result.dtype != torch.int8:
        raise RuntimeError(f"expected scalar type Char but found {result.dtype}")
    if scale.dtype != torch.float32:
        raise RuntimeError(f"expected scalar type Float but found {scale.dtype}")
    if azp is not None and azp.dtype != torch.int32:
        raise RuntimeError(f"expected scalar type Int but found {azp.dtype}")
    on_cuda(name, result, input, scale, azp)
    T, H = rows_of(input)
    numel_check(name, "result", result, T * H)
    numel_check(name, "scale", scale, T)
    if azp is not None:
        numel_check(name, "azp", azp, T)
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_dynamic_scaled_int8_quant(
            result.data_ptr(), scale.data_ptr(), None if azp is None else azp.data_ptr(),
            input.data_ptr(), T, H, _lib.DTYPE_CODE[input.dtype], _lib.stream_of(input)))


def dynamic_per_token_scaled_fp8_quant(result: torch.Tensor, input: torch.Tensor,
                                       scale: torch.Tensor,
                                       scale_ub: Optional[torch.Tensor] = None) -> None:
    """Per-token fp8-e4m3fn quantization (reference host function
    op/vllm/quantization/fp8/common.cu:375-411); rows of input and result may be strided."""
    name = "dynamic_per_token_scaled_fp8_quant"
    torch_check(input.stride(-1) == 1, "last dimension of input must be contiguous")
    torch_check(result.stride(-1) == 1, "last dimension of output must be contiguous")
    dispatch_check(input.dtype, "dynamic_per_token_scaled_fp8_quant_kernel_scalar_type")
    dispatch_check(result.dtype, "dynamic_per_token_scaled_fp8_quant_kernel_fp8_type",
                   allowed=(torch.float8_e4m3fn,))
    if scale.dtype != torch.float32:
        raise RuntimeError(f"expected scalar type Float but found {scale.dtype}")
    on_cuda(name, result, input, scale, scale_ub)
    T, H = rows_of(input)
    if result.shape != input.shape:
        raise RuntimeError(f"{name}: result shape {tuple(result.shape)} != input shape")
    numel_check(name, "scale", scale, T)
    contiguous_check(name, "scale", scale)
    if scale_ub is not None and (scale_ub.dtype != torch.float32 or scale_ub.numel() < 1):
        raise RuntimeError(f"{name}: scale_ub must be a float32 tensor with one element")

    def row_stride(t: torch.Tensor) -> int:
        if t.dim() < 2 or T <= 1:
            return H
        for d in range(t.dim() - 2):
            if t.size(d) > 1 and t.stride(d) != t.stride(d + 1) * t.size(d + 1):
                raise RuntimeError(f"{name}: rows must be uniformly strided")
        return t.stride(-2)

    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_dynamic_per_token_scaled_fp8_quant(
            result.data_ptr(), scale.data_ptr(), input.data_ptr(),
            None if scale_ub is None else scale_ub.data_ptr(), T, H, row_stride(input),
            row_stride(result), _lib.DTYPE_CODE[input.dtype], _lib.stream_of(input)))


_IMPLS = {
    "rms_norm": rms_norm,
    "fused_add_rms_norm": fused_add_rms_norm,
    "rms_norm_dynamic_per_token_quant": rms_norm_dynamic_per_token_quant,
    "dynamic_scaled_int8_quant": dynamic_scaled_int8_quant,
    "dynamic_per_token_scaled_fp8_quant": dynamic_per_token_scaled_fp8_quant,
    "rms_norm_per_block_quant": rms_norm_per_block_quant,
}

_library = torch.library.Library("_C", "FRAGMENT")


def _defined(name: str) -> bool:
    try:
        getattr(torch.ops._C, name)
        return True
    except (AttributeError, RuntimeError):
        return False


def _meta(*args, **kwargs) -> None:  # mutating ops with no return: nothing to compute
    return None


for _name, _schema in SCHEMAS.items():
    if not _defined(_name):
        _library.define(_schema)
        _library.impl(_name, _meta, "Meta")
    _library.impl(_name, _IMPLS[_name], "CUDA")
