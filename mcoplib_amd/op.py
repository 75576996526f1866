"""``mcoplib.op`` surface of the fused norm/quant path, backed by libmcop_norm.so (gfx950).

Functions keep the reference pybind signatures (op/pybind.cpp:42-44, 51, 54, 55; declarations
in include/fused_rms_norm_dq.h:3-24, include/rms_norm_dynamic_per_token_quant.h:2-8,
include/scale_dynamic_quant.h:6-10,
include/fused_add_layernorm_per_token_quant_padding_output.h:3-11), their positional argument
order, in-place outputs and error behaviour.  Every call enqueues one kernel on torch's current
stream of the tensors' device and returns without synchronizing.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._checks import (contiguous_check, dispatch_check, numel_check, on_cuda, rows_of,
                      torch_check)

__all__ = [
    "rms_norm_dynamic_per_token_quant",
    "rms_norm_dynamic_per_token_quant_custom",
    "scale_dynamic_quant",
    "fused_add_rms_norm_dynamic_per_token_quant_padding_output",
    "rms_norm",
    "head_rms_norm",
]


def rms_norm_dynamic_per_token_quant(out: torch.Tensor, input: torch.Tensor,
                                     weight: torch.Tensor, smooth_scale: torch.Tensor,
                                     scales: torch.Tensor, var_epsilon: float,
                                     after_res: torch.Tensor, after_norm: torch.Tensor,
                                     residual: Optional[torch.Tensor] = None,
                                     standard_norm: bool = False) -> None:
    """SmoothQuant (residual add +) RMSNorm + dynamic per-token quantization
    ("fused_rms_norm_dq"; reference entry op/fused_rms_norm_dq.cu:646-667).

    after_res <- input (+ residual); after_norm <- after_res / rsqrt(mean(after_res^2) + eps)
    * weight (the reference's literal form; ``standard_norm=True`` multiplies by the rsqrt
    instead); out <- per-token quantization of after_norm * smooth_scale; scales[t] <- absmax/127
    (int8) or absmax/448 (fp8-e4m3fn, an extension: the reference accepts int8 only).
    ``residual`` is read, not updated.  weight and smooth_scale are each the input dtype or fp32.
    """
    name = "rms_norm_dynamic_per_token_quant"
    torch_check(out.dtype in (torch.int8, torch.float8_e4m3fn),
                "out.dtype() == torch::kInt8 || out.dtype() == torch::kFloat8_e4m3fn")
    torch_check(out.is_contiguous() and input.is_contiguous(),
                "out.is_contiguous() && input.is_contiguous()")
    torch_check(scales.dtype == torch.float32, "scales.dtype() == torch::kFloat32")
    dispatch_check(input.dtype, "rms_norm_dynamic_per_token_quant_dispatch")
    on_cuda(name, out, input, weight, smooth_scale, scales, after_res, after_norm, residual)
    T, H = rows_of(input)
    numel_check(name, "out", out, T * H)
    numel_check(name, "weight", weight, H)
    numel_check(name, "smooth_scale", smooth_scale, H)
    numel_check(name, "scales", scales, T)
    for what, t in (("weight", weight), ("smooth_scale", smooth_scale), ("scales", scales),
                    ("after_res", after_res), ("after_norm", after_norm)):
        contiguous_check(name, what, t)
    for what, t in (("after_res", after_res), ("after_norm", after_norm)):
        numel_check(name, what, t, T * H)
        if t.dtype != input.dtype:
            raise RuntimeError(f"{name}: {what} must have the input dtype {input.dtype}")
    if residual is not None:
        if residual.dtype != input.dtype:
            raise RuntimeError(f"{name}: residual must have the input dtype {input.dtype}")
        contiguous_check(name, "residual", residual)
        numel_check(name, "residual", residual, T * H)
    for what, t in (("weight", weight), ("smooth_scale", smooth_scale)):
        if t.dtype not in (input.dtype, torch.float32):
            raise RuntimeError(f"{name}: {what} must be {input.dtype} or float32, got {t.dtype}")
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_rms_norm_smooth_quant(
            out.data_ptr(), _lib.DTYPE_CODE[out.dtype], scales.data_ptr(), input.data_ptr(),
            weight.data_ptr(), _lib.DTYPE_CODE[weight.dtype], smooth_scale.data_ptr(),
            _lib.DTYPE_CODE[smooth_scale.dtype], after_res.data_ptr(), after_norm.data_ptr(),
            None if residual is None else residual.data_ptr(), T, H,
            _lib.DTYPE_CODE[input.dtype], float(var_epsilon),
            _lib.SQ_STANDARD_NORM if standard_norm else 0, _lib.stream_of(input)))


def rms_norm_dynamic_per_token_quant_custom(out: torch.Tensor, input: torch.Tensor,
                                            weight: torch.Tensor, scales: torch.Tensor,
                                            var_epsilon: float,
                                            scale_ub: Optional[torch.Tensor] = None,
                                            residual: Optional[torch.Tensor] = None) -> None:
    """(Residual add +) RMSNorm + dynamic per-token int8 quantization with mcoplib's own
    arithmetic (reference entry op/rms_norm_dynamic_per_token_quant.cu:266-285): scale floor
    1.5e-6 and codes in [-127, 127]; at H == 7168 the reference's fp32 chain (codes from
    (x [+ r]) * w * rsqrt(...) without bf16 rounding, scale_ub unused).  ``residual`` is
    updated in place to input + residual; out and scales ([T] or [T, 1] fp32) are written."""
    name = "rms_norm_dynamic_per_token_quant_custom"
    torch_check(out.dtype == torch.int8, "out.dtype() == torch::kInt8")
    torch_check(out.is_contiguous() and input.is_contiguous(),
                "out.is_contiguous() && input.is_contiguous()")
    torch_check(scales.dtype == torch.float32, "scales.dtype() == torch::kFloat32")
    dispatch_check(input.dtype, " rms_norm_dynamic_per_token_quant_dispatch_")
    _norm_quant(name, out, input, weight, scales, var_epsilon, scale_ub, residual, custom=True)


def _norm_quant(name: str, out: torch.Tensor, input: torch.Tensor, weight: torch.Tensor,
                scales: torch.Tensor, eps: float, scale_ub: Optional[torch.Tensor],
                residual: Optional[torch.Tensor], custom: bool = False) -> None:
    """Shared launcher of the (residual add +) RMSNorm + per-token quant kernel (vLLM's
    arithmetic, or mcoplib's own with ``custom``)."""
    on_cuda(name, out, input, weight, scales, scale_ub, residual)
    T, H = rows_of(input)
    numel_check(name, "out", out, T * H)
    numel_check(name, "weight", weight, H)
    numel_check(name, "scales", scales, T)
    contiguous_check(name, "weight", weight)
    contiguous_check(name, "scales", scales)
    if weight.dtype != input.dtype:
        raise RuntimeError(f"{name}: weight must have the input dtype {input.dtype}")
    if residual is not None:
        if residual.dtype != input.dtype:
            raise RuntimeError(f"{name}: residual must have the input dtype {input.dtype}")
        contiguous_check(name, "residual", residual)
        numel_check(name, "residual", residual, T * H)
    if scale_ub is not None:
        if scale_ub.dtype != torch.float32 or scale_ub.numel() < 1:
            raise RuntimeError(f"{name}: scale_ub must be a float32 tensor with one element")
    ub = None if scale_ub is None else scale_ub.data_ptr()
    rp = None if residual is None else residual.data_ptr()
    with _lib.device_of(input):
        if custom:
            _lib.check(_lib.lib.mcop_rms_norm_dynamic_per_token_quant_custom(
                out.data_ptr(), scales.data_ptr(), input.data_ptr(), weight.data_ptr(), ub, rp,
                T, H, _lib.DTYPE_CODE[input.dtype], float(eps), _lib.stream_of(input)))
        else:
            _lib.check(_lib.lib.mcop_rms_norm_dynamic_per_token_quant(
                out.data_ptr(), _lib.DTYPE_CODE[out.dtype], scales.data_ptr(),
                input.data_ptr(), weight.data_ptr(), ub, rp, T, H,
                _lib.DTYPE_CODE[input.dtype], float(eps), _lib.stream_of(input)))


def scale_dynamic_quant(hidden_states: torch.Tensor, smooth_scales: torch.Tensor,
                        dst_dtype: torch.dtype = torch.int8
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """Smooth-scale multiply + dynamic per-token int8 quantization (reference entry
    op/scale_dynamic_quant.cu:127-153).  Returns new (codes shaped like hidden_states,
    scales [T] fp32)."""
    torch_check(hidden_states.is_cuda, "hidden_states.is_cuda()")
    torch_check(smooth_scales.is_cuda, "smooth_scales.is_cuda()")
    T, H = rows_of(hidden_states)
    output = torch.empty_like(hidden_states, dtype=dst_dtype)
    scales = torch.empty((T,), dtype=smooth_scales.dtype, device=smooth_scales.device)
    if not (hidden_states.dtype == torch.bfloat16 and dst_dtype == torch.int8):
        raise RuntimeError("Only support bfloat16")
    name = "scale_dynamic_quant"
    on_cuda(name, hidden_states, smooth_scales)
    contiguous_check(name, "hidden_states", hidden_states)
    contiguous_check(name, "smooth_scales", smooth_scales)
    numel_check(name, "smooth_scales", smooth_scales, H)
    if smooth_scales.dtype != torch.float32:
        raise RuntimeError(f"{name}: smooth_scales must be float32")
    with _lib.device_of(hidden_states):
        _lib.check(_lib.lib.mcop_scale_dynamic_quant(
            output.data_ptr(), scales.data_ptr(), hidden_states.data_ptr(),
            smooth_scales.data_ptr(), T, H, _lib.stream_of(hidden_states)))
    return output, scales


def fused_add_rms_norm_dynamic_per_token_quant_padding_output(
        output: torch.Tensor, output_rms: torch.Tensor, output_quant_int8: torch.Tensor,
        out_scales: torch.Tensor, input: torch.Tensor, residual: torch.Tensor,
        weight: torch.Tensor, pad_size: int, epsilon: float) -> None:
    """Residual add + RMSNorm + per-token int8 quantization with a padded per-row output
    (reference entry op/fused_add_layernorm_per_token_quant_padding_output.cu:397-416).

    ``output`` (int8, 2*pad_size bytes per row) receives each row's codes at bytes [0, H) and
    its fp32 scale at bytes [H, H+4); ``output_rms`` (bf16) the normalized row,
    ``output_quant_int8`` the codes again, ``out_scales`` the scales; ``residual`` becomes
    input + residual.  bf16 input, int8 output, as in the reference.  H == 7168 uses the
    reference's fp32 chain (its "opt" kernel); other H its bf16-rounded chain, and here every
    output is written for every H (the reference's generic kernel leaves output_rms,
    output_quant_int8 and out_scales unwritten)."""
    name = "fused_add_rms_norm_dynamic_per_token_quant_padding_output"
    torch_check(output.dtype == torch.int8, "output.dtype() == torch::kInt8")
    torch_check(input.dtype == torch.bfloat16, "input.dtype() == at::ScalarType::BFloat16")
    torch_check(output.is_contiguous() and input.is_contiguous(),
                "output.is_contiguous() && input.is_contiguous()")
    on_cuda(name, output, output_rms, output_quant_int8, out_scales, input, residual, weight)
    T, H = rows_of(input)
    pad = int(pad_size)
    if 2 * pad < H + 4:
        raise RuntimeError(f"{name}: a padded row of 2*pad_size = {2 * pad} bytes cannot hold "
                           f"{H} codes and a 4-byte scale")
    numel_check(name, "output", output, T * 2 * pad)
    for what, t, dt in (("output_rms", output_rms, torch.bfloat16),
                        ("output_quant_int8", output_quant_int8, torch.int8),
                        ("residual", residual, torch.bfloat16),
                        ("weight", weight, torch.bfloat16),
                        ("out_scales", out_scales, torch.float32)):
        if t.dtype != dt:
            raise RuntimeError(f"{name}: {what} must be {dt}, got {t.dtype}")
        contiguous_check(name, what, t)
    numel_check(name, "output_rms", output_rms, T * H)
    numel_check(name, "output_quant_int8", output_quant_int8, T * H)
    numel_check(name, "residual", residual, T * H)
    numel_check(name, "weight", weight, H)
    numel_check(name, "out_scales", out_scales, T)
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output(
            output.data_ptr(), output_rms.data_ptr(), output_quant_int8.data_ptr(),
            out_scales.data_ptr(), input.data_ptr(), residual.data_ptr(), weight.data_ptr(),
            T, H, pad, float(epsilon), _lib.stream_of(input)))


def rms_norm(out: torch.Tensor, input: torch.Tensor, weight: torch.Tensor, var_epsilon: float,
             after_res: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
             rms_div: bool = True) -> None:
    """(Residual add +) RMSNorm (reference entry op/fused_rms_norm_dq.cu:980-998).

    out <- (input [+ residual]) / rsqrt(mean(.^2) + eps) * weight when ``rms_div`` (the
    reference's convention, which its own test asserts), or * rsqrt(...) * weight otherwise;
    with a residual, after_res <- input + residual (the residual itself is not updated).
    weight is the input dtype or fp32."""
    name = "rms_norm"
    torch_check(out.is_contiguous() and input.is_contiguous(),
                "out.is_contiguous() && input.is_contiguous()")
    torch_check(weight.is_contiguous(), "weight.is_contiguous()")
    dispatch_check(input.dtype, "rms_norm_per_token_dispatch")
    on_cuda(name, out, input, weight, after_res, residual)
    T, H = rows_of(input)
    if out.dtype != input.dtype:
        raise RuntimeError(f"{name}: out must have the input dtype {input.dtype}")
    if weight.dtype not in (input.dtype, torch.float32):
        raise RuntimeError(f"{name}: weight must be {input.dtype} or float32, got {weight.dtype}")
    numel_check(name, "out", out, T * H)
    numel_check(name, "weight", weight, H)
    if residual is not None:
        if after_res is None:
            raise RuntimeError(f"{name}: a residual needs an after_res output")
        for what, t in (("residual", residual), ("after_res", after_res)):
            if t.dtype != input.dtype:
                raise RuntimeError(f"{name}: {what} must have the input dtype {input.dtype}")
            contiguous_check(name, what, t)
            numel_check(name, what, t, T * H)
    with _lib.device_of(input):
        _lib.check(_lib.lib.mcop_rms_norm(
            out.data_ptr(), input.data_ptr(), weight.data_ptr(), _lib.DTYPE_CODE[weight.dtype],
            None if residual is None else after_res.data_ptr(),
            None if residual is None else residual.data_ptr(), T, H,
            _lib.DTYPE_CODE[input.dtype], float(var_epsilon), 1 if rms_div else 0,
            _lib.stream_of(input)))


def head_rms_norm(out: torch.Tensor, hidden_states: torch.Tensor, weight: torch.Tensor,
                  var_epsilon: float, head_offset: int, head_norm: int) -> None:
    """Per-head RMSNorm of heads [head_offset, head_offset + head_norm) of
    hidden_states [num_tokens, num_heads, head_size] with per-head weights
    [num_heads, head_size] (bf16 or fp32); out (same shape) is written for those heads only
    (reference entry op/fused_rms_norm_dq.cu:804-812).  The reference's convention:
    x / rsqrt(mean(x^2) + eps) * weight."""
    name = "head_rms_norm"
    torch_check(out.is_contiguous() and weight.is_contiguous() and hidden_states.is_contiguous(),
                "out.is_contiguous() && weight.is_contiguous() && hidden_states.is_contiguous()")
    dispatch_check(hidden_states.dtype, "head_rms_norm_dispatch")
    on_cuda(name, out, hidden_states, weight)
    if hidden_states.dim() != 3:
        raise RuntimeError(f"{name}: hidden_states must be [num_tokens, num_heads, head_size]")
    T, NH, D = hidden_states.shape
    if out.shape != hidden_states.shape or out.dtype != hidden_states.dtype:
        raise RuntimeError(f"{name}: out must match hidden_states in shape and dtype")
    if weight.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"{name}: weight must be bfloat16 or float32, got {weight.dtype}")
    head_offset, head_norm = int(head_offset), int(head_norm)
    if head_offset < 0 or head_norm < 0 or head_offset + head_norm > NH:
        raise RuntimeError(f"{name}: heads [{head_offset}, {head_offset + head_norm}) are not "
                           f"inside the {NH} heads")
    if weight.numel() < (head_offset + head_norm) * D:
        raise RuntimeError(f"{name}: weight holds {weight.numel()} elements, needs "
                           f"{(head_offset + head_norm) * D}")
    with _lib.device_of(hidden_states):
        _lib.check(_lib.lib.mcop_head_rms_norm(
            out.data_ptr(), hidden_states.data_ptr(), weight.data_ptr(),
            _lib.DTYPE_CODE[weight.dtype], T, NH, D, head_offset, head_norm,
            _lib.DTYPE_CODE[hidden_states.dtype], float(var_epsilon),
            _lib.stream_of(hidden_states)))
