"""TEST INFRASTRUCTURE ONLY -- CPU oracle of the fused RMSNorm + per-token quantization path.

Python bindings (ctypes + torch CPU tensors) of ``mcop_oracle.c``, the plain-C restatement of the
reference's algorithms.  Only the tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
of ``bench.py`` use this package, and only as the checker / CPU baseline; the product
(``mcoplib_amd``) never imports it.

Every function returns new tensors (inputs are not modified) so the GPU results can be compared
with them.  Each one cites the reference code it restates; see ``mcop_oracle.c`` for the
arithmetic contract.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmcop_oracle.so"

_DT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.int8: 3,
       torch.float8_e4m3fn: 4}


def build() -> Path:
    """Compile mcop_oracle.c with gcc (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    P, I64, F, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
    lib.oracle_fused_add_rms_norm.argtypes = [P, I64, P, P, I64, I64, I, F]
    lib.oracle_rms_norm_quant.argtypes = [P, I, P, P, P, P, P, I64, I64, I, F]
    lib.oracle_rms_norm_smooth_quant.argtypes = [P, I, P, P, P, I, P, I, P, P, P, I64, I64, I, F, I]
    lib.oracle_scale_dynamic_quant.argtypes = [P, P, P, P, I64, I64]
    lib.oracle_fp8_e4m3fn_from_f32.argtypes = [P, P, I64, F]
    lib.oracle_dynamic_scaled_int8_quant.argtypes = [P, P, P, I64, I64, I]
    lib.oracle_dynamic_scaled_int8_azp_quant.argtypes = [P, P, P, P, I64, I64, I]
    lib.oracle_dynamic_per_token_fp8_quant.argtypes = [P, P, P, P, I64, I64, I64, I64, I]
    lib.oracle_add_rms_norm_quant_padded.argtypes = [P, I64, P, P, P, P, P, P, I64, I64, F]
    lib.oracle_rms_norm_per_block_quant.argtypes = [P, I, P, P, P, P, P, I64, I64, I, F, I64, I]
    lib.oracle_rms_norm.argtypes = [P, P, P, I, P, P, I64, I64, I, F, I]
    lib.oracle_rms_norm_quant_custom.argtypes = [P, P, P, P, P, P, I64, I64, I, F]
    lib.oracle_head_rms_norm.argtypes = [P, P, P, I, I64, I64, I64, I64, I64, I, F]
    lib.oracle_vllm_rms_norm.argtypes = [P, P, P, I64, I64, I, F]
    for name in ("oracle_f32_to_bf16_array", "oracle_f32_to_f16_array",
                 "oracle_f32_to_e4m3fn_array"):
        getattr(lib, name).argtypes = [P, P, I64]
    for name in ("oracle_fused_add_rms_norm", "oracle_rms_norm_quant",
                 "oracle_rms_norm_smooth_quant", "oracle_scale_dynamic_quant",
                 "oracle_fp8_e4m3fn_from_f32", "oracle_f32_to_bf16_array",
                 "oracle_f32_to_f16_array", "oracle_f32_to_e4m3fn_array", "oracle_set_threads",
                 "oracle_dynamic_scaled_int8_quant", "oracle_dynamic_scaled_int8_azp_quant",
                 "oracle_dynamic_per_token_fp8_quant", "oracle_add_rms_norm_quant_padded",
                 "oracle_rms_norm_per_block_quant", "oracle_rms_norm", "oracle_head_rms_norm",
                 "oracle_vllm_rms_norm", "oracle_rms_norm_quant_custom"):
        getattr(lib, name).restype = None
    lib.oracle_set_threads.argtypes = [I]
    lib.oracle_num_threads.restype = I
    return lib


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _cpu(t: torch.Tensor) -> torch.Tensor:
    assert t.device.type == "cpu", "the oracle takes CPU tensors"
    return t.contiguous()


def _rows(x: torch.Tensor) -> tuple[int, int]:
    H = x.shape[-1]
    return (x.numel() // H if H else 0), H


# ------------------------------------------------------------------------------------ H1
def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                       eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """vLLM ``_C::fused_add_rms_norm`` (op/vllm/layernorm_kernels.cu:92-182, 243-292).

    Returns (new input, new residual)."""
    xo, ro, w = _cpu(x).clone(), _cpu(residual).clone(), _cpu(weight)
    T, H = _rows(xo)
    lib().oracle_fused_add_rms_norm(xo.data_ptr(), H, ro.data_ptr(), w.data_ptr(), T, H,
                                    _DT[x.dtype], float(eps))
    return xo, ro


# ------------------------------------------------------------------------------------ H2/H3
def rms_norm_dynamic_per_token_quant(
        x: torch.Tensor, weight: torch.Tensor, eps: float, quant_dtype: torch.dtype,
        scale_ub: Optional[float] = None, residual: Optional[torch.Tensor] = None
) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """vLLM ``_C::rms_norm_dynamic_per_token_quant`` / mcoplib
    ``rms_norm_dynamic_per_token_quant_custom``
    (op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:14-90,
    layernorm_utils.cuh:223-535; op/rms_norm_dynamic_per_token_quant.cu:16-92).

    Returns (codes, scales [T,1] fp32, new residual or None)."""
    xc, w = _cpu(x), _cpu(weight)
    T, H = _rows(xc)
    out = torch.empty(xc.shape, dtype=quant_dtype)
    scales = torch.empty((T, 1), dtype=torch.float32)
    ro = None if residual is None else _cpu(residual).clone()
    ub = None if scale_ub is None else ctypes.byref(ctypes.c_float(float(scale_ub)))
    lib().oracle_rms_norm_quant(out.data_ptr(), _DT[quant_dtype], scales.data_ptr(),
                                xc.data_ptr(), w.data_ptr(), ub, _ptr(ro), T, H, _DT[x.dtype],
                                float(eps))
    return out, scales, ro


def rms_norm_per_block_quant(
        x: torch.Tensor, weight: torch.Tensor, eps: float, quant_dtype: torch.dtype,
        group_size: int, scale_ub: Optional[float] = None,
        residual: Optional[torch.Tensor] = None, is_scale_transposed: bool = False
) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """vLLM ``_C::rms_norm_per_block_quant``
    (op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:92-126,
    194-270; layernorm_utils.cuh:223-393, 455-535).

    Returns (codes, scales [T, H/G] or [H/G, T] fp32, new residual or None)."""
    xc, w = _cpu(x), _cpu(weight)
    T, H = _rows(xc)
    assert H % group_size == 0
    NG = H // group_size
    out = torch.empty(xc.shape, dtype=quant_dtype)
    scales = torch.empty((NG, T) if is_scale_transposed else (T, NG), dtype=torch.float32)
    ro = None if residual is None else _cpu(residual).clone()
    ub = None if scale_ub is None else ctypes.byref(ctypes.c_float(float(scale_ub)))
    lib().oracle_rms_norm_per_block_quant(out.data_ptr(), _DT[quant_dtype], scales.data_ptr(),
                                          xc.data_ptr(), w.data_ptr(), ub, _ptr(ro), T, H,
                                          _DT[x.dtype], float(eps), int(group_size),
                                          1 if is_scale_transposed else 0)
    return out, scales, ro


def rms_norm_dynamic_per_token_quant_custom(
        x: torch.Tensor, weight: torch.Tensor, eps: float, scale_ub: Optional[float] = None,
        residual: Optional[torch.Tensor] = None
) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """mcoplib ``op.rms_norm_dynamic_per_token_quant_custom`` (op/rms_norm_dynamic_per_token_quant.cu
    :52-285, kernel/rms_norm_vllm.cuh:330-454), int8 only.

    Returns (int8 codes, scales [T, 1] fp32, new residual or None)."""
    xc, w = _cpu(x), _cpu(weight)
    T, H = _rows(xc)
    out = torch.empty(xc.shape, dtype=torch.int8)
    scales = torch.empty((T, 1), dtype=torch.float32)
    ro = None if residual is None else _cpu(residual).clone()
    ub = None if scale_ub is None else ctypes.byref(ctypes.c_float(float(scale_ub)))
    lib().oracle_rms_norm_quant_custom(out.data_ptr(), scales.data_ptr(), xc.data_ptr(),
                                       w.data_ptr(), ub, _ptr(ro), T, H, _DT[x.dtype],
                                       float(eps))
    return out, scales, ro


# ------------------------------------------------------------------------------------ H4
def rms_norm_smooth_quant(
        x: torch.Tensor, weight: torch.Tensor, smooth: torch.Tensor, eps: float,
        quant_dtype: torch.dtype = torch.int8, residual: Optional[torch.Tensor] = None,
        standard_norm: bool = False
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """mcoplib ``op.rms_norm_dynamic_per_token_quant`` (fused_rms_norm_dq),
    op/fused_rms_norm_dq.cu:69-186, 260-303, 646-667.

    Returns (codes, scales [T] fp32, after_res, after_norm)."""
    xc, w, sm = _cpu(x), _cpu(weight), _cpu(smooth)
    T, H = _rows(xc)
    out = torch.empty(xc.shape, dtype=quant_dtype)
    scales = torch.empty((T,), dtype=torch.float32)
    after_res = torch.empty_like(xc)
    after_norm = torch.empty_like(xc)
    r = None if residual is None else _cpu(residual)
    lib().oracle_rms_norm_smooth_quant(out.data_ptr(), _DT[quant_dtype], scales.data_ptr(),
                                       xc.data_ptr(), w.data_ptr(), _DT[w.dtype], sm.data_ptr(),
                                       _DT[sm.dtype], after_res.data_ptr(), after_norm.data_ptr(),
                                       _ptr(r), T, H, _DT[x.dtype], float(eps),
                                       1 if standard_norm else 0)
    return out, scales, after_res, after_norm


# ------------------------------------------------------------------------------------ H5
def scale_dynamic_quant(h: torch.Tensor, smooth: torch.Tensor
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """mcoplib ``op.scale_dynamic_quant`` (op/scale_dynamic_quant.cu:40-153).

    Returns (int8 codes shaped like h, scales [T] fp32)."""
    hc, sm = _cpu(h), _cpu(smooth)
    assert hc.dtype == torch.bfloat16 and sm.dtype == torch.float32
    T, H = _rows(hc)
    out = torch.empty(hc.shape, dtype=torch.int8)
    scales = torch.empty((T,), dtype=torch.float32)
    lib().oracle_scale_dynamic_quant(out.data_ptr(), scales.data_ptr(), hc.data_ptr(),
                                     sm.data_ptr(), T, H)
    return out, scales


# ------------------------------------------------------------------------------------ quantizers
def dynamic_scaled_int8_quant(x: torch.Tensor, use_azp: bool = False
                              ) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """vLLM ``_C::dynamic_scaled_int8_quant``
    (op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:94-132, 370-422, 459-527).

    Returns (int8 codes shaped like x, scales [T, 1] fp32, azp [T, 1] int32 or None)."""
    xc = _cpu(x)
    T, H = _rows(xc)
    out = torch.empty(xc.shape, dtype=torch.int8)
    scales = torch.empty((T, 1), dtype=torch.float32)
    if use_azp:
        azp = torch.empty((T, 1), dtype=torch.int32)
        lib().oracle_dynamic_scaled_int8_azp_quant(out.data_ptr(), scales.data_ptr(),
                                                   azp.data_ptr(), xc.data_ptr(), T, H,
                                                   _DT[x.dtype])
        return out, scales, azp
    lib().oracle_dynamic_scaled_int8_quant(out.data_ptr(), scales.data_ptr(), xc.data_ptr(), T,
                                           H, _DT[x.dtype])
    return out, scales, None


def dynamic_per_token_scaled_fp8_quant(x: torch.Tensor, scale_ub: Optional[float] = None
                                       ) -> tuple[torch.Tensor, torch.Tensor]:
    """vLLM ``_C::dynamic_per_token_scaled_fp8_quant`` (op/vllm/quantization/fp8/common.cu:142-180,
    375-411).  x may have strided rows (unit last-dimension stride).

    Returns (fp8-e4m3fn codes shaped like x, contiguous; scales [T, 1] fp32)."""
    assert x.device.type == "cpu", "the oracle takes CPU tensors"
    xc = x if (x.dim() == 2 and x.stride(-1) == 1) else x.contiguous()
    T, H = _rows(xc)
    in_stride = xc.stride(0) if xc.dim() == 2 and T > 1 else H
    out = torch.empty(xc.shape, dtype=torch.float8_e4m3fn)
    scales = torch.empty((T, 1), dtype=torch.float32)
    ub = None if scale_ub is None else ctypes.byref(ctypes.c_float(float(scale_ub)))
    lib().oracle_dynamic_per_token_fp8_quant(out.data_ptr(), scales.data_ptr(), xc.data_ptr(),
                                             ub, T, H, in_stride, H, _DT[x.dtype])
    return out, scales


# ------------------------------------------------------------------------------------ norms
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: Optional[torch.Tensor] = None, rms_div: bool = True
             ) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """mcoplib ``op.rms_norm`` (op/fused_rms_norm_dq.cu:305-420, 814-998).

    Returns (out, after_res or None)."""
    xc, w = _cpu(x), _cpu(weight)
    T, H = _rows(xc)
    out = torch.empty_like(xc)
    r = None if residual is None else _cpu(residual)
    ares = None if residual is None else torch.empty_like(xc)
    lib().oracle_rms_norm(out.data_ptr(), xc.data_ptr(), w.data_ptr(), _DT[w.dtype], _ptr(ares),
                          _ptr(r), T, H, _DT[x.dtype], float(eps), 1 if rms_div else 0)
    return out, ares


def head_rms_norm(out: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float,
                  head_offset: int, head_norm: int) -> torch.Tensor:
    """mcoplib ``op.head_rms_norm`` (op/fused_rms_norm_dq.cu:493-578, 669-812): returns a copy
    of ``out`` with heads [head_offset, head_offset + head_norm) of x [T, NH, D] normalized."""
    o, xc, w = _cpu(out).clone(), _cpu(x), _cpu(weight)
    T, NH, D = xc.shape
    lib().oracle_head_rms_norm(o.data_ptr(), xc.data_ptr(), w.data_ptr(), _DT[w.dtype], T, NH, D,
                               int(head_offset), int(head_norm), _DT[x.dtype], float(eps))
    return o


def vllm_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """vLLM ``_C::rms_norm`` (op/vllm/layernorm_kernels.cu:15-86, 186-231); x of any rank, its
    rows are normalized in order.  Returns out [T, H] (contiguous, shaped like x)."""
    xc, w = _cpu(x), _cpu(weight)
    T, H = _rows(xc)
    out = torch.empty_like(xc)
    lib().oracle_vllm_rms_norm(out.data_ptr(), xc.data_ptr(), w.data_ptr(), T, H, _DT[x.dtype],
                               float(eps))
    return out


# ------------------------------------------------------------------------------------ padded
def add_rms_norm_quant_padded(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                              pad_size: int, eps: float, fill: int = 0):
    """mcoplib ``fused_add_rms_norm_dynamic_per_token_quant_padding_output``
    (op/fused_add_layernorm_per_token_quant_padding_output.cu:181-416).  bf16 only.

    Returns (padded uint8 [T, 2*pad_size] -- bytes the op does not write hold ``fill`` --,
    new residual, output_rms bf16, codes int8, scales [T, 1] fp32)."""
    xc, w = _cpu(x), _cpu(weight)
    assert xc.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
    T, H = _rows(xc)
    ro = _cpu(residual).clone()
    padded = torch.full((T, 2 * pad_size), fill, dtype=torch.uint8)
    rms = torch.empty_like(xc)
    q = torch.empty(xc.shape, dtype=torch.int8)
    scales = torch.empty((T, 1), dtype=torch.float32)
    lib().oracle_add_rms_norm_quant_padded(padded.data_ptr(), 2 * pad_size, rms.data_ptr(),
                                           q.data_ptr(), scales.data_ptr(), xc.data_ptr(),
                                           ro.data_ptr(), w.data_ptr(), T, H, float(eps))
    return padded, ro, rms, q, scales


# ------------------------------------------------------------------------------------ formats
def fp8_e4m3fn_from_f32(x: torch.Tensor, mul: float = 1.0) -> torch.Tensor:
    """e4m3fn(clamp(x * mul, +-448)) as uint8 codes (quant_conversions.cuh:23-28)."""
    xc = _cpu(x).to(torch.float32)
    out = torch.empty(xc.shape, dtype=torch.uint8)
    lib().oracle_fp8_e4m3fn_from_f32(out.data_ptr(), xc.data_ptr(), xc.numel(), float(mul))
    return out


def _conv(x: torch.Tensor, fn: str, dtype: torch.dtype) -> torch.Tensor:
    xc = _cpu(x).to(torch.float32)
    out = torch.empty(xc.shape, dtype=dtype)
    getattr(lib(), fn)(out.data_ptr(), xc.data_ptr(), xc.numel())
    return out


def f32_to_bf16_bits(x: torch.Tensor) -> torch.Tensor:
    return _conv(x, "oracle_f32_to_bf16_array", torch.int16)


def f32_to_f16_bits(x: torch.Tensor) -> torch.Tensor:
    return _conv(x, "oracle_f32_to_f16_array", torch.int16)


def f32_to_e4m3fn_bits(x: torch.Tensor) -> torch.Tensor:
    return _conv(x, "oracle_f32_to_e4m3fn_array", torch.uint8)


__all__ = [
    "build", "set_threads", "num_threads", "fused_add_rms_norm",
    "rms_norm_dynamic_per_token_quant", "rms_norm_dynamic_per_token_quant_custom",
    "rms_norm_smooth_quant", "scale_dynamic_quant",
    "dynamic_scaled_int8_quant", "dynamic_per_token_scaled_fp8_quant",
    "add_rms_norm_quant_padded", "rms_norm_per_block_quant", "rms_norm", "head_rms_norm",
    "vllm_rms_norm", "fp8_e4m3fn_from_f32", "f32_to_bf16_bits", "f32_to_f16_bits", "f32_to_e4m3fn_bits",
]

if os.environ.get("MCOP_ORACLE_THREADS"):
    set_threads(int(os.environ["MCOP_ORACLE_THREADS"]))
