"""ctypes binding of libmcop_norm.so (the gfx950 kernels and their C ABI, include/mcop_norm.h).

The library is loaded once at import, before the C++ operator surfaces (_torch_ops.so, which
links the same library).  There is no fallback: if the library is missing or does not export the
expected ABI, importing this module raises ImportError, and every operator of the package
therefore fails loudly instead of computing anything elsewhere.  The binding itself serves the
launch-shape override, the ABI checks of the tests, and callers that want the raw ABI from
Python.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmcop_norm.so"
ABI_VERSION = 2

# mcop_dtype codes (include/mcop_norm.h)
BF16, F16, F32, I8, FP8_E4M3FN = 0, 1, 2, 3, 4


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m mcoplib_amd._build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(LIB_PATH))
    P, I64, F, I, U32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_uint32
    lib.mcop_fused_add_rms_norm.argtypes = [P, I64, P, P, I64, I64, I, F, P]
    lib.mcop_rms_norm_dynamic_per_token_quant.argtypes = [P, I, P, P, P, P, P, I64, I64, I, F, P]
    lib.mcop_rms_norm_dynamic_per_token_quant_noalloc.argtypes = [P, I, P, P, P, P, P, I64, I64,
                                                                   I, F, P]
    lib.mcop_rms_norm_smooth_quant.argtypes = [P, I, P, P, P, I, P, I, P, P, P, I64, I64, I, F,
                                               U32, P]
    lib.mcop_scale_dynamic_quant.argtypes = [P, P, P, P, I64, I64, P]
    lib.mcop_fp8_e4m3fn_from_f32.argtypes = [P, P, I64, F, P]
    lib.mcop_dynamic_scaled_int8_quant.argtypes = [P, P, P, P, I64, I64, I, P]
    lib.mcop_dynamic_per_token_scaled_fp8_quant.argtypes = [P, P, P, P, I64, I64, I64, I64, I, P]
    lib.mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output.argtypes = [
        P, P, P, P, P, P, P, I64, I64, I64, F, P]
    lib.mcop_rms_norm_per_block_quant.argtypes = [P, I, P, P, P, P, P, I64, I64, I, F, I64, I,
                                                   P]
    lib.mcop_rms_norm.argtypes = [P, P, P, I, P, P, I64, I64, I, F, I, P]
    lib.mcop_head_rms_norm.argtypes = [P, P, P, I, I64, I64, I64, I64, I64, I, F, P]
    lib.mcop_vllm_rms_norm.argtypes = [P, P, P, I64, I64, I, I64, I64, I64, I64, I64, I, F, P]
    lib.mcop_rms_norm_dynamic_per_token_quant_custom.argtypes = [P, P, P, P, P, P, I64, I64, I,
                                                                  F, P]
    lib.mcop_debug_set_launch_override.argtypes = [I, I]
    lib.mcop_debug_set_split_rows.argtypes = [I]
    lib.mcop_debug_fail_split_waits.argtypes = [I]
    for fn in ("mcop_fused_add_rms_norm", "mcop_rms_norm_dynamic_per_token_quant",
               "mcop_rms_norm_dynamic_per_token_quant_noalloc",
               "mcop_rms_norm_smooth_quant", "mcop_scale_dynamic_quant",
               "mcop_fp8_e4m3fn_from_f32", "mcop_debug_set_launch_override",
               "mcop_debug_set_split_rows", "mcop_debug_fail_split_waits", "mcop_abi_version",
               "mcop_dynamic_scaled_int8_quant", "mcop_dynamic_per_token_scaled_fp8_quant",
               "mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output",
               "mcop_rms_norm_per_block_quant", "mcop_rms_norm", "mcop_head_rms_norm",
               "mcop_vllm_rms_norm", "mcop_rms_norm_dynamic_per_token_quant_custom"):
        getattr(lib, fn).restype = I
    lib.mcop_last_error.restype = ctypes.c_char_p
    lib.mcop_last_error.argtypes = []
    got = lib.mcop_abi_version()
    if got != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {got}, expected {ABI_VERSION}")
    return lib


lib = _load()


def check(rc: int) -> None:
    """Raise RuntimeError with the library's message on a non-zero status."""
    if rc != 0:
        msg = lib.mcop_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg or f"libmcop_norm status {rc}")


try:  # raw hipStream_t of the current torch stream without building a Stream object
    _raw_stream = torch._C._cuda_getCurrentRawStream  # type: ignore[attr-defined]
except AttributeError:  # pragma: no cover
    _raw_stream = None


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t (as an int) of torch's current stream on t's device."""
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(t.device).cuda_stream


def set_launch_override(vectors_per_lane: int = 0, lanes_per_row: int = 0) -> None:
    """Force the row kernels' launch shape for later calls from this thread (0, 0 = automatic;
    a debug hook for tests and tuning). Results do not change."""
    check(lib.mcop_debug_set_launch_override(int(vectors_per_lane), int(lanes_per_row)))


def set_split_rows(enabled: bool = True) -> None:
    """Whether rows too wide for one workgroup's registers may take the split-row kernels (the
    default) or always the multi-pass kernels, for later calls from this thread (a debug hook
    for tests and A/B timing). Results do not change."""
    check(lib.mcop_debug_set_split_rows(1 if enabled else 0))


def fail_split_waits(on: bool = True) -> None:
    """Make the split-row launches of later calls from this thread fail every exchange at once
    (their error word set before the kernel starts; a test hook for the failure path: such rows
    get NaN scales, or NaN outputs for the norms); False restores normal launches."""
    check(lib.mcop_debug_fail_split_waits(1 if on else 0))
