"""Argument checks shared by the operator surfaces.

The reference validates with TORCH_CHECK, which raises RuntimeError("Expected <condition> to be
true, but got false."); the checks here use the same condition text so failures read the same.
The reference's checks are not sufficient for memory safety (it trusts shapes and devices);
the extra checks below (all on CUDA, matching element counts) raise RuntimeError as well.
"""

from __future__ import annotations

from typing import Optional

import torch

_TORCH_NAMES = {
    torch.float32: "Float", torch.float16: "Half", torch.bfloat16: "BFloat16",
    torch.int8: "Char", torch.float8_e4m3fn: "Float8_e4m3fn", torch.int32: "Int",
    torch.int64: "Long", torch.float64: "Double", torch.uint8: "Byte",
}
FLOAT_TYPES = (torch.float32, torch.float16, torch.bfloat16)


def torch_check(cond: bool, text: str) -> None:
    if not cond:
        raise RuntimeError(f"Expected {text} to be true, but got false.")


def dispatch_check(dtype: torch.dtype, name: str, allowed=FLOAT_TYPES) -> None:
    """The AT_DISPATCH_SWITCH error for a dtype outside the dispatched list."""
    if dtype not in allowed:
        raise RuntimeError(f'"{name}" not implemented for \'{_TORCH_NAMES.get(dtype, str(dtype))}\'')


def on_cuda(name: str, *tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{name}: all tensors must be on a CUDA (HIP) device, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{name}: tensors on different devices ({dev} and {t.device})")
    assert dev is not None
    return dev


def numel_check(name: str, what: str, t: torch.Tensor, n: int) -> None:
    if t.numel() != n:
        raise RuntimeError(f"{name}: {what} has {t.numel()} elements, expected {n}")


def contiguous_check(name: str, what: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise RuntimeError(f"{name}: {what} must be contiguous")


def rows_of(t: torch.Tensor) -> tuple[int, int]:
    """(num_tokens, hidden_size) of a [..., hidden_size] tensor, as the reference computes them
    (numel / size(-1))."""
    if t.dim() == 0:
        raise RuntimeError("expected a tensor with at least one dimension")
    hidden = t.size(-1)
    if hidden == 0:
        raise RuntimeError("hidden_size (the last dimension) must be positive")
    return t.numel() // hidden, hidden
