"""Helpers of the GPU parity tests: seeded inputs (generated on the CPU, so the oracle sees the
same bits) and the parity bar of the path.

Parity bar (from the path's specification): bf16/fp16/fp32 outputs (residual, after_res,
after_norm, normalized x) bit-exact; fp32 scales within 1e-6 relative; int8 / fp8 codes exact
except at most one code step on at most 1e-4 of the elements.  The implementation is designed to
be bit-exact everywhere; the tests report how many elements differ at all.
"""

from __future__ import annotations

import os
import sys

import torch

DEV = "cuda:0"
SCALE_RTOL = 1e-6
CODE_FRAC = 1e-4
# MCOP_TEST_EXACT=1 tightens the bar to bit equality for codes and scales as well
EXACT = os.environ.get("MCOP_TEST_EXACT", "") == "1"


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(shape, seed, dtype, scale=1.0, mean=0.0):
    return (mean + scale * torch.randn(*shape, generator=gen(seed))).to(dtype)


def weight(H, seed, dtype):
    return (1.0 + 0.1 * torch.randn(H, generator=gen(seed))).to(dtype)


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _ordinal(q: torch.Tensor) -> torch.Tensor:
    """Signed position of each code on its format's number line (adjacent codes differ by 1)."""
    if q.dtype == torch.int8:
        return q.to(torch.int32)
    b = q.view(torch.uint8).to(torch.int32)
    mag = b & 0x7F
    return torch.where((b & 0x80) != 0, -mag, mag)


def assert_codes(q: torch.Tensor, q_ref: torch.Tensor, what: str) -> None:
    q = q.detach().cpu()
    d = (_ordinal(q) - _ordinal(q_ref)).abs()
    n_diff = int((d > 0).sum())
    frac = n_diff / max(1, d.numel())
    say(f"  {what}: {n_diff} of {d.numel()} codes differ (max step {int(d.max()) if d.numel() else 0})")
    assert int(d.max() if d.numel() else 0) <= 1, f"{what}: code differs by more than one step"
    assert frac <= CODE_FRAC, f"{what}: {n_diff} codes differ ({frac:.2e} > {CODE_FRAC})"
    assert not EXACT or n_diff == 0, f"{what}: {n_diff} codes differ (exact mode)"


def assert_scales(s: torch.Tensor, s_ref: torch.Tensor, what: str) -> None:
    s = s.detach().cpu().flatten().double()
    r = s_ref.flatten().double()
    zero = r == 0
    assert torch.all(s[zero] == 0), f"{what}: scale should be 0"
    same = (s == r) | (torch.isnan(s) & torch.isnan(r))  # equal infinities / NaNs included
    rel = ((s - r).abs() / r.abs().clamp_min(1e-300))[~zero & ~same]
    n_diff = int((~same).sum())
    say(f"  {what}: {n_diff} of {s.numel()} scales differ (max rel {float(rel.max()) if rel.numel() else 0:.3e})")
    assert rel.numel() == 0 or float(rel.max()) <= SCALE_RTOL, f"{what}: scale rel err"
    assert not EXACT or n_diff == 0, f"{what}: {n_diff} scales differ (exact mode)"


def assert_exact(t: torch.Tensor, ref: torch.Tensor, what: str) -> None:
    t = t.detach().cpu()
    assert t.dtype == ref.dtype and t.shape == ref.shape, f"{what}: {t.dtype}{tuple(t.shape)}"
    if t.dtype in (torch.bfloat16, torch.float16):
        a, b = t.view(torch.int16), ref.view(torch.int16)
    elif t.dtype == torch.float32:
        a, b = t.view(torch.int32), ref.view(torch.int32)
    else:
        a, b = t, ref
    diff = a != b
    if t.is_floating_point():  # NaN payloads may differ
        diff &= ~(torch.isnan(t) & torch.isnan(ref))
    n_diff = int(diff.sum())
    say(f"  {what}: {n_diff} of {t.numel()} values differ")
    assert n_diff == 0, f"{what}: not bit-exact"
