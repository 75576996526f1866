"""Tensors past 2^31 elements (bf16 buffers past 4 GiB): every row offset must be computed in 64
bits.  The inputs are generated on the GPU (a few GB); rows on both sides of element 2^31 (byte
2^32 of the bf16 buffers), the first rows and the last row are copied back and checked against
the oracle bit for bit, the rest by size-independent properties (finite scales, |code| <= 127).
"""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import custom_ops
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, say

pytestmark = pytest.mark.gpu


def _inputs(T, H, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    r = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    for t in (x, r):  # in slices, so the fp32 temporaries stay small
        for a in range(0, T, 16384):
            t[a:a + 16384] = torch.randn(min(16384, T - a), H, generator=g, device=DEV)
    w = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).to(torch.bfloat16)
    return x, r, w


def _sample_rows(T, H):
    cross = (1 << 31) // H  # the first row at or past element 2^31
    return sorted({0, 1, cross - 1, cross, cross + 1, T - 1})


@pytest.mark.parametrize("H", [8192, 131072])  # the register-resident and the multi-pass kernel
def test_h2_past_2_31_elements(H):
    T = (1 << 31) // H + 16
    say(f"large: custom rms_norm_dynamic_per_token_quant T={T} H={H} ({T * H} elements)")
    x, r, w = _inputs(T, H, 1)
    rows = _sample_rows(T, H)
    xs, rs = x[rows].cpu(), r[rows].cpu()
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8, residual=r)
    torch.cuda.synchronize()
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(xs, w.cpu(), 1e-6,
                                                                        residual=rs)
    assert_exact(r[rows], r_ref, "residual rows")
    assert_scales(s[rows], s_ref, "scale rows")
    assert_codes(q[rows], q_ref, "code rows")
    assert bool(torch.isfinite(s).all()) and bool((s > 0).all())
    assert int(q.abs().max()) <= 127
    del x, r, q, s
    torch.cuda.empty_cache()


def test_h1_past_2_31_elements():
    H = 8192
    T = (1 << 31) // H + 16
    say(f"large: fused_add_rms_norm T={T} H={H} ({T * H} elements)")
    x, r, w = _inputs(T, H, 2)
    rows = _sample_rows(T, H)
    xs, rs = x[rows].cpu(), r[rows].cpu()
    torch.ops._C.fused_add_rms_norm(x, r, w, 1e-6)
    torch.cuda.synchronize()
    x_ref, r_ref = oracle.fused_add_rms_norm(xs, rs, w.cpu(), 1e-6)
    assert_exact(r[rows], r_ref, "residual rows")
    assert_exact(x[rows], x_ref, "output rows")
    del x, r
    torch.cuda.empty_cache()
