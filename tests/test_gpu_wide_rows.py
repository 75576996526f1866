"""Rows wider than the register-resident kernels hold (65536 bf16/fp16 or 32768 fp32 elements
with 16-byte vectors; 16384 on the scalar path) take the multi-pass kernels (one 1024-lane
workgroup per row, re-reading the row each pass) for H1, H2, H3, H4 and H5: bit for bit against
the oracle, as the register-resident ones are."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import custom_ops, op
from gpu_util import (DEV, assert_codes, assert_exact, assert_scales, gen, say)

pytestmark = pytest.mark.gpu

# (dtype, H): just past the vector-path limit, a power of two far past it, and scalar-path rows
# (H not a multiple of the vector width) past the scalar limit
SHAPES = [(torch.bfloat16, 65544), (torch.bfloat16, 131072), (torch.bfloat16, 20001),
          (torch.float16, 65608), (torch.float32, 32772), (torch.float32, 16390)]


def _x(T, H, seed, dtype, scale=1.0):
    x = torch.randn(T, H, generator=gen(seed)) * scale
    x[0, 7] = 40.0 * scale  # an outlier: the absmax row element
    if T > 2:
        x[2].zero_()
    return x.to(dtype)


def _w(H, seed, dtype):
    return (1 + 0.1 * torch.randn(H, generator=gen(seed))).to(dtype)


@pytest.mark.parametrize("dtype,H", SHAPES)
def test_wide_h1_fused_add_rms_norm(dtype, H):
    say(f"wide H1 {dtype} H={H}")
    x, r, w = _x(3, H, 1, dtype), _x(3, H, 2, dtype), _w(H, 3, dtype)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    xd, rd = x.to(DEV), r.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_exact(xd, x_ref, "output")


@pytest.mark.parametrize("dtype,H", SHAPES)
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_wide_h2_norm_quant(dtype, H, qdt):
    say(f"wide H2 {dtype} H={H} {qdt}")
    x, r, w = _x(3, H, 4, dtype), _x(3, H, 5, dtype), _w(H, 6, dtype)
    ubs = (None, 0.05) if qdt == torch.float8_e4m3fn else (None,)
    for res in (None, r):
        for ub in ubs:
            q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, ub,
                                                                          res)
            q = torch.empty(x.shape, dtype=qdt, device=DEV)
            s = torch.empty(3, 1, device=DEV)
            rd = None if res is None else res.to(DEV)
            ubd = None if ub is None else torch.tensor([ub], device=DEV)
            torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, ubd,
                                                          rd)
            torch.cuda.synchronize()
            tag = f"res={res is not None} ub={ub}"
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")
            if res is not None:
                assert_exact(rd, r_ref, tag + " residual")


@pytest.mark.parametrize("dtype,H", SHAPES)
def test_wide_h3_custom(dtype, H):
    say(f"wide H3 {dtype} H={H}")
    x, r, w = _x(3, H, 7, dtype), _x(3, H, 8, dtype), _w(H, 9, dtype)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    rd = r.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x.to(DEV), w.to(DEV), 1e-6, torch.int8,
                                                       residual=rd)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")
    assert_exact(rd, r_ref, "residual")


@pytest.mark.parametrize("dtype,H", SHAPES)
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_wide_h4_smooth_quant(dtype, H, qdt):
    say(f"wide H4 {dtype} H={H} {qdt}")
    x, r = _x(3, H, 10, dtype, 3.0), _x(3, H, 11, dtype)
    for wdt, sdt, res, standard in ((dtype, torch.float32, None, False),
                                    (torch.float32, dtype, r, True)):
        w = _w(H, 12, wdt)
        sm = (0.5 + 1.5 * torch.rand(H, generator=gen(13))).to(sdt)
        q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, res,
                                                                    standard)
        q = torch.empty(x.shape, dtype=qdt, device=DEV)
        s = torch.empty(3, device=DEV)
        ar = torch.empty(x.shape, dtype=dtype, device=DEV)
        an = torch.empty(x.shape, dtype=dtype, device=DEV)
        op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                            None if res is None else res.to(DEV),
                                            standard_norm=standard)
        torch.cuda.synchronize()
        tag = f"w={wdt} s={sdt} res={res is not None} std={standard}"
        assert_exact(ar, ar_ref, tag + " after_res")
        assert_exact(an, an_ref, tag + " after_norm")
        assert_scales(s, s_ref, tag + " scales")
        assert_codes(q, q_ref, tag + " codes")


@pytest.mark.parametrize("H", [65544, 131072, 20001])
def test_wide_h5_scale_dynamic_quant(H):
    say(f"wide H5 H={H}")
    h = _x(3, H, 14, torch.bfloat16)
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(15))
    q_ref, s_ref = oracle.scale_dynamic_quant(h, sm)
    q, s = op.scale_dynamic_quant(h.to(DEV), sm.to(DEV), torch.int8)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


def test_wide_rows_many_rows():
    """More rows than resident workgroups, with a residual, through the headline surface."""
    say("wide rows: 600 x 65544")
    H = 65544
    x, r, w = _x(600, H, 16, torch.bfloat16), _x(600, H, 17, torch.bfloat16), _w(H, 18,
                                                                                 torch.bfloat16)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    rd = r.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x.to(DEV), w.to(DEV), 1e-6, torch.int8,
                                                       residual=rd)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")
    assert_exact(rd, r_ref, "residual")
