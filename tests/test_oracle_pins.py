"""Pins the CPU oracle (oracle/mcop_oracle.c) against what fixes its results independently of it:
the reference's own known-answer vectors and test oracles (restated from the reference's test
files), closed forms, invariants, and float64 computations.  No GPU needed."""

import math

import numpy as np
import pytest
import torch

import oracle

BF16_ULP = 2.0 ** -7  # relative spacing bound of bf16 (8 significant bits)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ============================================================== H5 scale_dynamic_quant
def _ref_test_loop_oracle(h, smooth):
    """The CPU oracle of unit_test/test_scale_dynamic_quant.py:4-20 (float64 python scalars)."""
    flat = h.reshape(-1, h.shape[-1]).float()
    q = torch.zeros_like(flat, dtype=torch.int8)
    s = torch.zeros(flat.shape[0], dtype=torch.float32)
    for t in range(flat.shape[0]):
        d = flat[t] * smooth
        m = torch.abs(d).max().item()
        sc = m / 127.0 if m > 0 else 1.0
        s[t] = sc
        q[t] = torch.round(d / sc).clamp(-128, 127).to(torch.int8)
    return q.reshape(h.shape), s


def test_h5_known_answers_from_reference_test():
    # unit_test/test_scale_dynamic_quant.py:56-60: scales 8/127 and 4/127 within 1e-5
    h = torch.tensor([[[1.0, 2.0, 3.0, 4.0], [4.0, 3.0, 2.0, 1.0]]], dtype=torch.bfloat16)
    sm = torch.tensor([1.0, 1.0, 2.0, 2.0], dtype=torch.float32)
    q, s = oracle.scale_dynamic_quant(h, sm)
    assert abs(s[0].item() - 8.0 / 127) < 1e-5
    assert abs(s[1].item() - 4.0 / 127) < 1e-5
    # codes by hand: v = [1,2,6,8] * 127/8 = [15.875, 31.75, 95.25, 127];
    #                v = [4,3,4,2] * 127/4 = [127, 95.25, 127, 63.5 -> 64 (ties to even)]
    assert q.reshape(2, 4).tolist() == [[16, 32, 95, 127], [127, 95, 127, 64]]


def test_h5_edge_cases_from_reference_test():
    sm8 = torch.ones(8)
    q, s = oracle.scale_dynamic_quant(torch.zeros(1, 4, 8, dtype=torch.bfloat16), sm8)
    assert torch.all(q == 0)                       # :62-67
    assert torch.all(s == 0)
    q, s = oracle.scale_dynamic_quant(torch.ones(1, 4, 8, dtype=torch.bfloat16) * 1000.0, sm8)
    assert torch.all(q.abs() <= 127)               # :68-73
    assert torch.all(q == 127)
    h = (torch.randn(2, 64, 256, generator=_gen(7)) * 1e-7).to(torch.bfloat16)
    q, s = oracle.scale_dynamic_quant(h, torch.ones(256))
    assert torch.all(torch.isfinite(s)) and torch.all(s > 0)   # :107-113


def test_h5_vs_reference_test_oracle_seeded():
    # unit_test/test_scale_dynamic_quant.py:47-54 (seed 13, [2,128,768], smooth = ones),
    # tolerances of the reference: codes atol 1, scales rtol 1e-5
    h = torch.randn(2, 128, 768, generator=_gen(13)).to(torch.bfloat16)
    sm = torch.ones(768)
    q, s = oracle.scale_dynamic_quant(h, sm)
    qr, sr = _ref_test_loop_oracle(h, sm)
    assert torch.allclose(q.float(), qr.float(), rtol=0, atol=1)
    assert torch.allclose(s, sr, rtol=1e-5)
    # and with a non-trivial smooth scale
    sm2 = 0.5 + 1.5 * torch.rand(768, generator=_gen(14))
    q, s = oracle.scale_dynamic_quant(h, sm2)
    qr, sr = _ref_test_loop_oracle(h, sm2)
    assert torch.allclose(q.float(), qr.float(), rtol=0, atol=1)
    assert torch.allclose(s, sr, rtol=1e-5)


def test_h5_scale_is_the_literal_multiplication():
    # scales[t] = A * 0.00787401574803f, a multiplication by the fp32 constant (not A / 127)
    h = torch.randn(64, 512, generator=_gen(15)).to(torch.bfloat16)
    sm = torch.ones(512)
    _, s = oracle.scale_dynamic_quant(h, sm)
    A = h.float().abs().amax(dim=1)
    assert torch.equal(s, A * torch.tensor(0.00787401574803, dtype=torch.float32))


# ============================================================== H2 / H3
def _vllm_forward_native(x, weight, eps, residual=None):
    """vLLM RMSNorm.forward_native, the oracle of unit_test/test_fused_rms_norm_dq.py:77-87."""
    orig = x.dtype
    xf = x.to(torch.float32)
    if residual is not None:
        xf = xf + residual.to(torch.float32)
        residual = xf.to(orig)
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    out = xf.to(orig) * weight
    return out, residual


def _dynamic_int8(y):
    """dynamic_scaled_int8_quant as the reference test uses it (:59-68): scale = absmax/127,
    code = rne(y * 127/absmax) saturated."""
    yf = y.float()
    A = yf.abs().amax(dim=-1, keepdim=True)
    s = A / 127.0
    q = torch.round(yf * (127.0 / A)).clamp(-128, 127).to(torch.int8)
    return q, s


@pytest.mark.parametrize("T,H", [(1, 64), (83, 1033), (83, 2048), (64, 5120), (16, 5137),
                                 (256, 4096)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("add_residual", [False, True])
def test_h2_vs_reference_test_oracle(T, H, dtype, add_residual):
    """The comparison unit_test/test_fused_rms_norm_dq.py:201-211 intends (it returns before
    running it): scales allclose, codes atol 1, residual allclose.  The oracle's sum and rsqrt
    are correctly rounded while the test oracle's are torch's, so the normalized value can
    differ by one bf16 ulp; at most 1% of rows may then show a scale difference of that size."""
    g = _gen(1000 + T + H)
    scale = 1.0 / H
    x = (torch.randn(T, H, generator=g) * scale).to(dtype)
    w = (1.0 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    r = (torch.randn(T, H, generator=g) * scale).to(dtype) if add_residual else None
    eps = 1e-6
    q, s, ro = oracle.rms_norm_dynamic_per_token_quant(x, w, eps, torch.int8, residual=r)
    y_ref, r_ref = _vllm_forward_native(x, w, eps, r)
    q_ref, s_ref = _dynamic_int8(y_ref)
    close = torch.isclose(s, s_ref, rtol=1e-5, atol=1e-8).flatten()
    assert close.float().mean() >= 0.99
    rel = ((s - s_ref).abs() / s_ref).flatten()
    assert rel.max() <= 2 * BF16_ULP
    rows = close.nonzero().flatten()
    assert torch.allclose(q[rows].float(), q_ref[rows].float(), atol=1)
    if add_residual:
        assert torch.equal(ro, r_ref)  # round(x + r) is exact on both sides


def _h2_float64_y(x, w, eps, r=None):
    a = x.double() + (0 if r is None else r.double())
    rho = 1.0 / torch.sqrt((a * a).mean(dim=-1, keepdim=True) + eps)
    return a * rho * w.double()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h2_invariants_and_float64_bound(dtype):
    g = _gen(21)
    T, H = 128, 1024
    x = torch.randn(T, H, generator=g).to(dtype)
    r = torch.randn(T, H, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    q, s, ro = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8, residual=r)
    y64 = _h2_float64_y(x, w, 1e-6, r)
    # scale: (max|y|)/127 with y within two roundings of the float64 value
    A64 = y64.abs().amax(dim=-1, keepdim=True)
    ulp = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 2 ** -22}[dtype]
    assert ((s.double() * 127 - A64).abs() / A64).max() <= 2 * ulp
    assert q.abs().max() <= 127
    # the absmax element of each row is coded +-127
    assert torch.all(q.abs().amax(dim=1) == 127)
    # reconstruction: |q*s - y| <= s/2 + 2 roundings of y
    err = (q.double() * s.double() - y64).abs()
    assert torch.all(err <= s.double() * 0.5001 + 2 * ulp * y64.abs())
    # signs agree wherever the code is non-zero
    nz = q != 0
    assert torch.all(torch.sign(q[nz].double()) == torch.sign(y64[nz]))
    assert torch.equal(ro, (x.float() + r.float()).to(dtype))


@pytest.mark.parametrize("c", [0.75, -3.0, 1e-3, 200.0])
@pytest.mark.parametrize("H", [64, 4096, 1029])
def test_h2_closed_form_constant_and_one_hot_rows(c, H):
    eps = 1e-6
    w = torch.ones(H, dtype=torch.bfloat16)
    # constant row: every element equals c -> every code is sign(c)*127
    x = torch.full((2, H), c, dtype=torch.bfloat16)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, eps, torch.int8)
    sgn = 1 if c > 0 else -1
    assert torch.all(q == sgn * 127)
    cb = float(x[0, 0].float())
    y = float(torch.tensor(cb / math.sqrt(cb * cb + eps)).to(torch.bfloat16))
    assert abs(s[0, 0].item() * 127 - abs(y)) <= 2 * BF16_ULP * abs(y)
    # one-hot row: rho = 1/sqrt(c^2/H + eps); only the hot element is non-zero
    x = torch.zeros(1, H, dtype=torch.bfloat16)
    x[0, H // 3] = c
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, eps, torch.int8)
    assert q[0, H // 3].item() == sgn * 127
    assert int((q != 0).sum()) == 1
    y = cb / math.sqrt(cb * cb / H + eps)
    assert abs(s[0, 0].item() * 127 - abs(y)) <= 2 * BF16_ULP * abs(y)


@pytest.mark.parametrize("k", [-3, 1, 5])
def test_h2_power_of_two_scaling_invariance(k):
    # with eps = 0, x -> 2^k x scales sum(x^2) by 4^k and rho by 2^-k exactly: y, codes and
    # scales are unchanged bit for bit
    g = _gen(31)
    x = torch.randn(32, 512, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(512, generator=g)).to(torch.bfloat16)
    q0, s0, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 0.0, torch.int8)
    q1, s1, _ = oracle.rms_norm_dynamic_per_token_quant(x * (2.0 ** k), w, 0.0, torch.int8)
    assert torch.equal(q0, q1) and torch.equal(s0, s1)


def test_h2_scale_floor_and_ub():
    w = torch.ones(64, dtype=torch.bfloat16)
    # a zero row: int8 scale floor FLT_EPSILON, fp8 floor 1/(448*512); codes 0
    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8)
    assert s.item() == np.finfo(np.float32).eps and torch.all(q == 0)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.float8_e4m3fn)
    assert s.item() == np.float32(1.0) / np.float32(448.0 * 512.0)
    assert torch.all(q.view(torch.uint8) == 0)
    # scale_ub caps A: codes saturate at +-448 for fp8
    x = torch.randn(4, 64, generator=_gen(5)).to(torch.bfloat16)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.float8_e4m3fn,
                                                     scale_ub=0.5)
    assert torch.all(s == np.float32(0.5) / np.float32(448))
    assert q.float().abs().max() == 448


def test_h2_fp8_codes_round_the_quotient():
    g = _gen(41)
    x = torch.randn(64, 2048, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.float8_e4m3fn)
    y64 = _h2_float64_y(x, w, 1e-6)
    A64 = y64.abs().amax(dim=-1, keepdim=True)
    assert ((s.double() * 448 - A64).abs() / A64).max() <= 2 * BF16_ULP
    # codes decode to y/s within half an fp8 step (2^-4 relative) plus y's own rounding
    dec = q.float().double()
    ratio = y64 / s.double()
    assert torch.all((dec - ratio).abs() <= 2 ** -4 * ratio.abs() + 2 * BF16_ULP * ratio.abs()
                     + 2 ** -9)
    assert q.float().abs().amax(dim=1).eq(448).all()


# ============================================================== H1
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h1_residual_exact_and_output_bound(dtype):
    g = _gen(51)
    T, H = 64, 4096
    x = torch.randn(T, H, generator=g).to(dtype)
    r = torch.randn(T, H, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    xo, ro = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    z = (x.float() + r.float()).to(dtype)
    assert torch.equal(ro, z)                       # residual <- round(x + r), bit exact
    z64 = z.double()
    y64 = z64 / torch.sqrt((z64 * z64).mean(-1, keepdim=True) + 1e-6) * w.double()
    ulp = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 2 ** -22}[dtype]
    assert torch.all((xo.double() - y64).abs() <= 2 * ulp * y64.abs() + 1e-30)


def test_h1_vs_vllm_forward_native():
    # vLLM's forward_native normalizes the unrounded sum x + r; the reference kernel (and the
    # oracle) the rounded residual -- outputs agree within the two bf16 roundings
    g = _gen(52)
    x = torch.randn(32, 2048, generator=g).to(torch.bfloat16)
    r = torch.randn(32, 2048, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16)
    xo, ro = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    y_ref, r_ref = _vllm_forward_native(x, w, 1e-6, r)
    assert torch.equal(ro, r_ref)
    d = (xo.float() - y_ref.float()).abs()
    assert torch.all(d <= 2 * BF16_ULP * y_ref.float().abs() + 1e-30)
    assert (d == 0).float().mean() > 0.75


# ============================================================== H4
def test_h4_literal_convention_vs_reference_asserting_test():
    """unit_test/test_rms_norm.py:24-38,70-74: normalized = after_res / rsqrt(ms + eps) * w,
    assert_close(atol=rtol=1e-5), fp32 (here 256 x 4096 instead of 4096^2, seed 42)."""
    g = _gen(42)
    m, n = 256, 4096
    x = torch.randn(m, n, generator=g)
    r = torch.randn(m, n, generator=g)
    w = torch.randn(n, generator=g)
    sm = torch.ones(n)
    q, s, after_res, after_norm = oracle.rms_norm_smooth_quant(x, w, sm, 1e-5, residual=r)
    ar_ref = x + r
    ms = torch.mean(ar_ref * ar_ref, dim=-1, keepdim=True)
    norm_ref = ar_ref / torch.rsqrt(ms + 1e-5) * w
    torch.testing.assert_close(norm_ref, after_norm, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(ar_ref, after_res, atol=1e-5, rtol=1e-5)
    assert torch.equal(after_res, ar_ref)


def test_h4_quant_stage_exact_for_fp32():
    # for fp32 input after_norm is the unrounded u, so the quant stage is reproducible exactly
    # with torch ops: v = u * sm; s = A/127; q = clamp(rne(v * (1/s)), +-127)
    g = _gen(61)
    x = torch.randn(64, 1024, generator=g) * 3
    w = 1 + 0.1 * torch.randn(1024, generator=g)
    sm = 0.5 + 1.5 * torch.rand(1024, generator=g)
    q, s, ar, an = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6)
    v = an * sm
    A = v.abs().amax(dim=1)
    s_ref = A / 127.0
    assert torch.equal(s, s_ref)
    inv = 1.0 / s_ref
    q_ref = torch.round(v * inv[:, None]).clamp(-127, 127).to(torch.int8)
    assert torch.equal(q, q_ref)
    # fp8 (this library's extension; the reference's operator has no fp8 form): s = A/448,
    # codes = e4m3fn(clamp(v / s)), dividing as the path's fp8 quantizers do
    q8, s8, _, _ = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, torch.float8_e4m3fn)
    s8_ref = A / 448.0
    assert torch.equal(s8, s8_ref)
    c = (v / s8_ref[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(q8.view(torch.uint8), c.view(torch.uint8))
    # (random data rarely tells v / s from v * (1/s) at fp8 precision; the hand-built tie of
    # test_oracle_rounding_points.py::test_h4_fp8_divides_by_the_scale does)


def test_h4_literal_vs_standard_forms():
    # literal u = a/rho*w = a*sqrt(ms+eps)*w; standard u = a*rho*w = a/sqrt(ms+eps)*w:
    # their ratio is ms + eps (rows scaled by 3 and 0.1 so that ms != 1)
    g = _gen(62)
    x = torch.randn(2, 512, generator=g)
    x[0] *= 3
    x[1] *= 0.1
    w = torch.ones(512)
    sm = torch.ones(512)
    _, _, ar, lit = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6)
    _, _, _, std = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, standard_norm=True)
    ms = (ar.double() ** 2).mean(dim=1, keepdim=True) + 1e-6
    ratio = lit.double() / std.double()
    assert torch.allclose(ratio, ms.expand_as(ratio), rtol=1e-5)


def test_h4_zero_row_gives_zero_codes_and_scale():
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    w = torch.ones(256, dtype=torch.bfloat16)
    sm = torch.ones(256)
    for qd in (torch.int8, torch.float8_e4m3fn):
        q, s, _, an = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qd)
        assert torch.all(q.view(torch.uint8) == 0) and torch.all(s == 0)


def test_h4_bf16_rounding_points():
    # the bf16 path rounds after_res (the later passes re-read it) and after_norm; the codes
    # come from the unrounded u * smooth
    g = _gen(63)
    x = torch.randn(16, 768, generator=g).to(torch.bfloat16)
    r = torch.randn(16, 768, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(768, generator=g)).to(torch.bfloat16)
    sm = 0.5 + 1.5 * torch.rand(768, generator=g)
    q, s, ar, an = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, residual=r)
    assert torch.equal(ar, (x.float() + r.float()).to(torch.bfloat16))
    a = x.double() + r.double()
    rho = 1 / torch.sqrt((a * a).mean(1, keepdim=True) + 1e-6)
    u64 = ar.double() / rho * w.double()
    assert torch.all((an.double() - u64).abs() <= 2 * BF16_ULP * u64.abs())
    v64 = u64 * sm.double()
    A = v64.abs().amax(1)
    assert torch.all(((s.double() * 127 - A).abs() / A) <= 1e-6)
