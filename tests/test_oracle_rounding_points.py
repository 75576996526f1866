"""The oracle's rounding points, pinned by hand-built rows (tests/rounding_points.py).

For each case the expected outputs were worked out by hand; the test checks that the oracle
gives them, and that the plausible alternative reading (computed here with torch, step by step)
gives a different answer -- so an oracle that followed the alternative would fail.  Reference
lines are cited in the case builders."""

import math

import numpy as np
import torch

import oracle
import rounding_points as rp

BF = torch.bfloat16


def _rho64(a: torch.Tensor, eps: float) -> torch.Tensor:
    return 1.0 / torch.sqrt((a.double() ** 2).mean(-1, keepdim=True) + eps)


def _rel(a, b) -> float:
    return abs(float(a) - float(b)) / abs(float(b))


def test_h1_variance_is_taken_over_the_rounded_sum():
    c = rp.h1_variance_of_rounded_sum()
    xo, ro = oracle.fused_add_rms_norm(c["x"], c["r"], c["w"], c["eps"])
    assert ro.float().view(-1).tolist() == c["r_out"]
    assert xo.float().view(-1).tolist() == c["x_out"]
    # alternative: rho from the unrounded x + r, applied to the rounded z
    a = c["x"].float() + c["r"].float()
    z = a.to(BF).float()
    alt = ((z * _rho64(a, c["eps"]).float()).to(BF).float() * c["w"].float()).to(BF).float()
    assert alt.view(-1).tolist() == c["x_out_alt"] != c["x_out"]


def test_h2_and_h3_round_y_twice():
    c = rp.h2_double_rounding_of_y()
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant(c["x"], c["w"], c["eps"], torch.int8)
    assert _rel(s.item(), c["int8_scale"]) <= 1e-6
    assert q.view(-1).tolist() == c["int8_codes"]
    q8, s8, _ = oracle.rms_norm_dynamic_per_token_quant(c["x"], c["w"], c["eps"],
                                                        torch.float8_e4m3fn)
    assert _rel(s8.item(), c["fp8_scale"]) <= 1e-6
    assert q8.float().view(-1).tolist() == c["fp8_values"]
    # mcoplib's own operator of the same name, generic chain: the same y
    qc, sc, _ = oracle.rms_norm_dynamic_per_token_quant_custom(c["x"], c["w"], c["eps"])
    assert _rel(sc.item(), c["int8_scale"]) <= 1e-6
    assert qc.view(-1).tolist() == c["int8_codes"]
    # alternative: one rounding, y = b(a * rho * w)
    a = c["x"].float()
    y1 = (a * _rho64(a, c["eps"]).float() * c["w"].float()).to(BF).float()
    s_alt = y1.abs().max().item() / 127.0
    assert _rel(s_alt, c["int8_scale_alt"]) <= 1e-6
    assert _rel(s_alt, c["int8_scale"]) > 1e-3


def test_h4_normalizes_the_rounded_after_res():
    c = rp.h4_rereads_rounded_after_res()
    q, s, ar, an = oracle.rms_norm_smooth_quant(c["x"], c["w"], c["sm"], c["eps"], torch.int8,
                                                c["r"])
    assert ar.float().view(-1).tolist() == c["after_res"]
    assert an.float().view(-1).tolist() == c["after_norm"]
    assert _rel(s.item(), c["int8_scale"]) <= 1e-6
    assert q.view(-1).tolist() == c["int8_codes"]
    _, _, _, an_std = oracle.rms_norm_smooth_quant(c["x"], c["w"], c["sm"], c["eps"],
                                                   torch.int8, c["r"], standard_norm=True)
    assert an_std.float().view(-1).tolist() == c["after_norm_std"]
    # alternative: the later passes use the unrounded a
    a = c["x"].float() + c["r"].float()
    rho = _rho64(a, c["eps"]).float()
    alt = (a / rho * c["w"].float()).to(BF).float()
    alt_std = (a * rho * c["w"].float()).to(BF).float()
    assert alt.view(-1).tolist() == c["after_norm_alt"] != c["after_norm"]
    assert alt_std.view(-1).tolist() == c["after_norm_std_alt"] != c["after_norm_std"]
    assert _rel(c["int8_scale_alt"], c["int8_scale"]) > 1e-3


def test_h3_at_7168_keeps_the_fp32_chain():
    c = rp.h3_7168_fp32_chain()
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant_custom(c["x"], c["w"], c["eps"])
    assert _rel(s.item(), c["scale"]) <= 1e-6
    assert q.view(-1).tolist() == c["codes"]
    # alternative: the generic chain (y rounded twice, 1.5e-6 floor) at this width
    a = c["x"].float()
    rho = _rho64(a, c["eps"]).float()
    y = ((a * rho).to(BF).float() * c["w"].float()).to(BF).float()
    s_alt = y.abs().max().item() / 127.0
    assert _rel(s_alt, c["scale_alt"]) <= 1e-6
    assert _rel(s_alt, c["scale"]) > 1e-3
    # one element off 7168 the generic chain applies
    x2 = torch.cat([c["x"], torch.zeros(1, 8, dtype=BF)], dim=1)
    w2 = torch.cat([c["w"], torch.ones(8, dtype=BF)])
    _, s2, _ = oracle.rms_norm_dynamic_per_token_quant_custom(x2, w2, c["eps"])
    rho2 = 1.0 / math.sqrt(20.0 / 7176 + c["eps"])
    y2 = float((torch.tensor(4.0 * rho2).to(BF).float() * 1.5).to(BF))
    assert _rel(s2.item(), y2 / 127.0) <= 1e-6


def test_fp8_quantizer_divides_by_the_scale():
    c = rp.fp8_quantizer_divides()
    q, s = oracle.dynamic_per_token_scaled_fp8_quant(c["x"])
    assert s.item() == c["scale"]
    assert q.float().view(-1).tolist() == c["values"]
    # alternative: multiply by the rounded reciprocal
    alt = (c["x"].float() * (1.0 / s)).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    assert alt.view(-1).tolist() == c["values_alt"] != c["values"]
    # H2's fp8 stage divides the same way (its quantizer is this one's, applied to y)


def test_fp8_quotient_beyond_448():
    c = rp.fp8_quotient_beyond_448()
    A = np.float32(1.0234375)
    s = A / np.float32(448.0)
    assert s.dtype == np.float32 and float(A / s) == c["quotient"]  # one ulp above 448
    q, sc = oracle.dynamic_per_token_scaled_fp8_quant(c["x"])
    assert sc.view(-1).tolist() == [float(s)] * 2
    assert q.float().tolist() == c["values"]


def test_h4_fp8_divides_by_the_scale():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 64, generator=g) * 2
    w = torch.ones(64)
    _, _, _, u = oracle.rms_norm_smooth_quant(x, w, torch.ones(64), rp.EPS)
    sm, i0, i1 = rp.h4_fp8_divides(u)
    q, s, _, _ = oracle.rms_norm_smooth_quant(x, w, sm, rp.EPS, torch.float8_e4m3fn)
    assert s.item() == 7.0 / 512.0
    assert q.float()[0, [i0, i1]].tolist() == [448.0, 1.75]
    v = u * sm
    alt = (v * (1.0 / s)[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    assert alt[0, [i0, i1]].tolist() == [448.0, 1.875]
