"""The kernels' rounding points on the hand-built rows of tests/rounding_points.py: each operator,
called through its drop-in surface on the GPU, must give the hand-derived answer (the same one the
oracle is pinned to in test_oracle_rounding_points.py), not the alternative reading's."""

import pytest
import torch

import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C)
import rounding_points as rp
from gpu_util import DEV, say
from mcoplib_amd import op

pytestmark = pytest.mark.gpu


def _rel(a, b) -> float:
    return abs(float(a) - float(b)) / abs(float(b))


def test_h1_rounding_points_on_gpu():
    c = rp.h1_variance_of_rounded_sum()
    say("H1 hand-built row, 1 x 8 bf16")
    x, r = c["x"].to(DEV), c["r"].to(DEV)
    torch.ops._C.fused_add_rms_norm(x, r, c["w"].to(DEV), c["eps"])
    assert r.float().cpu().view(-1).tolist() == c["r_out"]
    assert x.float().cpu().view(-1).tolist() == c["x_out"]


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_h2_rounding_points_on_gpu(qdt):
    c = rp.h2_double_rounding_of_y()
    say(f"H2 hand-built row, 1 x 8 bf16 -> {qdt}")
    q = torch.empty(1, 8, dtype=qdt, device=DEV)
    s = torch.empty(1, 1, dtype=torch.float32, device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, c["x"].to(DEV), c["w"].to(DEV), s,
                                                  c["eps"], None, None)
    if qdt == torch.int8:
        assert _rel(s.item(), c["int8_scale"]) <= 1e-6
        assert q.cpu().view(-1).tolist() == c["int8_codes"]
    else:
        assert _rel(s.item(), c["fp8_scale"]) <= 1e-6
        assert q.cpu().float().view(-1).tolist() == c["fp8_values"]


def test_h3_rounding_points_on_gpu():
    for c, codes, scale in ((rp.h2_double_rounding_of_y(), "int8_codes", "int8_scale"),
                            (rp.h3_7168_fp32_chain(), "codes", "scale")):
        H = c["x"].shape[1]
        say(f"H3 hand-built row, 1 x {H} bf16")
        q = torch.empty(1, H, dtype=torch.int8, device=DEV)
        s = torch.empty(1, 1, dtype=torch.float32, device=DEV)
        op.rms_norm_dynamic_per_token_quant_custom(q, c["x"].to(DEV), c["w"].to(DEV), s,
                                                   c["eps"], None, None)
        assert _rel(s.item(), c[scale]) <= 1e-6
        assert q.cpu().view(-1).tolist() == c[codes]


@pytest.mark.parametrize("standard", [False, True])
def test_h4_rounding_points_on_gpu(standard):
    c = rp.h4_rereads_rounded_after_res()
    say(f"H4 hand-built row, 1 x 8 bf16, standard_norm={standard}")
    q = torch.empty(1, 8, dtype=torch.int8, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    ar = torch.empty(1, 8, dtype=torch.bfloat16, device=DEV)
    an = torch.empty_like(ar)
    op.rms_norm_dynamic_per_token_quant(q, c["x"].to(DEV), c["w"].to(DEV), c["sm"].to(DEV), s,
                                        c["eps"], ar, an, c["r"].to(DEV), standard)
    assert ar.float().cpu().view(-1).tolist() == c["after_res"]
    assert an.float().cpu().view(-1).tolist() == c["after_norm_std" if standard else "after_norm"]
    if not standard:
        assert _rel(s.item(), c["int8_scale"]) <= 1e-6
        assert q.cpu().view(-1).tolist() == c["int8_codes"]


def test_fp8_quantizer_rounding_points_on_gpu():
    c = rp.fp8_quantizer_divides()
    say("fp8 quantizer hand-built row, 1 x 8 bf16")
    q = torch.empty(1, 8, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(1, 1, dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, c["x"].to(DEV), s, None)
    assert s.item() == c["scale"]
    assert q.cpu().float().view(-1).tolist() == c["values"]


def test_fp8_quotient_beyond_448_on_gpu():
    """A quotient one ulp beyond +-448 codes +-448 in the bounded short form of the fp8
    epilogues (the standalone quantizer here); H2's fp8 codes of the same rows against the
    oracle."""
    c = rp.fp8_quotient_beyond_448()
    say("fp8 quotient one ulp beyond 448, 2 x 8 bf16")
    x = c["x"].to(DEV)
    q = torch.empty(2, 8, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(2, 1, dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, x, s, None)
    assert q.cpu().float().tolist() == c["values"]
    import oracle  # the expected H2 codes of the same rows

    w = torch.ones(8, dtype=torch.bfloat16)
    q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant(c["x"], w, 0.0,
                                                              torch.float8_e4m3fn)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w.to(DEV), s, 0.0, None, None)
    assert torch.equal(s.cpu(), s_ref) and torch.equal(q.cpu().view(torch.uint8),
                                                       q_ref.view(torch.uint8))


def test_h4_fp8_rounding_points_on_gpu():
    import oracle  # only to obtain the row's after_norm, from which the smooth scales are built

    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 64, generator=g) * 2
    w = torch.ones(64)
    _, _, _, u = oracle.rms_norm_smooth_quant(x, w, torch.ones(64), rp.EPS)
    sm, i0, i1 = rp.h4_fp8_divides(u)
    say("H4 fp8 hand-built row, 1 x 64 fp32")
    q = torch.empty(1, 64, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(1, dtype=torch.float32, device=DEV)
    ar = torch.empty(1, 64, dtype=torch.float32, device=DEV)
    an = torch.empty_like(ar)
    op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, rp.EPS, ar, an,
                                        None)
    assert torch.equal(an.cpu(), u)
    assert s.item() == 7.0 / 512.0
    assert q.cpu().float()[0, [i0, i1]].tolist() == [448.0, 1.75]
