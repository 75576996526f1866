"""Special parameters on every kernel path, GPU against the oracle bit for bit: weights and
smooth scales holding zeros, +-inf, NaN, huge and subnormal values; scale bounds of 0, a tiny
value, +inf and NaN; eps of 0 (a zero row then has an infinite rho) and a large eps.  The rows
are ordinary (seeded normal values, one row of zeros); the paths are those of
test_gpu_special_paths.py (latency, bandwidth, element-wise, split-row, multi-pass)."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib, op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say

pytestmark = pytest.mark.gpu

# path -> (row width, rows, split-row kernels allowed)
PATHS = {"exact": (1024, 6, True), "bandwidth": (1024, 300, True), "scalar": (1030, 6, True),
         "split": (65544, 4, True), "multipass": (65544, 4, False)}
UBS = [0.0, 1e-30, float("inf"), float("nan")]


def _special_vec(H, seed, base):
    """A per-channel vector around `base` with zeros, +-inf, NaN, a huge, a subnormal and a
    negative entry at fixed positions."""
    v = base * (1 + 0.1 * torch.randn(H, generator=gen(seed)))
    for k, val in ((3, 0.0), (H // 3, 0.0), (5, float("inf")), (H // 2, float("-inf")),
                   (11, float("nan")), (17, 3.0e38), (23, 1e-39), (29, -2.0)):
        v[k] = val
    return v


def _setup(path, dtype, seed):
    H, T, split = PATHS[path]
    x = torch.randn(T, H, generator=gen(seed))
    x[1] = 0.0
    r = torch.randn(T, H, generator=gen(seed + 1))
    w = _special_vec(H, seed + 2, 1.0)
    return x.to(dtype), r.to(dtype), w.to(dtype), split


def _on(split, fn):
    _lib.set_split_rows(split)
    try:
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        _lib.set_split_rows(True)


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("eps", [1e-6, 0.0, 10.0])
def test_fused_add_rms_norm_params(path, eps):
    say(f"special params: fused_add_rms_norm {path} eps={eps}")
    x, r, w, split = _setup(path, torch.bfloat16, 300)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, eps)
    xd, rd = x.to(DEV), r.to(DEV)
    _on(split, lambda: torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), eps))
    assert_exact(rd, r_ref, "residual")
    assert_exact(xd, x_ref, "output")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("eps", [1e-6, 0.0])
def test_rms_norm_dynamic_per_token_quant_params(path, qdt, eps):
    say(f"special params: vLLM norm-quant {path} {qdt} eps={eps}")
    x, r, w, split = _setup(path, torch.bfloat16, 310)
    for ub in ([None] + UBS if qdt == torch.float8_e4m3fn else [None]):
        for res in (None, r):
            tag = f"ub={ub} res={res is not None}"
            q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, eps, qdt, ub, res)
            q = torch.empty(x.shape, dtype=qdt, device=DEV)
            s = torch.empty(x.shape[0], 1, device=DEV)
            rd = None if res is None else res.to(DEV)
            ubd = None if ub is None else torch.tensor([ub], device=DEV)
            _on(split, lambda: torch.ops._C.rms_norm_dynamic_per_token_quant(
                q, x.to(DEV), w.to(DEV), s, eps, ubd, rd))
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")
            if res is not None:
                assert_exact(rd, r_ref, tag + " residual")


@pytest.mark.parametrize("path", list(PATHS))
def test_custom_op_params(path):
    say(f"special params: mcoplib custom norm-quant {path}")
    x, r, w, split = _setup(path, torch.bfloat16, 320)
    for ub in (None, 0.0, float("inf")):
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, ub, r)
        q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
        s = torch.empty(x.shape[0], 1, device=DEV)
        rd = r.to(DEV)
        ubd = None if ub is None else torch.tensor([ub], device=DEV)
        _on(split, lambda: op.rms_norm_dynamic_per_token_quant_custom(q, x.to(DEV), w.to(DEV), s,
                                                                      1e-6, ubd, rd))
        assert_exact(rd, r_ref, f"ub={ub} residual")
        assert_scales(s, s_ref, f"ub={ub} scales")
        assert_codes(q, q_ref, f"ub={ub} codes")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("standard", [False, True])
def test_smooth_quant_params(path, qdt, standard):
    say(f"special params: smooth quant {path} {qdt} standard={standard}")
    x, r, w, split = _setup(path, torch.bfloat16, 330)
    sm = _special_vec(x.shape[1], 334, 1.2)
    for eps in (1e-6, 0.0):
        for res in (None, r):
            tag = f"eps={eps} res={res is not None}"
            q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, eps, qdt, res,
                                                                        standard)
            q = torch.empty(x.shape, dtype=qdt, device=DEV)
            s = torch.empty(x.shape[0], device=DEV)
            ar = torch.empty(x.shape, dtype=x.dtype, device=DEV)
            an = torch.empty_like(ar)
            _on(split, lambda: op.rms_norm_dynamic_per_token_quant(
                q, x.to(DEV), w.to(DEV), sm.to(DEV), s, eps, ar, an,
                None if res is None else res.to(DEV), standard_norm=standard))
            assert_exact(ar, ar_ref, tag + " after_res")
            assert_exact(an, an_ref, tag + " after_norm")
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")


@pytest.mark.parametrize("path", list(PATHS))
def test_scale_dynamic_quant_params(path):
    say(f"special params: scale_dynamic_quant {path}")
    x, _, _, split = _setup(path, torch.bfloat16, 340)
    sm = _special_vec(x.shape[1], 341, 1.0)
    q_ref, s_ref = oracle.scale_dynamic_quant(x, sm)
    q, s = _on(split, lambda: op.scale_dynamic_quant(x.to(DEV), sm.to(DEV), torch.int8))
    assert_scales(s.reshape(-1), s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("path", list(PATHS))
def test_fp8_quantizer_scale_bounds(path):
    say(f"special params: fp8 quantizer scale bounds {path}")
    x, _, _, split = _setup(path, torch.bfloat16, 350)
    for ub in UBS:
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x, scale_ub=ub)
        q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
        s = torch.empty(x.shape[0], 1, device=DEV)
        ubd = torch.tensor([ub], device=DEV)
        _on(split, lambda: torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, x.to(DEV), s, ubd))
        assert_scales(s, s_ref, f"ub={ub} scales")
        assert_codes(q, q_ref, f"ub={ub} codes")


@pytest.mark.parametrize("path", ["exact", "bandwidth", "split", "multipass"])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_per_block_quant_params(path, qdt):
    say(f"special params: per-block quant {path} {qdt}")
    H = 65664 if path in ("split", "multipass") else None
    x, r, w, split = _setup(path, torch.bfloat16, 360)
    if H:
        g = gen(361)
        x = torch.randn(x.shape[0], H, generator=g).to(torch.bfloat16)
        r = torch.randn(x.shape[0], H, generator=g).to(torch.bfloat16)
        w = _special_vec(H, 362, 1.0).to(torch.bfloat16)
    for ub in ([None] + UBS if qdt == torch.float8_e4m3fn else [None]):
        tag = f"ub={ub}"
        q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, 128, ub, r)
        q = torch.empty(x.shape, dtype=qdt, device=DEV)
        s = torch.empty(x.shape[0], x.shape[1] // 128, device=DEV)
        rd = r.to(DEV)
        ubd = None if ub is None else torch.tensor([ub], device=DEV)
        _on(split, lambda: torch.ops._C.rms_norm_per_block_quant(q, x.to(DEV), w.to(DEV), s, 1e-6,
                                                                  ubd, rd, 128, False))
        assert_exact(rd, r_ref, tag + " residual")
        assert_scales(s, s_ref, tag + " scales")
        assert_codes(q, q_ref, tag + " codes")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("eps", [1e-6, 0.0])
def test_norm_params(path, eps):
    say(f"special params: mcoplib and vLLM rms_norm {path} eps={eps}")
    x, r, w, split = _setup(path, torch.bfloat16, 370)
    for res in (None, r):
        for rms_div in (True, False):
            tag = f"res={res is not None} rms_div={rms_div}"
            out_ref, ares_ref = oracle.rms_norm(x, w, eps, residual=res, rms_div=rms_div)
            out = torch.empty(x.shape, dtype=x.dtype, device=DEV)
            ares = None if res is None else torch.empty(x.shape, dtype=x.dtype, device=DEV)
            _on(split, lambda: op.rms_norm(out, x.to(DEV), w.to(DEV), eps, ares,
                                           None if res is None else res.to(DEV), rms_div))
            assert_exact(out, out_ref, tag + " out")
            if res is not None:
                assert_exact(ares, ares_ref, tag + " after_res")
    o = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    _on(split, lambda: torch.ops._C.rms_norm(o, x.to(DEV), w.to(DEV), eps))
    assert_exact(o, oracle.vllm_rms_norm(x, w, eps), "vLLM rms_norm")


@pytest.mark.parametrize("path", list(PATHS))
def test_padded_op_params(path):
    say(f"special params: padded op {path}")
    x, r, w, split = _setup(path, torch.bfloat16, 380)
    H = x.shape[1]
    pad = (H + 4 + 63) // 64 * 32
    refs = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6)
    T = x.shape[0]
    p = torch.zeros(T, 2 * pad, dtype=torch.int8, device=DEV)
    rms = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(T, 1, device=DEV)
    rd = r.to(DEV)
    _on(split, lambda: op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
        p, rms, q, s, x.to(DEV), rd, w.to(DEV), pad, 1e-6))
    assert torch.equal(p.cpu().view(torch.uint8), refs[0]), "padded rows"
    assert_exact(rd, refs[1], "residual")
    assert_exact(rms, refs[2], "output_rms")
    assert_codes(q, refs[3], "codes")
    assert_scales(s, refs[4], "scales")
