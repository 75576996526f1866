"""Special values on every kernel path of every operator, GPU against the oracle bit for bit.

The rows: zeros, squares that overflow fp32, subnormals, +-inf and NaN elements, an ordinary row,
one large element among tiny ones, values near the bf16 maximum, and a row of values so small
that 1 / absmax overflows binary32; residual rows include one whose sums overflow.  Each
operator runs them on each of its kernel paths, chosen by the row width, the row count and the
library's split-row hook:

- ``exact``: 1024-wide rows, at most 256 rows (the latency path: one row per workgroup, the
  exact-row form where the operator has one);
- ``bandwidth``: the same rows repeated past 256 rows (the generic register form);
- ``scalar``: 1030-wide rows (not a whole number of 16-byte vectors: the element-wise path);
- ``split``: 65544-wide rows (past the register kernels: the split-row kernels);
- ``multipass``: the same width with the split-row kernels switched off (the multi-pass kernels);
- ``scalar-wide``: 20002-wide rows (the element-wise multi-pass kernels).

Special values of the configured widths and of the split path are tested beside each operator's
parity tests as well; this file crosses every path with every operator."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say
from test_gpu_special_values import _rows
from test_gpu_split_rows import (_h1, _h2, _h4, _h5, _mc_norm, _padded, _per_block, _ptq_fp8,
                                 _ptq_int8)
from test_gpu_split_specials import _h3

pytestmark = pytest.mark.gpu

EPS = 1e-6
# path -> (row width, repeats of the special rows, split-row kernels allowed)
PATHS = {"exact": (1024, 1, True), "bandwidth": (1024, 28, True), "scalar": (1030, 1, True),
         "split": (65544, 1, True), "multipass": (65544, 1, False),
         "scalar-wide": (20002, 1, True)}
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _inputs(path, dtype, seed, H=None):
    """x, residual and weight of the path's shape (`H` overrides its width)."""
    H0, reps, _ = PATHS[path]
    H = H or H0
    x = torch.cat([_rows(H, seed), torch.randn(1, H, generator=gen(seed + 1)) * 1e-38])
    r = torch.randn(x.shape[0], H, generator=gen(seed + 2))
    r[8] = 3.0e38  # x + r overflows in fp32 (and rounds to inf in bf16 / fp16)
    w = 1 + 0.1 * torch.randn(H, generator=gen(seed + 3))
    x, r = x.repeat(reps, 1), r.repeat(reps, 1)
    return x.to(dtype), r.to(dtype), w.to(dtype)


def _run(path, fn, *args):
    """fn(*args) on the path's kernels (the split-row kernels off for `multipass`)."""
    split = PATHS[path][2]
    _lib.set_split_rows(split)
    try:
        return fn(*args)
    finally:
        _lib.set_split_rows(True)


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_add_rms_norm(path, dtype):
    say(f"special paths: fused_add_rms_norm {path} {dtype}")
    x, r, w = _inputs(path, dtype, 200)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, EPS)
    out, res = _run(path, _h1, x, r, w, 0)
    assert_exact(res, r_ref, "residual")
    assert_exact(out, x_ref, "output")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_rms_norm_dynamic_per_token_quant(path, dtype, qdt):
    say(f"special paths: vLLM norm-quant {path} {dtype} {qdt}")
    x, r, w = _inputs(path, dtype, 210)
    for res in (None, r):
        for ub in ((None, 0.05) if qdt == torch.float8_e4m3fn else (None,)):
            tag = f"res={res is not None} ub={ub}"
            q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, EPS, qdt, ub,
                                                                          res)
            q, s, rr = _run(path, _h2, x, w, res, qdt, ub)
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")
            if res is not None:
                assert_exact(rr, r_ref, tag + " residual")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", DTYPES)
def test_custom_op(path, dtype):
    say(f"special paths: mcoplib custom norm-quant {path} {dtype}")
    x, r, w = _inputs(path, dtype, 220)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, EPS, residual=r)
    q, s, rr = _run(path, _h3, x, w, r)
    assert_exact(rr, r_ref, "residual")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_smooth_quant(path, dtype, qdt):
    say(f"special paths: smooth quant {path} {dtype} {qdt}")
    x, r, w = _inputs(path, dtype, 230)
    sm = 0.5 + 1.5 * torch.rand(x.shape[1], generator=gen(234))
    for res in (None, r):
        for standard in (False, True):
            tag = f"res={res is not None} standard={standard}"
            q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, EPS, qdt, res,
                                                                        standard)
            q, s, ar, an = _run(path, _h4, x, w, sm, res, qdt, standard)
            assert_exact(ar, ar_ref, tag + " after_res")
            assert_exact(an, an_ref, tag + " after_norm")
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")


@pytest.mark.parametrize("path", list(PATHS))
def test_scale_dynamic_quant(path):
    say(f"special paths: scale_dynamic_quant {path}")
    x, _, _ = _inputs(path, torch.bfloat16, 240)
    sm = 0.5 + 1.5 * torch.rand(x.shape[1], generator=gen(241))
    q_ref, s_ref = oracle.scale_dynamic_quant(x, sm)
    q, s = _run(path, _h5, x, sm)
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", DTYPES)
def test_standalone_quantizers(path, dtype):
    say(f"special paths: standalone quantizers {path} {dtype}")
    x, _, _ = _inputs(path, dtype, 250)
    for use_azp in (False, True):
        tag = f"int8 azp={use_azp}"
        q_ref, s_ref, zp_ref = oracle.dynamic_scaled_int8_quant(x, use_azp=use_azp)
        q, s, zp = _run(path, _ptq_int8, x, use_azp)
        assert_scales(s, s_ref, tag + " scales")
        assert_codes(q, q_ref, tag + " codes")
        if use_azp:
            assert_exact(zp, zp_ref, tag + " azp")
    xd = x.to(DEV)
    for ub in (None, 0.05):
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x, scale_ub=ub)
        q, s = _run(path, _ptq_fp8, xd, ub)
        assert_scales(s, s_ref, f"fp8 ub={ub} scales")
        assert_codes(q, q_ref, f"fp8 ub={ub} codes")


@pytest.mark.parametrize("path", list(PATHS) + ["h7168"])
def test_padded_op(path):
    say(f"special paths: padded op {path}")
    if path == "h7168":  # the reference's 7168 chain, on the latency path
        x, r, w = _inputs("exact", torch.bfloat16, 260, H=7168)
        path = "exact"
    else:
        x, r, w = _inputs(path, torch.bfloat16, 260)
    H = x.shape[1]
    pad = (H + 4 + 63) // 64 * 32
    refs = oracle.add_rms_norm_quant_padded(x, r, w, pad, EPS)
    p, rr, rms, q, s = _run(path, _padded, x, r, w, pad)
    assert torch.equal(p.view(torch.uint8), refs[0]), "padded rows"
    assert_exact(rr, refs[1], "residual")
    assert_exact(rms, refs[2], "output_rms")
    assert_codes(q, refs[3], "codes")
    assert_scales(s, refs[4], "scales")


@pytest.mark.parametrize("path", ["exact", "bandwidth", "split", "multipass"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_per_block_quant(path, dtype, qdt):
    say(f"special paths: per-block quant {path} {dtype} {qdt}")
    # whole groups a row: 65664 = 513 * 128 for the wide paths
    x, r, w = _inputs(path, dtype, 270, H=65664 if path in ("split", "multipass") else None)
    for G in (64, 128):
        for res, ub in ((None, None), (r, None), (r, 0.05)):
            if ub is not None and qdt == torch.int8:
                continue
            tag = f"G={G} res={res is not None} ub={ub}"
            q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, EPS, qdt, G, ub, res)
            q, s, rr = _run(path, _per_block, x, w, res, qdt, G, ub, False)
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")
            if res is not None:
                assert_exact(rr, r_ref, tag + " residual")


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dtype", DTYPES)
def test_norms(path, dtype):
    say(f"special paths: mcoplib and vLLM rms_norm {path} {dtype}")
    x, r, w = _inputs(path, dtype, 280)
    for res in (None, r):
        for rms_div in (True, False):
            tag = f"res={res is not None} rms_div={rms_div}"
            out_ref, ares_ref = oracle.rms_norm(x, w, EPS, residual=res, rms_div=rms_div)
            out, ares = _run(path, _mc_norm, x, w, res, rms_div)
            assert_exact(out, out_ref, tag + " out")
            if res is not None:
                assert_exact(ares, ares_ref, tag + " after_res")

    def vllm(xx, ww):
        o = torch.empty(xx.shape, dtype=xx.dtype, device=DEV)
        torch.ops._C.rms_norm(o, xx.to(DEV), ww.to(DEV), EPS)
        torch.cuda.synchronize()
        return o.cpu()
    assert_exact(_run(path, vllm, x, w), oracle.vllm_rms_norm(x, w, EPS), "vLLM rms_norm")
