"""Rows wider than the register-resident kernels hold (65536 bf16/fp16 or 32768 fp32 elements
with 16-byte vectors; 16384 on the scalar path) take the multi-pass kernels (one 1024-lane
workgroup per row, re-reading the row each pass) in every operator: bit for bit against the
oracle, as the register-resident ones are."""

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


@pytest.mark.parametrize("dtype,H", SHAPES + [(torch.bfloat16, 163848)])  # past the LDS-held part
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


@pytest.mark.parametrize("H", [65544, 131072, 20001, 163848])
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


# --------------------------------------------- the operators beyond the north-star path


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 65544), (torch.bfloat16, 65537),
                                     (torch.float32, 32772), (torch.bfloat16, 163848)])
def test_wide_standalone_quantizers(dtype, H):
    say(f"wide quantizers {dtype} H={H}")
    x = _x(3, H, 20, dtype)
    x[1, 3] = -80.0
    for azp in (False, True):
        q_ref, s_ref, z_ref = oracle.dynamic_scaled_int8_quant(x, use_azp=azp)
        q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
        s = torch.empty(3, 1, device=DEV)
        z = torch.empty(3, 1, dtype=torch.int32, device=DEV) if azp else None
        torch.ops._C.dynamic_scaled_int8_quant(q, x.to(DEV), s, z)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, f"int8 azp={azp} scales")
        assert_codes(q, q_ref, f"int8 azp={azp} codes")
        if azp:
            assert torch.equal(z.cpu().flatten(), z_ref.flatten())
    # fp8 with strided rows on both sides and a scale bound
    big = torch.zeros(3, H + 24, dtype=dtype)
    big[:, :H] = x
    xd = big.to(DEV)[:, :H]
    for ub in (None, 0.05):
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x, ub)
        qb = torch.empty(3, H + 40, dtype=torch.float8_e4m3fn, device=DEV)
        s = torch.empty(3, 1, device=DEV)
        ubd = None if ub is None else torch.tensor([ub], device=DEV)
        torch.ops._C.dynamic_per_token_scaled_fp8_quant(qb[:, :H], xd, s, ubd)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, f"fp8 ub={ub} scales")
        assert_codes(qb[:, :H].contiguous(), q_ref, f"fp8 ub={ub} codes")


@pytest.mark.parametrize("H", [65544, 65540, 163848])
def test_wide_padded(H):
    say(f"wide padded H={H}")
    pad = (H + 4 + 63) // 64 * 32
    x, r, w = _x(3, H, 21, torch.bfloat16), _x(3, H, 22, torch.bfloat16), _w(H, 23,
                                                                             torch.bfloat16)
    p_ref, r_ref, rms_ref, q_ref, s_ref = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6)
    p = torch.zeros(3, 2 * pad, dtype=torch.int8, device=DEV)
    rms = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(3, 1, device=DEV)
    rd = r.to(DEV)
    op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(p, rms, q, s, x.to(DEV), rd,
                                                                  w.to(DEV), pad, 1e-6)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_exact(rms, rms_ref, "output_rms")
    assert_codes(q, q_ref, "codes")
    assert_scales(s, s_ref, "scales")
    assert torch.equal(p.cpu().view(torch.uint8), p_ref), "padded rows"


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("misaligned", [False, True])
@pytest.mark.parametrize("with_res", [True, False])
def test_wide_per_block(qdt, G, misaligned, with_res):
    say(f"wide per-block {qdt} G={G} misaligned={misaligned} res={with_res}")
    H = 65536 + 128 if with_res else 131072 + 128  # past the on-chip head either way
    x, w = _x(3, H, 24, torch.bfloat16), _w(H, 26, torch.bfloat16)
    r = _x(3, H, 25, torch.bfloat16) if with_res else None
    for transposed, ub in ((False, None), (True, 0.05 if qdt == torch.float8_e4m3fn else None)):
        q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, ub, r,
                                                              transposed)
        if misaligned:  # one element into a buffer: the scalar path
            xb = torch.empty(3 * H + 1, dtype=torch.bfloat16, device=DEV)
            xb[1:] = x.flatten().to(DEV)
            xd = xb[1:].view(3, H)
        else:
            xd = x.to(DEV)
        q = torch.empty(x.shape, dtype=qdt, device=DEV)
        s = torch.empty(H // G, 3, device=DEV) if transposed else torch.empty(3, H // G,
                                                                               device=DEV)
        rd = r.to(DEV) if with_res else None
        ubd = None if ub is None else torch.tensor([ub], device=DEV)
        torch.ops._C.rms_norm_per_block_quant(q, xd, w.to(DEV), s, 1e-6, ubd, rd, G, transposed)
        torch.cuda.synchronize()
        tag = f"transposed={transposed} ub={ub}"
        if with_res:
            assert_exact(rd, r_ref, tag + " residual")
        assert_scales(s, s_ref, tag + " scales")
        assert_codes(q, q_ref, tag + " codes")


@pytest.mark.parametrize("dtype,wdtype,H", [(torch.bfloat16, torch.bfloat16, 65544),
                                            (torch.float16, torch.float32, 65608),
                                            (torch.float32, torch.float32, 32776),
                                            (torch.bfloat16, torch.bfloat16, 20001),
                                            (torch.bfloat16, torch.float32, 163848)])
def test_wide_norms(dtype, wdtype, H):
    say(f"wide norms {dtype} w={wdtype} H={H}")
    x, r, w = _x(3, H, 27, dtype), _x(3, H, 28, dtype), _w(H, 29, wdtype)
    for res in (None, r):
        for rms_div in (True, False):
            out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=res, rms_div=rms_div)
            out = torch.empty(x.shape, dtype=dtype, device=DEV)
            ares = torch.empty(x.shape, dtype=dtype, device=DEV) if res is not None else None
            op.rms_norm(out, x.to(DEV), w.to(DEV), 1e-6, ares,
                        None if res is None else res.to(DEV), rms_div)
            torch.cuda.synchronize()
            tag = f"res={res is not None} rms_div={rms_div}"
            assert_exact(out, out_ref, tag + " out")
            if res is not None:
                assert_exact(ares, ares_ref, tag + " after_res")
    if dtype != torch.float16:
        # vLLM rms_norm on a 3-D view with strided rows
        big = torch.randn(2, 3, H + 16, generator=gen(30)).to(dtype)
        xv = big[:, :, :H]
        wv = _w(H, 31, dtype)
        ref = oracle.vllm_rms_norm(xv.contiguous().view(6, H), wv, 1e-6)
        o = torch.empty(2, 3, H, dtype=dtype, device=DEV)
        torch.ops._C.rms_norm(o, big.to(DEV)[:, :, :H], wv.to(DEV), 1e-6)
        torch.cuda.synchronize()
        assert_exact(o.view(6, H), ref, "vLLM rms_norm 3-D strided")


def test_wide_head_rms_norm():
    say("wide head_rms_norm D=65544")
    T, NH, D = 2, 3, 65544
    hs = torch.randn(T, NH, D, generator=gen(32)).to(torch.bfloat16)
    w = _w(NH * D, 33, torch.bfloat16).view(NH, D)
    base = torch.zeros_like(hs)
    ref = oracle.head_rms_norm(base, hs, w, 1e-6, 1, 2)
    out = base.to(DEV)
    op.head_rms_norm(out, hs.to(DEV), w.to(DEV), 1e-6, 1, 2)
    torch.cuda.synchronize()
    assert_exact(out, ref, "head_rms_norm")


# Widths whose only fitting register-resident kernel spills registers (eight or sixteen vectors
# a lane; the build's resource remarks list them): the launch code sends these rows to the
# multi-pass kernel as well.  fp16 SmoothQuant with fp32 weight and smooth needs eight vectors a
# lane from 16392 on; bf16 H2 fp8 sixteen from 32776 on; the fp16 padded op and the fp16 norm
# with fp32 weights sixteen from 32776 on.
@pytest.mark.parametrize("H", [20480, 32768])
def test_spilling_widths_h4_fp16_fp32_weights(H):
    say(f"spilling-width H4 fp16 x, fp32 w/smooth, H={H}")
    x, w = _x(3, H, 30, torch.float16), _w(H, 31, torch.float32)
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(32))
    for qdt in (torch.int8, torch.float8_e4m3fn):
        q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt)
        q = torch.empty(x.shape, dtype=qdt, device=DEV)
        s = torch.empty(3, device=DEV)
        ar = torch.empty(x.shape, dtype=torch.float16, device=DEV)
        an = torch.empty_like(ar)
        op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                            None)
        torch.cuda.synchronize()
        assert_exact(ar, ar_ref, f"{qdt} after_res")
        assert_exact(an, an_ref, f"{qdt} after_norm")
        assert_scales(s, s_ref, f"{qdt} scales")
        assert_codes(q, q_ref, f"{qdt} codes")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_spilling_widths_h2_fp8(dtype):
    H = 49152
    say(f"spilling-width H2 {dtype} fp8 H={H}")
    x, r, w = _x(3, H, 33, dtype), _x(3, H, 34, dtype), _w(H, 35, dtype)
    for res in (None, r):
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6,
                                                                      torch.float8_e4m3fn,
                                                                      None, res)
        q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
        s = torch.empty(3, 1, device=DEV)
        rd = None if res is None else res.to(DEV)
        torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, None, rd)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
        if res is not None:
            assert_exact(rd, r_ref, "residual")


# Rows whose maximum sits in different places relative to the multi-pass kernel's on-chip head
# (with a residual the bf16 head is the first 9 x 1024 vectors, 73728 elements; the tail, re-read
# from memory each pass, starts there): constant rows, zero and tiny tails, near-equal maxima in
# one lane or spread over lanes, non-finite values, huge and zero weights.  Bit for bit against
# the oracle.
TAIL0 = 73728


def _tail_rows(H, seed):
    g = gen(seed)
    x = torch.randn(10, H, generator=g)
    r = torch.randn(10, H, generator=g) * 0.5
    lane0 = [TAIL0 + 8 * 1024 * k for k in range((H - TAIL0) // 8192)]  # lane 0's tail vectors
    x[1] = 1.0
    r[1] = 0.0                                  # a constant row
    x[2, TAIL0:] = 0.0
    r[2, TAIL0:] = 0.0                          # a zero tail
    for k, p in enumerate(lane0[:6]):           # six near-equal maxima in one lane
        x[3, p] = 30.0 - 0.01 * k
    for k, p in enumerate((TAIL0 + 8 * 5, TAIL0 + 8 * 1500 + 3, H - 1)):  # near-ties, 3 lanes
        x[4, p] = 40.0 - 0.15 * k
    x[5] *= 1e-34                               # tiny values: products below 2^-100
    r[5] *= 1e-34
    x[6, TAIL0 + 77] = float("inf")             # a non-finite value in the tail
    x[7, :TAIL0] *= 5.0                         # the maximum in the head, a small tail
    x[8, TAIL0:] *= 5.0                         # the maximum in the tail
    x[9, H - 8:] = 50.0                         # the maximum at the row's end
    return x.to(torch.bfloat16), r.to(torch.bfloat16)


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_wide_tail_maxima_h2(qdt):
    H = 163840
    x, r = _tail_rows(H, 40)
    for wname, w in (("normal", _w(H, 41, torch.bfloat16)),
                     ("large tail weights", _w(H, 42, torch.float32))):
        if wname != "normal":
            w = w.clone()
            w[TAIL0 + 1000::4099] = 3e30  # a few huge weights among the tail
            w[TAIL0 + 9::7001] = 0.0
            w = w.to(torch.bfloat16)
        say(f"wide tail maxima H2 {qdt} weights: {wname}")
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt,
                                                                      residual=r)
        q = torch.empty(x.shape, dtype=qdt, device=DEV)
        s = torch.empty(x.shape[0], 1, device=DEV)
        rd = r.to(DEV)
        torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, None, rd)
        torch.cuda.synchronize()
        assert_exact(rd, r_ref, "residual")
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")


def test_wide_tail_maxima_h3_and_no_residual():
    H = 163840
    x, r = _tail_rows(H, 43)
    w = _w(H, 44, torch.bfloat16)
    say("wide tail maxima H3 (custom op)")
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    rd = r.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x.to(DEV), w.to(DEV), 1e-6, torch.int8,
                                                       residual=rd)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")
    # without a residual the bf16 head holds 16 x 1024 vectors: a 262144-wide row has a tail
    H2 = 262144
    g = gen(45)
    xs = torch.randn(4, H2, generator=g)
    xs[1, 131072 + 5] = 80.0
    xs[2, 131072:] = 2.0                        # a constant tail
    xs[3, 131072 + 16::8192] = 33.0             # many equal maxima spread over lanes
    xs = xs.to(torch.bfloat16)
    w2 = _w(H2, 46, torch.bfloat16)
    say("wide tail maxima H2 no residual 262144")
    q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant(xs, w2, 1e-6, torch.int8)
    q = torch.empty(xs.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(4, 1, device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, xs.to(DEV), w2.to(DEV), s, 1e-6, None, None)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


# Exact-row (EX) instantiations that spill where their generic form does not (the build's
# resource remarks list them): fp32 H1 at eight vectors a lane, and fp16 SmoothQuant with fp32
# weights and fp16 smooth scales at eight.  On the latency path (at most 256 rows) the launch
# code would take the EX form for these exact rows; it must keep the generic one instead.  A
# child process with MCOP_DEBUG_TRACE=1 (the trace switch is read once per process) runs both
# and checks them against the oracle.
_EX_SPILL_SCRIPT = r"""
import sys, torch
sys.path.insert(0, "tests")
import oracle, mcoplib_amd._C
from mcoplib_amd import op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen
x = torch.randn(4, 16384, generator=gen(40)).float()
r = torch.randn(4, 16384, generator=gen(41)).float()
w = (1 + 0.1 * torch.randn(16384, generator=gen(42))).float()
x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
xd, rd = x.to(DEV), r.to(DEV)
torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), 1e-6)
torch.cuda.synchronize()
assert_exact(rd, r_ref, "H1 residual")
assert_exact(xd, x_ref, "H1 output")
H = 20480
x = torch.randn(4, H, generator=gen(43)).half()
r = torch.randn(4, H, generator=gen(44)).half()
w = (1 + 0.1 * torch.randn(H, generator=gen(45))).float()
sm = (0.5 + 1.5 * torch.rand(H, generator=gen(46))).half()
q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6,
                                                            torch.float8_e4m3fn, r)
q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
s = torch.empty(4, device=DEV)
ar, an = torch.empty_like(x, device=DEV), torch.empty_like(x, device=DEV)
op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                    r.to(DEV))
torch.cuda.synchronize()
assert_exact(ar, ar_ref, "H4 after_res")
assert_exact(an, an_ref, "H4 after_norm")
assert_scales(s, s_ref, "H4 scales")
assert_codes(q, q_ref, "H4 codes")
print("children ok", flush=True)
"""


def test_exact_form_that_spills_takes_the_generic_form():
    import os
    import subprocess
    import sys

    from conftest import ROOT

    say("exact-row forms that spill: H1 fp32 4x16384, H4 fp16 (fp32 w, fp16 smooth) 4x20480")
    env = dict(os.environ, MCOP_DEBUG_TRACE="1")
    out = subprocess.run([sys.executable, "-c", _EX_SPILL_SCRIPT], cwd=str(ROOT), env=env,
                         capture_output=True, text=True, timeout=300)
    say(out.stdout[-3000:])
    assert out.returncode == 0, out.stderr[-3000:]
    assert "children ok" in out.stdout
    launches = [ln for ln in out.stdout.splitlines() if ln.startswith("[mcop] ")
                and " rows=4 " in ln and " nv=8 " in ln]
    assert len(launches) == 2, launches
    assert out.stdout.count("exact-row form spills registers: generic form") == 2
