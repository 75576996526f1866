"""Rows too wide for one workgroup's registers on the split-row kernels (H1 / H2 / H3 / H4 / H5,
the per-block quant, the norms, the quantizers and the padded op: each row shared by several
workgroups that exchange partial results through a device workspace): bit for bit against the
oracle and against the multi-pass kernels (forced with the library's test hook), over several
row counts and calls that take several launches, two streams at once, and a HIP graph capture
(which takes the multi-pass kernel)."""

import os
import re
import subprocess
import sys
import threading

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from conftest import ROOT
from mcoplib_amd import _lib, custom_ops, op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say

pytestmark = pytest.mark.gpu


def _x(T, H, seed, dtype, scale=1.0):
    x = torch.randn(T, H, generator=gen(seed)) * scale
    x[0, 7] = 40.0 * scale  # an outlier: the absmax row element
    if T > 2:
        x[2].zero_()
    return x.to(dtype)


def _w(H, seed, dtype):
    return (1 + 0.1 * torch.randn(H, generator=gen(seed))).to(dtype)


def _h2(x, w, r, qdt, ub):
    """One vLLM-surface call on the GPU; returns (codes, scales, residual or None) on the CPU."""
    q = torch.empty(x.shape, dtype=qdt, device=DEV)
    s = torch.empty(x.shape[0], 1, device=DEV)
    rd = None if r is None else r.to(DEV)
    ubd = None if ub is None else torch.tensor([ub], device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, ubd, rd)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu(), None if rd is None else rd.cpu()


def _same(a, b, what):
    if a is None:
        assert b is None
        return
    assert torch.equal(a.view(torch.uint8) if a.element_size() == 1 else a,
                       b.view(torch.uint8) if b.element_size() == 1 else b), what


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 65544), (torch.bfloat16, 131072),
                                     (torch.bfloat16, 262144), (torch.float16, 65608),
                                     (torch.float32, 32772), (torch.float32, 65536)])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_split_h2_against_oracle_and_multipass(dtype, H, qdt):
    say(f"split H2 {dtype} H={H} {qdt}")
    T = 5
    x, r, w = _x(T, H, 60, dtype), _x(T, H, 61, dtype), _w(H, 62, dtype)
    ubs = (None, 0.05) if qdt == torch.float8_e4m3fn else (None,)
    for res in (None, r):
        for ub in ubs:
            tag = f"res={res is not None} ub={ub}"
            q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, ub, res)
            got = _h2(x, w, res, qdt, ub)
            assert_scales(got[1], s_ref, tag + " scales")
            assert_codes(got[0], q_ref, tag + " codes")
            if res is not None:
                assert_exact(got[2], r_ref, tag + " residual")
            _lib.set_split_rows(False)
            try:
                mp = _h2(x, w, res, qdt, ub)
            finally:
                _lib.set_split_rows(True)
            for a, b, what in zip(got, mp, ("codes", "scales", "residual")):
                _same(a, b, f"{tag} {what}: split-row and multi-pass kernels differ")


def _h4(x, w, sm, r, qdt, standard):
    """One fused_rms_norm_dq call on the GPU; returns (codes, scales, after_res, after_norm)."""
    q = torch.empty(x.shape, dtype=qdt, device=DEV)
    s = torch.empty(x.shape[0], device=DEV)
    ar = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    an = torch.empty_like(ar)
    op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                        None if r is None else r.to(DEV),
                                        standard_norm=standard)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu(), ar.cpu(), an.cpu()


@pytest.mark.parametrize("dtype,wdt,sdt,H", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, 65544),
    (torch.bfloat16, torch.bfloat16, torch.float32, 131072),
    (torch.bfloat16, torch.float32, torch.float32, 262144),
    (torch.float16, torch.float16, torch.float16, 65608),
    (torch.float32, torch.float32, torch.float32, 32772),
])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_split_h4_against_oracle_and_multipass(dtype, wdt, sdt, H, qdt):
    say(f"split H4 {dtype} w={wdt} s={sdt} H={H} {qdt}")
    T = 4
    x, r = _x(T, H, 90, dtype, 3.0), _x(T, H, 91, dtype, 3.0)
    w = _w(H, 92, wdt)
    sm = (0.5 + 1.5 * torch.rand(H, generator=gen(93))).to(sdt)
    for res in (None, r):
        for standard in (False, True):
            tag = f"res={res is not None} std={standard}"
            q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, res,
                                                                        standard)
            got = _h4(x, w, sm, res, qdt, standard)
            assert_exact(got[2], ar_ref, tag + " after_res")
            assert_exact(got[3], an_ref, tag + " after_norm")
            assert_scales(got[1], s_ref, tag + " scales")
            assert_codes(got[0], q_ref, tag + " codes")
            _lib.set_split_rows(False)
            try:
                mp = _h4(x, w, sm, res, qdt, standard)
            finally:
                _lib.set_split_rows(True)
            for a, b, what in zip(got, mp, ("codes", "scales", "after_res", "after_norm")):
                _same(a, b, f"{tag} {what}: split-row and multi-pass kernels differ")


def test_split_h4_wide_fp8_workload_rows():
    """The bench's wide-fp8 workload, 2048 x 131072 bf16 SmoothQuant to fp8 (bf16 weight, fp32
    smooth): blocks of rows at the start, the middle and the end against the oracle."""
    T, H = 2048, 131072
    say(f"split: the wide-fp8 workload {T}x{H}")
    x = _x(T, H, 94, torch.bfloat16)
    w = _w(H, 95, torch.bfloat16)
    sm = (0.5 + 1.5 * torch.rand(H, generator=gen(96))).to(torch.float32)
    q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(T, device=DEV)
    ar = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    an = torch.empty_like(ar)
    op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                        None)
    torch.cuda.synchronize()
    for b0 in (0, 1000, 1984):
        sel = slice(b0, b0 + 64)
        q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x[sel], w, sm, 1e-6,
                                                                    torch.float8_e4m3fn)
        assert_exact(ar[sel], ar_ref, f"after_res rows {b0}+")
        assert_exact(an[sel], an_ref, f"after_norm rows {b0}+")
        assert_scales(s[sel], s_ref, f"scales rows {b0}+")
        assert_codes(q[sel], q_ref, f"codes rows {b0}+")


def _h5(h, sm):
    q, s = op.scale_dynamic_quant(h.to(DEV), sm.to(DEV), torch.int8)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu().reshape(-1)


@pytest.mark.parametrize("T,H", [(1, 65544), (5, 131072), (3, 262152), (130, 524288)])
def test_split_h5_against_oracle_and_multipass(T, H):
    say(f"split H5 {T}x{H}")
    h = _x(T, H, 97, torch.bfloat16, 3.0)
    sm = (0.5 + 1.5 * torch.rand(H, generator=gen(98))).to(torch.float32)
    q_ref, s_ref = oracle.scale_dynamic_quant(h, sm)
    got = _h5(h, sm)
    assert_scales(got[1], s_ref, "scales")
    assert_codes(got[0], q_ref, "codes")
    _lib.set_split_rows(False)
    try:
        mp = _h5(h, sm)
    finally:
        _lib.set_split_rows(True)
    for a, b, what in zip(got, mp, ("codes", "scales")):
        _same(a, b, f"{what}: split-row and multi-pass kernels differ")


def test_split_h5_wide_sdq_workload_rows():
    """The bench's wide-sdq workload, 2048 x 131072 bf16 with fp32 smooth scales: blocks of rows
    at the start, the middle and the end against the oracle."""
    T, H = 2048, 131072
    say(f"split: the wide-sdq workload {T}x{H}")
    h = _x(T, H, 99, torch.bfloat16)
    sm = (0.5 + 1.5 * torch.rand(H, generator=gen(100))).to(torch.float32)
    q, s = op.scale_dynamic_quant(h.to(DEV), sm.to(DEV), torch.int8)
    torch.cuda.synchronize()
    s = s.reshape(-1)
    for b0 in (0, 1000, 1984):
        sel = slice(b0, b0 + 64)
        q_ref, s_ref = oracle.scale_dynamic_quant(h[sel], sm)
        assert_scales(s[sel], s_ref, f"scales rows {b0}+")
        assert_codes(q[sel], q_ref, f"codes rows {b0}+")


def _h1(x, r, w, pad):
    """One vLLM fused_add_rms_norm call on the GPU (x a row-strided view when pad > 0); returns
    (x, residual) on the CPU, and checks that the padding columns are untouched."""
    T, H = x.shape
    big = torch.randn(T, H + pad, generator=gen(101)).to(x.dtype)
    big[:, :H] = x
    bigd = big.to(DEV)
    xd = bigd[:, :H]
    rd = r.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(bigd[:, H:].cpu(), big[:, H:]), "padding columns changed"
    return xd.contiguous().cpu(), rd.cpu()


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 65544), (torch.bfloat16, 131072),
                                     (torch.bfloat16, 524288), (torch.float16, 65608),
                                     (torch.float32, 32772), (torch.float32, 65536)])
@pytest.mark.parametrize("pad", [0, 24])
def test_split_h1_against_oracle_and_multipass(dtype, H, pad):
    say(f"split H1 {dtype} H={H} pad={pad}")
    T = 4
    x, r, w = _x(T, H, 102, dtype), _x(T, H, 103, dtype), _w(H, 104, dtype)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    got = _h1(x, r, w, pad)
    assert_exact(got[1], r_ref, "residual")
    assert_exact(got[0], x_ref, "output")
    _lib.set_split_rows(False)
    try:
        mp = _h1(x, r, w, pad)
    finally:
        _lib.set_split_rows(True)
    for a, b, what in zip(got, mp, ("output", "residual")):
        _same(a, b, f"{what}: split-row and multi-pass kernels differ")


def test_split_h1_wide_fused_workload_rows():
    """The bench's wide-fused workload, 2048 x 131072 bf16: blocks of rows at the start, the
    middle and the end against the oracle."""
    T, H = 2048, 131072
    say(f"split: the wide-fused workload {T}x{H}")
    x, r, w = _x(T, H, 105, torch.bfloat16), _x(T, H, 106, torch.bfloat16), _w(H, 107,
                                                                                torch.bfloat16)
    xd, rd = x.to(DEV), r.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    for b0 in (0, 1000, 1984):
        sel = slice(b0, b0 + 64)
        x_ref, r_ref = oracle.fused_add_rms_norm(x[sel], r[sel], w, 1e-6)
        assert_exact(rd[sel], r_ref, f"residual rows {b0}+")
        assert_exact(xd[sel], x_ref, f"output rows {b0}+")


def _per_block(x, w, r, qdt, G, ub, transposed):
    """One vLLM rms_norm_per_block_quant call on the GPU; returns (codes, scales, residual)."""
    T, H = x.shape
    q = torch.empty(T, H, dtype=qdt, device=DEV)
    s = torch.empty((H // G, T) if transposed else (T, H // G), device=DEV)
    rd = None if r is None else r.to(DEV)
    ubd = None if ub is None else torch.tensor([ub], device=DEV)
    torch.ops._C.rms_norm_per_block_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, ubd, rd, G,
                                          transposed)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu(), None if rd is None else rd.cpu()


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 65664), (torch.bfloat16, 131072),
                                     (torch.float16, 65792), (torch.float32, 32896),
                                     (torch.float32, 65536)])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_split_per_block_against_oracle_and_multipass(dtype, H, qdt):
    """Slices hold whole groups (64 or 128 elements): every scale and code against the oracle,
    and the split and multi-pass kernels bit for bit, row-major and transposed scales."""
    say(f"split per-block {dtype} H={H} {qdt}")
    T = 3
    x, r = _x(T, H, 108, dtype, 0.01), _x(T, H, 109, dtype)
    w = _w(H, 110, dtype)
    for G in (64, 128):
        for res, transposed, ub in ((None, False, None), (r, True, None), (r, False, 0.02)):
            if ub is not None and qdt == torch.int8:
                continue
            tag = f"G={G} res={res is not None} tr={transposed} ub={ub}"
            q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, ub, res,
                                                                  transposed)
            got = _per_block(x, w, res, qdt, G, ub, transposed)
            assert_scales(got[1], s_ref, tag + " scales")
            assert_codes(got[0], q_ref, tag + " codes")
            if res is not None:
                assert_exact(got[2], r_ref, tag + " residual")
            _lib.set_split_rows(False)
            try:
                mp = _per_block(x, w, res, qdt, G, ub, transposed)
            finally:
                _lib.set_split_rows(True)
            for a, b, what in zip(got, mp, ("codes", "scales", "residual")):
                _same(a, b, f"{tag} {what}: split-row and multi-pass kernels differ")


def test_split_per_block_wide_block_workload_rows():
    """The bench's wide-block workload, 2048 x 131072 bf16 to fp8 with G = 128 and a residual:
    blocks of rows at the start, the middle and the end against the oracle."""
    T, H, G = 2048, 131072, 128
    say(f"split: the wide-block workload {T}x{H}")
    x, r, w = _x(T, H, 111, torch.bfloat16), _x(T, H, 112, torch.bfloat16), _w(H, 113,
                                                                                torch.bfloat16)
    q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(T, H // G, device=DEV)
    rd = r.to(DEV)
    torch.ops._C.rms_norm_per_block_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, None, rd, G, False)
    torch.cuda.synchronize()
    for b0 in (0, 1000, 1984):
        sel = slice(b0, b0 + 64)
        q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x[sel], w, 1e-6,
                                                              torch.float8_e4m3fn, G, None,
                                                              r[sel])
        assert_exact(rd[sel], r_ref, f"residual rows {b0}+")
        assert_scales(s[sel], s_ref, f"scales rows {b0}+")
        assert_codes(q[sel], q_ref, f"codes rows {b0}+")


def _mc_norm(x, w, r, rms_div):
    out = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    ares = None if r is None else torch.empty(x.shape, dtype=x.dtype, device=DEV)
    op.rms_norm(out, x.to(DEV), w.to(DEV), 1e-6, ares, None if r is None else r.to(DEV),
                rms_div)
    torch.cuda.synchronize()
    return out.cpu(), None if ares is None else ares.cpu()


@pytest.mark.parametrize("dtype,wdtype,H", [(torch.bfloat16, torch.bfloat16, 65544),
                                            (torch.bfloat16, torch.float32, 131072),
                                            (torch.float16, torch.float16, 65608),
                                            (torch.float32, torch.float32, 32772)])
def test_split_norms_against_oracle_and_multipass(dtype, wdtype, H):
    """mcoplib rms_norm (its element-wise chain at these widths, both rms_div forms, with and
    without a residual), vLLM rms_norm on a strided 3-D view and head_rms_norm: against the
    oracle and, bit for bit, against the multi-pass kernel."""
    say(f"split norms {dtype} w={wdtype} H={H}")
    x, r, w = _x(3, H, 114, dtype), _x(3, H, 115, dtype), _w(H, 116, wdtype)
    for res in (None, r):
        for rms_div in (True, False):
            tag = f"res={res is not None} rms_div={rms_div}"
            out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=res, rms_div=rms_div)
            got = _mc_norm(x, w, res, rms_div)
            assert_exact(got[0], out_ref, tag + " out")
            if res is not None:
                assert_exact(got[1], ares_ref, tag + " after_res")
            _lib.set_split_rows(False)
            try:
                mp = _mc_norm(x, w, res, rms_div)
            finally:
                _lib.set_split_rows(True)
            for a, b, what in zip(got, mp, ("out", "after_res")):
                _same(a, b, f"{tag} {what}: split-row and multi-pass kernels differ")
    if dtype != torch.float16 and wdtype == dtype:
        big = torch.randn(2, 3, H + 16, generator=gen(117)).to(dtype)
        ref = oracle.vllm_rms_norm(big[:, :, :H].contiguous().view(6, H), w, 1e-6)
        o = torch.empty(2, 3, H, dtype=dtype, device=DEV)
        torch.ops._C.rms_norm(o, big.to(DEV)[:, :, :H], w.to(DEV), 1e-6)
        torch.cuda.synchronize()
        assert_exact(o.view(6, H), ref, "vLLM rms_norm 3-D strided")
    if dtype == torch.bfloat16 and wdtype == dtype:
        T, NH = 2, 3
        hs = torch.randn(T, NH, H, generator=gen(118)).to(dtype)
        hw = _w(NH * H, 119, dtype).view(NH, H)
        base = torch.zeros_like(hs)
        ref = oracle.head_rms_norm(base, hs, hw, 1e-6, 1, 2)
        out = base.to(DEV)
        op.head_rms_norm(out, hs.to(DEV), hw.to(DEV), 1e-6, 1, 2)
        torch.cuda.synchronize()
        assert_exact(out, ref, "head_rms_norm")


def test_split_norm_strided_rows_over_several_launches():
    """vLLM rms_norm over a strided 3-D view with more rows than one launch's workspace holds
    (8400 rows of 131072 bf16: 4095 rows a launch at 16 slices, 8191 at 8): rows on both sides
    of every launch boundary against the oracle, generated on the GPU."""
    A, B, H = 2, 4200, 131072
    say(f"split: vLLM rms_norm [{A}, {B}, {H}] strided (several launches)")
    g = torch.Generator(device=DEV).manual_seed(120)
    big = torch.randn(A, B, H + 16, device=DEV, generator=g).to(torch.bfloat16)
    w = _w(H, 121, torch.bfloat16)
    o = torch.empty(A, B, H, dtype=torch.bfloat16, device=DEV)
    torch.ops._C.rms_norm(o, big[:, :, :H], w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    xs = big[:, :, :H].reshape(A * B, H)
    os_ = o.view(A * B, H)
    for r0 in (0, 4090, 8186, A * B - 6):
        sel = slice(r0, r0 + 6)
        ref = oracle.vllm_rms_norm(xs[sel].cpu(), w, 1e-6)
        assert_exact(os_[sel], ref, f"rows {r0}+")
    del big, o


def _ptq_int8(x, use_azp):
    T = x.shape[0]
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty((T, 1), device=DEV)
    zp = torch.empty((T, 1), dtype=torch.int32, device=DEV) if use_azp else None
    torch.ops._C.dynamic_scaled_int8_quant(q, x.to(DEV), s, zp)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu(), None if zp is None else zp.cpu()


def _ptq_fp8(xd, ub):
    T = xd.shape[0]
    q = torch.empty(xd.shape, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty((T, 1), device=DEV)
    ubd = None if ub is None else torch.tensor([ub], device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, xd, s, ubd)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu()


def _mp(fn, *args):
    _lib.set_split_rows(False)
    try:
        return fn(*args)
    finally:
        _lib.set_split_rows(True)


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 65544), (torch.bfloat16, 262144),
                                     (torch.float16, 65608), (torch.float32, 32772),
                                     (torch.float32, 131072)])
def test_split_quantizers_against_oracle_and_multipass(dtype, H):
    """int8 symmetric, int8 with zero points (the max and the min in one exchange) and fp8 (with
    and without scale_ub, rows strided on the input side): against the oracle and, bit for bit,
    against the multi-pass kernels."""
    say(f"split quantizers {dtype} H={H}")
    T = 4
    x = _x(T, H, 122, dtype, 2.0)
    x[1] += 3.0  # an all-positive-leaning row: the zero point moves
    for use_azp in (False, True):
        tag = f"int8 azp={use_azp}"
        q_ref, s_ref, zp_ref = oracle.dynamic_scaled_int8_quant(x, use_azp=use_azp)
        got = _ptq_int8(x, use_azp)
        assert_scales(got[1], s_ref, tag + " scales")
        assert_codes(got[0], q_ref, tag + " codes")
        if use_azp:
            assert_exact(got[2], zp_ref, tag + " azp")
        for a, b, what in zip(got, _mp(_ptq_int8, x, use_azp), ("codes", "scales", "azp")):
            _same(a, b, f"{tag} {what}: split-row and multi-pass kernels differ")
    big = torch.randn(T, H + 64, generator=gen(123)).to(dtype)
    xs = big.to(DEV)[:, :H]  # rows strided on the input side
    for ub in (None, 0.05):
        tag = f"fp8 ub={ub}"
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(big[:, :H].contiguous(),
                                                                 scale_ub=ub)
        got = _ptq_fp8(xs, ub)
        assert_scales(got[1], s_ref, tag + " scales")
        assert_codes(got[0], q_ref, tag + " codes")
        for a, b, what in zip(got, _mp(_ptq_fp8, xs, ub), ("codes", "scales")):
            _same(a, b, f"{tag} {what}: split-row and multi-pass kernels differ")


def test_split_quantizer_wide_ptq_workload_rows():
    """The bench's wide-ptq workload, 2048 x 131072 bf16 to int8: blocks of rows at the start,
    the middle and the end against the oracle."""
    T, H = 2048, 131072
    say(f"split: the wide-ptq workload {T}x{H}")
    x = _x(T, H, 124, torch.bfloat16)
    q = torch.empty(T, H, dtype=torch.int8, device=DEV)
    s = torch.empty((T, 1), device=DEV)
    torch.ops._C.dynamic_scaled_int8_quant(q, x.to(DEV), s, None)
    torch.cuda.synchronize()
    for b0 in (0, 1000, 1984):
        sel = slice(b0, b0 + 64)
        q_ref, s_ref, _ = oracle.dynamic_scaled_int8_quant(x[sel])
        assert_scales(s[sel], s_ref, f"scales rows {b0}+")
        assert_codes(q[sel], q_ref, f"codes rows {b0}+")


def _padded(x, r, w, pad):
    T, H = x.shape
    p = torch.zeros(T, 2 * pad, dtype=torch.int8, device=DEV)
    rms = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(T, 1, device=DEV)
    rd = r.to(DEV)
    op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(p, rms, q, s, x.to(DEV), rd,
                                                                  w.to(DEV), pad, 1e-6)
    torch.cuda.synchronize()
    return p.cpu(), rd.cpu(), rms.cpu(), q.cpu(), s.cpu()


@pytest.mark.parametrize("H,extra", [(65544, 0), (131072, 64), (163848, 8)])
def test_split_padded_against_oracle_and_multipass(H, extra):
    """The padded wire-format op (its generic chain): every padded row byte, the residual,
    output_rms, codes and scales against the oracle and, bit for bit, against the multi-pass
    kernel; the spare bytes (at least `extra`) after each row's scale stay untouched."""
    say(f"split padded H={H} extra={extra}")
    T = 3
    # whole 8-byte units a padded row (the vector path, hence the split-row kernel, needs them)
    pad = (H + 4 + extra + 7) // 8 * 4
    x, r, w = _x(T, H, 125, torch.bfloat16), _x(T, H, 126, torch.bfloat16), _w(H, 127,
                                                                                 torch.bfloat16)
    refs = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6)
    got = _padded(x, r, w, pad)
    assert torch.equal(got[0].view(torch.uint8), refs[0]), "padded rows"
    assert_exact(got[1], refs[1], "residual")
    assert_exact(got[2], refs[2], "output_rms")
    assert_codes(got[3], refs[3], "codes")
    assert_scales(got[4], refs[4], "scales")
    for a, b, what in zip(got, _mp(_padded, x, r, w, pad),
                          ("padded", "residual", "output_rms", "codes", "scales")):
        _same(a, b, f"{what}: split-row and multi-pass kernels differ")


def test_split_padded_wide_padded_workload_rows():
    """The bench's wide-padded workload, 2048 x 131072: blocks of rows at the start, the middle
    and the end against the oracle, padded bytes included."""
    T, H = 2048, 131072
    pad = (H + 4 + 63) // 64 * 32  # the bench's padded rows
    say(f"split: the wide-padded workload {T}x{H}")
    x, r, w = _x(T, H, 128, torch.bfloat16), _x(T, H, 129, torch.bfloat16), _w(H, 130,
                                                                                 torch.bfloat16)
    p, rd, rms, q, s = _padded(x, r, w, pad)
    for b0 in (0, 1000, 1984):
        sel = slice(b0, b0 + 64)
        refs = oracle.add_rms_norm_quant_padded(x[sel], r[sel], w, pad, 1e-6)
        assert torch.equal(p[sel].view(torch.uint8), refs[0]), f"padded rows {b0}+"
        assert_exact(rd[sel], refs[1], f"residual rows {b0}+")
        assert_exact(rms[sel], refs[2], f"output_rms rows {b0}+")
        assert_codes(q[sel], refs[3], f"codes rows {b0}+")
        assert_scales(s[sel], refs[4], f"scales rows {b0}+")


@pytest.mark.parametrize("T", [1, 3, 250])
def test_split_h3_row_counts(T):
    """mcoplib's operator (1.5e-6 floor, +-127 codes) over a few row counts."""
    H = 131072
    say(f"split H3 T={T} H={H}")
    x, r, w = _x(T, H, 63, torch.bfloat16), _x(T, H, 64, torch.bfloat16), _w(H, 65,
                                                                               torch.bfloat16)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    rd = r.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x.to(DEV), w.to(DEV), 1e-6, torch.int8,
                                                       residual=rd)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")
    assert_exact(rd, r_ref, "residual")


def test_split_launches_in_chunks():
    """More rows than one launch's workspace holds (524288-wide bf16 rows with a residual: 1023
    rows a launch at 64 slices of 1024 vectors, 2047 at 32 slices of 2048): several launches,
    each later one on the rows, residual and codes after the one before.  Inputs are generated on
    the GPU; rows on both sides of every launch boundary are checked against the oracle."""
    T, H = 2050, 524288
    say(f"split: {T}x{H} bf16 with a residual (several launches)")
    g = torch.Generator(device=DEV).manual_seed(84)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    r = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    w = _w(H, 85, torch.bfloat16)
    sel = [slice(0, 3), slice(1020, 1027), slice(2044, 2050)]
    x_rows = [x[s].cpu() for s in sel]
    r_rows = [r[s].cpu() for s in sel]
    q = torch.empty(T, H, dtype=torch.int8, device=DEV)
    s_all = torch.empty(T, 1, device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w.to(DEV), s_all, 1e-6, None, r)
    torch.cuda.synchronize()
    for s, xs, rs in zip(sel, x_rows, r_rows):
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(xs, w, 1e-6, torch.int8,
                                                                      None, rs)
        assert_exact(r[s], r_ref, f"residual rows {s.start}+")
        assert_scales(s_all[s], s_ref, f"scales rows {s.start}+")
        assert_codes(q[s], q_ref, f"codes rows {s.start}+")
    del x, r, q


def test_split_wide_int8_workload_all_rows():
    """The bench's wide-int8 workload, 2048 x 131072 bf16 with a residual, through the headline
    surface: every row against the oracle (in blocks of 256 rows)."""
    T, H = 2048, 131072
    say(f"split: the wide-int8 workload {T}x{H}, all rows")
    x, r, w = _x(T, H, 66, torch.bfloat16), _x(T, H, 67, torch.bfloat16), _w(H, 68,
                                                                               torch.bfloat16)
    rd = r.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x.to(DEV), w.to(DEV), 1e-6, torch.int8,
                                                       residual=rd)
    torch.cuda.synchronize()
    B = 256
    for b0 in range(0, T, B):
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(
            x[b0:b0 + B], w, 1e-6, residual=r[b0:b0 + B])
        assert_exact(rd[b0:b0 + B], r_ref, f"residual rows {b0}+")
        assert_scales(s[b0:b0 + B], s_ref, f"scales rows {b0}+")
        assert_codes(q[b0:b0 + B], q_ref, f"codes rows {b0}+")


def test_split_two_streams():
    """Two host threads, each on its own stream, run wide rows (split-row launches) at the same
    time, 20 calls each; every call matches the single-stream result."""
    say("split: two threads, two streams, 20 wide calls each")
    H = 131072
    cases = []
    for i, T in enumerate((40, 96)):
        x, r, w = (_x(T, H, 70 + 3 * i, torch.bfloat16).to(DEV),
                   _x(T, H, 71 + 3 * i, torch.bfloat16).to(DEV),
                   _w(H, 72 + 3 * i, torch.bfloat16).to(DEV))
        cases.append((x, r, w))

    def run(x, r, w):
        q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
        s = torch.empty(x.shape[0], 1, device=DEV)
        rr = r.clone()
        torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w, s, 1e-6, None, rr)
        return q, s, rr
    expected = [run(*c) for c in cases]
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for _ in range(20):
                    got = run(*cases[i])
                    stream.synchronize()
                    if not all(torch.equal(a, b) for a, b in zip(got, expected[i])):
                        errors.append(f"thread {i}: result differs")
                        return
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors


def test_split_graph_capture_takes_the_multipass_kernel():
    """A wide-row call captured into a HIP graph runs the multi-pass kernel (no cooperative
    launch, no workspace in the graph); replays match the eager split-row result."""
    say("split: graph capture of a wide-row call")
    T, H = 6, 131072
    x, r, w = (_x(T, H, 80, torch.bfloat16).to(DEV), _x(T, H, 81, torch.bfloat16).to(DEV),
               _w(H, 82, torch.bfloat16).to(DEV))
    q0 = torch.empty(T, H, dtype=torch.int8, device=DEV)
    s0 = torch.empty(T, 1, device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q0, x, w, s0, 1e-6, None, None)
    q = torch.empty(T, H, dtype=torch.int8, device=DEV)
    s = torch.empty(T, 1, device=DEV)
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w, s, 1e-6, None, None)
    torch.cuda.current_stream().wait_stream(cap)
    for i in range(3):
        q.zero_()
        s.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(q, q0) and torch.equal(s, s0), f"replay {i}"


_TRACE_SCRIPT = r"""
import sys, torch
sys.path.insert(0, "tests")
import mcoplib_amd._C
from mcoplib_amd import _lib
from gpu_util import DEV
x = torch.randn(4, 131072, device=DEV).to(torch.bfloat16)
w = torch.ones(131072, device=DEV, dtype=torch.bfloat16)
q = torch.empty(4, 131072, dtype=torch.int8, device=DEV)
s = torch.empty(4, 1, device=DEV)
torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w, s, 1e-6, None, None)
_lib.set_split_rows(False)
torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w, s, 1e-6, None, None)
torch.cuda.synchronize()
print("child ok", flush=True)
"""


def test_split_launch_decisions_are_traced():
    say("split: MCOP_DEBUG_TRACE names the split-row and the multi-pass launches")
    env = dict(os.environ, MCOP_DEBUG_TRACE="1")
    out = subprocess.run([sys.executable, "-c", _TRACE_SCRIPT], cwd=str(ROOT), env=env,
                         capture_output=True, text=True, timeout=300)
    say(out.stdout[-2000:])
    assert out.returncode == 0, out.stderr[-3000:]
    assert "child ok" in out.stdout
    assert re.search(r"rows=4: split-row kernel, (8 slices of 2048|16 slices of 1024) vectors "
                     r"over 256 lanes", out.stdout)
    assert "rows=4: multi-pass kernel" in out.stdout
