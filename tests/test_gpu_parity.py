"""GPU parity: the HIP kernels (through the drop-in surfaces and the C ABI) against the CPU oracle
on the same seeded inputs, at the benchmark configurations (cfg1-cfg5, on the exact inputs
bench.py times: bench.config_inputs) and at the shapes the reference's own test enumerates
(unit_test/test_fused_rms_norm_dq.py:13-24)."""

import pytest
import torch

import bench
import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib, custom_ops, op
from gpu_util import (DEV, assert_codes, assert_exact, assert_scales, gen, randn, say, weight)

pytestmark = pytest.mark.gpu

# (num_tokens, hidden_size) of the reference test, plus the shapes around the launch geometry
REF_SHAPES = [
    *[(1, h) for h in [1, 64, 1024, 1025, 1026, 1027, 1028, 1029, 5120, 5137]],
    *[(83, h) for h in [1, 1033, 2048, 5120]],
    *[(2048, h) for h in [1, 64, 1024, 1029, 5137]],
    *[(4096, h) for h in [1, 64]],
    (7, 8192), (5, 16384), (3, 32768), (33, 7168), (9, 4096), (17, 200),
]


def _h2_case(T, H, dtype, qdt, with_res, seed, eps=1e-6, scale_ub=None, x_scale=1.0):
    x = randn((T, H), seed, dtype, scale=x_scale)
    w = weight(H, seed + 1, dtype)
    r = randn((T, H), seed + 2, dtype, scale=x_scale) if with_res else None
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, eps, qdt, scale_ub, r)
    xd, wd = x.to(DEV), w.to(DEV)
    rd = r.to(DEV) if with_res else None
    q = torch.empty((T, H), dtype=qdt, device=DEV)
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    ub = None if scale_ub is None else torch.tensor([scale_ub], dtype=torch.float32, device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, xd, wd, s, eps, ub, rd)
    torch.cuda.synchronize()
    tag = f"T={T} H={H} {dtype} {qdt} res={with_res}"
    assert_scales(s, s_ref, tag + " scales")
    assert_codes(q, q_ref, tag + " codes")
    if with_res:
        assert_exact(rd, r_ref, tag + " residual")


@pytest.mark.parametrize("T,H", REF_SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h2_reference_shapes(T, H, dtype):
    say(f"h2 shapes T={T} H={H} {dtype}")
    seed = T * 7919 + H
    for qdt in (torch.int8, torch.float8_e4m3fn):
        for with_res in (False, True):
            _h2_case(T, H, dtype, qdt, with_res, seed, x_scale=1.0 / max(H, 1) ** 0.5)


def test_h2_scale_ub_fp8():
    say("h2 scale_ub")
    _h2_case(256, 2048, torch.bfloat16, torch.float8_e4m3fn, True, 11, scale_ub=0.05)


def test_config1_norm_int8_no_residual():
    say("config 1: 256x4096 bf16, no residual, int8 (the bench's inputs)")
    c = bench.config_inputs("cfg1")
    x, w = c["x"], c["w"]
    q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, c["eps"], torch.int8)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(x.shape[0], 1, device=DEV)
    torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, c["eps"], None,
                                                  None)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "cfg1 scales")
    assert_codes(q, q_ref, "cfg1 codes")


def test_config3_add_norm_int8_outliers():
    """Config 3 (the headline workload) on the bench's exact inputs: x, residual [8192, 8192]
    bf16, 1% outlier channels x20, eps 1e-5."""
    T = H = 8192
    say("config 3: 8192x8192 add + rmsnorm + int8, outliers (the bench's inputs)")
    c = bench.config_inputs("cfg3")
    x, r, w = c["x"], c["r"], c["w"]
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-5,
                                                                        residual=r)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(xd, wd, 1e-5, torch.int8, residual=rd)
    torch.cuda.synchronize()
    assert s.shape == (T, 1) and q.dtype == torch.int8
    assert_exact(rd, r_ref, "cfg3 residual")
    assert_scales(s, s_ref, "cfg3 scales")
    assert_codes(q, q_ref, "cfg3 codes")


def test_config2_fused_add_rms_norm():
    """Config 2: in-place fused_add_rms_norm, [4096, 4096] bf16, eps 1e-6 (the bench's inputs)."""
    say("config 2: fused_add_rms_norm 4096x4096 (the bench's inputs)")
    c = bench.config_inputs("cfg2")
    x, r, w = c["x"], c["r"], c["w"]
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, wd, 1e-6)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "cfg2 residual")
    assert_exact(xd, x_ref, "cfg2 output")


@pytest.mark.parametrize("T,H", [(1, 1), (1, 64), (83, 1033), (2048, 1029), (64, 5137),
                                 (300, 4096), (5, 16384), (2, 32768), (37, 200)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h1_shapes(T, H, dtype):
    say(f"h1 T={T} H={H} {dtype}")
    x = randn((T, H), T + H, dtype)
    r = randn((T, H), T + H + 1, dtype)
    w = weight(H, T + H + 2, dtype)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, wd, 1e-6)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_exact(xd, x_ref, "output")


@pytest.mark.parametrize("T,H", [(128, 2048), (64, 4096)])
@pytest.mark.parametrize("pad", [64, 3])
def test_h1_row_strided_input(pad, T, H):
    """vLLM passes `input` as a row-strided view (input.stride(-2) != hidden_size); 64 x 4096
    takes the kernel's exact-row form (one row per workgroup, every lane in the row)."""
    say(f"h1 strided pad={pad} T={T} H={H}")
    big = randn((T, H + pad), 40, torch.bfloat16)
    x = big[:, :H]
    r = randn((T, H), 41, torch.bfloat16)
    w = weight(H, 42, torch.bfloat16)
    x_ref, r_ref = oracle.fused_add_rms_norm(x.contiguous(), r, w, 1e-6)
    bigd = big.to(DEV)
    xd = bigd[:, :H]
    rd, wd = r.to(DEV), w.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, wd, 1e-6)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_exact(xd.contiguous(), x_ref, "output")
    assert_exact(bigd[:, H:], big[:, H:], "padding untouched")


def _h4_case(T, H, dtype, wdt, sdt, qdt, with_res, standard, seed, eps=1e-6, x_scale=1.0):
    x = randn((T, H), seed, dtype, scale=x_scale)
    w = weight(H, seed + 1, wdt)
    sm = (0.5 + 1.5 * torch.rand(H, generator=gen(seed + 2))).to(sdt)
    r = randn((T, H), seed + 3, dtype, scale=x_scale) if with_res else None
    q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, eps, qdt, r, standard)
    xd, wd, smd = x.to(DEV), w.to(DEV), sm.to(DEV)
    rd = r.to(DEV) if with_res else None
    q = torch.empty((T, H), dtype=qdt, device=DEV)
    s = torch.empty((T,), dtype=torch.float32, device=DEV)
    ar = torch.empty_like(xd)
    an = torch.empty_like(xd)
    op.rms_norm_dynamic_per_token_quant(q, xd, wd, smd, s, eps, ar, an, rd, standard_norm=standard)
    torch.cuda.synchronize()
    tag = f"T={T} H={H} {dtype} w={wdt} s={sdt} {qdt} res={with_res} std={standard}"
    assert_exact(ar, ar_ref, tag + " after_res")
    assert_exact(an, an_ref, tag + " after_norm")
    assert_scales(s, s_ref, tag + " scales")
    assert_codes(q, q_ref, tag + " codes")
    if with_res:
        assert_exact(rd, r, tag + " residual unchanged")


@pytest.mark.parametrize("T,H", [(1, 64), (83, 1033), (256, 4096), (64, 5137), (33, 7168),
                                 (4, 16384)])
@pytest.mark.parametrize("dtype,wdt,sdt", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (torch.bfloat16, torch.float32, torch.float32),
    (torch.bfloat16, torch.bfloat16, torch.float32),
    (torch.float16, torch.float16, torch.float16),
    (torch.float32, torch.float32, torch.float32),
])
def test_h4_shapes(T, H, dtype, wdt, sdt):
    say(f"h4 T={T} H={H} {dtype} {wdt} {sdt}")
    seed = 3 * T + H
    for qdt in (torch.int8, torch.float8_e4m3fn):
        for with_res in (False, True):
            for standard in (False, True):
                _h4_case(T, H, dtype, wdt, sdt, qdt, with_res, standard, seed, x_scale=3.0)


def test_config4_smooth_quant_fp8():
    """Config 4 on the bench's inputs: fused_rms_norm_dq to fp8-e4m3fn with SmoothQuant,
    [16384, 7168] bf16, bf16 weight, fp32 smooth ~U(0.5, 2)."""
    say("config 4: 16384x7168 smooth quant fp8 (the bench's inputs)")
    c = bench.config_inputs("cfg4")
    x, w, sm = c["x"], c["w"], c["sm"]
    q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, c["eps"],
                                                                torch.float8_e4m3fn)
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty(x.shape[0], device=DEV)
    ar = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    an = torch.empty_like(ar)
    op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, c["eps"], ar, an,
                                        None)
    torch.cuda.synchronize()
    assert_exact(ar, ar_ref, "cfg4 after_res")
    assert_exact(an, an_ref, "cfg4 after_norm")
    assert_scales(s, s_ref, "cfg4 scales")
    assert_codes(q, q_ref, "cfg4 codes")


@pytest.mark.parametrize("dtype,wdt,sdt,qdt,with_res,standard", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.int8, True, False),
    (torch.float16, torch.float32, torch.float32, torch.float8_e4m3fn, False, True),
    (torch.float32, torch.float32, torch.float32, torch.int8, True, True),
])
def test_h4_many_rows_row_loop(dtype, wdt, sdt, qdt, with_res, standard):
    """Many rows (8192 x 4096: more workgroups than stay resident) with mixed dtypes."""
    say(f"h4 many rows 8192x4096 {dtype} {qdt} res={with_res} std={standard}")
    _h4_case(8192, 4096, dtype, wdt, sdt, qdt, with_res, standard, 21, x_scale=2.0)


@pytest.mark.parametrize("T,H,ov", [(2049, 7168, (0, 0)), (2051, 7168, (1, 0)),
                                    (2053, 4096, (4, 0)), (3001, 128, (0, 0)),
                                    (2050, 200, (0, 0)), (4097, 1024, (0, 0)),
                                    (2048, 16384, (0, 0))])
def test_h4_large_row_counts(T, H, ov):
    """Odd row counts past 2048, several rows per workgroup (short rows), forced one / four
    vectors per lane and a 16384-wide row, against the oracle bit for bit."""
    say(f"h4 large row counts T={T} H={H} override={ov}")
    try:
        _lib.set_launch_override(*ov)
        _h4_case(T, H, torch.bfloat16, torch.bfloat16, torch.float32, torch.float8_e4m3fn,
                 False, False, T + H, x_scale=2.0)
        _h4_case(T, H, torch.bfloat16, torch.float32, torch.bfloat16, torch.int8, True, True,
                 T + H + 1, x_scale=3.0)
    finally:
        _lib.set_launch_override(0, 0)


@pytest.mark.parametrize("T", [1, 4, 16, 64])
def test_config5_decode(T):
    say(f"config 5 decode T={T} (the bench's inputs)")
    c = bench.config_inputs(f"cfg5-decode{T}")
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(c["x"], c["w"], c["eps"],
                                                                        residual=c["r"])
    rd = c["r"].to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(c["x"].to(DEV), c["w"].to(DEV), c["eps"],
                                                       torch.int8, residual=rd)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "cfg5 decode residual")
    assert_scales(s, s_ref, "cfg5 decode scales")
    assert_codes(q, q_ref, "cfg5 decode codes")
    _h2_case(T, 5120, torch.bfloat16, torch.int8, True, 500 + T)


def test_config5_large_all_rows():
    """Config 5 (bandwidth leg): [32768, 16384] bf16 add + norm + int8 on the bench's inputs, one
    call over the whole tensor; every row's residual, scale and codes against the oracle (in
    blocks of 4096 rows), plus whole-tensor properties: every scale finite and > 0, every code
    within [-127, 127]."""
    T, H = 32768, 16384
    say("config 5 large: 32768x16384 (the bench's inputs), all rows")
    c = bench.config_inputs("cfg5-large")
    xd, rd, wd = c["x"].to(DEV), c["r"].to(DEV), c["w"].to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(xd, wd, 1e-6, torch.int8, residual=rd)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(s).all()) and bool((s > 0).all()), "scales finite and > 0"
    assert int(q.min()) >= -127 and int(q.max()) <= 127, "codes within [-127, 127]"
    del xd
    B = 4096
    for b0 in range(0, T, B):
        say(f"  rows {b0}-{b0 + B - 1}")
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(
            c["x"][b0:b0 + B], c["w"], 1e-6, residual=c["r"][b0:b0 + B])
        assert_exact(rd[b0:b0 + B], r_ref, f"cfg5 residual rows {b0}+")
        assert_scales(s[b0:b0 + B], s_ref, f"cfg5 scales rows {b0}+")
        assert_codes(q[b0:b0 + B], q_ref, f"cfg5 codes rows {b0}+")
    del rd, q, c


def test_h5_parity_shapes():
    for (shape, seed) in [((2, 128, 768), 13), ((1, 2048, 4096), 14), ((4, 512, 768), 15),
                          ((8, 128, 1024), 16), ((3, 5, 1027), 17), ((64, 7168), 18)]:
        say(f"h5 {shape}")
        h = randn(shape, seed, torch.bfloat16)
        sm = 0.5 + 1.5 * torch.rand(shape[-1], generator=gen(seed + 1))
        q_ref, s_ref = oracle.scale_dynamic_quant(h, sm)
        q, s = op.scale_dynamic_quant(h.to(DEV), sm.to(DEV), torch.int8)
        torch.cuda.synchronize()
        assert q.shape == h.shape and s.shape == (h.numel() // shape[-1],)
        assert_scales(s, s_ref, "h5 scales")
        assert_codes(q, q_ref, "h5 codes")


@pytest.mark.parametrize("T,H,ov", [(2049, 7168, (0, 0)), (2048, 7168, (2, 0)),
                                    (2051, 4096, (1, 0)), (4099, 1024, (0, 0)),
                                    (3001, 128, (0, 0)), (2050, 200, (0, 0)),
                                    (2053, 8192, (4, 0))])
def test_h5_two_rows_per_lane(T, H, ov):
    """From 2048 rows on, each lane quantizes two rows with one load of the smooth scales:
    odd row counts (a workgroup's second row past the end), several rows per workgroup (short
    rows) and forced vectors per lane, against the oracle bit for bit."""
    say(f"h5 two rows per lane T={T} H={H} override={ov}")
    h = randn((T, H), T + H, torch.bfloat16)
    h[T // 2].zero_()
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(T))
    q_ref, s_ref = oracle.scale_dynamic_quant(h, sm)
    try:
        _lib.set_launch_override(*ov)
        q, s = op.scale_dynamic_quant(h.to(DEV), sm.to(DEV), torch.int8)
        torch.cuda.synchronize()
    finally:
        _lib.set_launch_override(0, 0)
    assert_scales(s, s_ref, "h5 scales")
    assert_codes(q, q_ref, "h5 codes")


@pytest.mark.parametrize("T", [512, 517])
def test_launch_shape_does_not_change_bits(T):
    """The row sum is accumulated in fp64 and rounded once: every split of a row over lanes
    gives the same bits (all four row kernels)."""
    H = 4096
    say(f"launch shape independence T={T}")
    x = randn((T, H), 60, torch.bfloat16).to(DEV)
    r0 = randn((T, H), 61, torch.bfloat16).to(DEV)
    w = weight(H, 62, torch.bfloat16).to(DEV)
    sm = (0.5 + 1.5 * torch.rand(H, generator=gen(63))).to(DEV)
    shapes = [(0, 0), (1, 512), (2, 256), (4, 128), (8, 64), (2, 1024), (4, 512), (1, 1024)]
    outs = []
    try:
        for nv, tpr in shapes:
            _lib.set_launch_override(nv, tpr)
            r = r0.clone()
            q, s = custom_ops.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8,
                                                               residual=r)
            x1, r1 = x.clone(), r0.clone()
            torch.ops._C.fused_add_rms_norm(x1, r1, w, 1e-6)
            q4 = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=DEV)
            s4 = torch.empty(T, device=DEV)
            ar, an = torch.empty_like(x), torch.empty_like(x)
            op.rms_norm_dynamic_per_token_quant(q4, x, w, sm, s4, 1e-6, ar, an, r0)
            q5, s5 = op.scale_dynamic_quant(x, sm, torch.int8)
            outs.append([t.cpu() for t in (q, s, r, x1, r1, q4.view(torch.uint8), s4, ar, an,
                                           q5, s5)])
    finally:
        _lib.set_launch_override(0, 0)
    for o in outs[1:]:
        for a, b in zip(o, outs[0]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("T", [1, 64, 256])
def test_exact_row_forms_match_the_generic_form(T):
    """Rows that fill their workgroup exactly (one row per workgroup, every lane in it) take the
    kernel's exact-row form on the latency path (at most 256 rows) at two, four and eight
    vectors a lane; the generic form (several rows per workgroup, or lanes past the row end) must
    give the same bits, and both the oracle's."""
    H = 16384
    say(f"exact-row forms T={T}")
    x = randn((T, H), 64, torch.bfloat16)
    r0 = randn((T, H), 65, torch.bfloat16)
    w = weight(H, 66, torch.bfloat16)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r0)
    xd, wd = x.to(DEV), w.to(DEV)
    # 2048 vectors a row: (0, 0) = (2, 1024), (4, 512), (8, 256) exact; (8, 512): lanes past the
    # row end; (16, 128): two rows per workgroup
    shapes = [(0, 0), (4, 512), (8, 256), (8, 512), (16, 128)]
    try:
        for nv, tpr in shapes:
            _lib.set_launch_override(nv, tpr)
            rd = r0.to(DEV)
            q = torch.empty(T, H, dtype=torch.int8, device=DEV)
            s = torch.empty(T, 1, dtype=torch.float32, device=DEV)
            op.rms_norm_dynamic_per_token_quant_custom(q, xd, wd, s, 1e-6, None, rd)
            torch.cuda.synchronize()
            tag = f"T={T} nv={nv} tpr={tpr}"
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")
            assert_exact(rd, r_ref, tag + " residual")
    finally:
        _lib.set_launch_override(0, 0)


def test_repeatable():
    T, H = 1024, 8192
    x = randn((T, H), 70, torch.bfloat16).to(DEV)
    w = weight(H, 71, torch.bfloat16).to(DEV)
    first = None
    for _ in range(5):
        q, s = custom_ops.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8)
        if first is None:
            first = (q.clone(), s.clone())
        else:
            assert torch.equal(q, first[0]) and torch.equal(s, first[1])


def test_misaligned_views_take_the_scalar_path():
    """Pointers that are not 16-byte aligned (offset views) are handled (scalar kernels)."""
    T, H = 64, 1024
    say("misaligned views")
    buf_x = randn((T * H + 1,), 80, torch.bfloat16)
    buf_r = randn((T * H + 3,), 81, torch.bfloat16)
    w = weight(H, 82, torch.bfloat16)
    x = buf_x[1:].view(T, H)
    r = buf_r[3:].view(T, H)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6,
                                                                        residual=r)
    bxd, brd = buf_x.to(DEV), buf_r.to(DEV)
    xd, rd = bxd[1:].view(T, H), brd[3:].view(T, H)
    q = torch.empty((T, H), dtype=torch.int8, device=DEV)
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    op.rms_norm_dynamic_per_token_quant_custom(q, xd, w.to(DEV), s, 1e-6, None, rd)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


def test_special_values():
    """Rows with zeros, huge values, subnormals, infinities and NaN follow the oracle's defined
    semantics (NaN codes 0 for int8; clamp gives +448 for fp8)."""
    H = 256
    say("special values")
    rows = []
    rows.append(torch.zeros(H))
    big = torch.randn(H, generator=gen(90)) * 1e30
    rows.append(big)
    rows.append(torch.randn(H, generator=gen(91)) * 1e-39)
    t = torch.randn(H, generator=gen(92))
    t[5] = float("inf")
    rows.append(t)
    t = torch.randn(H, generator=gen(93))
    t[7] = float("nan")
    rows.append(t)
    x = torch.stack(rows).to(torch.bfloat16)
    w = weight(H, 94, torch.bfloat16)
    for qdt in (torch.int8, torch.float8_e4m3fn):
        q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt)
        q = torch.empty(x.shape, dtype=qdt, device=DEV)
        s = torch.empty((x.shape[0], 1), dtype=torch.float32, device=DEV)
        torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, None, None)
        torch.cuda.synchronize()
        sc, sr = s.cpu(), s_ref
        same = (sc == sr) | (torch.isnan(sc) & torch.isnan(sr))
        assert torch.all(same), (sc.flatten(), sr.flatten())
        assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))
    hq_ref, hs_ref = oracle.scale_dynamic_quant(x, torch.ones(H))
    hq, hs = op.scale_dynamic_quant(x.to(DEV), torch.ones(H, device=DEV), torch.int8)
    torch.cuda.synchronize()
    assert torch.equal(hq.cpu(), hq_ref)
    same = (hs.cpu() == hs_ref) | (torch.isnan(hs.cpu()) & torch.isnan(hs_ref))
    assert torch.all(same)


def test_fp8_conversion_matches_ocp_definition():
    """The hardware conversion (v_cvt_pk_fp8_f32) after the fmin/fmax clamp, against the oracle's
    conversion written from the OCP e4m3fn definition: every bf16 value, every fp8 midpoint and
    its neighbours, and random fp32."""
    say("fp8 conversion sweep")
    allbf = (torch.arange(1 << 16, dtype=torch.int32) << 16).view(torch.float32)
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    v = torch.unique(codes[torch.isfinite(codes)].double())
    mids = ((v[1:] + v[:-1]) / 2).float()
    mb = mids.view(torch.int32)
    around = torch.cat([mb, mb + 1, mb - 1]).view(torch.float32)
    rnd = torch.empty(1 << 22).uniform_(-500, 500, generator=gen(95))
    tiny = torch.empty(1 << 20).uniform_(-0.05, 0.05, generator=gen(96))
    x = torch.cat([allbf, around, rnd, tiny]).contiguous()
    for mul in (1.0, 0.37):
        ref = oracle.fp8_e4m3fn_from_f32(x, mul)
        xd = x.to(DEV)
        out = torch.empty(x.shape, dtype=torch.uint8, device=DEV)
        _lib.check(_lib.lib.mcop_fp8_e4m3fn_from_f32(out.data_ptr(), xd.data_ptr(), x.numel(),
                                                     mul, _lib.stream_of(xd)))
        torch.cuda.synchronize()
        bad = (out.cpu() != ref)
        assert int(bad.sum()) == 0, (x[bad][:8], out.cpu()[bad][:8], ref[bad][:8])


@pytest.mark.parametrize("T,H", [(1, 7168), (83, 7168), (2048, 7168), (3, 64), (83, 1033),
                                 (256, 4096), (7, 16384), (5, 7176)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h3_custom_op_shapes(T, H, dtype):
    """mcoplib's rms_norm_dynamic_per_token_quant_custom: its fp32 chain at H == 7168 and its
    generic chain (1.5e-6 floor, codes in [-127, 127]) elsewhere, with and without residual
    and scale_ub (which the 7168 chain ignores)."""
    say(f"h3 custom T={T} H={H} {dtype}")
    for with_res in (False, True):
        for ub in (None, 0.05):
            x = randn((T, H), T + H, dtype, scale=2.0)
            w = weight(H, T + H + 1, dtype)
            r = randn((T, H), T + H + 2, dtype) if with_res else None
            q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(
                x, w, 1e-6, scale_ub=ub, residual=r)
            rd = r.to(DEV) if with_res else None
            q = torch.empty((T, H), dtype=torch.int8, device=DEV)
            s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
            ubd = None if ub is None else torch.tensor([ub], device=DEV)
            op.rms_norm_dynamic_per_token_quant_custom(q, x.to(DEV), w.to(DEV), s, 1e-6, ubd, rd)
            torch.cuda.synchronize()
            tag = f"h3 T={T} H={H} {dtype} res={with_res} ub={ub}"
            assert_scales(s, s_ref, tag + " scales")
            assert_codes(q, q_ref, tag + " codes")
            if with_res:
                assert_exact(rd, r_ref, tag + " residual")


def test_h3_custom_op_zero_rows_and_specials():
    say("h3 custom special rows")
    for H in (7168, 4096):
        rows = [torch.zeros(H), torch.randn(H, generator=gen(95)) * 1e-30,
                torch.randn(H, generator=gen(96)) * 1e30]
        t = torch.randn(H, generator=gen(97))
        t[9] = float("nan")
        rows.append(t)
        x = torch.stack(rows).to(torch.bfloat16)
        w = weight(H, 98, torch.bfloat16)
        q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6)
        q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
        s = torch.empty((x.shape[0], 1), dtype=torch.float32, device=DEV)
        op.rms_norm_dynamic_per_token_quant_custom(q, x.to(DEV), w.to(DEV), s, 1e-6, None, None)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, f"h3 specials H={H} scales")
        assert_codes(q, q_ref, f"h3 specials H={H} codes")
