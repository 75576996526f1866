"""GPU parity of the standalone per-token quantizers (``torch.ops._C.dynamic_scaled_int8_quant``
with and without azp, ``torch.ops._C.dynamic_per_token_scaled_fp8_quant``) against the CPU oracle,
plus the reference's own verification recipes (benchmark/runners/
mcoplib_mxbenchmark_dynamic_scaled_int8_quant_runners.py:40-60,
mcoplib_mxbenchmark_dynamic_per_token_scaled_fp8_quant_runners.py:40-57) run on the GPU output."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, randn, say

pytestmark = pytest.mark.gpu

SHAPES = [
    *[(1, h) for h in [1, 64, 1024, 1025, 1029, 5120, 5137]],
    *[(83, h) for h in [1, 1033, 2048, 5120]],
    *[(2048, h) for h in [1, 64, 1024, 1029, 5137]],
    (4096, 64), (7, 8192), (5, 16384), (3, 32768), (33, 7168), (17, 200), (128, 4096),
]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _int8_case(x, use_azp, tag):
    T, H = x.shape[0] if x.dim() > 1 else 1, x.shape[-1]
    q_ref, s_ref, zp_ref = oracle.dynamic_scaled_int8_quant(x, use_azp=use_azp)
    xd = x.to(DEV)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    zp = torch.empty((T, 1), dtype=torch.int32, device=DEV) if use_azp else None
    torch.ops._C.dynamic_scaled_int8_quant(q, xd, s, zp)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, tag + " scales")
    assert_codes(q, q_ref, tag + " codes")
    if use_azp:
        assert_exact(zp, zp_ref, tag + " azp")
    return q, s


def _fp8_case(x, tag, ub=None):
    T = x.numel() // x.shape[-1]
    q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x.cpu(), scale_ub=ub)
    xd = x.to(DEV) if x.device.type == "cpu" else x
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    ubd = None if ub is None else torch.tensor([ub], dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, xd, s, ubd)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, tag + " scales")
    assert_codes(q, q_ref, tag + " codes")
    return q, s


@pytest.mark.parametrize("T,H", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_int8_shapes(T, H, dtype):
    say(f"int8 T={T} H={H} {dtype}")
    x = randn((T, H), T * 131 + H, dtype, scale=2.0)
    _int8_case(x, False, f"int8 T={T} H={H} {dtype}")
    _int8_case(x, True, f"int8-azp T={T} H={H} {dtype}")


@pytest.mark.parametrize("T,H", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_fp8_shapes(T, H, dtype):
    say(f"fp8 T={T} H={H} {dtype}")
    x = randn((T, H), T * 137 + H, dtype, scale=3.0)
    _fp8_case(x, f"fp8 T={T} H={H} {dtype}")
    _fp8_case(x, f"fp8-ub T={T} H={H} {dtype}", ub=1.5)


def test_azp_offset_rows():
    say("int8-azp rows with offsets and spreads")
    T, H = 256, 3000
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(5))
         * torch.logspace(-3, 3, T)[:, None] + torch.linspace(-100, 100, T)[:, None])
    for dtype in DTYPES:
        _int8_case(x.to(dtype), True, f"int8-azp offsets {dtype}")


def test_three_dim_input():
    say("3-D input [4, 33, 1536]")
    x = randn((4, 33, 1536), 7, torch.bfloat16)
    q_ref, s_ref, _ = oracle.dynamic_scaled_int8_quant(x)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty((4 * 33, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_scaled_int8_quant(q, x.to(DEV), s, None)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "3-D scales")
    assert_codes(q, q_ref, "3-D codes")


@pytest.mark.parametrize("pad", [64, 3])
def test_fp8_row_strided_input(pad):
    say(f"fp8 strided rows pad={pad}")
    T, H = 300, 2048
    base = randn((T, H + pad), 21 + pad, torch.bfloat16, scale=2.0).to(DEV)
    view = base[:, pad:pad + H] if pad % 8 == 0 else base[:, :H]
    _fp8_case(view, f"fp8 strided pad={pad}")


def test_fp8_row_strided_output():
    say("fp8 strided output")
    T, H = 128, 1024
    x = randn((T, H), 23, torch.float16, scale=2.0)
    q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x)
    big = torch.zeros((T, H + 128), dtype=torch.float8_e4m3fn, device=DEV)
    q = big[:, :H]
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, x.to(DEV), s, None)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "fp8 strided-out scales")
    assert_codes(q, q_ref, "fp8 strided-out codes")
    assert int(big[:, H:].view(torch.uint8).count_nonzero()) == 0, "wrote past the row"


@pytest.mark.parametrize("pad", [64, 8])
def test_exact_rows_with_strided_views(pad):
    """64 x 4096 rows take the exact-row form (one row per workgroup, every lane in the row):
    row-strided input and output views, fp8 and int8 with and without azp."""
    T, H = 64, 4096
    say(f"exact-row quantizers, strided views pad={pad}")
    base = randn((T, H + pad), 27 + pad, torch.bfloat16, scale=2.0).to(DEV)
    view = base[:, pad:pad + H]
    q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(view.cpu())
    big = torch.zeros((T, H + 128), dtype=torch.float8_e4m3fn, device=DEV)
    q = big[:, :H]
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, view, s, None)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "fp8 scales")
    assert_codes(q, q_ref, "fp8 codes")
    assert int(big[:, H:].view(torch.uint8).count_nonzero()) == 0, "wrote past the row"
    for use_azp in (False, True):
        _int8_case(view.cpu(), use_azp, f"int8 azp={use_azp}")


def test_misaligned_views_take_the_scalar_path():
    say("misaligned views")
    base = randn((65 * 1001 + 1,), 31, torch.bfloat16)
    x = base[1:].view(65, 1001)  # 2-byte offset: no 16-byte vectors
    q_ref, s_ref, _ = oracle.dynamic_scaled_int8_quant(x.contiguous())
    q = torch.empty((65, 1001), dtype=torch.int8, device=DEV)
    s = torch.empty((65, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_scaled_int8_quant(q, base.to(DEV)[1:].view(65, 1001), s, None)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, "int8 misaligned scales")
    assert_codes(q, q_ref, "int8 misaligned codes")
    _fp8_case(base.to(DEV)[1:].view(65, 1001), "fp8 misaligned")


def test_special_values():
    say("special values: zero, constant, inf, nan, huge, tiny rows")
    H = 512
    # the 1e-38 row's absmax lies below 127 / FLT_MAX in bf16 and fp32: 127 / A is infinite
    rows = [torch.zeros(H), torch.full((H,), 2.5), torch.full((H,), -7.0), torch.randn(H) * 1e-30,
            torch.randn(H).clamp(-3, 3) * 1e38, torch.randn(H) * 1e-38]
    r = torch.randn(H)
    r[7] = float("inf")
    rows.append(r)
    r = torch.randn(H)
    r[9] = float("nan")
    rows.append(r)
    r = torch.randn(H)
    r[3] = float("-inf")
    rows.append(r)
    x = torch.stack(rows)
    for dtype in (torch.float32, torch.bfloat16):
        xx = x.to(dtype)
        _int8_case(xx, False, f"special int8 {dtype}")
        _fp8_case(xx, f"special fp8 {dtype}")
    for dtype in (torch.float32, torch.bfloat16):
        _int8_case(x.to(dtype), True, f"special int8-azp {dtype}")


@pytest.mark.parametrize("nv", [1, 2, 4, 8, 16])
def test_launch_shape_does_not_change_bits(nv):
    say(f"launch override nv={nv}")
    T, H = 517, 4096
    x = randn((T, H), 41, torch.bfloat16, scale=2.0)
    try:
        _lib.set_launch_override(nv, 0)
        _int8_case(x, False, f"int8 nv={nv}")
        _int8_case(x, True, f"int8-azp nv={nv}")
        _fp8_case(x, f"fp8 nv={nv}")
    finally:
        _lib.set_launch_override(0, 0)


def test_reference_verification_recipes():
    say("reference benchmark verification recipes (fp16 128x1024, 128x4096)")
    x = randn((128, 1024), 51, torch.float16).to(DEV)
    q = torch.empty((128, 1024), dtype=torch.int8, device=DEV)
    s = torch.empty((128, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_scaled_int8_quant(q, x, s, None)
    safe = s.clone()
    safe[safe == 0] = 1.0
    ref = torch.clamp(torch.round(x.float() / safe), -128, 127).to(torch.int8)
    assert int((q.int() - ref.int()).abs().max()) <= 1
    x = randn((128, 4096), 52, torch.float16).to(DEV)
    q = torch.empty((128, 4096), dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty((128, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, x, s, None)
    safe = s.clone()
    safe[safe == 0] = 1.0
    ref = (x.float() / safe).to(torch.float8_e4m3fn)
    assert torch.equal(q.view(torch.uint8), ref.view(torch.uint8))


def test_large_rows_sampled():
    say("large: 8192 x 8192 bf16, int8 / azp / fp8 over sampled rows")
    T, H = 8192, 8192
    x = randn((T, H), 61, torch.bfloat16, scale=2.0)
    xd = x.to(DEV)
    idx = torch.arange(0, T, 61)
    for use_azp in (False, True):
        q = torch.empty((T, H), dtype=torch.int8, device=DEV)
        s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
        zp = torch.empty((T, 1), dtype=torch.int32, device=DEV) if use_azp else None
        torch.ops._C.dynamic_scaled_int8_quant(q, xd, s, zp)
        torch.cuda.synchronize()
        q_ref, s_ref, zp_ref = oracle.dynamic_scaled_int8_quant(x[idx], use_azp=use_azp)
        assert_scales(s.cpu()[idx], s_ref, f"large azp={use_azp} scales")
        assert_codes(q.cpu()[idx], q_ref, f"large azp={use_azp} codes")
        if use_azp:
            assert_exact(zp.cpu()[idx], zp_ref, "large azp")
    q = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=DEV)
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    torch.ops._C.dynamic_per_token_scaled_fp8_quant(q, xd, s, None)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x[idx])
    assert_scales(s.cpu()[idx], s_ref, "large fp8 scales")
    assert_codes(q.cpu()[idx], q_ref, "large fp8 codes")


def test_argument_errors():
    say("argument checks")
    x = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    s = torch.empty((4, 1), dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError):
        torch.ops._C.dynamic_scaled_int8_quant(torch.empty((4, 64), dtype=torch.uint8, device=DEV),
                                               x, s, None)
    with pytest.raises(RuntimeError):
        torch.ops._C.dynamic_scaled_int8_quant(torch.empty((4, 64), dtype=torch.int8, device=DEV),
                                               x.t(), s, None)
    with pytest.raises(RuntimeError):
        torch.ops._C.dynamic_per_token_scaled_fp8_quant(
            torch.empty((4, 64), dtype=torch.int8, device=DEV), x, s, None)
    with pytest.raises(RuntimeError):
        torch.ops._C.dynamic_per_token_scaled_fp8_quant(
            torch.empty((4, 64), dtype=torch.float8_e4m3fn, device=DEV), x,
            torch.empty((3, 1), dtype=torch.float32, device=DEV), None)
    # empty input: nothing launched, nothing raised
    torch.ops._C.dynamic_scaled_int8_quant(torch.empty((0, 64), dtype=torch.int8, device=DEV),
                                           torch.empty((0, 64), device=DEV), s[:0], None)
