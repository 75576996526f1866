"""Special values through every operator of the path, GPU against the oracle bit for bit: rows
of zeros, subnormals, values whose squares overflow fp32, +-inf and NaN elements, and residual
sums that overflow.  The oracle defines the results (fmax ignores NaN in the absmax, an infinite
sum of squares gives rho = 0, 0 * inf = NaN propagates, NaN codes follow each converter); the
kernels must reproduce them exactly.  (H2, H3, H5 and the standalone quantizers have their own
special-value tests next to their parity tests.)"""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say

pytestmark = pytest.mark.gpu


def _rows(H, seed):
    """[9, H] fp32 rows: zeros, huge (squares overflow fp32), subnormal, one +inf, one NaN,
    one -inf, ordinary, one large element among tiny ones, all near the bf16 maximum."""
    g = gen(seed)
    rows = [torch.zeros(H), torch.randn(H, generator=g) * 1e30,
            torch.randn(H, generator=g) * 1e-39]
    for k, v in ((5, float("inf")), (7, float("nan")), (3, float("-inf"))):
        t = torch.randn(H, generator=g)
        t[k % H] = v
        rows.append(t)
    rows.append(torch.randn(H, generator=g))
    t = torch.randn(H, generator=g) * 1e-20
    t[H // 2] = 6e4
    rows.append(t)
    rows.append(torch.full((H,), 3.0e38))
    return torch.stack(rows)


def _res_rows(H, seed):
    r = torch.randn(9, H, generator=gen(seed))
    r[8] = 3.0e38  # x + r overflows to inf in fp32
    return r


def _w(H, seed, dtype):
    return (1 + 0.1 * torch.randn(H, generator=gen(seed))).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h1_fused_add_rms_norm_specials(dtype):
    say(f"specials: fused_add_rms_norm {dtype}")
    H = 1024
    x = _rows(H, 1).to(dtype)
    r = _res_rows(H, 2).to(dtype)
    w = _w(H, 3, dtype)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    xd, rd = x.to(DEV), r.to(DEV)
    torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_exact(xd, x_ref, "output")


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("standard", [False, True])
@pytest.mark.parametrize("with_res", [False, True])
def test_h4_smooth_quant_specials(qdt, standard, with_res):
    say(f"specials: smooth quant {qdt} standard={standard} res={with_res}")
    H = 2048
    x = _rows(H, 4).to(torch.bfloat16)
    r = _res_rows(H, 5).to(torch.bfloat16) if with_res else None
    w = _w(H, 6, torch.bfloat16)
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(7))
    q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, r, standard)
    q = torch.empty(x.shape, dtype=qdt, device=DEV)
    s = torch.empty(x.shape[0], device=DEV)
    ar, an = torch.empty(x.shape, dtype=x.dtype, device=DEV), torch.empty(x.shape, dtype=x.dtype,
                                                                           device=DEV)
    op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                        None if r is None else r.to(DEV), standard_norm=standard)
    torch.cuda.synchronize()
    assert_exact(ar, ar_ref, "after_res")
    assert_exact(an, an_ref, "after_norm")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("H", [7168, 1024])
def test_padded_specials(H):
    say(f"specials: padded H={H}")
    pad = (H + 4 + 63) // 64 * 32
    x = _rows(H, 8).to(torch.bfloat16)
    r = _res_rows(H, 9).to(torch.bfloat16)
    w = _w(H, 10, torch.bfloat16)
    p_ref, r_ref, rms_ref, q_ref, s_ref = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6)
    T = x.shape[0]
    p = torch.zeros(T, 2 * pad, dtype=torch.int8, device=DEV)
    rms = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(T, 1, device=DEV)
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
def test_per_block_specials(qdt):
    say(f"specials: per-block quant {qdt}")
    H, G = 1024, 128
    x = _rows(H, 11).to(torch.bfloat16)
    r = _res_rows(H, 12).to(torch.bfloat16)
    w = _w(H, 13, torch.bfloat16)
    q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, None, r)
    q = torch.empty(x.shape, dtype=qdt, device=DEV)
    s = torch.empty(x.shape[0], H // G, device=DEV)
    rd = r.to(DEV)
    torch.ops._C.rms_norm_per_block_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, None, rd, G, False)
    torch.cuda.synchronize()
    assert_exact(rd, r_ref, "residual")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("H", [4096, 1030])  # the reference's vectorized / element-wise chains
@pytest.mark.parametrize("rms_div", [True, False])
def test_mc_rms_norm_specials(H, rms_div):
    say(f"specials: mcoplib rms_norm H={H} rms_div={rms_div}")
    x = _rows(H, 14).to(torch.bfloat16)
    r = _res_rows(H, 15).to(torch.bfloat16)
    w = _w(H, 16, torch.bfloat16)
    for res in (None, r):
        out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=res, rms_div=rms_div)
        out = torch.empty(x.shape, dtype=x.dtype, device=DEV)
        ares = torch.empty(x.shape, dtype=x.dtype, device=DEV) if res is not None else None
        op.rms_norm(out, x.to(DEV), w.to(DEV), 1e-6, ares, None if res is None else res.to(DEV),
                    rms_div)
        torch.cuda.synchronize()
        assert_exact(out, out_ref, "out")
        if res is not None:
            assert_exact(ares, ares_ref, "after_res")


def test_head_and_vllm_rms_norm_specials():
    say("specials: head_rms_norm and vLLM rms_norm")
    D = 128
    hs = _rows(D, 17).to(torch.bfloat16).view(9, 1, D).expand(9, 4, D).contiguous()
    w = _w(4 * D, 18, torch.bfloat16).view(4, D)
    base = torch.zeros_like(hs)
    ref = oracle.head_rms_norm(base, hs, w, 1e-6, 1, 3)
    out = base.to(DEV)
    op.head_rms_norm(out, hs.to(DEV), w.to(DEV), 1e-6, 1, 3)
    torch.cuda.synchronize()
    assert_exact(out, ref, "head_rms_norm")
    for dtype in (torch.bfloat16, torch.float32):
        x = _rows(512, 19).to(dtype)
        wv = _w(512, 20, dtype)
        ref = oracle.vllm_rms_norm(x, wv, 1e-6)
        o = torch.empty(x.shape, dtype=dtype, device=DEV)
        torch.ops._C.rms_norm(o, x.to(DEV), wv.to(DEV), 1e-6)
        torch.cuda.synchronize()
        assert_exact(o, ref, f"vLLM rms_norm {dtype}")


def _fp16_overflow_rows(H, seed):
    """fp16 x and residual [5, H] whose sums round to +-inf in fp16 while the fp32 sums (and so
    the sum of squares) stay finite: one element 60000 + 60000; every element 40000 + 40000; one
    element 33024 + 32496 = 65520 (the tie between 65504 and the overflow, which rounds to inf);
    a control row whose sums reach 65504, the largest finite fp16; an ordinary row."""
    g = gen(seed)
    x = torch.randn(5, H, generator=g)
    r = torch.randn(5, H, generator=g)
    x[0, 3], r[0, 3] = 60000.0, 60000.0
    x[1], r[1] = 40000.0, 40000.0
    x[2, H // 2], r[2, H // 2] = 33024.0, 32496.0
    x[3, 7], r[3, 7] = 32752.0, 32752.0
    return x.to(torch.float16), r.to(torch.float16)


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("standard", [False, True])
def test_h4_fp16_residual_sum_overflow(qdt, standard):
    """fp16 SmoothQuant with a residual whose rounded sums overflow: after_res is +-inf where the
    fp32 sum is finite, and the literal form's division must see those infinities (the short
    division form is only valid for finite b(a))."""
    say(f"specials: smooth quant fp16 residual overflow {qdt} standard={standard}")
    H = 2048
    x, r = _fp16_overflow_rows(H, 21)
    w = _w(H, 22, torch.float16)
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(23))
    q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, r, standard)
    assert torch.isinf(ar_ref[:3].float()).any(dim=1).all(), "rows 0-2 must overflow"
    q = torch.empty(x.shape, dtype=qdt, device=DEV)
    s = torch.empty(x.shape[0], device=DEV)
    ar, an = torch.empty(x.shape, dtype=x.dtype, device=DEV), torch.empty(x.shape, dtype=x.dtype,
                                                                           device=DEV)
    op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, 1e-6, ar, an,
                                        r.to(DEV), standard_norm=standard)
    torch.cuda.synchronize()
    assert_exact(ar, ar_ref, "after_res")
    assert_exact(an, an_ref, "after_norm")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("H", [4096, 1030])  # the reference's vectorized / element-wise chains
def test_mc_rms_norm_fp16_residual_sum_overflow(H):
    """mcoplib rms_norm, fp16, rms_div, with a residual whose rounded sums overflow (the
    element-wise chain at H = 1030 divides the rounded sum by rho)."""
    say(f"specials: mcoplib rms_norm fp16 residual overflow H={H}")
    x, r = _fp16_overflow_rows(H, 24)
    w = _w(H, 25, torch.float16)
    out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=r, rms_div=True)
    assert torch.isinf(ares_ref[:3].float()).any(dim=1).all(), "rows 0-2 must overflow"
    out = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    ares = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    op.rms_norm(out, x.to(DEV), w.to(DEV), 1e-6, ares, r.to(DEV), True)
    torch.cuda.synchronize()
    assert_exact(out, out_ref, "out")
    assert_exact(ares, ares_ref, "after_res")
