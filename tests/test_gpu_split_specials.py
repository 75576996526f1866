"""Special values and failed exchanges on the split-row kernels (rows too wide for one
workgroup's registers, each row shared by several workgroups that exchange partial results
through a device workspace).

- Rows of zeros, subnormals, values whose squares overflow fp32, +-inf and NaN elements and
  overflowing residual sums, at widths that take the split-row kernels, through every operator
  that has one: against the oracle bit for bit, and against the multi-pass kernel (forced with
  the library's test hook).
- The failure path of the exchange: with every wait of a launch failing at once (the test hook
  `mcop_debug_fail_split_waits` sets the workspace's error word before the kernel starts, as a
  timed-out wait leaves it), each call still returns, and every row's scales (for the norms and
  H1, every output) are NaN instead of a result built from partial sums; what the kernels write
  before their first exchange (the residual) is still exact.  The next call without the hook is
  bit-exact again, and narrow rows (no split-row kernel) are unaffected by the hook."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib, custom_ops, op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say
from test_gpu_special_values import _fp16_overflow_rows, _res_rows, _rows, _w
from test_gpu_split_rows import (_h1, _h2, _h4, _h5, _mc_norm, _mp, _padded, _per_block,
                                 _ptq_fp8, _ptq_int8)

pytestmark = pytest.mark.gpu

WIDE = 131072  # bf16 rows past the register kernels' 65536 elements


def _sm(H, seed):
    return 0.5 + 1.5 * torch.rand(H, generator=gen(seed))


_INT_OF_SIZE = {1: torch.uint8, 2: torch.int16, 4: torch.int32}


def _bits(t):
    return t.view(_INT_OF_SIZE[t.element_size()])


def _both(fn, *args):
    """The call on the split-row kernel and on the multi-pass kernel; asserts they agree bit for
    bit (NaNs included) and returns the split-row result."""
    got = fn(*args)
    mp = _mp(fn, *args)
    for k, (a, b) in enumerate(zip(got, mp)):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(_bits(a), _bits(b)), \
                f"output {k}: split-row and multi-pass kernels differ"
    return got


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, WIDE), (torch.float16, 65608)])
def test_split_h1_specials(dtype, H):
    say(f"split specials: fused_add_rms_norm {dtype} H={H}")
    x, r, w = _rows(H, 1).to(dtype), _res_rows(H, 2).to(dtype), _w(H, 3, dtype)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    got = _both(_h1, x, r, w, 0)
    assert_exact(got[1], r_ref, "residual")
    assert_exact(got[0], x_ref, "output")


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_split_h2_specials(qdt):
    say(f"split specials: vLLM rms_norm_dynamic_per_token_quant {qdt}")
    x, r, w = (_rows(WIDE, 4).to(torch.bfloat16), _res_rows(WIDE, 5).to(torch.bfloat16),
               _w(WIDE, 6, torch.bfloat16))
    for res in (None, r):
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, None, res)
        got = _both(_h2, x, w, res, qdt, None)
        assert_scales(got[1], s_ref, "scales")
        assert_codes(got[0], q_ref, "codes")
        if res is not None:
            assert_exact(got[2], r_ref, "residual")


def _h3(x, w, r):
    rd = r.to(DEV)
    q, s = custom_ops.rms_norm_dynamic_per_token_quant(x.to(DEV), w.to(DEV), 1e-6, torch.int8,
                                                       residual=rd)
    torch.cuda.synchronize()
    return q.cpu(), s.cpu(), rd.cpu()


def test_split_h3_specials():
    say("split specials: mcoplib custom op")
    x, r, w = (_rows(WIDE, 7).to(torch.bfloat16), _res_rows(WIDE, 8).to(torch.bfloat16),
               _w(WIDE, 9, torch.bfloat16))
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    got = _both(_h3, x, w, r)
    assert_exact(got[2], r_ref, "residual")
    assert_scales(got[1], s_ref, "scales")
    assert_codes(got[0], q_ref, "codes")


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("standard", [False, True])
def test_split_h4_specials(qdt, standard):
    say(f"split specials: smooth quant {qdt} standard={standard}")
    x, r, w = (_rows(WIDE, 10).to(torch.bfloat16), _res_rows(WIDE, 11).to(torch.bfloat16),
               _w(WIDE, 12, torch.bfloat16))
    sm = _sm(WIDE, 13)
    for res in (None, r):
        q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, res,
                                                                    standard)
        got = _both(_h4, x, w, sm, res, qdt, standard)
        assert_exact(got[2], ar_ref, "after_res")
        assert_exact(got[3], an_ref, "after_norm")
        assert_scales(got[1], s_ref, "scales")
        assert_codes(got[0], q_ref, "codes")


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_split_h4_fp16_residual_sum_overflow(qdt):
    """fp16 rows whose rounded residual sums overflow to inf while the sum of squares stays
    finite: the split kernel's division must see the infinities as the register kernel's does."""
    H = 65608
    say(f"split specials: smooth quant fp16 residual overflow {qdt} H={H}")
    x, r = _fp16_overflow_rows(H, 14)
    w = _w(H, 15, torch.float16)
    sm = _sm(H, 16)
    q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, r, False)
    assert torch.isinf(ar_ref[:3].float()).any(dim=1).all(), "rows 0-2 must overflow"
    got = _both(_h4, x, w, sm, r, qdt, False)
    assert_exact(got[2], ar_ref, "after_res")
    assert_exact(got[3], an_ref, "after_norm")
    assert_scales(got[1], s_ref, "scales")
    assert_codes(got[0], q_ref, "codes")


def test_split_h5_specials():
    say("split specials: scale_dynamic_quant")
    h = _rows(WIDE, 17).to(torch.bfloat16)
    sm = _sm(WIDE, 18)
    q_ref, s_ref = oracle.scale_dynamic_quant(h, sm)
    got = _both(_h5, h, sm)
    assert_scales(got[1], s_ref, "scales")
    assert_codes(got[0], q_ref, "codes")


def test_split_quantizer_specials():
    say("split specials: standalone quantizers")
    x = _rows(WIDE, 19).to(torch.bfloat16)
    for use_azp in (False, True):
        q_ref, s_ref, zp_ref = oracle.dynamic_scaled_int8_quant(x, use_azp=use_azp)
        got = _both(_ptq_int8, x, use_azp)
        assert_scales(got[1], s_ref, f"int8 azp={use_azp} scales")
        assert_codes(got[0], q_ref, f"int8 azp={use_azp} codes")
        if use_azp:
            assert_exact(got[2], zp_ref, "azp")
    xd = x.to(DEV)
    for ub in (None, 0.05):
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x, scale_ub=ub)
        got = _both(_ptq_fp8, xd, ub)
        assert_scales(got[1], s_ref, f"fp8 ub={ub} scales")
        assert_codes(got[0], q_ref, f"fp8 ub={ub} codes")


def test_split_padded_specials():
    say("split specials: padded op")
    H = WIDE
    pad = (H + 4 + 63) // 64 * 32  # whole 64-byte units: the vector path
    x, r, w = (_rows(H, 20).to(torch.bfloat16), _res_rows(H, 21).to(torch.bfloat16),
               _w(H, 22, torch.bfloat16))
    refs = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6)
    got = _both(_padded, x, r, w, pad)
    assert torch.equal(got[0].view(torch.uint8), refs[0]), "padded rows"
    assert_exact(got[1], refs[1], "residual")
    assert_exact(got[2], refs[2], "output_rms")
    assert_codes(got[3], refs[3], "codes")
    assert_scales(got[4], refs[4], "scales")


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_split_per_block_specials(qdt):
    say(f"split specials: per-block quant {qdt}")
    G = 128
    x, r, w = (_rows(WIDE, 23).to(torch.bfloat16), _res_rows(WIDE, 24).to(torch.bfloat16),
               _w(WIDE, 25, torch.bfloat16))
    q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, None, r)
    got = _both(_per_block, x, w, r, qdt, G, None, False)
    assert_exact(got[2], r_ref, "residual")
    assert_scales(got[1], s_ref, "scales")
    assert_codes(got[0], q_ref, "codes")


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, WIDE), (torch.float16, 65608)])
def test_split_norm_specials(dtype, H):
    say(f"split specials: mcoplib and vLLM rms_norm {dtype} H={H}")
    x, r, w = _rows(H, 26).to(dtype), _res_rows(H, 27).to(dtype), _w(H, 28, dtype)
    for res in (None, r):
        for rms_div in (True, False):
            out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=res, rms_div=rms_div)
            got = _both(_mc_norm, x, w, res, rms_div)
            assert_exact(got[0], out_ref, f"res={res is not None} rms_div={rms_div} out")
            if res is not None:
                assert_exact(got[1], ares_ref, "after_res")
    if dtype == torch.float16:
        x, r = _fp16_overflow_rows(H, 29)
        out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=r, rms_div=True)
        got = _both(_mc_norm, x, w, r, True)
        assert_exact(got[0], out_ref, "fp16 overflow out")
        assert_exact(got[1], ares_ref, "fp16 overflow after_res")
    ref = oracle.vllm_rms_norm(x, w, 1e-6)

    def vllm(xx, ww):
        o = torch.empty(xx.shape, dtype=xx.dtype, device=DEV)
        torch.ops._C.rms_norm(o, xx.to(DEV), ww.to(DEV), 1e-6)
        torch.cuda.synchronize()
        return (o.cpu(),)
    assert_exact(_both(vllm, x, w)[0], ref, "vLLM rms_norm")


# ------------------------------------------------------------------ failed exchanges
def _failing(fn, *args):
    """fn(*args) with every split-row exchange of its launches failing at once."""
    _lib.fail_split_waits(True)
    try:
        return fn(*args)
    finally:
        _lib.fail_split_waits(False)


def _all_nan(t, what):
    t = t.float()
    assert bool(torch.isnan(t).all()), f"{what}: {int((~torch.isnan(t)).sum())} of {t.numel()} " \
                                       f"values are not NaN"


def _inputs(T, seed, dtype=torch.bfloat16, H=WIDE):
    g = gen(seed)
    x = torch.randn(T, H, generator=g).to(dtype)
    r = torch.randn(T, H, generator=g).to(dtype)
    return x, r, _w(H, seed + 1, dtype)


@pytest.mark.parametrize("kind", ["h1", "h2", "h2-fp8-ub", "h3", "h4", "h5", "h5-one-row",
                                  "int8", "int8-azp", "fp8-ub", "padded", "per-block",
                                  "mc-norm", "vllm-norm"])
def test_split_failed_exchange_gives_nan_scales(kind):
    T = 5
    say(f"split: failed exchanges, {kind}, {T}x{WIDE}")
    x, r, w = _inputs(T, 40)
    sm = _sm(WIDE, 42)
    if kind == "h1":
        out, res = _failing(_h1, x, r, w, 0)
        _all_nan(out, "output")
        assert_exact(res, oracle.fused_add_rms_norm(x, r, w, 1e-6)[1], "residual")
        assert_exact(_h1(x, r, w, 0)[0], oracle.fused_add_rms_norm(x, r, w, 1e-6)[0], "after")
    elif kind in ("h2", "h2-fp8-ub"):
        qdt, ub = ((torch.int8, None) if kind == "h2" else (torch.float8_e4m3fn, 0.05))
        q, s, res = _failing(_h2, x, w, r, qdt, ub)
        _all_nan(s, "scales")
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, ub, r)
        assert_exact(res, r_ref, "residual")
        q, s, _ = _h2(x, w, r, qdt, ub)
        assert_scales(s, s_ref, "scales after")
        assert_codes(q, q_ref, "codes after")
    elif kind == "h3":
        q, s, res = _failing(_h3, x, w, r)
        _all_nan(s, "scales")
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6,
                                                                            residual=r)
        assert_exact(res, r_ref, "residual")
        assert_scales(_h3(x, w, r)[1], s_ref, "scales after")
    elif kind == "h4":
        q, s, ar, an = _failing(_h4, x, w, sm, r, torch.float8_e4m3fn, False)
        _all_nan(s, "scales")
        q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6,
                                                                    torch.float8_e4m3fn, r,
                                                                    False)
        assert_exact(ar, ar_ref, "after_res")
        got = _h4(x, w, sm, r, torch.float8_e4m3fn, False)
        assert_scales(got[1], s_ref, "scales after")
        assert_codes(got[0], q_ref, "codes after")
    elif kind in ("h5", "h5-one-row"):
        h = x[:1] if kind == "h5-one-row" else x  # one row: the one-row-a-workgroup kernel
        q, s = _failing(_h5, h, sm)
        _all_nan(s, "scales")
        q_ref, s_ref = oracle.scale_dynamic_quant(h, sm)
        assert_scales(_h5(h, sm)[1], s_ref, "scales after")
    elif kind in ("int8", "int8-azp"):
        azp = kind == "int8-azp"
        q, s, zp = _failing(_ptq_int8, x, azp)
        _all_nan(s, "scales")
        q_ref, s_ref, _ = oracle.dynamic_scaled_int8_quant(x, use_azp=azp)
        assert_scales(_ptq_int8(x, azp)[1], s_ref, "scales after")
    elif kind == "fp8-ub":
        q, s = _failing(_ptq_fp8, x.to(DEV), 0.05)
        _all_nan(s, "scales")
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x, scale_ub=0.05)
        assert_scales(_ptq_fp8(x.to(DEV), 0.05)[1], s_ref, "scales after")
    elif kind == "padded":
        pad = (WIDE + 4 + 63) // 64 * 32
        p, res, rms, q, s = _failing(_padded, x, r, w, pad)
        _all_nan(s, "scales")
        _all_nan(p[:, WIDE:WIDE + 4].contiguous().view(torch.float32), "scales in the rows")
        refs = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6)
        assert_exact(res, refs[1], "residual")
        got = _padded(x, r, w, pad)
        assert torch.equal(got[0].view(torch.uint8), refs[0]), "padded rows after"
    elif kind == "per-block":
        q, s, res = _failing(_per_block, x, w, r, torch.float8_e4m3fn, 128, None, True)
        _all_nan(s, "group scales")
        q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, torch.float8_e4m3fn,
                                                              128, None, r, True)
        assert_exact(res, r_ref, "residual")
        assert_scales(_per_block(x, w, r, torch.float8_e4m3fn, 128, None, True)[1], s_ref,
                      "scales after")
    elif kind == "mc-norm":
        out, ares = _failing(_mc_norm, x, w, r, True)
        _all_nan(out, "output")
        out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=r, rms_div=True)
        assert_exact(ares, ares_ref, "after_res")
        assert_exact(_mc_norm(x, w, r, True)[0], out_ref, "output after")
    else:
        o = torch.empty(x.shape, dtype=x.dtype, device=DEV)
        xd, wd = x.to(DEV), w.to(DEV)
        _failing(torch.ops._C.rms_norm, o, xd, wd, 1e-6)
        torch.cuda.synchronize()
        _all_nan(o, "output")
        torch.ops._C.rms_norm(o, xd, wd, 1e-6)
        torch.cuda.synchronize()
        assert_exact(o, oracle.vllm_rms_norm(x, w, 1e-6), "output after")


def test_failed_exchange_hook_leaves_narrow_rows_alone():
    """Rows that fit one workgroup take no split-row kernel, so the hook changes nothing."""
    say("split: failed-exchange hook on narrow rows")
    x, r, w = _inputs(64, 50, H=4096)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8, None,
                                                                  r)
    q, s, res = _failing(_h2, x, w, r, torch.int8, None)
    assert_exact(res, r_ref, "residual")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")
