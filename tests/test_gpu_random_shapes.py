"""Seeded random shapes through every operator of the path, GPU against the oracle: odd and even
widths from 1 element to past the register-resident limits, 1 to 300 rows, every input dtype an
operator takes.  They exercise the launch geometry's corners (rows packed into one workgroup,
ragged last vectors, the scalar path for widths not a multiple of the vector, the multi-pass
kernels) that the configuration-shaped tests leave between them.  The case is a function of the
seed alone, so a failure names its seed, operator and shape."""

import random

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say

pytestmark = pytest.mark.gpu

OPS = ["h1", "h2", "h3", "h4", "h5", "ptq_int8", "ptq_azp", "ptq_fp8", "norm", "vllm_norm",
       "padded", "per_block"]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _shape(rng: random.Random):
    kind = rng.random()
    if kind < 0.4:
        H = rng.randint(1, 12000)
    elif kind < 0.8:
        H = 8 * rng.randint(1, 2500)
    elif kind < 0.95:
        H = rng.choice([7168, 8192, 5120, 4096, 16384, 32768]) + rng.choice([-8, -1, 0, 1, 8])
    else:
        H = rng.choice([65536 + 8, 70001, 131072])
    T = rng.choice([1, 2, 3, 5, 17, 40, rng.randint(1, 300)])
    if H >= 65536:
        T = min(T, 5)
    return T, H


def _x(T, H, seed, dtype, scale=1.0):
    x = torch.randn(T, H, generator=gen(seed)) * scale
    if T > 1:
        x[T // 2, H // 3] = 30.0 * scale  # an outlier
    return x.to(dtype)


def _w(H, seed, dtype):
    return (1 + 0.1 * torch.randn(H, generator=gen(seed))).to(dtype)


@pytest.mark.parametrize("seed", range(400))
def test_random_shape(seed):
    rng = random.Random(seed)
    name = OPS[seed % len(OPS)]
    T, H = _shape(rng)
    dtype = rng.choice(DTYPES)
    say(f"random seed={seed}: {name} T={T} H={H} {dtype}")
    _check(seed, rng, name, T, H, dtype)


def _wide_shape(rng: random.Random):
    """Rows past the register-resident kernels: mostly whole 16-byte vectors (the split-row
    kernels, 2 to 64 slices), a few odd widths (the element-wise multi-pass kernels)."""
    kind = rng.random()
    if kind < 0.85:
        H = 8 * rng.randint(8193, 48000)
    elif kind < 0.95:
        H = rng.choice([65544, 131072, 262144, 393216])
    else:
        H = rng.randint(65537, 140000) | 1
    T = rng.choice([1, 2, 3, 5, 9, rng.randint(1, 24)])
    return T, H


@pytest.mark.parametrize("seed", range(1000, 1096))
def test_random_wide_shape(seed):
    """Seeded random rows wider than one workgroup's registers through every operator."""
    rng = random.Random(seed)
    name = OPS[seed % len(OPS)]
    T, H = _wide_shape(rng)
    dtype = rng.choice(DTYPES)
    say(f"random wide seed={seed}: {name} T={T} H={H} {dtype}")
    _check(seed, rng, name, T, H, dtype)


def _check(seed, rng, name, T, H, dtype):
    """One seeded case of operator `name` at [T, H] in `dtype` against the oracle."""
    eps = rng.choice([1e-6, 1e-5])
    if name == "h1":
        x, r, w = _x(T, H, seed, dtype), _x(T, H, seed + 1, dtype), _w(H, seed + 2, dtype)
        x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, eps)
        pad = rng.choice([0, 0, 8, 3])  # x rows may be strided (input.stride(-2) > H)
        big = torch.zeros(T, H + pad, dtype=dtype)
        big[:, :H] = x
        bigd, rd = big.to(DEV), r.to(DEV)
        xd = bigd[:, :H]
        torch.ops._C.fused_add_rms_norm(xd, rd, w.to(DEV), eps)
        torch.cuda.synchronize()
        assert_exact(rd, r_ref, "residual")
        assert_exact(xd.contiguous(), x_ref, "output")
        assert not pad or bool((bigd[:, H:] == 0).all()), "row padding written"
    elif name == "h2":
        qdt = rng.choice([torch.int8, torch.float8_e4m3fn])
        with_res = rng.random() < 0.5
        x, w = _x(T, H, seed, dtype), _w(H, seed + 2, dtype)
        r = _x(T, H, seed + 1, dtype) if with_res else None
        ub = 0.5 if qdt == torch.float8_e4m3fn and rng.random() < 0.3 else None
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, eps, qdt, ub, r)
        q = torch.empty(T, H, dtype=qdt, device=DEV)
        s = torch.empty(T, 1, device=DEV)
        rd = None if r is None else r.to(DEV)
        ubd = None if ub is None else torch.tensor([ub], device=DEV)
        torch.ops._C.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), s, eps, ubd, rd)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
        if r is not None:
            assert_exact(rd, r_ref, "residual")
    elif name == "h3":
        x, w = _x(T, H, seed, dtype), _w(H, seed + 2, dtype)
        r = _x(T, H, seed + 1, dtype) if rng.random() < 0.7 else None
        q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, eps,
                                                                            residual=r)
        q = torch.empty(T, H, dtype=torch.int8, device=DEV)
        s = torch.empty(T, 1, device=DEV)
        rd = None if r is None else r.to(DEV)
        op.rms_norm_dynamic_per_token_quant_custom(q, x.to(DEV), w.to(DEV), s, eps, None, rd)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
        if r is not None:
            assert_exact(rd, r_ref, "residual")
    elif name == "h4":
        qdt = rng.choice([torch.int8, torch.float8_e4m3fn])
        standard = rng.random() < 0.5
        x = _x(T, H, seed, dtype, rng.choice([0.1, 1.0, 3.0]))
        r = _x(T, H, seed + 1, dtype) if rng.random() < 0.5 else None
        w = _w(H, seed + 2, rng.choice([dtype, torch.float32]))
        sm = (0.5 + 1.5 * torch.rand(H, generator=gen(seed + 3))).to(rng.choice([dtype,
                                                                                 torch.float32]))
        q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, eps, qdt, r,
                                                                    standard)
        q = torch.empty(T, H, dtype=qdt, device=DEV)
        s = torch.empty(T, device=DEV)
        ar = torch.empty(T, H, dtype=dtype, device=DEV)
        an = torch.empty(T, H, dtype=dtype, device=DEV)
        op.rms_norm_dynamic_per_token_quant(q, x.to(DEV), w.to(DEV), sm.to(DEV), s, eps, ar, an,
                                            None if r is None else r.to(DEV),
                                            standard_norm=standard)
        torch.cuda.synchronize()
        assert_exact(ar, ar_ref, "after_res")
        assert_exact(an, an_ref, "after_norm")
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
    elif name == "h5":
        x = _x(T, H, seed, torch.bfloat16)
        sm = 0.5 + 1.5 * torch.rand(H, generator=gen(seed + 3))
        q_ref, s_ref = oracle.scale_dynamic_quant(x, sm)
        q, s = op.scale_dynamic_quant(x.to(DEV), sm.to(DEV), torch.int8)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
    elif name in ("ptq_int8", "ptq_azp"):
        azp = name == "ptq_azp"
        x = _x(T, H, seed, dtype)
        q_ref, s_ref, z_ref = oracle.dynamic_scaled_int8_quant(x, use_azp=azp)
        q = torch.empty(T, H, dtype=torch.int8, device=DEV)
        s = torch.empty(T, 1, device=DEV)
        z = torch.empty(T, 1, dtype=torch.int32, device=DEV) if azp else None
        torch.ops._C.dynamic_scaled_int8_quant(q, x.to(DEV), s, z)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
        if azp:
            assert torch.equal(z.cpu().flatten(), z_ref.flatten()), "zero points"
    elif name == "ptq_fp8":
        x = _x(T, H, seed, dtype)
        ub = 0.05 if rng.random() < 0.3 else None
        q_ref, s_ref = oracle.dynamic_per_token_scaled_fp8_quant(x, ub)
        pin, pout = rng.choice([0, 0, 16, 5]), rng.choice([0, 0, 32, 7])  # strided rows
        big = torch.zeros(T, H + pin, dtype=dtype)
        big[:, :H] = x
        qb = torch.zeros(T, H + pout, dtype=torch.float8_e4m3fn, device=DEV)
        s = torch.empty(T, 1, device=DEV)
        ubd = None if ub is None else torch.tensor([ub], device=DEV)
        torch.ops._C.dynamic_per_token_scaled_fp8_quant(qb[:, :H], big.to(DEV)[:, :H], s, ubd)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(qb[:, :H].contiguous(), q_ref, "codes")
        assert not pout or bool((qb[:, H:].view(torch.uint8) == 0).all()), "row padding written"
    elif name == "norm":
        x, w = _x(T, H, seed, dtype), _w(H, seed + 2, rng.choice([dtype, torch.float32]))
        r = _x(T, H, seed + 1, dtype) if rng.random() < 0.5 else None
        rms_div = rng.random() < 0.5
        out_ref, ares_ref = oracle.rms_norm(x, w, eps, residual=r, rms_div=rms_div)
        out = torch.empty(T, H, dtype=dtype, device=DEV)
        ares = torch.empty(T, H, dtype=dtype, device=DEV) if r is not None else None
        op.rms_norm(out, x.to(DEV), w.to(DEV), eps, ares, None if r is None else r.to(DEV),
                    rms_div)
        torch.cuda.synchronize()
        assert_exact(out, out_ref, "out")
        if r is not None:
            assert_exact(ares, ares_ref, "after_res")
    elif name == "padded":
        x, r, w = (_x(T, H, seed, torch.bfloat16), _x(T, H, seed + 1, torch.bfloat16),
                   _w(H, seed + 2, torch.bfloat16))
        pad = (H + 4 + 63) // 64 * 32 + rng.choice([0, 0, 32])
        p_ref, r_ref, rms_ref, q_ref, s_ref = oracle.add_rms_norm_quant_padded(x, r, w, pad, eps)
        p = torch.zeros(T, 2 * pad, dtype=torch.int8, device=DEV)
        rms = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
        q = torch.empty(T, H, dtype=torch.int8, device=DEV)
        s = torch.empty(T, 1, device=DEV)
        rd = r.to(DEV)
        op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(p, rms, q, s, x.to(DEV), rd,
                                                                      w.to(DEV), pad, eps)
        torch.cuda.synchronize()
        assert_exact(rd, r_ref, "residual")
        assert_exact(rms, rms_ref, "output_rms")
        assert_codes(q, q_ref, "codes")
        assert_scales(s, s_ref, "scales")
        assert torch.equal(p.cpu().view(torch.uint8), p_ref), "padded rows"
    elif name == "per_block":
        G = rng.choice([64, 128])
        H = G * max(1, H // G)
        qdt = rng.choice([torch.int8, torch.float8_e4m3fn])
        transposed = rng.random() < 0.3
        x, w = _x(T, H, seed, dtype), _w(H, seed + 2, dtype)
        r = _x(T, H, seed + 1, dtype) if rng.random() < 0.5 else None
        q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, eps, qdt, G, None, r,
                                                              transposed)
        q = torch.empty(T, H, dtype=qdt, device=DEV)
        s = (torch.empty(H // G, T, device=DEV) if transposed
             else torch.empty(T, H // G, device=DEV))
        rd = None if r is None else r.to(DEV)
        torch.ops._C.rms_norm_per_block_quant(q, x.to(DEV), w.to(DEV), s, eps, None, rd, G,
                                              transposed)
        torch.cuda.synchronize()
        assert_scales(s, s_ref, "scales")
        assert_codes(q, q_ref, "codes")
        if r is not None:
            assert_exact(rd, r_ref, "residual")
    else:  # vllm_norm, on a 2-D or a 3-D input with strided rows
        x, w = _x(T, H, seed, dtype), _w(H, seed + 2, dtype)
        ref = oracle.vllm_rms_norm(x, w, eps)
        out = torch.empty(T, H, dtype=dtype, device=DEV)
        if T % 2 == 0 and rng.random() < 0.5:
            big = torch.zeros(2, T // 2, H + 16, dtype=dtype)
            big[:, :, :H] = x.view(2, T // 2, H)
            torch.ops._C.rms_norm(out.view(2, T // 2, H), big.to(DEV)[:, :, :H], w.to(DEV), eps)
        else:
            torch.ops._C.rms_norm(out, x.to(DEV), w.to(DEV), eps)
        torch.cuda.synchronize()
        assert_exact(out, ref, "out")
