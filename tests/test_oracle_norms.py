"""Pins of the oracle's RMSNorms without quantization: mcoplib ``op.rms_norm`` and
``op.head_rms_norm`` (op/fused_rms_norm_dq.cu:305-420, 493-578, 669-998) and vLLM
``_C::rms_norm`` (op/vllm/layernorm_kernels.cu:15-86, 186-231).

  - the reference's own asserting tests, at their tolerances (atol = rtol = 1e-5):
    unit_test/test_rms_norm.py:53-68 (fp32, residual, rms_div) and
    unit_test/test_head_rms_norm.py:46-57 (fp32 heads, per-head fp32 weights, the untouched
    heads included), at reduced sizes;
  - bit-exact torch restatements of each rounding chain, on both sides of the reference's
    switch between its vectorized and element-wise kernels;
  - vLLM's chain against vLLM's forward_native convention (two bf16 roundings).
"""

import numpy as np
import pytest
import torch

import oracle


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _rho(a: torch.Tensor, eps: float) -> torch.Tensor:
    H = a.shape[-1]
    ss = (a.double() * a.double()).sum(-1, keepdim=True).float()
    ms = (ss.double() / float(np.float32(H))).float()
    v = ms + torch.tensor(eps, dtype=torch.float32)
    r = torch.sqrt(v.double()).float()
    return (1.0 / r.double()).float()


def _vectorized(H, dtype, wdtype):
    n = 4 if torch.float32 in (dtype, wdtype) else 8
    return H % n == 0 and H <= 3 * 1024 * n


# ------------------------------------------------------------------------- mcoplib rms_norm

def test_reference_rms_norm_test():
    # unit_test/test_rms_norm.py: fp32, residual, weight N(0,1), eps 1e-5, rms_div=True
    m, n = 256, 4096
    g = _gen(42)
    h = torch.randn(m, n, generator=g)
    r = torch.randn(m, n, generator=g)
    w = torch.randn(n, generator=g)
    out, ares = oracle.rms_norm(h, w, 1e-5, residual=r, rms_div=True)
    after = h + r
    rms = torch.rsqrt(torch.mean(after * after, dim=-1, keepdim=True) + 1e-5)
    ref = after / rms * w
    torch.testing.assert_close(ref, out, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(after, ares, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype,wdtype,H", [
    (torch.bfloat16, torch.bfloat16, 4096),    # vectorized
    (torch.bfloat16, torch.bfloat16, 1030),    # element-wise: not a multiple of 8
    (torch.bfloat16, torch.bfloat16, 24576),   # vectorized: the largest
    (torch.bfloat16, torch.bfloat16, 24584),   # element-wise: longer than 3 * 1024 * 8
    (torch.float16, torch.float32, 12288),     # vectorized with fp32 weights (n = 4)
    (torch.float16, torch.float32, 12296),     # element-wise with fp32 weights
    (torch.float32, torch.float32, 1028),      # vectorized fp32
    (torch.float32, torch.float32, 1026),      # element-wise fp32
])
@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("rms_div", [True, False])
def test_rms_norm_restatement(dtype, wdtype, H, with_res, rms_div):
    g = _gen(H + 7)
    T = 6
    x = (torch.randn(T, H, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(wdtype)
    r = torch.randn(T, H, generator=g).to(dtype) if with_res else None
    out, ares = oracle.rms_norm(x, w, 1e-6, residual=r, rms_div=rms_div)
    a = x.float() + (r.float() if with_res else 0.0)
    rho = _rho(a, 1e-6)
    if _vectorized(H, dtype, wdtype):
        d = (1.0 / rho.double()).float() if rms_div else rho
        ref = ((a * d) * w.float()).to(dtype)
    else:
        at = a.to(dtype).float() if with_res else a
        n = at / rho if rms_div else at * rho
        ref = (n * w.float()).to(dtype)
    assert torch.equal(out, ref)
    if with_res:
        assert torch.equal(ares, a.to(dtype))
    else:
        assert ares is None


def test_rms_div_is_the_reciprocal_convention():
    # rms_div: x / rsqrt(ms + eps) = x * sqrt(ms + eps); without: x * rsqrt(ms + eps)
    x = torch.full((1, 64), 3.0)
    w = torch.ones(64)
    out_div, _ = oracle.rms_norm(x, w, 0.0, rms_div=True)
    out_mul, _ = oracle.rms_norm(x, w, 0.0, rms_div=False)
    assert torch.allclose(out_div, torch.full((1, 64), 9.0))
    assert torch.allclose(out_mul, torch.full((1, 64), 1.0))


# ------------------------------------------------------------------------- head_rms_norm

@pytest.mark.parametrize("D", [4096, 4096 * 2, 4096 * 3])
def test_reference_head_rms_norm_test(D):
    # unit_test/test_head_rms_norm.py: fp32 heads and weights, head_offset 0, eps 1e-5
    T, NH, hn = 4, 16, 8
    g = _gen(42)
    hs = torch.randn(T, NH, D, generator=g)
    w = torch.randn(NH, D, generator=g)
    out = oracle.head_rms_norm(hs.clone(), hs, w, 1e-5, 0, hn)
    ref = hs.clone()
    for h in range(hn):
        sel = hs[:, h, :]
        var = sel.pow(2).mean(-1, keepdim=True)
        ref[:, h, :] = w[h, :] * (sel / torch.rsqrt(var + 1e-5))
    torch.testing.assert_close(ref, out, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype,wdtype,D", [(torch.bfloat16, torch.bfloat16, 128),
                                            (torch.bfloat16, torch.float32, 128),
                                            (torch.float16, torch.bfloat16, 100),
                                            (torch.float32, torch.bfloat16, 256),
                                            (torch.float32, torch.float32, 12290)])
def test_head_rms_norm_restatement(dtype, wdtype, D):
    T, NH, off, hn = 5, 12, 3, 6
    g = _gen(D)
    hs = torch.randn(T, NH, D, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(NH, D, generator=g)).to(wdtype)
    base = torch.randn(T, NH, D, generator=g).to(dtype)
    out = oracle.head_rms_norm(base, hs, w, 1e-6, off, hn)
    ref = base.clone()
    for h in range(off, off + hn):
        a = hs[:, h, :].float()
        rho = _rho(a, 1e-6)
        if _vectorized(D, dtype, wdtype):
            y = (a * (1.0 / rho.double()).float()) * w[h].float()
        else:
            y = (a / rho) * w[h].float()
        ref[:, h, :] = y.to(dtype)
    assert torch.equal(out, ref)


# ------------------------------------------------------------------------- vLLM rms_norm

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_vllm_rms_norm_restatement(dtype):
    g = _gen(9)
    x = (torch.randn(33, 1000, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(1000, generator=g)).to(dtype)
    out = oracle.vllm_rms_norm(x, w, 1e-6)
    rho = _rho(x.float(), 1e-6)
    ref = ((x.float() * rho).to(dtype).float() * w.float()).to(dtype)
    assert torch.equal(out, ref)


def test_vllm_rms_norm_vs_forward_native():
    # vLLM RMSNorm.forward_native: x * rsqrt(mean(x^2) + eps) in fp32, cast, times weight
    g = _gen(10)
    x = torch.randn(64, 4096, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    out = oracle.vllm_rms_norm(x, w, 1e-6)
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * w
    d = (out.float() - ref.float()).abs()
    assert torch.all(d <= 2 * 2.0 ** -8 * ref.float().abs() + 1e-6)
