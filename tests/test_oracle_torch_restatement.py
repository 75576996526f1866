"""Bit-level cross-check of the C oracle against an independent restatement in torch.

The restatement follows the reference kernels operation by operation with torch's own dtype
conversions and arithmetic (where the C oracle uses hand-written bit manipulation), and takes the
row statistic from torch's float64 sum.  Every rounding point of the reference (the bf16 residual,
b(a*rho), b(. * w), the fp32 scale and its reciprocal, the code rounding) must then agree bit for
bit, so a dropped rounding step, a wrong operand or an index mistake in either implementation
fails here.  Reference lines: op/vllm/layernorm_kernels.cu:118-143 with
op/vllm/type_convert.cuh:104-165 (H1); op/vllm/quantization/fused_kernels/layernorm_utils.cuh:
245-276, 436-447, 503-531 and fused_layernorm_dynamic_per_token_quant.cu:37 (H2);
op/fused_rms_norm_dq.cu:77-94, 136-154, 176-182 (H4)."""

import numpy as np
import pytest
import torch

import oracle


def _rho(a: torch.Tensor, eps: float) -> torch.Tensor:
    """1/sqrt(fl32(sum a^2)/H + eps) with each fp32 step rounded once (computed in float64,
    rounded to float32 after each operation; exact for these operations)."""
    H = a.shape[-1]
    ss = (a.double() * a.double()).sum(-1, keepdim=True).float()
    ms = (ss.double() / float(np.float32(H))).float()
    v = ms + torch.tensor(eps, dtype=torch.float32)
    r = torch.sqrt(v.double()).float()
    return (1.0 / r.double()).float()


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_h1_restatement(dtype):
    g = _gen(11)
    x = torch.randn(64, 1000, generator=g).to(dtype)
    r = torch.randn(64, 1000, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(1000, generator=g)).to(dtype)
    xo, ro = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    z = (x.float() + r.float()).to(dtype)            # packed add: one rounding of the sum
    rho = _rho(z.float(), 1e-6)                        # variance of the rounded residual
    y = (z.float() * rho).to(dtype).float() * w.float()
    assert torch.equal(ro, z)
    assert torch.equal(xo, y.to(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("with_res", [False, True])
def test_h2_restatement(dtype, qdt, with_res):
    g = _gen(12)
    x = (torch.randn(96, 777, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(777, generator=g)).to(dtype)
    r = torch.randn(96, 777, generator=g).to(dtype) if with_res else None
    q, s, ro = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, residual=r)
    a = x.float() + (r.float() if with_res else 0.0)  # unrounded sum
    rho = _rho(a, 1e-6)
    y = ((a * rho).to(dtype).float() * w.float()).to(dtype).float()
    A = y.abs().amax(-1, keepdim=True)
    if qdt == torch.int8:
        s_ref = torch.maximum(A / 127.0, torch.tensor(np.finfo(np.float32).eps))
        inv = 1.0 / s_ref
        q_ref = torch.round(y * inv).clamp(-128, 127).to(torch.int8)
        assert torch.equal(q, q_ref)
    else:
        s_ref = torch.maximum(A / 448.0, torch.tensor(1.0, dtype=torch.float32) / (448.0 * 512.0))
        q_ref = (y / s_ref).clamp(-448, 448).to(torch.float8_e4m3fn)
        assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))
    assert torch.equal(s, s_ref)
    if with_res:
        assert torch.equal(ro, a.to(dtype))


@pytest.mark.parametrize("dtype,wdt,sdt", [(torch.bfloat16, torch.bfloat16, torch.bfloat16),
                                           (torch.bfloat16, torch.bfloat16, torch.float32),
                                           (torch.float16, torch.float32, torch.float32),
                                           (torch.float32, torch.float32, torch.float32)])
@pytest.mark.parametrize("standard", [False, True])
def test_h4_restatement(dtype, wdt, sdt, standard):
    g = _gen(13)
    x = (torch.randn(64, 900, generator=g) * 3).to(dtype)
    r = torch.randn(64, 900, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(900, generator=g)).to(wdt)
    sm = (0.5 + 1.5 * torch.rand(900, generator=g)).to(sdt)
    for qdt in (torch.int8, torch.float8_e4m3fn):
        q, s, ar, an = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, r, standard)
        a = x.float() + r.float()
        rho = _rho(a, 1e-6)
        at = a.to(dtype).float()                       # after_res, re-read by the later passes
        n = at * rho if standard else at / rho
        u = n * w.float()
        v = u * sm.float()
        A = v.abs().amax(-1)
        s_ref = A / (127.0 if qdt == torch.int8 else 448.0)
        inv = torch.where(A > 0, 1.0 / s_ref, torch.zeros_like(s_ref))
        t = v * inv[:, None]
        assert torch.equal(ar, a.to(dtype))
        assert torch.equal(an, u.to(dtype))
        assert torch.equal(s, s_ref)
        if qdt == torch.int8:
            assert torch.equal(q, torch.round(t).clamp(-127, 127).to(torch.int8))
        else:  # fp8 (this library's extension) divides by the scale
            t8 = torch.where(A[:, None] > 0, v / s_ref[:, None], torch.zeros_like(v))
            assert torch.equal(q.view(torch.uint8),
                               t8.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8))
