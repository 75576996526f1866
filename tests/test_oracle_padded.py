"""Pins of the oracle's padded wire-format op (mcoplib
``fused_add_rms_norm_dynamic_per_token_quant_padding_output``,
op/fused_add_layernorm_per_token_quant_padding_output.cu:181-416, wrapper
mcoplib/custom_ops.py:7-27).

The reference's own test (unit_test/test_fused_add_rms_norm_custom.py) asserts nothing; its
intended comparison -- residual against x + residual, output_rms against torch.rms_norm -- is run
here at a bf16 tolerance.  The rest pins the layout by construction (codes at bytes [0, H), the
fp32 scale at [H, H+4), untouched bytes after), both rounding chains through an independent torch
restatement, and the quantization invariants.
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


def _inputs(T, H, seed):
    g = _gen(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.randn(H, generator=g).to(torch.bfloat16)  # the reference test's N(0, 1) weight
    return x, r, w


@pytest.mark.parametrize("T,H,pad", [(3, 7168, 3840), (5, 4096, 2050), (4, 1030, 517)])
def test_layout(T, H, pad):
    x, r, w = _inputs(T, H, 1)
    padded, ro, rms, q, s = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6, fill=0xA5)
    assert padded.shape == (T, 2 * pad)
    assert torch.equal(padded[:, :H].view(torch.int8), q)
    assert torch.equal(padded[:, H:H + 4].contiguous().view(torch.float32), s)
    assert torch.all(padded[:, H + 4:] == 0xA5)


@pytest.mark.parametrize("T,H", [(16, 7168), (16, 4096), (9, 1030)])
def test_torch_restatement(T, H):
    x, r, w = _inputs(T, H, 2)
    eps = 1e-6
    _, ro, rms, q, s = oracle.add_rms_norm_quant_padded(x, r, w, H // 2 + 8, eps)
    a = x.float() + r.float()
    rho = _rho(a, eps)
    rb = a.to(torch.bfloat16)
    wf = w.float()
    if H == 7168:  # the reference's fp32 chain
        p = a * wf
        A = p.abs().amax(-1, keepdim=True)
        y = p * rho
        rms_ref = y.to(torch.bfloat16)
    else:          # the bf16-rounded chain
        A = (rb.float() * wf).to(torch.bfloat16).float().abs().amax(-1, keepdim=True)
        rms_ref = ((rb.float() * rho).to(torch.bfloat16).float() * wf).to(torch.bfloat16)
        y = rms_ref.float()
    s_ref = torch.maximum((A * rho) / 127.0, torch.tensor(np.finfo(np.float32).eps))
    inv = torch.ones_like(s_ref) / s_ref
    q_ref = torch.round(y * inv).clamp(-127, 127).to(torch.int8)
    assert torch.equal(ro, rb)
    assert torch.equal(s, s_ref)
    assert torch.equal(rms, rms_ref)
    assert torch.equal(q, q_ref)


@pytest.mark.parametrize("H", [7168, 4096])
def test_reference_test_intent(H):
    # unit_test/test_fused_add_rms_norm_custom.py:23-27,43-44: sum = x + residual,
    # rms = torch.rms_norm(sum, weight, eps); batch 1, N(0, 1) weight
    x, r, w = _inputs(1, H, 3)
    _, ro, rms, _, _ = oracle.add_rms_norm_quant_padded(x, r, w, 3840 if H == 7168 else 2100,
                                                         1e-6)
    total = x + r
    ref = torch.rms_norm(total.float(), total.shape, weight=w.float().unsqueeze(0), eps=1e-6)
    assert torch.equal(ro, total)
    # two bf16 roundings apart at most (the reference's chains round at different points)
    err = (rms.float() - ref).abs()
    assert torch.all(err <= 2 * 2.0 ** -8 * ref.abs() + 1e-6)


@pytest.mark.parametrize("H", [7168, 5120])
def test_invariants(H):
    T = 32
    x, r, w = _inputs(T, H, 4)
    x = (x.float() * torch.logspace(-2, 2, T)[:, None]).to(torch.bfloat16)
    _, _, rms, q, s = oracle.add_rms_norm_quant_padded(x, r, w, H, 1e-6)
    assert q.abs().max().item() <= 127 and q.min().item() >= -127
    top = q.gather(-1, rms.float().abs().argmax(-1, keepdim=True)).int().abs()
    assert torch.all(top >= 126)
    deq = q.double() * s.double()
    err = (deq - rms.double()).abs()
    assert torch.all(err <= 0.5 * s.double() * (1 + 1e-5) + 0.02 * rms.double().abs())


def test_zero_row_floor():
    x = torch.zeros(2, 7168, dtype=torch.bfloat16)
    r = torch.zeros_like(x)
    w = torch.ones(7168, dtype=torch.bfloat16)
    _, _, rms, q, s = oracle.add_rms_norm_quant_padded(x, r, w, 3840, 1e-6)
    assert torch.all(s == float(np.finfo(np.float32).eps))
    assert torch.count_nonzero(q) == 0 and torch.count_nonzero(rms.float()) == 0
