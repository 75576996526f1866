"""Pins of the oracle's mcoplib ``rms_norm_dynamic_per_token_quant_custom`` restatement
(op/rms_norm_dynamic_per_token_quant.cu:52-285, kernel/rms_norm_vllm.cuh:330-454).

  - at H == 7168 the reference runs a kernel whose chain (p = a * w in fp32, scale from
    max|p| * rsqrt, codes of p * rsqrt) is the same as the "opt" kernel of the padded wire-format
    op (op/fused_add_layernorm_per_token_quant_padding_output.cu:181-283): the two restatements,
    written separately, must agree bit for bit on codes, scales and residual;
  - elsewhere the chain is vLLM's (pinned separately) with a 1.5e-6 scale floor and codes
    clamped to [-127, 127]: identical to the vLLM restatement whenever neither bites, and the
    floor / clamp themselves by closed forms;
  - the reference test's intended comparison (unit_test/test_rms_norm_custom.py:21-47:
    torch.rms_norm, then absmax/127 and round) within one code and a bf16 ulp of scale;
  - a torch restatement of both chains.
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


def _inputs(T, H, dtype, seed):
    g = _gen(seed)
    x = (torch.randn(T, H, generator=g) * 2).to(dtype)
    r = torch.randn(T, H, generator=g).to(dtype)
    w = torch.randn(H, generator=g).to(dtype)
    return x, r, w


def test_7168_chain_equals_the_padded_op_chain():
    x, r, w = _inputs(24, 7168, torch.bfloat16, 1)
    q, s, ro = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    _, ro2, _, q2, s2 = oracle.add_rms_norm_quant_padded(x, r, w, 3840, 1e-6)
    assert torch.equal(q, q2) and torch.equal(s, s2) and torch.equal(ro, ro2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("H", [4096, 1033, 7176])
def test_generic_chain_equals_vllm_chain_when_floor_and_clamp_are_idle(dtype, H):
    x, r, w = _inputs(32, H, dtype, 2)
    q, s, ro = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    q2, s2, ro2 = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8, residual=r)
    assert torch.equal(q, q2) and torch.equal(s, s2) and torch.equal(ro, ro2)


def test_generic_floor_and_clamp():
    H = 256
    x = torch.zeros(2, H, dtype=torch.bfloat16)
    x[1, 3] = 1.0
    w = torch.ones(H, dtype=torch.bfloat16)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6)
    # zero row: the floor (1.5e-6 as the nearest float); vLLM's floor is FLT_EPSILON
    assert s[0].item() == float(np.float32(1.5e-6))
    assert torch.count_nonzero(q[0]) == 0
    # a scale bound below the row maximum: codes saturate at +-127 (vLLM's range is -128..127)
    # y = b(b(x * rho)) with rho = 1/sqrt(32.3125): -1.40625, 1.40625, 0.17578125, 0.087890625;
    # s = 0.127 / 127 = 0.001, so y / s = -1406, 1406, 175.8, 87.9
    x2 = torch.tensor([[-8.0, 8.0, 1.0, 0.5]], dtype=torch.bfloat16)
    q2, s2, _ = oracle.rms_norm_dynamic_per_token_quant_custom(
        x2, torch.ones(4, dtype=torch.bfloat16), 0.0, scale_ub=0.127)
    assert s2.item() == float(np.float32(np.float32(0.127) / np.float32(127.0)))
    assert q2.tolist() == [[-127, 127, 127, 88]]


@pytest.mark.parametrize("H", [7168, 4096])
def test_torch_restatement(H):
    x, r, w = _inputs(16, H, torch.bfloat16, 3)
    q, s, ro = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6, residual=r)
    a = x.float() + r.float()
    rho = _rho(a, 1e-6)
    if H == 7168:
        p = a * w.float()
        A = p.abs().amax(-1, keepdim=True)
        s_ref = torch.maximum((A * rho) / 127.0, torch.tensor(np.finfo(np.float32).eps))
        t = p * rho
    else:
        y = ((a * rho).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16).float()
        A = y.abs().amax(-1, keepdim=True)
        s_ref = torch.maximum(A / 127.0, torch.tensor(np.float32(1.5e-6)))
        t = y
    q_ref = torch.round(t * (torch.ones_like(s_ref) / s_ref)).clamp(-127, 127).to(torch.int8)
    assert torch.equal(s, s_ref)
    assert torch.equal(q, q_ref)
    assert torch.equal(ro, a.to(torch.bfloat16))


def test_reference_test_intent_7168():
    # torch.rms_norm(bf16) then absmax / 127 and round (the reference test's quantize helper)
    g = _gen(4)
    x = torch.randn(1, 7168, generator=g).to(torch.bfloat16)
    w = torch.randn(7168, generator=g).to(torch.bfloat16)
    q, s, _ = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-6)
    y = torch.rms_norm(x.float(), x.shape, weight=w.float().unsqueeze(0), eps=1e-6)
    y = y.to(torch.bfloat16).float()
    sc = y.abs().max() / 127.0
    ref = torch.clamp(torch.round(y / sc), -128, 127)
    assert abs(s.item() / sc.item() - 1) < 2 ** -7
    assert (q.float() - ref).abs().max() <= 1
