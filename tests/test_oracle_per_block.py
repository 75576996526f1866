"""Pins of the oracle's per-group quantization (vLLM ``_C::rms_norm_per_block_quant``,
op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:92-126,194-270,
layernorm_utils.cuh:283-393,455-535).

The reference ships no test for this op, so the pins are:
  - reduction to the per-token op: with one group per row (H == group_size) the scales and codes
    equal the per-token oracle's (a separately pinned function) bit for bit, int8 and fp8;
  - consistency across groupings: y is the same for every group size, so every group-64 scale
    is at most the group-128 scale of the pair it belongs to, and the larger of the pair equals
    it; the per-token scale is the largest group scale;
  - a torch restatement of every rounding point, both scale layouts;
  - invariants: each group's absmax element codes to +-127 (int8) or +-448 (fp8), dequantised
    error within half a step.
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


def _inputs(T, H, dtype, seed, res=True):
    g = _gen(seed)
    x = (torch.randn(T, H, generator=g) * torch.logspace(-1, 1, H)[None, :]).to(dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    r = torch.randn(T, H, generator=g).to(dtype) if res else None
    return x, w, r


@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_one_group_per_row_is_the_per_token_op(G, qdt, dtype):
    x, w, r = _inputs(50, G, dtype, 1)
    q, s, ro = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, residual=r)
    q2, s2, ro2 = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, residual=r)
    assert torch.equal(s.view(-1), s2.view(-1))
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(ro, ro2)


def test_scale_ub_matches_per_token_op_with_one_group():
    x, w, r = _inputs(40, 64, torch.bfloat16, 2)
    q, s, _ = oracle.rms_norm_per_block_quant(x, w, 1e-6, torch.float8_e4m3fn, 64,
                                              scale_ub=0.02, residual=r)
    q2, s2, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.float8_e4m3fn,
                                                        scale_ub=0.02, residual=r)
    assert torch.equal(s.view(-1), s2.view(-1))
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_groupings_are_consistent(qdt):
    x, w, r = _inputs(30, 1024, torch.bfloat16, 3)
    _, s64, _ = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, 64, residual=r)
    _, s128, _ = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, 128, residual=r)
    _, st, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, residual=r)
    pairs = s64.view(30, 8, 2)
    assert torch.equal(pairs.amax(-1), s128)
    assert torch.equal(s128.amax(-1, keepdim=True), st)


@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("transposed", [False, True])
def test_torch_restatement(G, qdt, transposed):
    T, H = 24, 768
    x, w, r = _inputs(T, H, torch.bfloat16, 4)
    q, s, ro = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, residual=r,
                                               is_scale_transposed=transposed)
    a = x.float() + r.float()
    rho = _rho(a, 1e-6)
    y = ((a * rho).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16).float()
    yg = y.view(T, H // G, G)
    A = yg.abs().amax(-1, keepdim=True)
    if qdt == torch.int8:
        s_ref = torch.maximum(A / 127.0, torch.tensor(np.finfo(np.float32).eps))
        q_ref = torch.round(yg * (torch.ones_like(s_ref) / s_ref)).clamp(-128, 127)
        assert torch.equal(q, q_ref.to(torch.int8).view(T, H))
    else:
        s_ref = torch.maximum(A / 448.0, torch.tensor(1.0, dtype=torch.float32) / (448 * 512))
        q_ref = (yg / s_ref).clamp(-448, 448).to(torch.float8_e4m3fn).view(T, H)
        assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))
    s_ref = s_ref.view(T, H // G)
    assert torch.equal(s, s_ref.t().contiguous() if transposed else s_ref)
    assert torch.equal(ro, a.to(torch.bfloat16))


@pytest.mark.parametrize("qdt,top", [(torch.int8, 127), (torch.float8_e4m3fn, 448.0)])
def test_invariants(qdt, top):
    T, H, G = 16, 2048, 128
    x, w, _ = _inputs(T, H, torch.float32, 5, res=False)
    q, s, _ = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G)
    qf = q.float().view(T, H // G, G)
    assert torch.all(qf.abs().amax(-1) == top)
    if qdt == torch.int8:
        a = x.double()
        y = a * _rho(x.float(), 1e-6).double() * w.double()
        err = (qf.double() * s.double().unsqueeze(-1) - y.view(T, H // G, G)).abs()
        assert torch.all(err <= s.double().unsqueeze(-1) * 0.5 + 1e-6 * y.abs().view(T, H // G, G))
