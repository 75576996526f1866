"""The CPU legs of bench.py compute the benchmarked operation: its vectorized torch restatement
(the `cpu_torch` figure) equals the C oracle bit for bit, residual, scales and codes."""

import torch

import bench
import oracle


def test_torch_cpu_leg_equals_the_oracle():
    g = torch.Generator().manual_seed(3)
    T, H = 64, 4096
    x = torch.randn(T, H, generator=g)
    x[:, :40] *= 20.0  # outlier channels, as in the headline workload
    x = x.to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    q, s, res = bench.torch_cpu_add_norm_int8(x, r, w, 1e-5)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-5, torch.int8,
                                                                  residual=r)
    assert torch.equal(res, r_ref)
    assert torch.equal(s.view(-1), s_ref.view(-1))
    assert torch.equal(q, q_ref)
