"""The CPU legs and inputs of bench.py: the vectorized torch restatement (the `cpu_torch` figure)
equals the C oracle bit for bit for both operators it restates, and the seeded inputs follow the
stated recipe (the same builder feeds the GPU parity tests, so the benchmarked bits are the
parity-checked bits)."""

import torch

import bench
import oracle


def _rows(seed, T, H):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    x[:, :40] *= 20.0  # outlier channels, as in the headline workload
    x = x.to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    return x, r, w


def test_torch_cpu_leg_equals_the_oracle():
    x, r, w = _rows(3, 64, 4096)
    q, s, res = bench.torch_cpu_add_norm_int8(x, r, w, 1e-5)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-5, torch.int8,
                                                                  residual=r)
    assert torch.equal(res, r_ref)
    assert torch.equal(s.view(-1), s_ref.view(-1))
    assert torch.equal(q, q_ref)
    # without a residual (cfg1)
    q, s, res = bench.torch_cpu_add_norm_int8(x, None, w, 1e-6)
    q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8)
    assert res is None and torch.equal(q, q_ref) and torch.equal(s.view(-1), s_ref.view(-1))


def test_torch_cpu_leg_of_the_mcoplib_operator_equals_the_oracle():
    # the benchmarked surface is mcoplib's own operator (1.5e-6 scale floor, codes +-127)
    x, r, w = _rows(4, 64, 8192)
    x[3].zero_()
    r[3].zero_()  # a zero row: the floor decides the scale
    q, s, res = bench.torch_cpu_add_norm_int8(x, r, w, 1e-5, floor=1.5e-6, lo=-127)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-5, residual=r)
    assert torch.equal(res, r_ref)
    assert torch.equal(s.view(-1), s_ref.view(-1))
    assert s[3].item() == torch.tensor(1.5e-6, dtype=torch.float32).item()
    assert torch.equal(q, q_ref)


def test_config_inputs_follow_the_recipe():
    c = bench.config_inputs("cfg3")
    x, r, w = c["x"], c["r"], c["w"]
    assert x.shape == r.shape == (8192, 8192) and w.shape == (8192,) and c["eps"] == 1e-5
    assert x.dtype == r.dtype == w.dtype == torch.bfloat16
    # 82 outlier channels: column RMS ~20 there, ~1 elsewhere
    col = x.float().pow(2).mean(0).sqrt()
    assert int((col > 10).sum()) == 82 and float(col[col < 10].max()) < 1.2
    g = torch.Generator().manual_seed(3)
    assert set(torch.nonzero(col > 10).view(-1).tolist()) == \
        set(torch.randperm(8192, generator=g)[:82].tolist())
    # residual and weight statistics
    assert abs(float(r.float().std()) - 1) < 0.01 and abs(float(w.float().mean()) - 1) < 0.01
    c4 = bench.config_inputs("cfg4")
    assert c4["r"] is None and c4["sm"].dtype == torch.float32
    assert 0.5 <= float(c4["sm"].min()) and float(c4["sm"].max()) <= 2.0
    # deterministic: the same bits every time
    assert torch.equal(bench.config_inputs("cfg5-decode4")["x"],
                       bench.config_inputs("cfg5-decode4")["x"])
