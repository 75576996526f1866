"""The reference's own hot-path tests, restated against this implementation on the GPU.

- unit_test/test_scale_dynamic_quant.py: shapes, known answers, edge cases and the seeded
  comparison with its CPU loop oracle (codes atol 1, scales rtol 1e-5);
- unit_test/test_fused_rms_norm_dq.py: the comparison it intends (it returns before calling the
  op): torch.ops._C.rms_norm_dynamic_per_token_quant against vLLM's RMSNorm.forward_native plus
  per-token int8 quantization, over its shape list, with and without residual;
- unit_test/test_rms_norm_custom.py: mcoplib.custom_ops.rms_norm_dynamic_per_token_quant at
  hidden 7168 (its dedicated one-pass kernel in the reference);
- unit_test/test_rms_norm.py: the divide-by-rsqrt convention of mcoplib's norms, asserted with
  assert_close(atol=rtol=1e-5), here through after_norm of op.rms_norm_dynamic_per_token_quant.
"""

import pytest
import torch

import oracle

# the reference's own import lines (README.md:149,155; unit_test/test_rms_norm_custom.py:2)
from mcoplib import op as ops
import mcoplib._C  # noqa: F401
from mcoplib.custom_ops import rms_norm_dynamic_per_token_quant
from gpu_util import DEV, say

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------ test_scale_dynamic_quant.py
def _loop_oracle(h, smooth):
    flat = h.reshape(-1, h.shape[-1]).float()
    q = torch.zeros_like(flat, dtype=torch.int8)
    s = torch.zeros(flat.shape[0], dtype=torch.float32, device=h.device)
    for t in range(flat.shape[0]):
        d = flat[t] * smooth
        m = torch.abs(d).max().item()
        sc = m / 127.0 if m > 0 else 1.0
        s[t] = sc
        q[t] = torch.round(d / sc).clamp(-128, 127).to(torch.int8)
    return q.view(h.shape), s


def test_scale_dynamic_quant_reference_suite():
    torch.manual_seed(13)
    h = torch.randn(2, 128, 768, device=DEV, dtype=torch.bfloat16)
    sm = torch.ones(768, device=DEV, dtype=torch.float32)
    q, s = ops.scale_dynamic_quant(h, sm, torch.int8)
    assert q.shape == (2, 128, 768) and s.shape == (2 * 128,)
    qr, sr = _loop_oracle(h, sm)
    assert torch.allclose(q.cpu(), qr.cpu(), rtol=0, atol=1)
    assert torch.allclose(s.cpu(), sr.cpu(), rtol=1e-5)

    h = torch.tensor([[[1.0, 2.0, 3.0, 4.0], [4.0, 3.0, 2.0, 1.0]]], device=DEV,
                     dtype=torch.bfloat16)
    sm = torch.tensor([1.0, 1.0, 2.0, 2.0], device=DEV, dtype=torch.float32)
    q, s = ops.scale_dynamic_quant(h, sm, torch.int8)
    assert abs(s[0].item() - 8.0 / 127) < 1e-5
    assert abs(s[1].item() - 4.0 / 127) < 1e-5

    q, s = ops.scale_dynamic_quant(torch.zeros(1, 4, 8, device=DEV, dtype=torch.bfloat16),
                                  torch.ones(8, device=DEV), torch.int8)
    assert torch.all(q == 0)
    q, s = ops.scale_dynamic_quant(torch.ones(1, 4, 8, device=DEV, dtype=torch.bfloat16) * 1000.0,
                                  torch.ones(8, device=DEV), torch.int8)
    assert torch.all(torch.abs(q) <= 127)
    for shape in [(1, 1, 768), (4, 512, 768), (1, 2048, 4096), (8, 128, 1024)]:
        h = torch.randn(*shape, device=DEV, dtype=torch.bfloat16)
        q, s = ops.scale_dynamic_quant(h, torch.ones(shape[-1], device=DEV), torch.int8)
        assert q.shape == shape and s.shape == (shape[0] * shape[1],)
    h = torch.randn(2, 64, 256, device=DEV, dtype=torch.bfloat16) * 1e-7
    q, s = ops.scale_dynamic_quant(h, torch.ones(256, device=DEV), torch.int8)
    assert torch.all(torch.isfinite(s)) and torch.all(s > 0)
    with pytest.raises(RuntimeError, match="Only support bfloat16"):
        ops.scale_dynamic_quant(h.float(), torch.ones(256, device=DEV), torch.int8)


# ------------------------------------------------------------ test_fused_rms_norm_dq.py
VEC_HIDDEN_SIZES = range(1024, 1030)
NUM_TOKENS_HIDDEN_SIZES = [
    *[(1, i) for i in [1, 64, *VEC_HIDDEN_SIZES, 5120, 5137]],
    *[(83, i) for i in [1, 1033, 2048, 5120]],
    *[(2048, i) for i in [1, 64, *VEC_HIDDEN_SIZES, 5137]],
    *[(4096, i) for i in [1, 64, 5137]],
]
EPS = 1e-6


def _forward_native(x, weight, residual):
    orig = x.dtype
    xf = x.to(torch.float32)
    if residual is not None:
        xf = xf + residual.to(torch.float32)
        residual = xf.to(orig)
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(var + EPS)
    return xf.to(orig) * weight, residual


def _per_token_int8(y):
    yf = y.float()
    A = yf.abs().amax(dim=-1, keepdim=True)
    s = A / 127.0
    return torch.round(yf * (127.0 / A)).clamp(-128, 127).to(torch.int8), s


@pytest.mark.parametrize("num_tokens,hidden_size", NUM_TOKENS_HIDDEN_SIZES)
@pytest.mark.parametrize("add_residual", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float])
@torch.inference_mode()
def test_fused_rms_norm_dq_reference(num_tokens, hidden_size, add_residual, dtype):
    """Tolerances of the reference test (scales allclose, codes atol 1, residual allclose).  Its
    oracle normalizes with torch's mean/rsqrt; rows where that moves the normalized absmax by one
    bf16 ulp (at most 1% of rows) get a scale one ulp apart and are excluded from the code check."""
    torch.random.manual_seed(0)
    torch.cuda.manual_seed(0)
    w = torch.empty(hidden_size, dtype=dtype, device=DEV).normal_(mean=1.0, std=0.1)
    scale = 1 / hidden_size
    x = torch.randn(num_tokens, hidden_size, dtype=dtype, device=DEV) * scale
    residual = torch.randn_like(x) * scale if add_residual else None
    ref_out, ref_res = _forward_native(x, w, None if residual is None else residual.clone())
    ref_q, ref_s = _per_token_int8(ref_out)
    ops_res = None if residual is None else residual.clone()
    out = torch.empty_like(x, dtype=torch.int8)
    scales = torch.empty((x.numel() // x.shape[-1], 1), device=DEV, dtype=torch.float32)
    torch.ops._C.rms_norm_dynamic_per_token_quant(out, x, w, scales, EPS, None, ops_res)
    # rows whose normalized values are all zero (x == -residual, frequent at hidden 1): the test
    # oracle gives scale 0, the kernel the int8 scale floor FLT_EPSILON; both code zeros
    zero = (ref_s == 0).flatten()
    assert torch.all(scales.flatten()[zero] == torch.finfo(torch.float32).eps)
    assert torch.all(out[zero] == 0)
    close = (torch.isclose(ref_s, scales).flatten() & ~zero) | zero
    assert close.float().mean() >= 0.99
    nz = ~zero
    assert ((scales.flatten()[nz] - ref_s.flatten()[nz]).abs() / ref_s.flatten()[nz]).max() <= 2 ** -6
    rows = (close & nz).nonzero().flatten()
    assert torch.allclose(ref_q[rows].float(), out[rows].float(), atol=1)
    if add_residual:
        assert torch.allclose(ref_res, ops_res)


# ------------------------------------------------------------ test_rms_norm_custom.py
def test_rms_norm_custom_7168():
    hidden, tokens = 7168, 1
    x = torch.randn(tokens, hidden, dtype=torch.bfloat16, device=DEV)
    res = torch.randn(tokens, hidden, dtype=torch.bfloat16, device=DEV)
    w = torch.randn(hidden, dtype=torch.bfloat16, device=DEV)
    res_in = res.clone()
    q, s = rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8, None, res)
    ref_res = (x.float() + res_in.float()).to(torch.bfloat16)
    assert torch.equal(res, ref_res)
    y = torch.rms_norm(ref_res.float(), (hidden,), None, 1e-6).to(torch.bfloat16) * w
    yq, ys = _per_token_int8(y)
    assert torch.allclose(s, ys, rtol=2 ** -6)
    assert (q.float() - yq.float()).abs().max() <= 2
    # and exactly the reference kernel's own (fp32) chain at this width
    q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant_custom(
        x.cpu(), w.cpu(), 1e-6, residual=res_in.cpu())
    assert torch.equal(q.cpu(), q_ref) and torch.equal(s.cpu(), s_ref)


# ------------------------------------------------------------ test_rms_norm.py
@pytest.mark.parametrize("m,n", [(4096, 4096), (512, 7168)])
def test_rms_div_convention(m, n):
    """The reference's norms divide by rsqrt(ms + eps) (unit_test/test_rms_norm.py:24-38), as
    the literal form of op.rms_norm_dynamic_per_token_quant does."""
    say(f"rms_div m={m} n={n}")
    torch.manual_seed(42)
    x = torch.randn(m, n, dtype=torch.float32, device=DEV)
    r = torch.randn(m, n, dtype=torch.float32, device=DEV)
    w = torch.randn(n, dtype=torch.float32, device=DEV)
    after_res_ref = x + r
    ms = torch.mean(after_res_ref * after_res_ref, dim=-1, keepdim=True)
    norm_ref = after_res_ref / torch.rsqrt(ms + 1e-5) * w
    out = torch.empty(m, n, dtype=torch.int8, device=DEV)
    scales = torch.empty(m, dtype=torch.float32, device=DEV)
    after_res = torch.empty_like(x)
    after_norm = torch.empty_like(x)
    ops.rms_norm_dynamic_per_token_quant(out, x, w, torch.ones(n, device=DEV), scales, 1e-5,
                                        after_res, after_norm, r)
    torch.testing.assert_close(norm_ref, after_norm, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(after_res_ref.reshape(-1), after_res.reshape(-1), atol=1e-5,
                               rtol=1e-5)
