"""The torch.ops._C operators under tracing: their Meta kernels accept meta tensors (CPU test),
and a function calling them compiles with torch.compile (aot_eager: functionalization of the
mutating schemas, no code generation) and matches the eager results bit for bit (GPU test)."""

import pytest
import torch

import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)


def test_meta_kernels_accept_meta_tensors():
    m = torch.device("meta")
    x = torch.empty(4, 64, dtype=torch.bfloat16, device=m)
    w = torch.empty(64, dtype=torch.bfloat16, device=m)
    r = torch.empty_like(x)
    q = torch.empty(4, 64, dtype=torch.int8, device=m)
    s = torch.empty(4, 1, dtype=torch.float32, device=m)
    assert torch.ops._C.fused_add_rms_norm(x, r, w, 1e-6) is None
    assert torch.ops._C.rms_norm(torch.empty_like(x), x, w, 1e-6) is None
    assert torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w, s, 1e-6, None, r) is None
    assert torch.ops._C.rms_norm_per_block_quant(q, x, w, torch.empty(4, 1, device=m), 1e-6,
                                                 None, r, 64, False) is None
    assert torch.ops._C.dynamic_scaled_int8_quant(q, x, s, None) is None
    assert torch.ops._C.dynamic_per_token_scaled_fp8_quant(
        torch.empty(4, 64, dtype=torch.float8_e4m3fn, device=m), x, s, None) is None


@pytest.mark.gpu
def test_torch_compile_aot_eager_matches_eager():
    dev = "cuda:0"
    g = torch.Generator().manual_seed(5)
    x0 = torch.randn(33, 4096, generator=g).to(torch.bfloat16).to(dev)
    r0 = torch.randn(33, 4096, generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(dev)

    def step(x, r):
        q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
        s = torch.empty(x.shape[0], 1, dtype=torch.float32, device=x.device)
        torch.ops._C.rms_norm_dynamic_per_token_quant(q, x, w, s, 1e-6, None, r)
        torch.ops._C.fused_add_rms_norm(x, r, w, 1e-6)
        return q, s

    xe, re_ = x0.clone(), r0.clone()
    qe, se = step(xe, re_)
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    xc, rc = x0.clone(), r0.clone()
    qc, sc = compiled(xc, rc)
    torch.cuda.synchronize()
    assert torch.equal(qc, qe) and torch.equal(sc, se)
    assert torch.equal(xc, xe) and torch.equal(rc, re_)
