"""The operators can be captured in a HIP graph (they only enqueue kernels on torch's current
stream, allocate nothing and never synchronize): each replay, with fresh inputs copied into the
captured buffers and eager work in between, must equal the eager result."""

import pytest
import torch

import mcoplib_amd._C  # noqa: F401
from mcoplib_amd import op
from gpu_util import DEV, randn, weight, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H", [(64, 5120), (4, 131072)])  # register and multi-pass kernels
def test_graph_replays_match_eager(T, H):
    say(f"graph capture: add + rmsnorm + int8, then fused_add_rms_norm, T={T} H={H}")
    x = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    r = torch.empty_like(x)
    w = weight(H, 1, torch.bfloat16).to(DEV)
    q = torch.empty(T, H, dtype=torch.int8, device=DEV)
    s = torch.empty(T, 1, dtype=torch.float32, device=DEV)
    x2 = torch.empty_like(x)
    r2 = torch.empty_like(x)
    x.copy_(randn((T, H), 2, torch.bfloat16))
    r.copy_(randn((T, H), 3, torch.bfloat16))
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            op.rms_norm_dynamic_per_token_quant_custom(q, x, w, s, 1e-6, None, r)
            x2.copy_(x)
            r2.copy_(r)
            torch.ops._C.fused_add_rms_norm(x2, r2, w, 1e-6)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        xi = randn((T, H), 10 + rep, torch.bfloat16).to(DEV)
        ri = randn((T, H), 20 + rep, torch.bfloat16).to(DEV)
        x.copy_(xi)
        r.copy_(ri)
        g.replay()
        # eager reference on separate buffers
        qe = torch.empty_like(q)
        se = torch.empty_like(s)
        re_ = ri.clone()
        op.rms_norm_dynamic_per_token_quant_custom(qe, xi, w, se, 1e-6, None, re_)
        xe2, re2 = xi.clone(), re_.clone()
        torch.ops._C.fused_add_rms_norm(xe2, re2, w, 1e-6)
        torch.cuda.synchronize()
        assert torch.equal(q, qe) and torch.equal(s, se) and torch.equal(r, re_)
        assert torch.equal(x2, xe2) and torch.equal(r2, re2)
        _ = (xi * 2).sum().item()  # unrelated eager work between replays
