"""The no-allocation entry point, mcop_rms_norm_dynamic_per_token_quant_noalloc, through the C ABI
against the allocating mcop_rms_norm_dynamic_per_token_quant on the same inputs: identical codes,
scales and residual (residual bit-exact, scales within 1e-6 relative, codes
within one step on at most 1e-4 of elements; both run the same kernels, so they agree bit for
bit), on two calls in a row, the second with a smaller input, for rows that take the split-row
kernel (whose workspace this entry point keeps in its static scratch) and for rows that fit one
workgroup; and a traced child process that shows the split launches using the scratch."""

import os
import subprocess
import sys

import pytest
import torch

from conftest import ROOT
from mcoplib_amd import _lib
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, gen, say

pytestmark = pytest.mark.gpu

_DT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.int8: 3,
       torch.float8_e4m3fn: 4}


def _inputs(T, H, dtype, seed, res):
    g = gen(seed)
    x = (torch.randn(T, H, generator=g) * 2).to(dtype).to(DEV)
    r = torch.randn(T, H, generator=g).to(dtype).to(DEV) if res else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype).to(DEV)
    return x, r, w


def _call(fn, x, r, w, qdt, ub):
    T, H = x.shape
    q = torch.empty(T, H, dtype=qdt, device=DEV)
    s = torch.empty(T, 1, device=DEV)
    rr = None if r is None else r.clone()
    ubt = None if ub is None else torch.tensor([ub], device=DEV)
    rc = fn(q.data_ptr(), _DT[qdt], s.data_ptr(), x.data_ptr(), w.data_ptr(),
            None if ubt is None else ubt.data_ptr(), None if rr is None else rr.data_ptr(),
            T, H, _DT[x.dtype], 1e-6, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, _lib.lib.mcop_last_error().decode()
    return q.cpu(), s.cpu(), None if rr is None else rr.cpu()


@pytest.mark.parametrize("cases", [
    # (T, H, dtype, out dtype, residual, scale bound): the second smaller than the first
    ((300, 131072, torch.bfloat16, torch.int8, True, None),
     (7, 65544, torch.bfloat16, torch.int8, True, None)),
    ((64, 262144, torch.float16, torch.float8_e4m3fn, False, 0.05),
     (3, 40000, torch.float32, torch.float8_e4m3fn, True, None)),
    ((256, 8192, torch.bfloat16, torch.int8, True, None),
     (1, 5120, torch.bfloat16, torch.int8, True, None)),
])
def test_noalloc_matches_the_allocating_entry_point(cases):
    L = _lib.lib
    for i, (T, H, dtype, qdt, res, ub) in enumerate(cases):
        say(f"no-alloc call {i}: {T}x{H} {dtype} -> {qdt} res={res} ub={ub}")
        x, r, w = _inputs(T, H, dtype, 90 + i, res)
        want = _call(L.mcop_rms_norm_dynamic_per_token_quant, x, r, w, qdt, ub)
        got = _call(L.mcop_rms_norm_dynamic_per_token_quant_noalloc, x, r, w, qdt, ub)
        assert_codes(got[0], want[0], "codes")
        assert_scales(got[1], want[1], "scales")
        if res:
            assert_exact(got[2], want[2], "residual")
        assert torch.equal(got[0].view(torch.uint8), want[0].view(torch.uint8)), "codes bits"
        assert torch.equal(got[1].view(torch.int32), want[1].view(torch.int32)), "scale bits"


_TRACE_SCRIPT = r"""
import sys, torch
sys.path.insert(0, "tests")
from mcoplib_amd import _lib
from gpu_util import DEV
x = torch.randn(3, 131072, device=DEV).to(torch.bfloat16)
w = torch.ones(131072, device=DEV, dtype=torch.bfloat16)
q = torch.empty(3, 131072, dtype=torch.int8, device=DEV)
s = torch.empty(3, 1, device=DEV)
st = torch.cuda.current_stream().cuda_stream
for fn in (_lib.lib.mcop_rms_norm_dynamic_per_token_quant_noalloc,
           _lib.lib.mcop_rms_norm_dynamic_per_token_quant):
    assert fn(q.data_ptr(), 3, s.data_ptr(), x.data_ptr(), w.data_ptr(), None, None, 3, 131072,
              0, 1e-6, st) == 0
torch.cuda.synchronize()
print("child ok", flush=True)
"""


def test_noalloc_split_launch_uses_the_scratch():
    say("no-alloc: traced child process")
    env = dict(os.environ, MCOP_DEBUG_TRACE="1")
    out = subprocess.run([sys.executable, "-c", _TRACE_SCRIPT], cwd=str(ROOT), env=env,
                         capture_output=True, text=True, timeout=300)
    say(out.stdout[-2000:])
    assert out.returncode == 0, out.stderr[-3000:]
    lines = [ln for ln in out.stdout.splitlines() if "split-row kernel" in ln]
    assert len(lines) == 2, lines
    assert lines[0].startswith("[mcop] rms_norm_dynamic_per_token_quant_noalloc rows=3:")
    assert lines[0].endswith("workspace in the no-allocation scratch")
    assert lines[1].endswith("workspace from the stream-ordered allocator")
