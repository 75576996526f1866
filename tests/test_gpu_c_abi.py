"""The C ABI driven from a plain C caller on the GPU: tests/c_caller/abi_example.c (the example
INTEGRATION.md quotes) allocates device memory with hipMalloc, creates a stream of its own, passes
raw device pointers to mcop_fused_add_rms_norm, mcop_rms_norm_dynamic_per_token_quant,
mcop_rms_norm_smooth_quant and mcop_scale_dynamic_quant, and copies the results back; this test
loads it with ctypes (host buffers only, no torch device tensors) and compares every output with
the CPU oracle bit for bit (the reference's C++ entry points it stands in for:
include/rms_norm_dynamic_per_token_quant.h:2-8, include/fused_rms_norm_dq.h:3-12,
include/scale_dynamic_quant.h:6-10 and op/vllm/torch_bindings.cpp:161-164,216-221)."""

import ctypes

import pytest
import torch

import oracle
from conftest import ROOT
from gpu_util import assert_codes, assert_exact, assert_scales, gen, say

pytestmark = pytest.mark.gpu

LIB = ROOT / "tests" / "c_caller" / "libabi_example.so"
P, I64, F, I, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_size_t


@pytest.fixture(scope="module")
def c():
    if not LIB.exists():
        raise RuntimeError(f"{LIB} is not built (make -C tests/c_caller, or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    lib.example_fused_add_rms_norm.argtypes = [P, P, P, I64, I64, F, P, SZ]
    lib.example_rms_norm_quant.argtypes = [P, I, P, P, P, P, I64, I64, F, P, SZ]
    lib.example_rms_norm_smooth_quant.argtypes = [P, I, P, P, P, P, P, P, P, I64, I64, F, P, SZ]
    lib.example_scale_dynamic_quant.argtypes = [P, P, P, P, I64, I64, P, SZ]
    for f in (lib.example_fused_add_rms_norm, lib.example_rms_norm_quant,
              lib.example_rms_norm_smooth_quant, lib.example_scale_dynamic_quant):
        f.restype = I
    return lib


def _call(fn, *args):
    err = ctypes.create_string_buffer(512)
    rc = fn(*args, err, 512)
    assert rc == 0, f"rc={rc}: {err.value.decode()}"


def _bf16(T, H, seed, scale=1.0):
    return (scale * torch.randn(T, H, generator=gen(seed))).to(torch.bfloat16)


def _w(H, seed):
    return (1 + 0.1 * torch.randn(H, generator=gen(seed))).to(torch.bfloat16)


@pytest.mark.parametrize("T,H", [(64, 5120), (257, 4096), (3, 4104)])
def test_c_caller_fused_add_rms_norm(c, T, H):
    say(f"C caller: mcop_fused_add_rms_norm {T}x{H}")
    x, r, w = _bf16(T, H, 1), _bf16(T, H, 2), _w(H, 3)
    x_ref, r_ref = oracle.fused_add_rms_norm(x, r, w, 1e-6)
    xo, ro = x.clone(), r.clone()
    _call(c.example_fused_add_rms_norm, xo.data_ptr(), ro.data_ptr(), w.data_ptr(), T, H, 1e-6)
    assert_exact(ro, r_ref, "residual")
    assert_exact(xo, x_ref, "output")


@pytest.mark.parametrize("T,H", [(64, 5120), (300, 8192), (5, 2056)])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("with_res", [True, False])
def test_c_caller_rms_norm_quant(c, T, H, qdt, with_res):
    say(f"C caller: mcop_rms_norm_dynamic_per_token_quant {T}x{H} {qdt} res={with_res}")
    x, w = _bf16(T, H, 4), _w(H, 5)
    r = _bf16(T, H, 6) if with_res else None
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, qdt, None, r)
    q = torch.empty(T, H, dtype=qdt)
    s = torch.empty(T, dtype=torch.float32)
    ro = r.clone() if with_res else None
    _call(c.example_rms_norm_quant, q.data_ptr(), int(qdt == torch.float8_e4m3fn), s.data_ptr(),
          x.data_ptr(), w.data_ptr(), None if ro is None else ro.data_ptr(), T, H, 1e-6)
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")
    if with_res:
        assert_exact(ro, r_ref, "residual")


@pytest.mark.parametrize("T,H", [(128, 7168), (2, 4096)])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("with_res", [False, True])
def test_c_caller_rms_norm_smooth_quant(c, T, H, qdt, with_res):
    say(f"C caller: mcop_rms_norm_smooth_quant {T}x{H} {qdt} res={with_res}")
    x, w = _bf16(T, H, 7, 3.0), _w(H, 8)
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(9))
    r = _bf16(T, H, 10) if with_res else None
    q_ref, s_ref, ar_ref, an_ref = oracle.rms_norm_smooth_quant(x, w, sm, 1e-6, qdt, r)
    q = torch.empty(T, H, dtype=qdt)
    s = torch.empty(T, dtype=torch.float32)
    ar, an = torch.empty_like(x), torch.empty_like(x)
    _call(c.example_rms_norm_smooth_quant, q.data_ptr(), int(qdt == torch.float8_e4m3fn),
          s.data_ptr(), x.data_ptr(), w.data_ptr(), sm.data_ptr(), ar.data_ptr(), an.data_ptr(),
          None if r is None else r.data_ptr(), T, H, 1e-6)
    assert_exact(ar, ar_ref, "after_res")
    assert_exact(an, an_ref, "after_norm")
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


@pytest.mark.parametrize("T,H", [(200, 7168), (2, 768)])
def test_c_caller_scale_dynamic_quant(c, T, H):
    say(f"C caller: mcop_scale_dynamic_quant {T}x{H}")
    x = _bf16(T, H, 11)
    sm = 0.5 + 1.5 * torch.rand(H, generator=gen(12))
    q_ref, s_ref = oracle.scale_dynamic_quant(x, sm)
    q = torch.empty(T, H, dtype=torch.int8)
    s = torch.empty(T, dtype=torch.float32)
    _call(c.example_scale_dynamic_quant, q.data_ptr(), s.data_ptr(), x.data_ptr(), sm.data_ptr(),
          T, H)
    assert_scales(s, s_ref, "scales")
    assert_codes(q, q_ref, "codes")


def test_c_caller_reports_an_error_status(c):
    """A hidden size the operator rejects (0) comes back as the C status MCOP_E_INVALID with
    mcop_last_error()'s message, after the caller's buffers and stream were set up."""
    say("C caller: error status")
    x, w = _bf16(2, 64, 13), _w(64, 14)
    q, s = torch.empty(2, 64, dtype=torch.int8), torch.empty(2, dtype=torch.float32)
    err = ctypes.create_string_buffer(512)
    rc = c.example_rms_norm_quant(q.data_ptr(), 0, s.data_ptr(), x.data_ptr(), w.data_ptr(), None,
                                  2, 0, 1e-6, err, 512)
    assert rc == -1, (rc, err.value)
    assert b"bad shape num_tokens=2 hidden_size=0" in err.value, err.value
