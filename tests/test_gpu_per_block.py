"""GPU parity of ``torch.ops._C.rms_norm_per_block_quant`` (per-group scales, group 64 / 128,
row-major or transposed scales) against the CPU oracle: codes, scales and the residual."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, randn, say, weight

pytestmark = pytest.mark.gpu

SHAPES = [(1, 128), (1, 4096), (83, 1024), (83, 5120), (2048, 128), (2048, 7168), (7, 8192),
          (5, 16384), (3, 32768), (300, 2048), (17, 192)]


def _case(T, H, dtype, qdt, G, with_res, transposed, seed, scale_ub=None, x=None):
    tag = f"T={T} H={H} {dtype} {qdt} G={G} res={with_res} tr={transposed} ub={scale_ub}"
    if x is None:
        x = randn((T, H), seed, dtype, scale=1.0 / max(H, 1) ** 0.5)
    w = weight(H, seed + 1, dtype)
    r = randn((T, H), seed + 2, dtype) if with_res else None
    q_ref, s_ref, r_ref = oracle.rms_norm_per_block_quant(x, w, 1e-6, qdt, G, scale_ub, r,
                                                          transposed)
    q = torch.empty((T, H), dtype=qdt, device=DEV)
    s = torch.empty(s_ref.shape, dtype=torch.float32, device=DEV)
    rd = r.to(DEV) if with_res else None
    ub = None if scale_ub is None else torch.tensor([scale_ub], dtype=torch.float32, device=DEV)
    torch.ops._C.rms_norm_per_block_quant(q, x.to(DEV), w.to(DEV), s, 1e-6, ub, rd, G,
                                          transposed)
    torch.cuda.synchronize()
    assert_scales(s, s_ref, tag + " scales")
    assert_codes(q, q_ref, tag + " codes")
    if with_res:
        assert_exact(rd, r_ref, tag + " residual")


@pytest.mark.parametrize("T,H", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_shapes(T, H, dtype):
    say(f"per-block T={T} H={H} {dtype}")
    seed = 31 * T + H
    for qdt in (torch.int8, torch.float8_e4m3fn):
        for G in (64, 128):
            if H % G == 0:
                _case(T, H, dtype, qdt, G, with_res=(G == 64),
                      transposed=(qdt == torch.int8), seed=seed)


@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("with_res", [False, True])
def test_layouts_and_residual(transposed, with_res):
    say(f"per-block layouts tr={transposed} res={with_res}")
    for qdt in (torch.int8, torch.float8_e4m3fn):
        for G in (64, 128):
            _case(517, 4096, torch.bfloat16, qdt, G, with_res, transposed, 5)


def test_scale_ub_fp8():
    say("per-block fp8 scale_ub")
    for G in (64, 128):
        _case(256, 2048, torch.bfloat16, torch.float8_e4m3fn, G, True, False, 11,
              scale_ub=0.02)


def test_misaligned_views_take_the_element_path():
    say("per-block misaligned views")
    T, H = 65, 1024
    base = randn((T * H + 1,), 13, torch.bfloat16)
    x = base[1:].view(T, H)
    w = weight(H, 14, torch.bfloat16)
    for qdt in (torch.int8, torch.float8_e4m3fn):
        for G in (64, 128):
            q_ref, s_ref, _ = oracle.rms_norm_per_block_quant(x.contiguous(), w, 1e-6, qdt, G)
            q = torch.empty((T, H), dtype=qdt, device=DEV)
            s = torch.empty(s_ref.shape, dtype=torch.float32, device=DEV)
            xd = base.to(DEV)[1:].view(T, H)
            torch.ops._C.rms_norm_per_block_quant(q, xd, w.to(DEV), s, 1e-6, None, None, G,
                                                  False)
            torch.cuda.synchronize()
            assert_scales(s, s_ref, f"misaligned {qdt} G={G} scales")
            assert_codes(q, q_ref, f"misaligned {qdt} G={G} codes")


def test_group_outliers_and_zero_groups():
    say("per-block outlier and zero groups")
    T, H = 64, 2048
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(3))
    x[:, 128:256] = 0.0          # a zero group at G = 64 and G = 128
    x[:, 700] *= 1000.0          # an outlier channel
    x[5] = 0.0                   # a zero row
    for dtype in (torch.bfloat16, torch.float32):
        for qdt in (torch.int8, torch.float8_e4m3fn):
            for G in (64, 128):
                _case(T, H, dtype, qdt, G, False, False, 17, x=x.to(dtype))


@pytest.mark.parametrize("nv", [1, 2, 4, 8, 16])
def test_launch_shape_does_not_change_bits(nv):
    say(f"per-block launch override nv={nv}")
    try:
        _lib.set_launch_override(nv, 0)
        for G in (64, 128):
            _case(129, 4096, torch.bfloat16, torch.int8, G, True, False, 19)
            _case(129, 4096, torch.float32, torch.float8_e4m3fn, G, False, True, 20)
    finally:
        _lib.set_launch_override(0, 0)


def test_argument_errors():
    say("per-block argument checks")
    x = torch.randn(4, 192, device=DEV, dtype=torch.bfloat16)
    w = torch.ones(192, device=DEV, dtype=torch.bfloat16)
    q = torch.empty((4, 192), dtype=torch.int8, device=DEV)
    with pytest.raises(RuntimeError):  # group size
        torch.ops._C.rms_norm_per_block_quant(q, x, w, torch.empty(4 * 6, device=DEV), 1e-6,
                                              None, None, 32, False)
    with pytest.raises(RuntimeError):  # 192 is not a multiple of 128
        torch.ops._C.rms_norm_per_block_quant(q, x, w, torch.empty(4 * 2, device=DEV), 1e-6,
                                              None, None, 128, False)
    with pytest.raises(RuntimeError):  # scale_ub needs fp8 output
        torch.ops._C.rms_norm_per_block_quant(q, x, w, torch.empty(4 * 3, device=DEV), 1e-6,
                                              torch.ones(1, device=DEV), None, 64, False)
    with pytest.raises(RuntimeError):  # wrong number of scales
        torch.ops._C.rms_norm_per_block_quant(q, x, w, torch.empty(4 * 2, device=DEV), 1e-6,
                                              None, None, 64, False)
