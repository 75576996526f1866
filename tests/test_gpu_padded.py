"""GPU parity of the padded wire-format op (``mcoplib_amd.custom_ops`` /
``mcoplib_amd.op.fused_add_rms_norm_dynamic_per_token_quant_padding_output``) against the CPU
oracle: every output bit-exact, bytes of the padded rows past the scale left untouched, both
rounding chains (H == 7168 and other H), the vector and scalar paths, and the reference test's
own call (batch 1, H = 7168, pad 3840)."""

import pytest
import torch

import oracle
from mcoplib_amd import _lib, custom_ops, op
from gpu_util import DEV, assert_codes, assert_exact, assert_scales, say

pytestmark = pytest.mark.gpu


def _inputs(T, H, seed, x_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, generator=g) * x_scale).to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.randn(H, generator=g).to(torch.bfloat16)
    return x, r, w


def _case(T, H, pad, seed, x_scale=1.0):
    tag = f"padded T={T} H={H} pad={pad}"
    say(tag)
    x, r, w = _inputs(T, H, seed, x_scale)
    p_ref, r_ref, rms_ref, q_ref, s_ref = oracle.add_rms_norm_quant_padded(x, r, w, pad, 1e-6,
                                                                           fill=0xA5)
    padded = torch.full((T, 2 * pad), 0xA5, dtype=torch.uint8, device=DEV)
    rms = torch.empty((T, H), dtype=torch.bfloat16, device=DEV)
    q = torch.empty((T, H), dtype=torch.int8, device=DEV)
    s = torch.empty((T, 1), dtype=torch.float32, device=DEV)
    rd = r.to(DEV)
    op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
        padded.view(torch.int8), rms, q, s, x.to(DEV), rd, w.to(DEV), pad, 1e-6)
    torch.cuda.synchronize()
    assert_exact(padded, p_ref, tag + " padded rows (codes, scale, untouched tail)")
    assert_exact(rd, r_ref, tag + " residual")
    assert_exact(rms, rms_ref, tag + " output_rms")
    assert_codes(q, q_ref, tag + " codes")
    assert_scales(s, s_ref, tag + " scales")


@pytest.mark.parametrize("T", [1, 7, 83, 2048])
def test_deepseek_shape(T):
    _case(T, 7168, 3840, 100 + T)


@pytest.mark.parametrize("T,H,pad", [(1, 4096, 2050), (83, 4096, 2052), (300, 5120, 2600),
                                     (17, 1024, 516), (64, 8192, 4100), (9, 64, 36),
                                     (5, 16384, 8200)])
def test_other_widths(T, H, pad):
    _case(T, H, pad, 7 * T + H)


@pytest.mark.parametrize("T,H,pad", [(33, 1030, 517), (65, 7168, 3587), (12, 2000, 1003)])
def test_scalar_path_and_unaligned_scale(T, H, pad):
    # pad_bytes not a multiple of 8 (and, for 1030 / 2000, a scale at a byte offset that is not
    # a multiple of 4 on odd rows): the element-wise kernel and byte stores of the scale
    _case(T, H, pad, 3 * T + H)


def test_large_values_and_scaled_rows():
    _case(256, 7168, 3840, 5, x_scale=300.0)
    _case(256, 4096, 2048 + 4, 6, x_scale=1e-3)


@pytest.mark.parametrize("nv", [1, 2, 4, 8, 16])
def test_launch_shape_does_not_change_bits(nv):
    try:
        _lib.set_launch_override(nv, 0)
        _case(129, 7168, 3840, 9)
        _case(129, 4096, 2056, 10)
    finally:
        _lib.set_launch_override(0, 0)


def test_reference_unit_test_call():
    # unit_test/test_fused_add_rms_norm_custom.py:29-44 (batch 1, H 7168, pad 3840, eps 1e-6)
    say("reference unit test call")
    x, r, w = _inputs(1, 7168, 11)
    xd, rd, wd = x.to(DEV), r.to(DEV), w.to(DEV)
    output, residual_, output_rms, q, scales = \
        custom_ops.fused_add_rms_norm_dynamic_per_token_quant_padding_output(xd, rd, wd, 3840,
                                                                             1e-6)
    torch.cuda.synchronize()
    assert output.dtype == torch.bfloat16 and output.shape == (1, 3840)
    assert residual_ is rd
    total = x + r
    assert torch.equal(residual_.cpu(), total)
    ref = torch.rms_norm(total.float(), total.shape, weight=w.float().unsqueeze(0), eps=1e-6)
    err = (output_rms.float().cpu() - ref).abs()
    assert torch.all(err <= 2 * 2.0 ** -8 * ref.abs() + 1e-6)
    raw = output.view(torch.uint8).cpu()
    assert torch.equal(raw[:, :7168].view(torch.int8), q.cpu())
    assert torch.equal(raw[:, 7168:7172].contiguous().view(torch.float32), scales.cpu())


def test_argument_errors():
    say("argument checks")
    x = torch.randn(2, 64, device=DEV).to(torch.bfloat16)
    r = torch.randn(2, 64, device=DEV).to(torch.bfloat16)
    w = torch.randn(64, device=DEV).to(torch.bfloat16)
    rms, q = torch.empty_like(x), torch.empty((2, 64), dtype=torch.int8, device=DEV)
    s = torch.empty((2, 1), device=DEV)
    with pytest.raises(RuntimeError):  # row too short for codes + scale
        op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
            torch.empty((2, 66), dtype=torch.int8, device=DEV), rms, q, s, x, r, w, 33, 1e-6)
    with pytest.raises(RuntimeError):  # output must be int8
        op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
            torch.empty((2, 36), dtype=torch.bfloat16, device=DEV), rms, q, s, x, r, w, 36, 1e-6)
    with pytest.raises(RuntimeError):  # input must be bf16
        op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
            torch.empty((2, 72), dtype=torch.int8, device=DEV), rms.float(), q, s, x.float(),
            r, w, 36, 1e-6)
