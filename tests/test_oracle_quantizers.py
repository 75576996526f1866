"""Pins of the oracle's standalone per-token quantizers (vLLM ``_C::dynamic_scaled_int8_quant``,
op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:94-132, 370-422, 459-527, and
``_C::dynamic_per_token_scaled_fp8_quant``, op/vllm/quantization/fp8/common.cu:142-180, 375-411).

What pins them:
  - hand-worked known answers (ties to even, saturation, the zero-point formula);
  - the reference's own verification recipes (benchmark/runners/
    mcoplib_mxbenchmark_dynamic_scaled_int8_quant_runners.py:40-60 and
    mcoplib_mxbenchmark_dynamic_per_token_scaled_fp8_quant_runners.py:40-57): the fp8 recipe must
    agree bit for bit, the int8 one (which divides by the scale where the kernel multiplies by
    127/A) within one code on few elements;
  - a torch restatement operation by operation;
  - invariants: the absmax element maps to +-127 / +-448, the row minimum and maximum map to the
    ends of the asymmetric range, dequantisation error within half a step (one step with a zero
    point), and the fp8 quantizer reproducing the quantizer stage of the fused H2 oracle.
"""

import numpy as np
import pytest
import torch

import oracle


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------------------ int8 symmetric

def test_int8_known_answers():
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0], [-4.0, 2.0, 0.0, 1.0]], dtype=torch.bfloat16)
    q, s, azp = oracle.dynamic_scaled_int8_quant(x)
    assert azp is None
    # inv = 127/4 = 31.75: 31.75 -> 32, 63.5 -> 64 (tie to even), 95.25 -> 95, 127
    assert q.tolist() == [[32, 64, 95, 127], [-127, 64, 0, 32]]
    assert s.flatten().tolist() == [float(np.float32(4.0) / np.float32(127.0))] * 2


def test_int8_zero_and_inf_rows_give_zero_codes():
    x = torch.zeros(2, 64, dtype=torch.float16)
    x[1, 5] = float("inf")
    q, s, _ = oracle.dynamic_scaled_int8_quant(x)
    assert s[0].item() == 0.0 and s[1].item() == float("inf")
    # A == 0: inv = 0; A == inf: inv = 127/inf = 0 and inf * 0 = NaN converts to 0
    assert torch.count_nonzero(q) == 0


def test_int8_tiny_row_has_an_infinite_inverse():
    """A row whose absmax lies below 127 / FLT_MAX (bf16 and fp32 reach it; fp16 cannot): the
    binary32 quotient 127 / A overflows to inf, so every nonzero element's product is infinite
    and saturates to +-127, and 0 * inf = NaN converts to 0 -- not the codes of the exact
    quotient, which would round these elements to +-127 and +-64."""
    x = torch.tensor([[2e-38, -2e-38, 1e-38, 0.0, -1e-38]], dtype=torch.bfloat16)
    A = np.float32(x.float().abs().max().item())
    assert np.isinf(np.float32(127.0) / A)  # the premise: the binary32 quotient overflows
    q, s, _ = oracle.dynamic_scaled_int8_quant(x)
    assert q.tolist() == [[127, -127, 127, 0, -127]]
    assert s.item() == float(A / np.float32(127.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_int8_torch_restatement(dtype):
    x = (torch.randn(128, 1031, generator=_gen(1)) * 3).to(dtype)
    q, s, _ = oracle.dynamic_scaled_int8_quant(x)
    A = x.float().abs().amax(-1, keepdim=True)
    s_ref = A / 127.0
    # tensor / tensor: torch evaluates `127.0 / A` as 127 * reciprocal(A), two roundings
    inv = torch.where(A == 0, torch.zeros_like(A), torch.full_like(A, 127.0) / A)
    q_ref = torch.round(x.float() * inv).clamp(-127, 127).to(torch.int8)
    assert torch.equal(s, s_ref)
    assert torch.equal(q, q_ref)


def test_int8_vs_reference_benchmark_recipe():
    # runner: safe_scales[scales == 0] = 1; ref = clamp(round(x / scales), -128, 127)
    x = torch.randn(512, 4096, generator=_gen(2)).to(torch.float16)
    q, s, _ = oracle.dynamic_scaled_int8_quant(x)
    safe = s.clone()
    safe[safe == 0] = 1.0
    ref = torch.clamp(torch.round(x.float() / safe), -128, 127).to(torch.int8)
    d = (q.int() - ref.int()).abs()
    assert d.max().item() <= 1
    assert (d > 0).float().mean().item() < 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_int8_invariants(dtype):
    x = (torch.randn(64, 2000, generator=_gen(3)) * torch.logspace(-3, 3, 64)[:, None]).to(dtype)
    q, s, _ = oracle.dynamic_scaled_int8_quant(x)
    xf = x.double()
    arg = xf.abs().argmax(-1, keepdim=True)
    top = q.gather(-1, arg).int().abs()
    assert torch.all(top == 127)
    assert q.min().item() >= -127
    err = (q.double() * s.double() - xf).abs().amax(-1)
    assert torch.all(err <= s.double().flatten() * (0.5 + 1e-5))


# ------------------------------------------------------------------------------ int8 zero point

def test_azp_known_answers():
    x = torch.tensor([[-1.0, 0.0, 1.0, 2.0]], dtype=torch.float32)
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    s32 = np.float32(3.0) / np.float32(255.0)
    assert s.item() == float(s32)
    # zp = rne(-128 - (-1)/s) = rne(-128 + 85.00000x) = -43; codes rne(x * (1/s)) + zp
    assert azp.item() == -43
    assert q.tolist() == [[-128, -43, 42, 127]]


def test_azp_all_positive_row_has_large_zero_point():
    x = torch.tensor([[1000.0, 1000.5, 1001.0]], dtype=torch.float32)
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    assert s.item() == float(np.float32(1.0) / np.float32(255.0))
    assert azp.item() == -255128
    # 1/s rounds to 254.99998, so the middle value lands at 255127.48 -> 255127 -> -1
    assert q.tolist() == [[-128, -1, 127]]


def test_azp_tiny_row_saturates_infinite_products():
    """A row of tiny values: s = (max - min) / 255 is subnormal, so inv = 1 / s is infinite and
    every nonzero product is +-inf.  float_to_int32_rn clamps them to +-2^31, i.e. INT32_MAX /
    INT32_MIN, and the zero point is negative here, so the int32 sum of the reference would
    wrap for -inf; the restatement saturates instead: -inf codes -128 (not 127), +inf 127, and
    0 * inf = NaN 127 like any NaN product."""
    x = torch.tensor([[4e-39, -2e-39, 0.0]], dtype=torch.float32)
    mx, mn = np.float32(x[0, 0].item()), np.float32(x[0, 1].item())
    s32 = (mx - mn) / np.float32(255.0)
    assert np.isinf(np.float32(1.0) / s32)  # the premise: inv overflows
    zp = int(np.rint(np.float32(-128.0) - mn / s32))
    assert zp < 0
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    assert s.item() == float(s32) and azp.item() == zp
    assert q.tolist() == [[127, -128, 127]]


def test_azp_nan_element_codes_like_the_fmin_clamp():
    # float_to_int32_rn: min(NaN, 2^31) = 2^31 -> INT32_MAX; + zp saturates to 127
    x = torch.tensor([[-1.0, 0.0, float("nan"), 2.0]], dtype=torch.float32)
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    assert azp.item() == -43 and q.tolist() == [[-128, -43, 127, 127]]
    # the symmetric form converts directly: NaN -> 0
    q, _, _ = oracle.dynamic_scaled_int8_quant(x)
    assert q.tolist() == [[-64, 0, 0, 127]]


def test_azp_constant_row_is_defined():
    x = torch.full((3, 40), 2.5, dtype=torch.bfloat16)
    x[2] = 0
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    assert torch.all(s == 0) and torch.all(azp == -128) and torch.all(q == -128)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_azp_torch_restatement(dtype):
    x = (torch.randn(96, 777, generator=_gen(4)) * 2 + 0.7).to(dtype)
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    xf = x.float()
    mx, mn = xf.amax(-1, keepdim=True), xf.amin(-1, keepdim=True)
    s_ref = (mx - mn) / 255.0
    zp_ref = torch.round(-128.0 - mn / s_ref).to(torch.int32)
    inv = 1.0 / s_ref
    q_ref = (torch.round(xf * inv).to(torch.int64) + zp_ref).clamp(-128, 127).to(torch.int8)
    assert torch.equal(s, s_ref)
    assert torch.equal(azp, zp_ref)
    assert torch.equal(q, q_ref)


def test_azp_invariants():
    x = (torch.randn(64, 3001, generator=_gen(5)) * torch.logspace(-2, 2, 64)[:, None]
         + torch.linspace(-5, 5, 64)[:, None])
    q, s, azp = oracle.dynamic_scaled_int8_quant(x, use_azp=True)
    lo = q.gather(-1, x.argmin(-1, keepdim=True)).int()
    hi = q.gather(-1, x.argmax(-1, keepdim=True)).int()
    assert torch.all(lo <= -127) and torch.all(hi >= 126)
    deq = (q.double() - azp.double()) * s.double()
    err = (deq - x.double()).abs().amax(-1)
    assert torch.all(err <= s.double().flatten() * (1.0 + 1e-4))


# ------------------------------------------------------------------------------ fp8

def test_fp8_known_answers():
    x = torch.tensor([[896.0, -896.0, 1.0, 0.0], [0.0, 0.0, 0.0, 0.0]], dtype=torch.float32)
    q, s = oracle.dynamic_per_token_scaled_fp8_quant(x)
    assert s.flatten().tolist() == [2.0, float(np.float32(1.0) / np.float32(229376.0))]
    # 448 -> 0x7e, -448 -> 0xfe, 0.5 -> 0x30, zeros -> 0
    assert q.view(torch.uint8).tolist() == [[0x7E, 0xFE, 0x30, 0x00], [0, 0, 0, 0]]


def test_fp8_scale_ub():
    x = torch.tensor([[100.0, 10.0, -50.0]], dtype=torch.float32)
    q, s = oracle.dynamic_per_token_scaled_fp8_quant(x, scale_ub=44.8)
    assert s.item() == float(np.float32(np.float32(44.8) / np.float32(448.0)))
    # |x / s| beyond 448 clamps to the largest finite code
    assert q.view(torch.uint8)[0, 0].item() == 0x7E and q.view(torch.uint8)[0, 2].item() == 0xFE


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("ub", [None, 3.0])
def test_fp8_vs_reference_benchmark_recipe(dtype, ub):
    # runner: ref = (x / safe_scales).to(float8_e4m3fn) -- torch's own conversion
    x = (torch.randn(256, 1024, generator=_gen(6)) * 4).to(dtype)
    q, s = oracle.dynamic_per_token_scaled_fp8_quant(x, scale_ub=ub)
    A = x.float().abs().amax(-1, keepdim=True)
    if ub is not None:
        A = torch.minimum(A, torch.tensor(ub, dtype=torch.float32))
    s_ref = torch.maximum(A / 448.0, torch.tensor(1.0, dtype=torch.float32) / (448.0 * 512.0))
    assert torch.equal(s, s_ref)
    ref = (x.float() / s).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(q.view(torch.uint8), ref.view(torch.uint8))


def test_fp8_strided_rows():
    base = torch.randn(40, 300, generator=_gen(7)).to(torch.bfloat16)
    view = base[:, 10:266]
    q, s = oracle.dynamic_per_token_scaled_fp8_quant(view)
    q2, s2 = oracle.dynamic_per_token_scaled_fp8_quant(view.contiguous())
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_is_the_quantizer_stage_of_h2(dtype):
    # vLLM's H2 test quantizes the unfused RMSNorm output with this op; without a residual the
    # fused H2 fp8 path is that composition exactly (the H1 oracle with a zero residual is the
    # unfused b(b(x * rho) * w)).
    g = _gen(8)
    x = (torch.randn(64, 1536, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(1536, generator=g)).to(dtype)
    q_h2, s_h2, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.float8_e4m3fn)
    y, _ = oracle.fused_add_rms_norm(x, torch.zeros_like(x), w, 1e-6)
    q, s = oracle.dynamic_per_token_scaled_fp8_quant(y)
    assert torch.equal(s, s_h2)
    assert torch.equal(q.view(torch.uint8), q_h2.view(torch.uint8))
