"""Pins the oracle's number-format conversions (bf16, fp16, fp8-e4m3fn, all written in
oracle/mcop_oracle.c from the formats' definitions) against PyTorch's own CPU conversions, an
independent implementation, over sweeps that include every rounding tie."""

import numpy as np
import pytest
import torch

import oracle


def _f32_from_bits(u: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(u.astype(np.uint32).view(np.float32).copy())


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def _sweep_around(values_u32: np.ndarray) -> np.ndarray:
    """The given fp32 bit patterns and their neighbours one ulp away."""
    return np.concatenate([values_u32, values_u32 + 1, values_u32 - 1]).astype(np.uint32)


def test_bf16_matches_torch_including_ties():
    rng = np.random.default_rng(0)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    ties = hi | 0x8000  # exactly halfway between two bf16 values
    u = np.concatenate([rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32),
                        _sweep_around(ties)])
    x = _f32_from_bits(u)
    got = _bits16(oracle.f32_to_bf16_bits(x))
    ref = _bits16(x.to(torch.bfloat16))
    nan = torch.isnan(x).numpy()
    assert np.array_equal(got[~nan], ref[~nan])
    got_f = torch.from_numpy(got.astype(np.int16)).view(torch.bfloat16)
    assert torch.isnan(got_f.float()[torch.from_numpy(nan)]).all()


def test_f16_matches_torch_including_ties_subnormals_overflow():
    rng = np.random.default_rng(1)
    h = np.arange(1 << 16, dtype=np.uint16)
    vals = torch.from_numpy(h.view(np.int16)).view(torch.float16).float()
    finite = torch.isfinite(vals)
    v = vals[finite].numpy().astype(np.float64)
    v = np.unique(v)
    mids = ((v[1:] + v[:-1]) / 2).astype(np.float32)  # halfway points (exact in fp32)
    mids_u = mids.view(np.uint32)
    extra = np.array([65504, 65519.99, 65520, 65536, 1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                      2 ** -14, 2 ** -14 - 2 ** -25], dtype=np.float32)
    u = np.concatenate([_sweep_around(mids_u),
                        rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32),
                        extra.view(np.uint32), (-extra).view(np.uint32)])
    x = _f32_from_bits(u)
    got = _bits16(oracle.f32_to_f16_bits(x))
    ref = _bits16(x.to(torch.float16))
    nan = torch.isnan(x).numpy()
    assert np.array_equal(got[~nan], ref[~nan])


def test_e4m3fn_matches_torch_after_clamp():
    rng = np.random.default_rng(2)
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    finite = codes[torch.isfinite(codes)].numpy().astype(np.float64)
    v = np.unique(finite)
    mids = ((v[1:] + v[:-1]) / 2).astype(np.float32)
    # every bf16 value (as fp32) clamped to +-448, all fp8 midpoints and their neighbours,
    # random fp32 in the fp8 range and in its subnormal range
    bf = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    bf = bf[np.isfinite(bf)]
    x = np.concatenate([
        np.clip(bf, -448, 448),
        _sweep_around(mids.view(np.uint32)).view(np.float32),
        rng.uniform(-448, 448, 1 << 20).astype(np.float32),
        rng.uniform(-2 ** -5, 2 ** -5, 1 << 18).astype(np.float32),
    ]).astype(np.float32)
    xt = torch.from_numpy(x)
    got = oracle.f32_to_e4m3fn_bits(xt).numpy()
    ref = xt.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_fp8_epilogue_clamps_like_fmin_fmax():
    # clamp(v, +-448) uses fmin/fmax: NaN -> +448, +-inf -> +-448, beyond range saturates
    x = torch.tensor([float("nan"), float("inf"), -float("inf"), 1e6, -1e6, 448.0, -448.0, 0.0,
                      -0.0], dtype=torch.float32)
    got = oracle.fp8_e4m3fn_from_f32(x).tolist()
    assert got == [0x7e, 0x7e, 0xfe, 0x7e, 0xfe, 0x7e, 0xfe, 0x00, 0x80]


@pytest.mark.parametrize("mul", [1.0, 0.5, 3.0])
def test_fp8_epilogue_scaling(mul):
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.uniform(-300, 300, 4096).astype(np.float32))
    got = oracle.fp8_e4m3fn_from_f32(x, mul)
    ref = (x * mul).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(got, ref)
