"""Hand-built rows that pin where the reference rounds, shared by the CPU oracle tests
(test_oracle_rounding_points.py) and the GPU tests (test_gpu_rounding_points.py).

Each case is a tiny row whose expected outputs were worked out by hand (the derivation is in
the docstring) and whose plausible alternative reading -- a rounding step dropped or moved --
gives a different, also hand-derived, answer.  The tests check that the implementation gives
the expected answer and that the alternative differs from it, so a restatement that followed
the alternative reading fails.  Values chosen so that every rounding lands far from a boundary,
except where a tie is the point of the case (ties round to even).

bf16 spacing: 2^-8 in [0.5, 1), 2^-7 in [1, 2), 2^-6 in [2, 4), 2^-5 in [4, 8), 2^-4 in
[8, 16), 0.25 in [32, 64), 0.5 in [64, 128).
"""

from __future__ import annotations

import math

import numpy as np
import torch

EPS = 1e-6
F32_EPS = float(np.finfo(np.float32).eps)


def _bf16(vals, n=None):
    t = torch.tensor(vals, dtype=torch.float32)
    if n is not None and t.numel() < n:
        t = torch.cat([t, torch.zeros(n - t.numel())])
    return t.to(torch.bfloat16).view(1, -1)


def h1_variance_of_rounded_sum():
    """H1 (op/vllm/layernorm_kernels.cu:118-133, type_convert.cuh:167-183): the variance is taken
    over the ROUNDED residual z = b(x + r).

    x = 1, r = 2^-8 in all 8 lanes, w = 1, eps = 1e-6.  x + r = 1 + 2^-8 is the tie between 1 and
    1 + 2^-7, so z = 1 (even).  Sum z^2 / 8 = 1, rho = 1/sqrt(1 + 1e-6) = 0.9999995, and
    b(z * rho) = 1, so the new x is b(1 * 1) = 1 in every lane and the new residual is 1.
    Alternative (variance of the unrounded sum): mean = (1 + 2^-8)^2 = 1.0078278, rho' =
    0.9961089, b(1 * rho') = 0.99609375 (= 1 - 2^-8; 0.99611 is 1.5e-5 above it, 2^-8 below 1)."""
    H = 8
    return {
        "x": _bf16([1.0] * H), "r": _bf16([2.0 ** -8] * H), "w": _bf16([1.0] * H).view(-1),
        "eps": EPS,
        "x_out": [1.0] * H, "r_out": [1.0] * H,
        "x_out_alt": [0.99609375] * H,
    }


def h2_double_rounding_of_y():
    """H2 (layernorm_utils.cuh:531) and the generic H3 chain (kernel/rms_norm_vllm.cuh:445):
    y = b(b(a * rho) * w), two roundings.

    x = [3, 4, 0 x 6], w = [1, 1.5, 1 x 6], no residual, eps = 1e-6.  Sum a^2 = 25, mean 3.125,
    rho = 1/sqrt(3.125001) = 0.5656853.  4 rho = 2.2627417 -> b = 145/64 = 2.265625 (144.8 units
    of 2^-6); times 1.5 = 3.3984375 = 217.5 units of 2^-6, a tie -> 218/64 = 3.40625 (even).
    3 rho = 1.6970563 -> b = 217/128 = 1.6953125; times 1 -> 1.6953125.  So A = max|y| =
    3.40625, and the int8 scale is A/127 (FLT_EPSILON floor not reached), the codes
    [rne(1.6953125 * 127/3.40625), 127] = [rne(63.21), 127] = [63, 127]; fp8: s = A/448,
    codes [e4m3(1.6953125 * 448/3.40625) = e4m3(222.97) = 224, 448].
    Alternative (one rounding, b(a * rho * w)): 4 rho * 1.5 = 3.3941125 -> 217.2 units ->
    3.390625, so A' = 3.390625 and the scale A'/127 differs by 0.46%."""
    H = 8
    A = 3.40625
    return {
        "x": _bf16([3.0, 4.0], H), "w": _bf16([1.0, 1.5], H).view(-1), "eps": EPS,
        "int8_scale": A / 127.0, "int8_codes": [63, 127] + [0] * (H - 2),
        "fp8_scale": A / 448.0, "fp8_values": [224.0, 448.0] + [0.0] * (H - 2),
        "int8_scale_alt": 3.390625 / 127.0,
    }


def h4_rereads_rounded_after_res():
    """H4 (op/fused_rms_norm_dq.cu:82-84 writes after_res = b(a); :243-245 and :176-179 read it
    back): the normalization uses a~ = b(x + r), while rho comes from the unrounded a.

    x = [3, 4, 0 x 6], r = [0, 2^-6, 0 x 6], w = 1, smooth = 1, eps = 1e-6.  a = [3, 4.015625,
    0...]; 4.015625 is the tie between 4 and 4 + 2^-5, so after_res = [3, 4, 0...].  Sum a^2 =
    9 + 16.125244 = 25.125244, mean 3.1406555, rho = 1/sqrt(3.1406565) = 0.5642737.
    Literal form u = (a~ / rho) * w: u = [5.3165712, 7.0887616, 0...];
      after_norm = b(u) = [170/32 = 5.3125, 227/32 = 7.09375] (170.13 and 226.84 units of 2^-5);
      v = u * 1; int8 scale = 7.0887616/127.
    Alternative (the later passes use the unrounded a): u'_1 = 4.015625 / rho = 7.1164524 ->
    b = 228/32 = 7.125; scale 7.1164524/127 (0.39% larger).
    int8 codes [rne(127 * 5.3165712/7.0887616), 127] = [rne(95.25), 127] = [95, 127].
    Standard form u = (a~ * rho) * w: u = [1.6928211, 2.2570948] -> b = [217/128 = 1.6953125,
    144/64 = 2.25] (216.68 and 144.45 units); alternative 4.015625 * rho = 2.2659117 -> 145/64 =
    2.265625."""
    H = 8
    rho = 1.0 / math.sqrt((9.0 + 4.015625 ** 2) / 8.0 + EPS)
    return {
        "x": _bf16([3.0, 4.0], H), "r": _bf16([0.0, 2.0 ** -6], H),
        "w": _bf16([1.0] * H).view(-1), "sm": torch.ones(H), "eps": EPS,
        "after_res": [3.0, 4.0] + [0.0] * (H - 2),
        "after_norm": [5.3125, 7.09375] + [0.0] * (H - 2),
        "after_norm_alt": [5.3125, 7.125] + [0.0] * (H - 2),
        "int8_scale": 4.0 / rho / 127.0, "int8_scale_alt": 4.015625 / rho / 127.0,
        "int8_codes": [95, 127] + [0] * (H - 2),               # rne(127 * 5.3166/7.0888 = 95.25)
        "after_norm_std": [1.6953125, 2.25] + [0.0] * (H - 2),
        "after_norm_std_alt": [1.6953125, 2.265625] + [0.0] * (H - 2),
    }


def h3_7168_fp32_chain():
    """mcoplib's H3 at H == 7168 (op/rms_norm_dynamic_per_token_quant.cu:146-182) keeps
    p = a * w in fp32 and scales by rho at the end; every other width rounds y twice
    (kernel/rms_norm_vllm.cuh:330-454).

    x = [4, 2, 0 x 7166], w = [1.5, 1, 1 ...], no residual, eps = 1e-6.  Sum a^2 = 20,
    rho = 1/sqrt(20/7168 + 1e-6) = 18.927953.  7168 chain: p = [6, 2, 0...], A = 6,
    s = (A * rho)/127 = 0.8942340, codes [rne(6 rho / s), rne(2 rho / s)] = [127, rne(42.33)] =
    [127, 42].
    Alternative (the generic chain at this width): b(4 rho) = b(75.711812) = 75.5 (151.4 units
    of 0.5); times 1.5 = 113.25 = 226.5 units, a tie -> 113 (even); A' = 113, s' = 113/127 =
    0.8897638 (0.50% smaller)."""
    H = 7168
    rho = 1.0 / math.sqrt(20.0 / H + EPS)
    return {
        "x": _bf16([4.0, 2.0], H), "w": _bf16([1.5] + [1.0] * (H - 1)).view(-1), "eps": EPS,
        "scale": 6.0 * rho / 127.0, "codes": [127, 42] + [0] * (H - 2),
        "scale_alt": 113.0 / 127.0,
    }


def fp8_quantizer_divides():
    """vLLM's fp8 per-token quantizer divides by the scale (op/vllm/quantization/fp8/
    common.cu:142-180 with quant_conversions.cuh:23-28 / ScaledQuant<.., false>).

    x = [6.125, 0.0247802734375 (= 203/8192), 0 x 6] (both bf16 values).  A = 6.125 = 448 * 7/512,
    so s = 7/512 exactly (the 1/(448*512) floor not reached), and x_1 / s = 1.8125 exactly: the
    tie between the e4m3 values 1.75 and 1.875, which rounds to 1.75 (even mantissa).
    Alternative (multiply by the rounded reciprocal): RN(1/s) = 73.14286 is above 512/7 by
    3e-6 relative, x_1 * RN(1/s) rounds to 1.8125001 and codes 1.875."""
    H = 8
    return {
        "x": _bf16([6.125, 203.0 / 8192.0], H), "scale": 7.0 / 512.0,
        "values": [448.0, 1.75] + [0.0] * (H - 2), "values_alt": [448.0, 1.875] + [0.0] * (H - 2),
    }


def fp8_quotient_beyond_448():
    """The fp8 quotient of a row's absmax element can land one ulp above 448: with
    A = 1.0234375 (= 131/128, a bf16 value), s = RN(A/448) is below A/448, and RN(A/s) =
    448 + 2^-15.  Such a quotient codes +-448 (the clamp to [-448, 448], or the conversion's
    round-to-nearest: the next e4m3 magnitude would be 480, the midpoint 464), never NaN.
    Two rows: the absmax negative, then positive; the other element 0.5 gives 0.5/s = 218.87,
    coding 224 (between 208 and 224, above the midpoint 216)."""
    H = 8
    x = torch.cat([_bf16([-1.0234375, 0.5], H), _bf16([1.0234375, -0.5], H)])
    return {"x": x, "quotient": 448.0 + 2.0 ** -15,
            "values": [[-448.0, 224.0] + [0.0] * (H - 2), [448.0, -224.0] + [0.0] * (H - 2)]}


def h4_fp8_divides(u: torch.Tensor):
    """H4's fp8 output, this library's extension (the reference's operator has no fp8 form:
    op/fused_rms_norm_dq.cu:51-66 defines ScaledQuant for int8 only): q = e4m3(clamp(v / s)),
    dividing by the scale as the path's fp8 quantizers do (quant_conversions.cuh:52-59).

    fp32 input; `u` is the row's after_norm (unrounded for fp32 input, independent of the smooth
    scales).  The smooth scales are chosen so that v = RN(u * sm) is 6.125 at one element (the
    absmax: s = 6.125/448 = 7/512 exactly) and 203/8192 = 1.8125 s at another, and tiny
    elsewhere: the second element's quotient is the e4m3 tie 1.8125 -> 1.75, while v * RN(1/s)
    codes 1.875 (as in fp8_quantizer_divides).  Returns (fp32 smooth vector, index of the
    absmax element, index of the tie element)."""
    f32 = np.float32
    un = u.double().view(-1).numpy().astype(np.float32)
    sm = np.full(un.shape, f32(2.0 ** -12), dtype=np.float32)

    def hit(target, ui):
        # an fp32 smooth value near target/u whose product with u rounds to the target, or None
        up = down = f32(target / float(ui))
        for _ in range(64):
            for c in (up, down):
                if f32(f32(ui) * c) == f32(target):
                    return c
            up, down = np.nextafter(up, f32(np.inf)), np.nextafter(down, f32(-np.inf))
        return None

    picked = []
    for target in (6.125, 203.0 / 8192.0):
        for i in range(un.size):
            c = hit(target, un[i]) if i not in picked and abs(un[i]) > 1e-3 else None
            if c is not None:
                sm[i] = c
                picked.append(i)
                break
        else:
            raise AssertionError("no element's smooth scale hits the target")
    return torch.from_numpy(sm), picked[0], picked[1]
