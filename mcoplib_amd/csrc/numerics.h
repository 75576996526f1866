// numerics.h -- scalar arithmetic shared by every row kernel of libmcop_norm.
//
// Everything here is plain IEEE-754 binary32/binary64 arithmetic, so the same source compiles
// for gfx950 (hipcc) and for the host (g++, used by the CPU test of mcop_fdiv_const).
#pragma once

#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#if defined(__HIP__)
#define MCOP_HD __host__ __device__ __attribute__((always_inline)) inline
#else
#define MCOP_HD static inline
#endif

// Correctly rounded quotient a / b for a divisor b that is fixed for a whole row, given
// inv == RN(1/b).  Markstein's correction: q0 = RN(a*inv) is within one ulp of a/b, the
// remainder r = a - q0*b is exact in one FMA, and RN(q0 + r*inv) == RN(a/b) (Markstein,
// IBM J. Res. Dev. 34(1), 1990; Muller et al., Handbook of Floating-Point Arithmetic, 2nd ed.,
// sec. 4.9).  The theorem excludes underflow and overflow of the intermediate terms, so
// numerators or quotients outside [2^-100, 2^100] (and every non-finite case) take the full
// division instead; a == +-0 returns q0 = a * inv, which carries the quotient's sign (the
// correction step would turn -0 into +0).
// `b_ok` is the caller's once-per-row check that b itself is in [2^-100, 2^100].
MCOP_HD float mcop_fdiv_const(float a, float b, float inv, bool b_ok) {
  const float q0 = a * inv;
  const float r = __builtin_fmaf(-q0, b, a);
  const float q = __builtin_fmaf(r, inv, q0);
  const float aa = __builtin_fabsf(a);
  const float aq = __builtin_fabsf(q);
  const bool fast = b_ok && aa >= 0x1p-100f && aq >= 0x1p-100f && aq <= 0x1p100f;
  return fast ? q : ((b_ok && a == 0.0f) ? q0 : a / b);
}

MCOP_HD bool mcop_divisor_ok(float b) {
  const float ab = __builtin_fabsf(b);
  return ab >= 0x1p-100f && ab <= 0x1p100f;
}

// 1/sqrt(ss/H + eps) with every step correctly rounded to binary32: the fp64 sum of squares is
// rounded once to fp32, then the fp32 quotient, the fp32 sum with eps, the fp32 square root and
// the fp32 reciprocal.  Each fp32 step is evaluated in binary64 and rounded once; for / and
// sqrt that equals the correctly rounded binary32 result because 53 >= 2*24 + 2.
MCOP_HD float mcop_inv_rms(double ss64, int64_t hidden, float eps) {
  const float ss = (float)ss64;
  const float ms = (float)((double)ss / (double)(float)hidden);
  const float v = ms + eps;
  const float r = (float)__builtin_sqrt((double)v);
  return (float)(1.0 / (double)r);
}

// Correctly rounded binary32 quotient n / d for the once-per-row scale computations.
MCOP_HD float mcop_div_rn(float n, float d) { return (float)((double)n / (double)d); }
