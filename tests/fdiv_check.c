/* Host check of mcop_fdiv_const (mcoplib_amd/csrc/numerics.h), the per-element division the
 * kernels use: it must equal the IEEE binary32 quotient a / b bit for bit.
 * Sweeps: every finite bf16 numerator x divisors (powers of two, small integers, their
 * reciprocals and random normal values over 2^-60..2^60); random fp32 numerators over the whole
 * exponent range (including subnormals, zeros, infinities and NaN) x random divisors.
 * Prints "checked N mismatches M" and exits non-zero on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../mcoplib_amd/csrc/numerics.h"

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int same(float x, float y) { return (isnan(x) && isnan(y)) || f2u(x) == f2u(y); }

static uint64_t mix(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int main(void) {
  long checked = 0, bad = 0;
  const int ND = 3000;
#pragma omp parallel for reduction(+ : checked, bad) schedule(dynamic, 16)
  for (int t = 0; t < ND; ++t) {
    float b;
    if (t < 64) b = ldexpf(1.0f, t - 32);
    else if (t < 192) b = (float)(t - 63);
    else if (t < 320) b = 1.0f / (float)(t - 191);
    else {
      const uint64_t z = mix((uint64_t)t);
      b = u2f((uint32_t)((67 + (z >> 40) % 120) << 23) | (uint32_t)(z & 0x7fffff));
    }
    const float inv = 1.0f / b;
    const bool ok = mcop_divisor_ok(b);
    for (uint32_t h = 0; h < 65536; ++h) {
      const float a = u2f(h << 16);
      if (isnan(a)) continue;
      const float q = mcop_fdiv_const(a, b, inv, ok);
      ++checked;
      if (!same(q, a / b)) ++bad;
    }
    uint64_t z = mix((uint64_t)t * 7919u + 1);
    for (int k = 0; k < 20000; ++k) {
      z = mix(z);
      const float a = u2f((uint32_t)z);
      const float q = mcop_fdiv_const(a, b, inv, ok);
      ++checked;
      if (!same(q, a / b)) ++bad;
    }
  }
  /* divisors outside the fast domain (and zero / infinity) always take the full division */
  const float odd[] = {0.0f, INFINITY, 1e-38f, 1e38f, 0x1p-101f, 0x1p101f};
  for (unsigned i = 0; i < sizeof(odd) / sizeof(odd[0]); ++i) {
    const float b = odd[i], inv = 1.0f / b;
    for (uint32_t h = 0; h < 65536; ++h) {
      const float a = u2f(h << 16);
      const float q = mcop_fdiv_const(a, b, inv, mcop_divisor_ok(b));
      ++checked;
      if (!same(q, a / b)) ++bad;
    }
  }
  printf("checked %ld mismatches %ld\n", checked, bad);
  return bad != 0;
}
