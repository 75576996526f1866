/*
 * mcop_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement, in plain C, of the reference (MetaX-MACA/mcoplib) algorithms of the fused
 * RMSNorm + per-token quantization path.  It is the checker for libmcop_norm.so and the CPU
 * baseline timed by bench.py; nothing in the product links, imports or calls it.
 *
 * Arithmetic contract (shared with the GPU kernels, stated here independently of them):
 *   - every fp32 operation is a single correctly rounded IEEE binary32 operation, in the order
 *     the reference writes it (compile with -ffp-contract=off, no fast-math);
 *   - the row sum of squares is the binary32 rounding of the (compensated, Neumaier) binary64
 *     sum of the exact squares -- i.e. the correctly rounded sum for all practical inputs.  The
 *     reference sums in binary32 in cub's BlockReduce order, which is unknowable; the
 *     difference is one of reduction order only;
 *   - rsqrtf of the reference is replaced by 1/sqrtf, both steps correctly rounded;
 *   - conversions to bf16 / fp16 / fp8-e4m3fn round to nearest even (written from the formats'
 *     definitions, not from any library).
 * Rows are independent; the row loops run in parallel with OpenMP (results do not depend on
 * the thread count).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2, DT_I8 = 3, DT_FP8 = 4 };

/* ---------------------------------------------------------------- format conversions */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16 = the upper 16 bits of binary32; RNE on the dropped 16 bits; NaN stays NaN (quiet). */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16: 1/5/10, bias 15.  Decoding is exact; encoding rounds to nearest even with
   gradual underflow and overflow to infinity. */
static float f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0x1f) return u2f(s | 0x7f800000u | (m << 13));
  if (e == 0) { float v = ldexpf((float)m, -24); return s ? -v : v; }
  return u2f(s | ((e + 112u) << 23) | (m << 13));
}
uint16_t oracle_f32_to_f16(float f) {
  const uint16_t s = (uint16_t)((f2u(f) >> 16) & 0x8000u);
  if (isnan(f)) return (uint16_t)(s | 0x7e00u);
  const float a = fabsf(f);
  if (a >= 65520.0f) return (uint16_t)(s | 0x7c00u); /* 65520 = midpoint 65504..65536 -> inf */
  if (a < 0x1p-14f) {                                 /* subnormal: multiples of 2^-24 */
    const float m = rintf(a * 0x1p24f);               /* exact scaling, RNE to an integer */
    return (uint16_t)(s | (uint16_t)m);               /* m == 1024 is the smallest normal */
  }
  int e2;
  frexpf(a, &e2);
  int E = e2 - 1;                                     /* a in [2^E, 2^(E+1)) */
  float m = rintf(ldexpf(a, 10 - E));                 /* in [1024, 2048] */
  if (m == 2048.0f) { m = 1024.0f; ++E; }
  if (E > 15) return (uint16_t)(s | 0x7c00u);
  return (uint16_t)(s | (uint16_t)((E + 15) << 10) | (uint16_t)((int)m - 1024));
}

/* OCP fp8 E4M3FN: 1/4/3, bias 7, no infinities, 0x7f / 0xff are NaN, max finite 448 (0x7e).
   RNE; finite magnitudes beyond 448 saturate to 448 (callers clamp first anyway). */
uint8_t oracle_f32_to_e4m3fn(float f) {
  const uint8_t s = (uint8_t)((f2u(f) >> 24) & 0x80u);
  if (isnan(f)) return (uint8_t)(s | 0x7fu);
  const float a = fabsf(f);
  if (a >= 448.0f) return (uint8_t)(s | 0x7eu);
  if (a < 0x1p-6f) {                                  /* subnormal: multiples of 2^-9 */
    const float m = rintf(a * 0x1p9f);                /* 0..8; 8 is the smallest normal */
    return (uint8_t)(s | (uint8_t)m);
  }
  int e2;
  frexpf(a, &e2);
  int E = e2 - 1;
  float m = rintf(ldexpf(a, 3 - E));                  /* in [8, 16] */
  if (m == 16.0f) { m = 8.0f; ++E; }
  unsigned code = (unsigned)((E + 7) << 3) | (unsigned)((int)m - 8);
  if (code > 0x7eu) code = 0x7eu;
  return (uint8_t)(s | code);
}

static inline float load_el(const void* p, int dt, int64_t i) {
  switch (dt) {
    case DT_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case DT_F16: return f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}
/* round to the dtype (the value a store followed by a load would give) */
static inline float rnd_el(float f, int dt) {
  switch (dt) {
    case DT_BF16: return bf16_to_f32(oracle_f32_to_bf16(f));
    case DT_F16: return f16_to_f32(oracle_f32_to_f16(f));
    default: return f;
  }
}
static inline void store_el(void* p, int dt, int64_t i, float f) {
  switch (dt) {
    case DT_BF16: ((uint16_t*)p)[i] = oracle_f32_to_bf16(f); break;
    case DT_F16: ((uint16_t*)p)[i] = oracle_f32_to_f16(f); break;
    default: ((float*)p)[i] = f; break;
  }
}

/* ---------------------------------------------------------------- shared steps */

/* Neumaier-compensated binary64 accumulation of exact squares (a*a is exact in binary64). */
typedef struct { double s, c; } acc64;
static inline void acc_add(acc64* A, double x) {
  const double t = A->s + x;
  if (fabs(A->s) >= fabs(x)) A->c += (A->s - t) + x; else A->c += (x - t) + A->s;
  A->s = t;
}
/* An infinite or NaN term makes the compensation NaN (inf - inf); the plain sum is then the
   binary64 sum of the terms, as for any other order. */
static inline double acc_val(const acc64* A) { return isfinite(A->s) ? A->s + A->c : A->s; }

/* rho = 1 / sqrt(ss/H + eps): the reference's `rsqrtf(ss / hidden_size + epsilon)`
   (e.g. op/vllm/quantization/fused_kernels/layernorm_utils.cuh:273-274) with each binary32
   step correctly rounded. */
static inline float inv_rms(double ss64, int64_t H, float eps) {
  const float ss = (float)ss64;
  const float ms = ss / (float)H;
  const float v = ms + eps;
  return 1.0f / sqrtf(v);
}

/* rne to int with NaN -> 0, then saturate to [lo, 127]. */
static inline int8_t q_int8(float v, int lo) {
  if (isnan(v)) return 0;
  float t = rintf(v);
  if (t < (float)lo) t = (float)lo;
  if (t > 127.0f) t = 127.0f;
  return (int8_t)(int)t;
}

/* fmin/fmax clamp as float_to_fp8 (quant_conversions.cuh:23-28): NaN -> +448. */
static inline uint8_t q_fp8(float v) { return oracle_f32_to_e4m3fn(fmaxf(-448.0f, fminf(v, 448.0f))); }

/* ---------------------------------------------------------------- H1 */

/* vLLM fused_add_rms_norm, op/vllm/layernorm_kernels.cu:92-144 (bf16/fp16 width-8 kernel, with
   the packed add/multiply of op/vllm/type_convert.cuh:104-165) and :149-182 (generic kernel):
     z = b(x + r); r <- z; V = sum z^2 on the rounded z; rho = 1/sqrt(V/H + eps);
     x <- b(b(z * rho) * w).
   A bf16x2/half2 add or multiply rounds the exact result once; the binary32 add/multiply of two
   16-bit values followed by one rounding gives the same value (binary32 holds the exact product,
   and for the sum 24 >= 2*11 + 2 makes the double rounding innocuous). */
void oracle_fused_add_rms_norm(void* x, int64_t xstride, void* r, const void* w, int64_t T,
                               int64_t H, int dt, float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    acc64 A = {0.0, 0.0};
    for (int64_t i = 0; i < H; ++i) {
      const float z = rnd_el(load_el(x, dt, t * xstride + i) + load_el(r, dt, t * H + i), dt);
      store_el(r, dt, t * H + i, z);
      acc_add(&A, (double)z * (double)z);
    }
    const float rho = inv_rms(acc_val(&A), H, eps);
    for (int64_t i = 0; i < H; ++i) {
      const float z = load_el(r, dt, t * H + i);
      const float y = rnd_el(z * rho, dt) * load_el(w, dt, i);
      store_el(x, dt, t * xstride + i, y);
    }
  }
}

/* ---------------------------------------------------------------- H2 / H3 */

/* vLLM rms_norm_dynamic_per_token_quant,
   op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:14-47 with
   vectorized::compute_rms (layernorm_utils.cuh:223-279), compute_dynamic_per_token_scales
   (:394-454) and norm_and_quant (:457-535); the same operation as mcoplib's
   rms_norm_dynamic_per_token_quant_custom (op/rms_norm_dynamic_per_token_quant.cu:16-92):
     a = x (+ r); r <- b(a); rho from sum a^2 (unrounded); y = b(b(a*rho) * w);
     A = max|y|, A = min(A, ub);
     int8: s = max(A/127, FLT_EPSILON) (op/vllm/quantization/utils.cuh:46-51), inv = 1/s
           (fused_..._quant.cu:37), q = sat[-128,127](rne(y*inv)) -- the intended
           float_to_int8_rn (the reference's MACA helper, quant_conversions.cuh:15-21, stores the
           rounded value in a uint32_t and cannot produce correct codes);
     fp8:  s = max(A/448, 1/(448*512)), q = e4m3fn(clamp(y/s, +-448)) (quant_conversions.cuh:23-28).
   `scale_ub` is a host pointer here (NULL = none). */
void oracle_rms_norm_quant(void* out, int out_dt, float* scales, const void* x, const void* w,
                           const float* scale_ub, void* r, int64_t T, int64_t H, int dt,
                           float eps) {
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      acc64 A = {0.0, 0.0};
      for (int64_t i = 0; i < H; ++i) {
        float v = load_el(x, dt, t * H + i);
        if (r) v += load_el(r, dt, t * H + i);
        a[i] = v;
        acc_add(&A, (double)v * (double)v);
      }
      if (r) for (int64_t i = 0; i < H; ++i) store_el(r, dt, t * H + i, a[i]);
      const float rho = inv_rms(acc_val(&A), H, eps);
      float amax = 0.0f;
      for (int64_t i = 0; i < H; ++i) {
        a[i] = rnd_el(rnd_el(a[i] * rho, dt) * load_el(w, dt, i), dt);
        amax = fmaxf(amax, fabsf(a[i]));
      }
      if (scale_ub) amax = fminf(amax, *scale_ub);
      if (out_dt == DT_I8) {
        const float s = fmaxf(amax / 127.0f, FLT_EPSILON);
        const float inv = 1.0f / s;
        scales[t] = s;
        for (int64_t i = 0; i < H; ++i) ((int8_t*)out)[t * H + i] = q_int8(a[i] * inv, -128);
      } else {
        const float s = fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
        scales[t] = s;
        for (int64_t i = 0; i < H; ++i) ((uint8_t*)out)[t * H + i] = q_fp8(a[i] / s);
      }
    }
    free(a);
  }
}

/* vLLM rms_norm_per_block_quant,
   op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:92-126,194-270
   with vectorized::compute_rms (layernorm_utils.cuh:223-279), the group branch of
   compute_dynamic_per_token_scales (:283-360) and norm_and_quant (:455-535):
     a, r <- b(a), rho and y = b(b(a*rho) * w) as in oracle_rms_norm_quant;
     per group g of G elements: A_g = max|y| (min with ub);
     int8: s_g = max(A_g/127, FLT_EPSILON), q = sat[-128,127](rne(y * (1/s_g)));
     fp8:  s_g = max(A_g/448, 1/(448*512)), q = e4m3fn(clamp(y/s_g, +-448));
     scales[t*(H/G) + g], or scales[g*T + t] when `transposed`. */
void oracle_rms_norm_per_block_quant(void* out, int out_dt, float* scales, const void* x,
                                     const void* w, const float* scale_ub, void* r, int64_t T,
                                     int64_t H, int dt, float eps, int64_t G, int transposed) {
  const int64_t NG = H / G;
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      acc64 A = {0.0, 0.0};
      for (int64_t i = 0; i < H; ++i) {
        float v = load_el(x, dt, t * H + i);
        if (r) v += load_el(r, dt, t * H + i);
        a[i] = v;
        acc_add(&A, (double)v * (double)v);
      }
      if (r) for (int64_t i = 0; i < H; ++i) store_el(r, dt, t * H + i, a[i]);
      const float rho = inv_rms(acc_val(&A), H, eps);
      for (int64_t i = 0; i < H; ++i) a[i] = rnd_el(rnd_el(a[i] * rho, dt) * load_el(w, dt, i), dt);
      for (int64_t g = 0; g < NG; ++g) {
        float amax = 0.0f;
        for (int64_t i = g * G; i < (g + 1) * G; ++i) amax = fmaxf(amax, fabsf(a[i]));
        if (scale_ub) amax = fminf(amax, *scale_ub);
        const float s = out_dt == DT_I8 ? fmaxf(amax / 127.0f, FLT_EPSILON)
                                        : fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
        scales[transposed ? g * T + t : t * NG + g] = s;
        if (out_dt == DT_I8) {
          const float inv = 1.0f / s;
          for (int64_t i = g * G; i < (g + 1) * G; ++i)
            ((int8_t*)out)[t * H + i] = q_int8(a[i] * inv, -128);
        } else {
          for (int64_t i = g * G; i < (g + 1) * G; ++i)
            ((uint8_t*)out)[t * H + i] = q_fp8(a[i] / s);
        }
      }
    }
    free(a);
  }
}

/* mcoplib rms_norm_dynamic_per_token_quant_custom (int8 only),
   op/rms_norm_dynamic_per_token_quant.cu:266-285 with its two kernels:
   H != 7168 (:52-92; kernel/rms_norm_vllm.cuh:330-454): y = b(b(a*rho) * w) as above;
     A = max|y| (min with ub); s = max(A / 127, 1.5e-6) evaluated as the reference writes it
     (a float quotient against a double literal, :382); inv = 1.0f / s (:89);
     q = sat[-127,127](rne(y * inv)) (float_to_int8_rn of kernel/utils.h:219-226);
   H == 7168 (:94-186): p = a * w (fp32, :146-149); A = max|p|; s = max((A * rho) / 127,
     FLT_EPSILON) (:170-171); inv = 1.0f / s (:172); q = sat[-127,127](rne((p * rho) * inv))
     (:179-182); ub is not read.  r <- b(a) in both. */
void oracle_rms_norm_quant_custom(int8_t* out, float* scales, const void* x, const void* w,
                                  const float* scale_ub, void* r, int64_t T, int64_t H, int dt,
                                  float eps) {
  const int h7168 = H == 7168;
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      acc64 S = {0.0, 0.0};
      for (int64_t i = 0; i < H; ++i) {
        float v = load_el(x, dt, t * H + i);
        if (r) v += load_el(r, dt, t * H + i);
        a[i] = v;
        acc_add(&S, (double)v * (double)v);
      }
      if (r) for (int64_t i = 0; i < H; ++i) store_el(r, dt, t * H + i, a[i]);
      const float rho = inv_rms(acc_val(&S), H, eps);
      float amax = 0.0f;
      for (int64_t i = 0; i < H; ++i) {
        const float wf = load_el(w, dt, i);
        a[i] = h7168 ? a[i] * wf : rnd_el(rnd_el(a[i] * rho, dt) * wf, dt);
        amax = fmaxf(amax, fabsf(a[i]));
      }
      float s;
      if (h7168) {
        s = fmaxf((amax * rho) / 127.0f, FLT_EPSILON);
      } else {
        if (scale_ub) amax = fminf(amax, *scale_ub);
        s = (float)fmax((double)(amax / 127.0f), 1.5e-6);
      }
      const float inv = 1.0f / s;
      scales[t] = s;
      for (int64_t i = 0; i < H; ++i)
        out[t * H + i] = q_int8((h7168 ? a[i] * rho : a[i]) * inv, -127);
    }
    free(a);
  }
}

/* ---------------------------------------------------------------- H4 */

/* mcoplib rms_norm_dynamic_per_token_quant (fused_rms_norm_dq), op/fused_rms_norm_dq.cu:260-303
   with compute_rms (:69-99), compute_dynamic_per_token_scales (:125-161), norm_and_quant
   (:163-186):
     a = x (+ r, not written back); after_res <- b(a); rho from sum a^2 (unrounded);
     the later passes read a~ = b(a) back (:244, :250);
     u = (a~ / rho) * w  -- the reference divides by rho = rsqrt(...) (:139, :179);
         with `standard` != 0: u = (a~ * rho) * w;
     after_norm <- b(u); v = u * sm; A = max|v|;
     int8: s = A / 127.0 (:154; binary64 quotient rounded to binary32 == the binary32 quotient),
           q = sat[-127,127](rne(v * (1/s))) (kernel/utils.h:219-226);
     fp8: this library's own extension (BASELINE cfg 4), with no counterpart in the reference:
          its entry accepts int8 only (:658), ScaledQuant is defined for int8 only (:51-66), so
          the fp8 branch at :299-301 cannot be instantiated, and its scale is A/127 for any
          output (:154).  Defined here as s = A/448, q = e4m3fn(clamp(v / s)) with the
          correctly rounded quotient, the form of the path's fp8 quantizers
          (op/vllm/quantization/fused_kernels/quant_conversions.cuh:52-59).
     A == 0: s = 0 and q = 0 (the reference computes 0 * inf, or 0 / 0 for fp8).
   w and sm are each stored as w_dt / sm_dt (the input dtype or fp32). */
void oracle_rms_norm_smooth_quant(void* out, int out_dt, float* scales, const void* x,
                                  const void* w, int w_dt, const void* sm, int sm_dt,
                                  void* after_res, void* after_norm, const void* r, int64_t T,
                                  int64_t H, int dt, float eps, int standard) {
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      acc64 A = {0.0, 0.0};
      for (int64_t i = 0; i < H; ++i) {
        float v = load_el(x, dt, t * H + i);
        if (r) v += load_el(r, dt, t * H + i);
        acc_add(&A, (double)v * (double)v);
        a[i] = rnd_el(v, dt);
        if (after_res) store_el(after_res, dt, t * H + i, v);
      }
      const float rho = inv_rms(acc_val(&A), H, eps);
      float amax = 0.0f;
      for (int64_t i = 0; i < H; ++i) {
        const float n = standard ? a[i] * rho : a[i] / rho;
        const float u = n * load_el(w, w_dt, i);
        if (after_norm) store_el(after_norm, dt, t * H + i, u);
        a[i] = u * load_el(sm, sm_dt, i);
        amax = fmaxf(amax, fabsf(a[i]));
      }
      const float s = amax / (out_dt == DT_I8 ? 127.0f : 448.0f);
      const float inv = amax > 0.0f ? 1.0f / s : 0.0f;
      scales[t] = s;
      for (int64_t i = 0; i < H; ++i) {
        if (out_dt == DT_I8) ((int8_t*)out)[t * H + i] = q_int8(a[i] * inv, -127);
        else ((uint8_t*)out)[t * H + i] = amax > 0.0f ? q_fp8(a[i] / s) : 0;
      }
    }
    free(a);
  }
}

/* ---------------------------------------------------------------- H5 */

/* mcoplib scale_dynamic_quant, op/scale_dynamic_quant.cu:40-104:
     v = f(h) * sm (fp32); A = max|v|; scales[t] = A * 0.00787401574803f (:75);
     inv = 127.0f / A (:79); q = sat[-128,127](rne(v * inv)) (:88-91); A == 0 gives q = 0. */
void oracle_scale_dynamic_quant(int8_t* out, float* scales, const uint16_t* h, const float* sm,
                                int64_t T, int64_t H) {
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      float amax = 0.0f;
      for (int64_t i = 0; i < H; ++i) {
        a[i] = bf16_to_f32(h[t * H + i]) * sm[i];
        amax = fmaxf(amax, fabsf(a[i]));
      }
      scales[t] = amax * 0.00787401574803f;
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      for (int64_t i = 0; i < H; ++i) out[t * H + i] = q_int8(a[i] * inv, -128);
    }
    free(a);
  }
}

/* ---------------------------------------------------------------- standalone per-token quant */

/* float -> int32, round to nearest even, saturating; NaN -> 0 (the hardware conversion's NaN
   result, as in the reference's azp_t(zp) at int8_quant_kernels.cu:406). */
static inline int32_t cvt_sat_i32(float v) {
  if (isnan(v)) return 0;
  const float t = rintf(v);
  if (t >= 2147483648.0f) return INT32_MAX;
  if (t <= -2147483648.0f) return INT32_MIN;
  return (int32_t)t;
}

/* The reference's float_to_int32_rn (int8_quant_kernels.cu:27-35): x = min(x, 2^31),
   x = max(x, -2^31) with fmin/fmax semantics, then the saturating conversion -- so NaN becomes
   2^31 and converts to INT32_MAX. */
static inline int32_t float_to_int32_rn(float v) {
  v = fminf(v, 2147483648.0f);
  v = fmaxf(v, -2147483648.0f);
  return cvt_sat_i32(v);
}

/* vLLM dynamic_scaled_int8_quant without azp,
   op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:94-132 (generic kernel) and the
   register / LDS variants the host selects for 16-bit inputs (:167-339, chosen at :480-518),
   which do the same arithmetic:
     A = max|x|; scales[t] = A / 127; inv = 127 / A (0 when A == 0);
     q = sat[-127,127](rne(x * inv)) (float_to_int8_rn, :14-24).
   The variants compute 127 / A without the zero test; for A == 0 that gives 0 * inf = NaN,
   which the conversion maps to 0 -- the same codes. */
void oracle_dynamic_scaled_int8_quant(int8_t* out, float* scales, const void* x, int64_t T,
                                      int64_t H, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    float amax = 0.0f;
    for (int64_t i = 0; i < H; ++i) amax = fmaxf(amax, fabsf(load_el(x, dt, t * H + i)));
    scales[t] = amax / 127.0f;
    const float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
    for (int64_t i = 0; i < H; ++i) out[t * H + i] = q_int8(load_el(x, dt, t * H + i) * inv, -127);
  }
}

/* vLLM dynamic_scaled_int8_quant with azp (asymmetric), int8_quant_kernels.cu:370-422:
     s = (max x - min x) / 255; zp = (int32) nearbyint(-128 - min x / s); inv = 1 / s;
     q = sat[-128,127](float_to_int32_rn(x * inv) + zp)  (int32_to_int8, :37-46);
   a NaN element therefore codes 127.  The integer sum is formed in 64 bits, so it saturates
   instead of overflowing: the reference's int32 sum overflows, which C leaves undefined, for a
   NaN element or a product of +inf with zp > 0, and for a product of -inf with zp < 0 (inv =
   1 / s is infinite when s is subnormal, a row of tiny values); here those code 127, 127 and
   -128, the codes of the clamped values.
   A constant row (s == 0) has no zero point -- the reference converts NaN / inf to int there,
   which has no defined result; this restatement writes s = 0, zp = -128 and q = -128. */
void oracle_dynamic_scaled_int8_azp_quant(int8_t* out, float* scales, int32_t* azp,
                                          const void* x, int64_t T, int64_t H, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    float mx = -INFINITY, mn = INFINITY;
    for (int64_t i = 0; i < H; ++i) {
      const float v = load_el(x, dt, t * H + i);
      mx = fmaxf(mx, v);
      mn = fminf(mn, v);
    }
    const float s = (mx - mn) / 255.0f;
    const int degenerate = !(s > 0.0f);
    const int32_t zp = degenerate ? -128 : cvt_sat_i32(-128.0f - mn / s);
    const float inv = degenerate ? 0.0f : 1.0f / s;
    scales[t] = s;
    azp[t] = zp;
    for (int64_t i = 0; i < H; ++i) {
      int64_t q = (int64_t)float_to_int32_rn(load_el(x, dt, t * H + i) * inv) + zp;
      q = q < -128 ? -128 : (q > 127 ? 127 : q);
      out[t * H + i] = (int8_t)q;
    }
  }
}

/* vLLM dynamic_per_token_scaled_fp8_quant, op/vllm/quantization/fp8/common.cu:142-180
   (host :375-411), rows at in_stride / out_stride elements:
     A = max|x| (min with *scale_ub); s = max(A / 448, 1/(448*512)); q = e4m3fn(clamp(x / s)).
   `scale_ub` is a host pointer here (NULL = none). */
void oracle_dynamic_per_token_fp8_quant(uint8_t* out, float* scales, const void* x,
                                        const float* scale_ub, int64_t T, int64_t H,
                                        int64_t in_stride, int64_t out_stride, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    float amax = 0.0f;
    for (int64_t i = 0; i < H; ++i) amax = fmaxf(amax, fabsf(load_el(x, dt, t * in_stride + i)));
    if (scale_ub) amax = fminf(amax, *scale_ub);
    const float s = fmaxf(amax / 448.0f, 1.0f / (448.0f * 512.0f));
    scales[t] = s;
    for (int64_t i = 0; i < H; ++i)
      out[t * out_stride + i] = q_fp8(load_el(x, dt, t * in_stride + i) / s);
  }
}

/* ---------------------------------------------------------------- RMSNorm without quant */

/* The reference's choice between its vectorized and element-wise mcoplib norm kernels
   (op/fused_rms_norm_dq.cu:669-802, 814-978): vectors of n elements, n = 4 when the input or
   the weight is fp32 (float4 of fp32, or float2 of 16-bit values against fp32 weights), else 8;
   vectorized when H is a multiple of n and at most three vectors per thread of 1024 threads. */
static int mc_vectorized(int64_t H, int dt, int wdt) {
  const int64_t n = (dt == DT_F32 || wdt == DT_F32) ? 4 : 8;
  return H % n == 0 && H <= 3 * 1024 * n;
}

/* One mcoplib norm row: vectorized kernel (rms_norm_kernel_align :305-382,
   head_rms_norm_kernel_align :493-557): y = b((a * d) * w), d = rms_div ? (float)(1.0 / rho)
   : rho, a unrounded; element-wise kernels (norm_without_smooth :189-209, do_head_norm
   :212-224): y = b((a~ / rho) * w) or b((a~ * rho) * w), a~ the after_res value re-read. */
static void mc_norm_row(void* out, int64_t oo, const float* a, const void* w, int wdt,
                        int64_t wo, int64_t H, int dt, float rho, int rms_div, int vec) {
  if (vec) {
    const float d = rms_div ? (float)(1.0 / (double)rho) : rho;
    for (int64_t i = 0; i < H; ++i) store_el(out, dt, oo + i, (a[i] * d) * load_el(w, wdt, wo + i));
  } else {
    for (int64_t i = 0; i < H; ++i) {
      const float n = rms_div ? a[i] / rho : a[i] * rho;
      store_el(out, dt, oo + i, n * load_el(w, wdt, wo + i));
    }
  }
}

/* mcoplib.op.rms_norm, op/fused_rms_norm_dq.cu:980-998 (dispatch :814-978, kernels :305-420,
   compute_rms :69-99): a = x (+ r); after_res <- b(a) with a residual (r is not updated);
   rho = 1/sqrt(S/H + eps); out row as mc_norm_row. */
void oracle_rms_norm(void* out, const void* x, const void* w, int wdt, void* after_res,
                     const void* r, int64_t T, int64_t H, int dt, float eps, int rms_div) {
  const int vec = mc_vectorized(H, dt, wdt);
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      acc64 S = {0.0, 0.0};
      for (int64_t i = 0; i < H; ++i) {
        float v = load_el(x, dt, t * H + i);
        if (r) v += load_el(r, dt, t * H + i);
        acc_add(&S, (double)v * (double)v);
        if (r) {
          store_el(after_res, dt, t * H + i, v);
          if (!vec) v = rnd_el(v, dt);
        }
        a[i] = v;
      }
      mc_norm_row(out, t * H, a, w, wdt, 0, H, dt, inv_rms(acc_val(&S), H, eps), rms_div, vec);
    }
    free(a);
  }
}

/* mcoplib.op.head_rms_norm, op/fused_rms_norm_dq.cu:804-812 (dispatch :669-802, kernels
   :493-578): for every token t and head h in [off, off + hn) of x [T, NH, D], the row
   x[t, h, :] is normalized with weight row w[h, :] (rms_div always set); other heads of out
   are not written. */
void oracle_head_rms_norm(void* out, const void* x, const void* w, int wdt, int64_t T,
                          int64_t NH, int64_t D, int64_t off, int64_t hn, int dt, float eps) {
  const int vec = mc_vectorized(D, dt, wdt);
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)D * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t k = 0; k < T * hn; ++k) {
      const int64_t t = k / hn, h = off + k % hn, ro = (t * NH + h) * D;
      acc64 S = {0.0, 0.0};
      for (int64_t i = 0; i < D; ++i) {
        a[i] = load_el(x, dt, ro + i);
        acc_add(&S, (double)a[i] * (double)a[i]);
      }
      mc_norm_row(out, ro, a, w, wdt, h * D, D, dt, inv_rms(acc_val(&S), D, eps), 1, vec);
    }
    free(a);
  }
}

/* vLLM _C::rms_norm, op/vllm/layernorm_kernels.cu:15-86 (host :186-231), on contiguous rows:
   rho from S = sum x^2; y = b(b(x * rho) * w) (the 16-bit product rounds to 16 bits, :82). */
void oracle_vllm_rms_norm(void* out, const void* x, const void* w, int64_t T, int64_t H, int dt,
                          float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    acc64 S = {0.0, 0.0};
    for (int64_t i = 0; i < H; ++i) {
      const double v = load_el(x, dt, t * H + i);
      acc_add(&S, v * v);
    }
    const float rho = inv_rms(acc_val(&S), H, eps);
    for (int64_t i = 0; i < H; ++i)
      store_el(out, dt, t * H + i, rnd_el(load_el(x, dt, t * H + i) * rho, dt) * load_el(w, dt, i));
  }
}

/* ---------------------------------------------------------------- padded wire format */

/* mcoplib fused_add_rms_norm_dynamic_per_token_quant_padding_output,
   op/fused_add_layernorm_per_token_quant_padding_output.cu (entry :397-416, dispatch :344-395).
   Row t of `padded` (pad_bytes per row) receives the H codes at bytes [0, H) and the fp32 scale
   at bytes [H, H+4) (:216, :246, :255, :320); nothing else of the row is written.
   H == 7168, the "opt" kernel (:181-283), a = x + r in fp32:
     r <- b(a); p = a * w; A = max|p|; rho = 1/sqrt(S/H + eps);
     s = max((A * rho) / 127, FLT_EPSILON); u = p * rho; rms <- b(u);
     q = sat[-127,127](rne(u * (1/s)))  (float_to_int8_rn of kernel/utils.h:219-226).
   Other H, the generic kernel (:287-340): A = max|b(b(a) * w)| (bf16 product, :308);
     y = b(b(b(a) * rho) * w) (:334); q = sat[-127,127](rne(y * (1/s))); the reference writes
     only `padded` and r -- here rms <- y, q and scales[t] are written too. */
void oracle_add_rms_norm_quant_padded(uint8_t* padded, int64_t pad_bytes, uint16_t* rms,
                                      int8_t* q, float* scales, const uint16_t* x, uint16_t* r,
                                      const uint16_t* w, int64_t T, int64_t H, float eps) {
  const int opt = H == 7168;
#pragma omp parallel
  {
    float* a = (float*)malloc((size_t)H * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      acc64 S = {0.0, 0.0};
      float amax = 0.0f;
      for (int64_t i = 0; i < H; ++i) {
        const float v = bf16_to_f32(x[t * H + i]) + bf16_to_f32(r[t * H + i]);
        acc_add(&S, (double)v * (double)v);
        r[t * H + i] = oracle_f32_to_bf16(v);
        const float wf = bf16_to_f32(w[i]);
        if (opt) {
          a[i] = v * wf;
          amax = fmaxf(amax, fabsf(a[i]));
        } else {
          a[i] = bf16_to_f32(r[t * H + i]);
          amax = fmaxf(amax, fabsf(rnd_el(a[i] * wf, DT_BF16)));
        }
      }
      const float rho = inv_rms(acc_val(&S), H, eps);
      const float s = fmaxf((amax * rho) / 127.0f, FLT_EPSILON);
      const float inv = 1.0f / s;
      scales[t] = s;
      memcpy(padded + t * pad_bytes + H, &s, 4);
      for (int64_t i = 0; i < H; ++i) {
        float y;
        if (opt) {
          y = a[i] * rho;
          rms[t * H + i] = oracle_f32_to_bf16(y);
        } else {
          y = rnd_el(rnd_el(a[i] * rho, DT_BF16) * bf16_to_f32(w[i]), DT_BF16);
          rms[t * H + i] = oracle_f32_to_bf16(y);
        }
        const int8_t c = q_int8(y * inv, -127);
        q[t * H + i] = c;
        padded[t * pad_bytes + i] = (uint8_t)c;
      }
    }
    free(a);
  }
}

/* ---------------------------------------------------------------- elementwise fp8 */

void oracle_fp8_e4m3fn_from_f32(uint8_t* out, const float* in, int64_t n, float mul) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = q_fp8(in[i] * mul);
}

void oracle_f32_to_bf16_array(uint16_t* out, const float* in, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(in[i]);
}
void oracle_f32_to_f16_array(uint16_t* out, const float* in, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}
void oracle_f32_to_e4m3fn_array(uint8_t* out, const float* in, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_e4m3fn(in[i]);
}

int oracle_num_threads(void);
#ifdef _OPENMP
#include <omp.h>
int oracle_num_threads(void) { return omp_get_max_threads(); }
void oracle_set_threads(int n) { omp_set_num_threads(n); }
#else
int oracle_num_threads(void) { return 1; }
void oracle_set_threads(int n) { (void)n; }
#endif
