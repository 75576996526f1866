// rms_norm_quant.hip -- (residual add +) RMSNorm + dynamic per-token int8 / fp8-e4m3fn
// quantization, one pass over HBM.
//
// Semantics (per row, a = x [+ r] in fp32, b() = round to the input dtype):
//   residual <- b(a)                                   fused_..._quant.cu / layernorm_utils.cuh:503-508
//   rho = 1/sqrt(sum(a^2)/H + eps)                     layernorm_utils.cuh:245-276 (order: fp64 sum)
//   y = b(b(a*rho) * w)                                layernorm_utils.cuh:436,531
//   A = max|y|, min(A, *scale_ub)                      layernorm_utils.cuh:440-445
//   int8: s = max(A/127, FLT_EPSILON); q = sat[-128,127](rne(y * (1/s)))
//                                                      utils.cuh:46-51, fused_..._quant.cu:37
//   fp8 : s = max(A/448, 1/(448*512)); q = e4m3fn(clamp(y / s, +-448))  quant_conversions.cuh:23-28
// (paths relative to op/vllm/quantization/fused_kernels/ and op/vllm/quantization/ of the
// reference).
//
// mcoplib's own operator of the same name (rms_norm_dynamic_per_token_quant_custom,
// op/rms_norm_dynamic_per_token_quant.cu:266-285) is int8 only and differs in two ways (MODE):
//   QM_MC (any H but 7168; kernel/rms_norm_vllm.cuh:330-454): s = max(A/127, 1.5e-6) and
//     q = sat[-127,127](rne(y * (1/s))) (float_to_int8_rn of kernel/utils.h:219-226);
//   QM_MC_7168 (H == 7168; op/rms_norm_dynamic_per_token_quant.cu:94-186): no bf16 rounding
//     between a and the code: p = a * w, A = max|p|, s = max((A * rho)/127, FLT_EPSILON),
//     q = sat[-127,127](rne((p * rho) * (1/s))); scale_ub is not used.
//
// One pass: every lane loads all of its vectors of x, residual and weight before the first
// reduction and keeps the row in VGPRs; the residual is written back from registers, the codes
// are produced from registers, so HBM sees x and residual read once, residual and the codes
// written once (7*H + 4 bytes per bf16 row with residual).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <mutex>
#include <type_traits>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

enum QuantMode { QM_VLLM = 0, QM_MC = 1, QM_MC_7168 = 2 };

// The row's scale from its absmax (and rho for QM_MC_7168); *A receives the absmax after the
// scale bound.
template <bool FP8, int MODE>
__device__ __forceinline__ float row_scale(float amax, float rho, const float* scale_ub,
                                           float* A) {
  float a = amax;
  if (MODE != QM_MC_7168 && scale_ub != nullptr) a = __builtin_fminf(a, *scale_ub);
  *A = a;
  if constexpr (FP8) {
    return __builtin_fmaxf(mcop_div_rn(a, 448.0f), 1.0f / 229376.0f);
  } else if constexpr (MODE == QM_MC_7168) {
    return __builtin_fmaxf(mcop_div_rn(a * rho, 127.0f), FLT_EPSILON);
  } else {
    return __builtin_fmaxf(mcop_div_rn(a, 127.0f), MODE == QM_MC ? 1.5e-6f : FLT_EPSILON);
  }
}

// Codes of one vector of y (of p = a * w for QM_MC_7168).  `bounded`: no scale bound cut the
// row's absmax; `has_ub`: a scale bound was given.
template <class E, int VEC, bool FP8, int MODE>
__device__ __forceinline__ Pack<uint8_t, VEC> row_codes(const float* y, float rho, float s,
                                                        float inv, bool s_ok, bool bounded,
                                                        bool has_ub) {
  Pack<uint8_t, VEC> q;
  constexpr int LO = MODE == QM_VLLM ? -128 : -127;
  if constexpr (FP8) {
    q = fp8_quotient_codes<VEC>(y, s, inv, s_ok, bounded);
  } else if (std::is_same_v<E, F32> || (MODE != QM_MC_7168 && has_ub)) {
    // fp32 inputs can carry NaN payloads in the low byte, and a scale bound lets |y * inv|
    // exceed 127: round, convert and saturate
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = MODE == QM_MC_7168 ? y[e] * rho : y[e];
      q.v[e] = q_i8<LO>(t * inv);
    }
  } else {
    // |t * inv| < 127.5: the code cannot saturate (nor reach -128)
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = MODE == QM_MC_7168 ? y[e] * rho : y[e];
      q.v[e] = q_i8_in_range(t, inv);
    }
  }
  return q;
}

// With eight vectors a lane the bf16 int8 kernel asks for four waves per SIMD (at most 128
// VGPRs, which it meets without spilling): left free it took 140 VGPRs and three waves, one
// 512-lane workgroup per CU, and rows of 20480-32768 bf16 elements ran 14-20% slower.  The fp8
// forms, and fp16 (whose conversions need more registers), would spill under that bound and keep
// the default.
// EX (exact): the workgroup holds one row and every lane owns NV vectors of it (tpr ==
// blockDim.x, NV * tpr == hidden / VEC, one workgroup per row).  The row index is then uniform,
// so the row's base addresses are scalar and each vector's 32-bit offset serves every tensor,
// and the bounds tests and the out-of-row handling drop out: a shorter per-row chain (measured
// 12% less per decode call at T = 1-64 x 5120, about 0.5% at 8192 x 8192).
template <class E, int VEC, int NV, bool FP8, bool RES, int MODE, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
__attribute__((amdgpu_waves_per_eu(NV == 8 && !FP8 && std::is_same<E, BF16>::value ? 4 : 1)))
k_rms_norm_quant(uint8_t* __restrict__ out, float* __restrict__ scales,
                 const typename E::S* __restrict__ x, const typename E::S* __restrict__ w,
                 const float* __restrict__ scale_ub, typename E::S* __restrict__ res,
                 int64_t rows, int hidden, int tpr, float eps) {
  using S = typename E::S;
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  RowPos p;
  if constexpr (EX) {
    p = row_pos_one();
  } else {
    p = row_pos(rows, tpr);
  }
  const int nvec = hidden / VEC;
  const int64_t base = p.row * (int64_t)hidden;
  const int64_t lbase = p.lrow * (int64_t)hidden;
  auto lj_of = [&](int v) {  // element offset of the lane's vector v (loads)
    const int j = vec_index(v, tpr, p.lt);
    return (int64_t)(EX ? j : load_index(j, nvec)) * VEC;
  };

  // All loads first, unconditionally (out-of-row lanes re-read vector 0 of their row).
  Pack<S, VEC> xv[NV], rv[NV], wv[NV];
  if constexpr (NV >= 4) {
#pragma unroll
    for (int v = 0; v < NV; ++v) wv[v] = ld<S, VEC>(row_elem<EX>(w, 0, lj_of(v)));
    shared_loads_first();
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t lj = lj_of(v);
    xv[v] = ld_nt<S, VEC>(row_elem<EX>(x, lbase, lj));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(row_elem<EX>(res, lbase, lj));
    // with fewer vectors per lane the weight loads interleave with the streamed ones (measured
    // 1.5% faster at 8192 x 8192, two vectors per lane; shared-first won at four)
    if constexpr (NV < 4) wv[v] = ld<S, VEC>(row_elem<EX>(w, 0, lj));
  }

  float a[NV][VEC];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    const bool in = EX || j < nvec;
    // Lanes past the row end hold a copy of vector 0: it must not count in the sum.
    double vs = 0.0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float t = E::to_f(xv[v].v[e]);
      if constexpr (RES) t += E::to_f(rv[v].v[e]);
      a[v][e] = t;
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
    }
    ss += in ? vs : 0.0;
    if constexpr (RES) {
      if (p.live && in) {
        Pack<S, VEC> o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(a[v][e]);
        st_nt<S, VEC>(row_elem<EX>(res, base, (int64_t)j * VEC), o);
      }
    }
  }

  ss = row_reduce<EX>(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);

  // The absmax must skip the copies of vector 0 held past the row end: with an in-place
  // residual that copy may read vector 0's residual after its owner stored the sum there.
  // Rows that fill every lane (the common case) skip the test.
  const bool full = EX || (int64_t)NV * tpr == nvec;
  float amax = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const bool in = full || vec_index(v, tpr, p.lt) < nvec;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      // QM_MC_7168 keeps p = a * w unrounded (its code is rne((p * rho) * inv))
      const float y = MODE == QM_MC_7168
                          ? a[v][e] * E::to_f(wv[v].v[e])
                          : rnd<E>(rnd<E>(a[v][e] * rho) * E::to_f(wv[v].v[e]));
      a[v][e] = y;
      amax = __builtin_fmaxf(amax, in ? __builtin_fabsf(y) : 0.0f);
    }
  }
  amax = row_reduce<EX>(amax, red_max, tpr, MaxOp());

  float A;
  const float s = row_scale<FP8, MODE>(amax, rho, scale_ub, &A);
  if (p.live && p.lt == 0) scales[p.row] = s;
  const float inv = mcop_div_rn(1.0f, s);
  const bool s_ok = mcop_divisor_ok(s);
  const bool bounded = A == amax && s <= 0x1p100f;  // no scale bound cut the row's absmax

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    if (p.live && (EX || j < nvec)) {
      const Pack<uint8_t, VEC> q =
          row_codes<E, VEC, FP8, MODE>(a[v], rho, s, inv, s_ok, bounded, scale_ub != nullptr);
      st_nt<uint8_t, VEC>(row_elem<EX>(out, base, (int64_t)j * VEC), q);
    }
  }
}

// Rows too wide for the registers (QM_VLLM and QM_MC; QM_MC_7168 rows always fit): one
// 1024-lane workgroup per row and three passes over it -- sum of squares; absmax of y; codes and
// the residual.  The row's head (the first NC vectors of every lane: 8 x 1024 16-byte vectors
// without a residual, 5 x 1024 with one -- as many as fit 128 VGPRs without spilling) stays in
// registers across the passes, the next NL vectors (128 KB) in LDS; the rest is re-read each
// pass.  The residual is written in the last pass only, by the lane that read it, as the
// reference's multi-pass kernels do.
template <class E, int VEC, bool FP8, bool RES, int MODE>
__global__ void __launch_bounds__(kWideLanes)
k_rms_norm_quant_wide(uint8_t* __restrict__ out, float* __restrict__ scales,
                      const typename E::S* __restrict__ x, const typename E::S* __restrict__ w,
                      const float* __restrict__ scale_ub, typename E::S* __restrict__ res,
                      int hidden, float eps) {
  static_assert(MODE != QM_MC_7168, "7168-wide rows fit the register-resident kernel");
  using S = typename E::S;
  constexpr int NC = VEC > 1 ? (RES ? 5 : (FP8 && std::is_same<E, F16>::value ? 7 : 8)) : 16;
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int64_t base = (int64_t)blockIdx.x * hidden;
  // the head, loaded once (lanes past the row end hold nothing and skip it)
  Pack<S, VEC> xc[NC], rc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = c * tpr + (int)threadIdx.x;
    if (j < nvec) {
      xc[c] = ld<S, VEC>(x + base + (int64_t)j * VEC);
      if constexpr (RES) rc[c] = ld<S, VEC>(res + base + (int64_t)j * VEC);
    }
  }
  // The next NL vectors of every lane are held in LDS: lane-private slots (vector c of lane t
  // at [c][t]: consecutive lanes, consecutive 16-byte slots), so no barrier is needed.  The
  // workgroup already fills a CU's registers, so the 128 KB cost no occupancy.
  constexpr int NL = VEC > 1 ? (RES ? 4 : 8) : 0;
  constexpr int NLS = NL > 0 ? NL * (RES ? 2 : 1) : 1;
  __shared__ Pack<S, VEC> lds[NLS][kWideLanes];
  const int tid = (int)threadIdx.x;
#pragma unroll
  for (int c = 0; c < NL; ++c) {
    const int j = (NC + c) * tpr + tid;
    if (j < nvec) {
      lds[c][tid] = ld<S, VEC>(x + base + (int64_t)j * VEC);
      if constexpr (RES) lds[NL + c][tid] = ld<S, VEC>(res + base + (int64_t)j * VEC);
    }
  }
  auto a_head = [&](int c, float* a) {  // c < NC + NL
    if (c < NC) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a[e] = E::to_f(xc[c].v[e]);
        if constexpr (RES) a[e] += E::to_f(rc[c].v[e]);
      }
    } else {
      const Pack<S, VEC> xv = lds[c - NC][tid];
      Pack<S, VEC> rv;
      if constexpr (RES) rv = lds[NL + c - NC][tid];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a[e] = E::to_f(xv.v[e]);
        if constexpr (RES) a[e] += E::to_f(rv.v[e]);
      }
    }
  };
  auto a_of = [&](int64_t o, float* a) {
    const Pack<S, VEC> xv = ld<S, VEC>(x + base + o);
    Pack<S, VEC> rv;
    if constexpr (RES) rv = ld<S, VEC>(res + base + o);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      a[e] = E::to_f(xv.v[e]);
      if constexpr (RES) a[e] += E::to_f(rv.v[e]);
    }
  };
  const int tail0 = (NC + NL) * tpr + (int)threadIdx.x;  // the lane's first re-read vector
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    if (c * tpr + (int)threadIdx.x < nvec) {
      float a[VEC];
      a_head(c, a);
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss = __builtin_fma((double)a[e], (double)a[e], ss);
    }
  }
  for (int j = tail0; j < nvec; j += tpr) {
    float a[VEC];
    a_of((int64_t)j * VEC, a);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss = __builtin_fma((double)a[e], (double)a[e], ss);
  }
  ss = row_reduce(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  auto y_of = [&](int64_t o, const float* a, float* y) {
    const Pack<S, VEC> wv = ld<S, VEC>(w + o);
#pragma unroll
    for (int e = 0; e < VEC; ++e) y[e] = rnd<E>(rnd<E>(a[e] * rho) * E::to_f(wv.v[e]));
  };
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + (int)threadIdx.x;
    if (j < nvec) {
      float a[VEC], y[VEC];
      a_head(c, a);
      y_of((int64_t)j * VEC, a, y);
#pragma unroll
      for (int e = 0; e < VEC; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(y[e]));
    }
  }
  for (int j = tail0; j < nvec; j += tpr) {
    float a[VEC], y[VEC];
    a_of((int64_t)j * VEC, a);
    y_of((int64_t)j * VEC, a, y);
#pragma unroll
    for (int e = 0; e < VEC; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(y[e]));
  }
  amax = row_reduce(amax, red_max, tpr, MaxOp());
  float A;
  const float s = row_scale<FP8, MODE>(amax, rho, scale_ub, &A);
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
  const float inv = mcop_div_rn(1.0f, s);
  const bool s_ok = mcop_divisor_ok(s);
  const bool bounded = A == amax && s <= 0x1p100f;
  auto emit = [&](int64_t o, const float* a) {
    if constexpr (RES) {
      Pack<S, VEC> r;
#pragma unroll
      for (int e = 0; e < VEC; ++e) r.v[e] = E::from_f(a[e]);
      st<S, VEC>(res + base + o, r);
    }
    float y[VEC];
    y_of(o, a, y);
    st<uint8_t, VEC>(out + base + o,
                     row_codes<E, VEC, FP8, MODE>(y, rho, s, inv, s_ok, bounded,
                                                  scale_ub != nullptr));
  };
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + (int)threadIdx.x;
    if (j < nvec) {
      float a[VEC];
      a_head(c, a);
      emit((int64_t)j * VEC, a);
    }
  }
  for (int j = tail0; j < nvec; j += tpr) {
    float a[VEC];
    a_of((int64_t)j * VEC, a);
    emit((int64_t)j * VEC, a);
  }
}

// Rows too wide for one workgroup's registers, read once: the row is split into `slices` slices
// of `slice_vecs` vectors, one per workgroup -- workgroup b takes slice b % slices of row
// b / slices -- each holding its slice in registers (NV vectors a lane, the lane mapping of the
// register kernels within the slice).  The row's sum of squares and absmax are the slices'
// partials combined through the workspace `ws` (split_row.h: split_sum in slice order,
// split_max); every other step is the register kernel's, element by element.
// The bf16 int8 form at eight vectors a lane asks for four waves per SIMD, as the register
// kernel does (left free it took 129 VGPRs and three: 348 against 308 us at 2048 x 131072).
template <class E, int VEC, int NV, bool FP8, bool RES, int MODE>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
__attribute__((amdgpu_waves_per_eu(NV == 8 && !FP8 && std::is_same<E, BF16>::value ? 4 : 1)))
k_rms_norm_quant_split(uint8_t* __restrict__ out, float* __restrict__ scales,
                       const typename E::S* __restrict__ x, const typename E::S* __restrict__ w,
                       const float* __restrict__ scale_ub, typename E::S* __restrict__ res,
                       int64_t rows, int hidden, int slices, int slice_vecs, float eps,
                       uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  static_assert(MODE != QM_MC_7168, "7168-wide rows fit the register-resident kernel");
  using S = typename E::S;
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  __shared__ double x_sum;
  __shared__ float x_max;
  __shared__ int x_fail;
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int lt = (int)threadIdx.x;
  const int sl = (int)(blockIdx.x % (unsigned)slices);
  const int64_t row = blockIdx.x / (unsigned)slices;
  const int j0 = sl * slice_vecs;                   // the slice's first vector
  const int jn = min(slice_vecs, nvec - j0);        // vectors in the slice
  uint64_t* err = ws + split_ws_words(rows, slices) - 1;
  const int64_t base = row * (int64_t)hidden;
  // the lane's vector v: element offset in the row (lanes past the slice end re-read the
  // slice's first vector, which does not count)
  auto in_of = [&](int v) { return vec_index(v, tpr, lt) < jn; };
  auto lj_of = [&](int v) {
    return (int64_t)(j0 + (in_of(v) ? vec_index(v, tpr, lt) : 0)) * VEC;
  };
  Pack<S, VEC> xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = ld<S, VEC>(w + lj_of(v));
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    xv[v] = ld_nt<S, VEC>(x + base + lj_of(v));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(res + base + lj_of(v));
  }
  float a[NV][VEC];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    double vs = 0.0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float t = E::to_f(xv[v].v[e]);
      if constexpr (RES) t += E::to_f(rv[v].v[e]);
      a[v][e] = t;
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
    }
    ss += in_of(v) ? vs : 0.0;
    if constexpr (RES) {
      if (in_of(v)) {
        Pack<S, VEC> o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(a[v][e]);
        st_nt<S, VEC>(res + base + lj_of(v), o);
      }
    }
  }
  SplitRowReduce red{red_sum, red_max, tpr, ws, row, slices, sl, err, timeout_ticks, &x_sum,
                     &x_max, &x_fail};
  ss = red.sum(ss);
  const float rho = mcop_inv_rms(ss, hidden, eps);
  float amax = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float y = rnd<E>(rnd<E>(a[v][e] * rho) * E::to_f(wv[v].v[e]));
      a[v][e] = y;
      amax = __builtin_fmaxf(amax, in_of(v) ? __builtin_fabsf(y) : 0.0f);
    }
  }
  amax = red.max(amax);
  float A;
  const float s = row_scale<FP8, MODE>(amax, rho, scale_ub, &A);
  // slice 0 stores the scale; a slice whose exchange failed stores NaN (split_row.h)
  const bool failed = red.failed();
  if (lt == 0 && (sl == 0 || failed)) scales[row] = failed ? __builtin_nanf("") : s;
  const float inv = mcop_div_rn(1.0f, s);
  const bool s_ok = mcop_divisor_ok(s);
  const bool bounded = A == amax && s <= 0x1p100f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (in_of(v)) {
      st_nt<uint8_t, VEC>(out + base + lj_of(v),
                          row_codes<E, VEC, FP8, MODE>(a[v], rho, s, inv, s_ok, bounded,
                                                       scale_ub != nullptr));
    }
  }
}

// Rows too wide for the register-resident kernels, vector path: the split-row kernel when it
// applies (split_plan), in launches of at most chunk_rows rows, with its workspace from
// `scratch` when given (the no-allocation entry point: kSplitWsWords words) or else from the
// stream-ordered allocator, released on the same stream; MCOP_E_UNSUPPORTED (no message) when it
// does not apply, so the caller runs the multi-pass kernel.
template <class E, int VEC, bool FP8, bool RES, int MODE>
static int launch_split(const char* name, void* out, float* scales, const void* x,
                        const void* w, const float* scale_ub, void* res, int64_t rows,
                        int hidden, float eps, uint64_t* scratch, hipStream_t st) {
  using S = typename E::S;
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  const SplitKernel k8{fn(&k_rms_norm_quant_split<E, VEC, 8, FP8, RES, MODE>), 8};
  const SplitKernel k4{fn(&k_rms_norm_quant_split<E, VEC, 4, FP8, RES, MODE>), 4};
  return split_run(name, {k8, k4}, rows, hidden / VEC, scratch, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    auto* o = static_cast<uint8_t*>(out) + r0 * (int64_t)hidden;
    float* sc = scales + r0;
    auto* xp = static_cast<const S*>(x) + r0 * (int64_t)hidden;
    auto* wp = static_cast<const S*>(w);
    auto* rp = res == nullptr ? nullptr : static_cast<S*>(res) + r0 * (int64_t)hidden;
    int slices = p.slices, slice_vecs = p.slice_vecs;
    int64_t timeout = p.timeout_ticks;
    const float* ub = scale_ub;
    int h = hidden;
    float e = eps;
    void* args[] = {&o, &sc, &xp, &wp, &ub, &rp, &n, &h, &slices, &slice_vecs, &e, &ws, &timeout};
    return launch(args);
  });
}

template <class E, int VEC, bool FP8, bool RES, int MODE>
static void launch_nv(const Geometry& g, void* out, float* scales, const void* x, const void* w,
                      const float* scale_ub, void* res, int64_t rows, int hidden, float eps,
                      hipStream_t st) {
  using S = typename E::S;
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* o = static_cast<uint8_t*>(out);
  auto* xp = static_cast<const S*>(x);
  auto* wp = static_cast<const S*>(w);
  auto* rp = static_cast<S*>(res);
#define MCOP_LAUNCH(NVV, EXX)                                                                  \
  hipLaunchKernelGGL((k_rms_norm_quant<E, VEC, NVV, FP8, RES, MODE, EXX>), grid, block, 0, st, o, \
                     scales, xp, wp, scale_ub, rp, rows, hidden, g.tpr, eps)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it) take the EX form at two vectors a
    // lane, and at four or eight for at most 256 rows (the latency path): at four and eight it
    // takes more registers (fewer resident waves) for no gain on bandwidth-bound shapes.  The
    // 7168 chain's rows (896 vectors) are exact only at two vectors over 448 lanes.
    constexpr bool wide_ex = MODE != QM_MC_7168;
    // The EX form only when it keeps its registers.
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == hidden / VEC &&
                    (g.nv == 2 || (wide_ex && rows <= 256));
#define MCOP_EX(NVV, EXX)                                                                      \
  (ex && exact_form_ok(                                                                        \
             reinterpret_cast<const void*>(&k_rms_norm_quant<E, VEC, NVV, FP8, RES, MODE, EXX>)))
    switch (g.nv) {
      case 1: MCOP_LAUNCH(1, false); break;
      case 2: if (MCOP_EX(2, true)) MCOP_LAUNCH(2, true); else MCOP_LAUNCH(2, false); break;
      case 4: if (MCOP_EX(4, wide_ex)) MCOP_LAUNCH(4, wide_ex); else MCOP_LAUNCH(4, false); break;
      case 8: if (MCOP_EX(8, wide_ex)) MCOP_LAUNCH(8, wide_ex); else MCOP_LAUNCH(8, false); break;
      default: MCOP_LAUNCH(16, false); break;
    }
#undef MCOP_EX
  }
#undef MCOP_LAUNCH
}

template <class E, int VEC, bool FP8, bool RES, int MODE>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_rms_norm_quant<E, 1, 4, FP8, RES, MODE>)
                   : reinterpret_cast<const void*>(&k_rms_norm_quant<E, 1, 16, FP8, RES, MODE>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_rms_norm_quant<E, VEC, 1, FP8, RES, MODE>);
      case 2: return reinterpret_cast<const void*>(&k_rms_norm_quant<E, VEC, 2, FP8, RES, MODE>);
      case 4: return reinterpret_cast<const void*>(&k_rms_norm_quant<E, VEC, 4, FP8, RES, MODE>);
      case 8: return reinterpret_cast<const void*>(&k_rms_norm_quant<E, VEC, 8, FP8, RES, MODE>);
      default: return reinterpret_cast<const void*>(&k_rms_norm_quant<E, VEC, 16, FP8, RES, MODE>);
    }
  }
}

// `scratch`: the split-row kernel's workspace for the no-allocation entry point (NULL: the
// stream-ordered allocator provides it).
template <class E, bool FP8, int MODE>
static int dispatch(const char* name, void* out, float* scales, const void* x, const void* w,
                    const float* scale_ub, void* res, int64_t rows, int64_t hidden, float eps,
                    hipStream_t st, uint64_t* scratch = nullptr) {
  constexpr int V = E::VEC;
  const bool vec_ok = hidden % V == 0 && aligned(16, x, w, res) && aligned(V, out);
  const KernelOfNv kernels =
      vec_ok ? (res ? &kernel_of<E, V, FP8, true, MODE> : &kernel_of<E, V, FP8, false, MODE>)
             : (res ? &kernel_of<E, 1, FP8, true, MODE> : &kernel_of<E, 1, FP8, false, MODE>);
  if constexpr (MODE != QM_MC_7168) {
    if (!row_fits(hidden, vec_ok ? V : 1, kernels)) {
      if (vec_ok && split_rows_enabled()) {
        const int rc =
            res ? launch_split<E, V, FP8, true, MODE>(name, out, scales, x, w, scale_ub, res,
                                                      rows, (int)hidden, eps, scratch, st)
                : launch_split<E, V, FP8, false, MODE>(name, out, scales, x, w, scale_ub, res,
                                                       rows, (int)hidden, eps, scratch, st);
        if (rc != MCOP_E_UNSUPPORTED) return rc;
      }
      if (!wide_rows_ok(name, rows)) return MCOP_E_UNSUPPORTED;
      using S = typename E::S;
      auto* o = static_cast<uint8_t*>(out);
      auto* xp = static_cast<const S*>(x);
      auto* wp = static_cast<const S*>(w);
      auto* rp = static_cast<S*>(res);
      const dim3 grid((unsigned)rows), block(kWideLanes);
#define MCOP_WIDE(VV, RR)                                                                     \
  hipLaunchKernelGGL((k_rms_norm_quant_wide<E, VV, FP8, RR, MODE>), grid, block, 0, st, o,     \
                     scales, xp, wp, scale_ub, rp, (int)hidden, eps)
      if (vec_ok) {
        if (res) MCOP_WIDE(V, true); else MCOP_WIDE(V, false);
      } else {
        if (res) MCOP_WIDE(1, true); else MCOP_WIDE(1, false);
      }
#undef MCOP_WIDE
      return check_launch(name);
    }
  }
  Geometry g;
  if (!choose_geometry(name, rows, hidden, vec_ok ? V : 1, kernels, &g, 16,
                       /*wide_nv4=*/false)) {
    return MCOP_E_UNSUPPORTED;
  }
  const int h = (int)hidden;
  if (g.vec == 1) {
    if (res) launch_nv<E, 1, FP8, true, MODE>(g, out, scales, x, w, scale_ub, res, rows, h, eps, st);
    else launch_nv<E, 1, FP8, false, MODE>(g, out, scales, x, w, scale_ub, res, rows, h, eps, st);
  } else {
    if (res) launch_nv<E, V, FP8, true, MODE>(g, out, scales, x, w, scale_ub, res, rows, h, eps, st);
    else launch_nv<E, V, FP8, false, MODE>(g, out, scales, x, w, scale_ub, res, rows, h, eps, st);
  }
  return check_launch(name);
}

static int check_args(const char* name, const void* out, const float* scales, const void* input,
                      const void* weight, int64_t num_tokens, int64_t hidden_size) {
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size > INT32_MAX) {
    return set_error(MCOP_E_INVALID, "%s: bad shape num_tokens=%lld hidden_size=%lld", name,
                     (long long)num_tokens, (long long)hidden_size);
  }
  if (num_tokens > 0 && (!out || !scales || !input || !weight)) {
    return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  }
  return MCOP_OK;
}

// vLLM's operator (QM_VLLM), int8 or fp8 codes; `scratch` as for dispatch.
static int h2_entry(const char* name, void* out, mcop_dtype out_dtype, float* scales,
                    const void* input, const void* weight, const float* scale_ub, void* residual,
                    int64_t num_tokens, int64_t hidden_size, mcop_dtype in_dtype, float epsilon,
                    void* stream, uint64_t* scratch) {
  if (int rc = check_args(name, out, scales, input, weight, num_tokens, hidden_size)) return rc;
  if (num_tokens == 0) return MCOP_OK;
  if (out_dtype != MCOP_I8 && out_dtype != MCOP_FP8_E4M3FN) {
    return set_error(MCOP_E_INVALID, "%s: out dtype %d is not int8 or fp8_e4m3fn", name,
                     (int)out_dtype);
  }
  const bool fp8 = out_dtype == MCOP_FP8_E4M3FN;
  auto st = static_cast<hipStream_t>(stream);
#define MCOP_CASE(E)                                                                         \
  return fp8 ? dispatch<E, true, QM_VLLM>(name, out, scales, input, weight, scale_ub,         \
                                          residual, num_tokens, hidden_size, epsilon, st,     \
                                          scratch)                                            \
             : dispatch<E, false, QM_VLLM>(name, out, scales, input, weight, scale_ub,        \
                                           residual, num_tokens, hidden_size, epsilon, st,    \
                                           scratch)
  switch (in_dtype) {
    case MCOP_BF16: MCOP_CASE(BF16);
    case MCOP_F16: MCOP_CASE(F16);
    case MCOP_F32: MCOP_CASE(F32);
    default:
      return set_error(MCOP_E_INVALID, "%s: input dtype %d is not bf16/fp16/fp32", name,
                       (int)in_dtype);
  }
#undef MCOP_CASE
}

// The no-allocation entry point's workspace for the split-row kernels: kSplitWsWords 64-bit
// words (2 MiB) on every GPU the library runs on, held until the process ends.  In host code
// the name is a stand-in, not a device address: scratch_address() resolves each device's copy.
static __device__ __align__(256) uint64_t scratch[kSplitWsWords];

// The device address of `scratch` on the current device: hipGetSymbolAddress once per device
// (with that device current, on its first call there), then the kept address.  NULL, with the
// message set, when the runtime cannot resolve it.
static uint64_t* scratch_address(const char* name) {
  static std::mutex mu;
  static uint64_t* addr[64] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    set_error(MCOP_E_LAUNCH, "%s: no current device (or device %d beyond 63)", name, dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      set_error(MCOP_E_LAUNCH, "%s: hipGetSymbolAddress of the scratch array failed on device "
                "%d: %s", name, dev, hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = static_cast<uint64_t*>(p);
  }
  return addr[dev];
}

}  // namespace mcop

extern "C" int mcop_rms_norm_dynamic_per_token_quant(void* out, mcop_dtype out_dtype,
                                                     float* scales, const void* input,
                                                     const void* weight, const float* scale_ub,
                                                     void* residual, int64_t num_tokens,
                                                     int64_t hidden_size, mcop_dtype in_dtype,
                                                     float epsilon, void* stream) {
  return mcop::h2_entry("rms_norm_dynamic_per_token_quant", out, out_dtype, scales, input,
                        weight, scale_ub, residual, num_tokens, hidden_size, in_dtype, epsilon,
                        stream, nullptr);
}

extern "C" int mcop_rms_norm_dynamic_per_token_quant_noalloc(
    void* out, mcop_dtype out_dtype, float* scales, const void* input, const void* weight,
    const float* scale_ub, void* residual, int64_t num_tokens, int64_t hidden_size,
    mcop_dtype in_dtype, float epsilon, void* stream) {
  using namespace mcop;
  const char* name = "rms_norm_dynamic_per_token_quant_noalloc";
  if (int rc = check_args(name, out, scales, input, weight, num_tokens, hidden_size)) return rc;
  if (num_tokens == 0) return MCOP_OK;
  uint64_t* ws = scratch_address(name);
  if (ws == nullptr) return MCOP_E_LAUNCH;
  return h2_entry(name, out, out_dtype, scales, input, weight, scale_ub, residual, num_tokens,
                  hidden_size, in_dtype, epsilon, stream, ws);
}

extern "C" int mcop_rms_norm_dynamic_per_token_quant_custom(
    int8_t* out, float* scales, const void* input, const void* weight, const float* scale_ub,
    void* residual, int64_t num_tokens, int64_t hidden_size, mcop_dtype in_dtype, float epsilon,
    void* stream) {
  using namespace mcop;
  const char* name = "rms_norm_dynamic_per_token_quant_custom";
  if (int rc = check_args(name, out, scales, input, weight, num_tokens, hidden_size)) return rc;
  if (num_tokens == 0) return MCOP_OK;
  auto st = static_cast<hipStream_t>(stream);
  // the reference's dispatch: its fp32-chain kernel for H == 7168, the generic one otherwise
  const bool h7168 = hidden_size == 7168;
#define MCOP_CASE(E)                                                                         \
  return h7168 ? dispatch<E, false, QM_MC_7168>(name, out, scales, input, weight, scale_ub,   \
                                                residual, num_tokens, hidden_size, epsilon,   \
                                                st)                                           \
               : dispatch<E, false, QM_MC>(name, out, scales, input, weight, scale_ub,        \
                                           residual, num_tokens, hidden_size, epsilon, st)
  switch (in_dtype) {
    case MCOP_BF16: MCOP_CASE(BF16);
    case MCOP_F16: MCOP_CASE(F16);
    case MCOP_F32: MCOP_CASE(F32);
    default:
      return set_error(MCOP_E_INVALID, "%s: input dtype %d is not bf16/fp16/fp32", name,
                       (int)in_dtype);
  }
#undef MCOP_CASE
}
