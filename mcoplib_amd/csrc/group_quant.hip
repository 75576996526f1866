// group_quant.hip -- (residual add +) RMSNorm + dynamic per-group int8 / fp8-e4m3fn
// quantization (vLLM `_C::rms_norm_per_block_quant`), one pass over HBM.
//
// Semantics (per row, a = x [+ r] in fp32, b() = round to the input dtype; paths relative to
// op/vllm/quantization/fused_kernels/ of the reference):
//   residual <- b(a)                           layernorm_utils.cuh:500-508
//   rho = 1/sqrt(sum(a^2)/H + eps)             layernorm_utils.cuh:223-279 (order: fp64 sum)
//   y = b(b(a*rho) * w)                        layernorm_utils.cuh:325-329, 530-531
//   per group g of G = 64 or 128 consecutive elements:
//     A_g = max|y| over the group, min(A_g, *scale_ub)          :303-352
//     int8: s_g = max(A_g/127, FLT_EPSILON); q = sat[-128,127](rne(y * (1/s_g)))
//     fp8 : s_g = max(A_g/448, 1/(448*512)); q = e4m3fn(clamp(y / s_g, +-448))
//   scales[t * (H/G) + g], or scales[g * T + t] when transposed   :352-357, 517-521
// (the int8 code is the intended round-to-nearest-even with saturation, as for the per-token
// kernel of the same file).
//
// Lane mapping: the vector paths keep the row kernels' strided mapping (vector j = v*tpr + lane),
// so the G/VEC vectors of one group sit in G/VEC consecutive lanes and the group maximum is a
// butterfly over those lanes of one wave; the element-wise path (misaligned tensors) gives each
// lane NV consecutive elements instead, so a group spans G/NV lanes.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

// max over aligned runs of `lanes` consecutive lanes (a power of two <= 64) of one wave: DPP
// moves within 16-lane rows, LDS-routed shuffles across them
__device__ __forceinline__ float group_max(float v, int lanes) {
  const MaxOp op;
  if (lanes >= 2) v = op(v, dpp_mov<kDppXor1>(v));
  if (lanes >= 4) v = op(v, dpp_mov<kDppXor2>(v));
  if (lanes >= 8) v = op(v, dpp_mov<kDppHalfMirror>(v));
  if (lanes >= 16) v = op(v, dpp_mov<kDppMirror>(v));
  if (lanes >= 32) v = op(v, __shfl_xor(v, 16, 64));
  if (lanes >= 64) v = op(v, __shfl_xor(v, 32, 64));
  return v;
}

// Scale (*s) and codes of one vector of y in a group whose absmax is m (the multi-pass kernel's
// form of the register-resident kernel's inline epilogue).
template <class E, int VEC, bool FP8>
__device__ __forceinline__ Pack<uint8_t, VEC> group_codes(const float* y, float m, bool has_ub,
                                                          float ub, float* s_out) {
  const float A = has_ub ? __builtin_fminf(m, ub) : m;
  const float s = FP8 ? __builtin_fmaxf(mcop_div_rn(A, 448.0f), 1.0f / 229376.0f)
                      : __builtin_fmaxf(mcop_div_rn(A, 127.0f), FLT_EPSILON);
  *s_out = s;
  const float inv = mcop_div_rn(1.0f, s);
  Pack<uint8_t, VEC> q;
  if constexpr (FP8) {
    const bool bounded = A == m && s <= 0x1p100f;
    q = fp8_quotient_codes<VEC>(y, s, inv, mcop_divisor_ok(s), bounded);
  } else if constexpr (std::is_same_v<E, F32>) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-128>(y[e] * inv);
  } else {
    // |y * inv| <= 127 * (1 + 2^-22) < 127.5 (int8 takes no scale bound)
#pragma unroll
    for (int e = 0; e < VEC; ++e) q.v[e] = q_i8_in_range(y[e], inv);
  }
  return q;
}

// EX (exact): one row per workgroup and every lane in the row (tpr == blockDim.x, NV * tpr ==
// hidden / VEC): uniform row index, scalar base addresses with 32-bit offsets, no bounds tests.
template <class E, int VEC, int NV, bool FP8, bool RES, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_rms_norm_group_quant(uint8_t* __restrict__ out, float* __restrict__ scales,
                       const typename E::S* __restrict__ x, const typename E::S* __restrict__ w,
                       const float* __restrict__ scale_ub, typename E::S* __restrict__ res,
                       int64_t rows, int hidden, int tpr, float eps, int group,
                       int64_t scale_row_stride, int64_t scale_group_stride) {
  using S = typename E::S;
  constexpr bool BLOCKED = VEC == 1;
  __shared__ double red_sum[16];
  RowPos p;
  if constexpr (EX) {
    p = row_pos_one();
  } else {
    p = row_pos(rows, tpr);
  }
  const int nvec = hidden / VEC;
  const int64_t base = p.row * (int64_t)hidden;
  const int64_t lbase = p.lrow * (int64_t)hidden;
  auto index = [&](int v) { return BLOCKED ? p.lt * NV + v : vec_index(v, tpr, p.lt); };
  auto lj_of = [&](int v) { return (int64_t)(EX ? index(v) : load_index(index(v), nvec)) * VEC; };

  Pack<S, VEC> xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = ld<S, VEC>(row_elem<EX>(w, 0, lj_of(v)));
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t lj = lj_of(v);
    xv[v] = ld_nt<S, VEC>(row_elem<EX>(x, lbase, lj));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(row_elem<EX>(res, lbase, lj));
  }

  float a[NV][VEC];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = index(v);
    const bool in = EX || j < nvec;
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

  // Groups are whole (hidden % group == 0), so a group's lanes are all inside the row or all
  // past its end; the latter compute on copies and store nothing.
  float m[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    m[v] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float y = rnd<E>(rnd<E>(a[v][e] * rho) * E::to_f(wv[v].v[e]));
      a[v][e] = y;
      m[v] = __builtin_fmaxf(m[v], __builtin_fabsf(y));
    }
  }
  if constexpr (BLOCKED) {
    float mm = m[0];
#pragma unroll
    for (int v = 1; v < NV; ++v) mm = __builtin_fmaxf(mm, m[v]);
    mm = group_max(mm, group / NV);
#pragma unroll
    for (int v = 0; v < NV; ++v) m[v] = mm;
  } else {
#pragma unroll
    for (int v = 0; v < NV; ++v) m[v] = group_max(m[v], group / VEC);
  }

  const float ub = scale_ub != nullptr ? *scale_ub : 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = index(v);
    if (!(p.live && (EX || j < nvec))) continue;
    // kept inline (group_codes computes the same): the helper's order (codes before the scale
    // store) measured 1.4% slower here
    const float A = scale_ub != nullptr ? __builtin_fminf(m[v], ub) : m[v];
    const float s = FP8 ? __builtin_fmaxf(mcop_div_rn(A, 448.0f), 1.0f / 229376.0f)
                        : __builtin_fmaxf(mcop_div_rn(A, 127.0f), FLT_EPSILON);
    const int g = (int)(((int64_t)j * VEC) / group);
    if ((((int64_t)j * VEC) % group) == 0) {
      scales[p.row * scale_row_stride + (int64_t)g * scale_group_stride] = s;
    }
    const float inv = mcop_div_rn(1.0f, s);
    Pack<uint8_t, VEC> q;
    if constexpr (FP8) {
      const bool bounded = A == m[v] && s <= 0x1p100f;
      q = fp8_quotient_codes<VEC>(a[v], s, inv, mcop_divisor_ok(s), bounded);
    } else if constexpr (std::is_same_v<E, F32>) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-128>(a[v][e] * inv);
    } else {
      // |y * inv| <= 127 * (1 + 2^-22) < 127.5 (int8 takes no scale bound)
#pragma unroll
      for (int e = 0; e < VEC; ++e) q.v[e] = q_i8_in_range(a[v][e], inv);
    }
    st_nt<uint8_t, VEC>(row_elem<EX>(out, base, (int64_t)j * VEC), q);
  }
}

// Rows too wide for one workgroup's registers, read once (split_row.h): workgroup b takes slice
// b % slices of row b / slices -- `slice_vecs` vectors, a multiple of the group's G / VEC
// vectors, NV a lane -- and combines the row's sum of squares with the other slices' through
// the workspace `ws` (split_sum, in slice order); groups lie inside one slice, in G / VEC
// aligned lanes of one wave, so their absmax, scales and codes are the register kernel's.  The
// row index is uniform: scalar row bases, 32-bit offsets.
template <class E, int VEC, int NV, bool FP8, bool RES>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
__attribute__((amdgpu_waves_per_eu(NV == 8 ? 4 : 1)))
k_rms_norm_group_quant_split(uint8_t* __restrict__ out, float* __restrict__ scales,
                             const typename E::S* __restrict__ x,
                             const typename E::S* __restrict__ w,
                             const float* __restrict__ scale_ub, typename E::S* __restrict__ res,
                             int64_t rows, int hidden, float eps, int group,
                             int64_t scale_row_stride, int64_t scale_group_stride, int slices,
                             int slice_vecs, uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  using S = typename E::S;
  __shared__ double red_sum[16];
  __shared__ double x_sum;
  __shared__ int x_fail;
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int lt = (int)threadIdx.x;
  const int sl = (int)(blockIdx.x % (unsigned)slices);
  const int64_t row = blockIdx.x / (unsigned)slices;
  const int j0 = sl * slice_vecs;
  const int jn = min(slice_vecs, nvec - j0);
  const int64_t base = row * (int64_t)hidden;
  // Lanes past the slice end (whole groups) re-read the slice's first vector and store nothing.
  auto in_of = [&](int v) { return vec_index(v, tpr, lt) < jn; };
  auto lj_of = [&](int v) {
    return (int64_t)(j0 + (in_of(v) ? vec_index(v, tpr, lt) : 0)) * VEC;
  };
  Pack<S, VEC> xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = ld<S, VEC>(row_elem<true>(w, 0, lj_of(v)));
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    xv[v] = ld_nt<S, VEC>(row_elem<true>(x, base, lj_of(v)));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(row_elem<true>(res, base, lj_of(v)));
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
        st_nt<S, VEC>(row_elem<true>(res, base, lj_of(v)), o);
      }
    }
  }
  SplitRowReduce red{red_sum, nullptr, tpr, ws, row, slices, sl,
                     ws + split_ws_words(rows, slices) - 1, timeout_ticks, &x_sum, nullptr,
                     &x_fail};
  ss = red.sum(ss);
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float ub = scale_ub != nullptr ? *scale_ub : 0.0f;
  const bool failed = red.failed();  // a failed exchange: NaN scales
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float y = rnd<E>(rnd<E>(a[v][e] * rho) * E::to_f(wv[v].v[e]));
      a[v][e] = y;
      m = __builtin_fmaxf(m, __builtin_fabsf(y));
    }
    m = group_max(m, group / VEC);
    if (!in_of(v)) continue;
    float s;
    const Pack<uint8_t, VEC> q =
        group_codes<E, VEC, FP8>(a[v], m, scale_ub != nullptr, ub, &s);
    const int64_t o = lj_of(v);
    if (o % group == 0) {
      scales[row * scale_row_stride + (o / group) * scale_group_stride] =
          failed ? __builtin_nanf("") : s;
    }
    st_nt<uint8_t, VEC>(row_elem<true>(out, base, o), q);
  }
}

// Rows too wide for the registers: one 1024-lane workgroup per row, two passes (sum of squares;
// codes, scales and the residual).  The row's head stays on chip between the passes -- the
// first NC units of x (and residual) of every lane in registers, the next NL in lane-private LDS
// slots (unit c of lane t at [c][t], so no barrier is needed; the workgroup already fills a
// CU's registers, so the 128 KB cost no occupancy) -- and the second pass re-reads the rest,
// and the weight; the residual is written in the last pass only, by the lane that read it.  A
// lane takes U consecutive elements per step (one 16-byte vector, or four scalars on the scalar
// path), so a group spans group / U aligned lanes (<= 64), 1024 lanes hold whole groups, and a
// unit's bound check is the same for all lanes of its group.
template <class E, int U, bool VECLD, bool FP8, bool RES>
__global__ void __launch_bounds__(kWideLanes)
k_rms_norm_group_quant_wide(uint8_t* __restrict__ out, float* __restrict__ scales,
                            const typename E::S* __restrict__ x,
                            const typename E::S* __restrict__ w,
                            const float* __restrict__ scale_ub, typename E::S* __restrict__ res,
                            int hidden, float eps, int group, int64_t scale_row_stride,
                            int64_t scale_group_stride) {
  using S = typename E::S;
  constexpr int NC = VECLD ? (RES ? 4 : 8) : 8, NL = VECLD ? (RES ? 4 : 8) : 0;
  constexpr int NLS = NL > 0 ? NL * (RES ? 2 : 1) : 1;
  __shared__ double red_sum[16];
  __shared__ Pack<S, U> lds[NLS][kWideLanes];
  const int nunit = hidden / U;
  const int tpr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * hidden;
  auto raw = [&](const S* p) {
    Pack<S, U> v;
    if constexpr (VECLD) {
      v = ld<S, U>(p);
    } else {
#pragma unroll
      for (int e = 0; e < U; ++e) v.v[e] = p[e];
    }
    return v;
  };
  auto t_from = [&](const Pack<S, U>& xv, const Pack<S, U>& rv, float* t) {
#pragma unroll
    for (int e = 0; e < U; ++e) {
      t[e] = E::to_f(xv.v[e]);
      if constexpr (RES) t[e] += E::to_f(rv.v[e]);
    }
  };
  auto t_of = [&](int64_t o, float* t) {
    Pack<S, U> rv;
    if constexpr (RES) rv = raw(res + base + o);
    t_from(raw(x + base + o), rv, t);
  };
  Pack<S, U> xc[NC], rc[NC];
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + tid;
    if (j < nunit) {
      const Pack<S, U> xv = raw(x + base + (int64_t)j * U);
      Pack<S, U> rv;
      if constexpr (RES) rv = raw(res + base + (int64_t)j * U);
      if (c < NC) {
        xc[c] = xv;
        if constexpr (RES) rc[c] = rv;
      } else {
        lds[c - NC][tid] = xv;
        if constexpr (RES) lds[NL + c - NC][tid] = rv;
      }
    }
  }
  auto t_head = [&](int c, float* t) {
    if (c < NC) {
      t_from(xc[c], rc[c], t);
    } else {
      Pack<S, U> rv;
      if constexpr (RES) rv = lds[NL + c - NC][tid];
      t_from(lds[c - NC][tid], rv, t);
    }
  };
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    if (c * tpr + tid < nunit) {
      float t[U];
      t_head(c, t);
#pragma unroll
      for (int e = 0; e < U; ++e) ss = __builtin_fma((double)t[e], (double)t[e], ss);
    }
  }
  const int tail0 = (NC + NL) * tpr + tid;
  for (int j = tail0; j < nunit; j += tpr) {
    float t[U];
    t_of((int64_t)j * U, t);
#pragma unroll
    for (int e = 0; e < U; ++e) ss = __builtin_fma((double)t[e], (double)t[e], ss);
  }
  ss = row_reduce(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float ub = scale_ub != nullptr ? *scale_ub : 0.0f;
  auto emit = [&](int64_t o, const float* t) {
    float wf[U], y[U];
    const Pack<S, U> wv = raw(w + o);
#pragma unroll
    for (int e = 0; e < U; ++e) wf[e] = E::to_f(wv.v[e]);
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < U; ++e) {
      y[e] = rnd<E>(rnd<E>(t[e] * rho) * wf[e]);
      m = __builtin_fmaxf(m, __builtin_fabsf(y[e]));
    }
    m = group_max(m, group / U);
    float s;
    const Pack<uint8_t, U> q = group_codes<E, U, FP8>(y, m, scale_ub != nullptr, ub, &s);
    if (o % group == 0) {
      scales[(int64_t)blockIdx.x * scale_row_stride + (o / group) * scale_group_stride] = s;
    }
    if constexpr (RES) {
      Pack<S, U> r;
#pragma unroll
      for (int e = 0; e < U; ++e) r.v[e] = E::from_f(t[e]);
      if constexpr (VECLD) {
        st<S, U>(res + base + o, r);
      } else {
#pragma unroll
        for (int e = 0; e < U; ++e) res[base + o + e] = r.v[e];
      }
    }
    if constexpr (VECLD) {
      st<uint8_t, U>(out + base + o, q);
    } else {
#pragma unroll
      for (int e = 0; e < U; ++e) out[base + o + e] = q.v[e];
    }
  };
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + tid;
    if (j < nunit) {
      float t[U];
      t_head(c, t);
      emit((int64_t)j * U, t);
    }
  }
  for (int j = tail0; j < nunit; j += tpr) {
    float t[U];
    t_of((int64_t)j * U, t);
    emit((int64_t)j * U, t);
  }
}

template <class E, int VEC, bool FP8, bool RES>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, 1, 4, FP8, RES>)
                   : reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, 1, 16, FP8, RES>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, VEC, 1, FP8, RES>);
      case 2: return reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, VEC, 2, FP8, RES>);
      case 4: return reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, VEC, 4, FP8, RES>);
      case 8: return reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, VEC, 8, FP8, RES>);
      default: return reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, VEC, 16, FP8, RES>);
    }
  }
}

struct GqArgs {
  void* out;
  float* scales;
  const void* x;
  const void* w;
  const float* scale_ub;
  void* res;
  int64_t rows;
  int hidden;
  float eps;
  int group;
  int64_t srow;
  int64_t sgrp;
};

template <class E, int VEC, bool FP8, bool RES>
static void launch_nv(const Geometry& g, const GqArgs& a, hipStream_t st) {
  using S = typename E::S;
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* o = static_cast<uint8_t*>(a.out);
  auto* xp = static_cast<const S*>(a.x);
  auto* wp = static_cast<const S*>(a.w);
  auto* rp = static_cast<S*>(a.res);
#define MCOP_LAUNCH(NVV, EXX)                                                                   \
  hipLaunchKernelGGL((k_rms_norm_group_quant<E, VEC, NVV, FP8, RES, EXX>), grid, block, 0, st, o, \
                     a.scales, xp, wp, a.scale_ub, rp, a.rows, a.hidden, g.tpr, a.eps, a.group, \
                     a.srow, a.sgrp)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it) on the latency path (at most 256
    // rows) take the EX form, when it keeps its registers
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == a.hidden / VEC && a.rows <= 256;
#define MCOP_EX(NVV)                                                                           \
  (ex && exact_form_ok(                                                                        \
             reinterpret_cast<const void*>(&k_rms_norm_group_quant<E, VEC, NVV, FP8, RES, true>)))
    switch (g.nv) {
      case 1: MCOP_LAUNCH(1, false); break;
      case 2: if (MCOP_EX(2)) MCOP_LAUNCH(2, true); else MCOP_LAUNCH(2, false); break;
      case 4: if (MCOP_EX(4)) MCOP_LAUNCH(4, true); else MCOP_LAUNCH(4, false); break;
      case 8: if (MCOP_EX(8)) MCOP_LAUNCH(8, true); else MCOP_LAUNCH(8, false); break;
      default: MCOP_LAUNCH(16, false); break;
    }
#undef MCOP_EX
  }
#undef MCOP_LAUNCH
}

// Rows too wide for the register kernels, vector path: the split-row kernel when it applies (its
// slices whole groups), its workspace from the stream-ordered allocator; MCOP_E_UNSUPPORTED (no
// message) when it does not.
template <class E, int VEC, bool FP8, bool RES>
static int launch_split(const char* name, const GqArgs& a, hipStream_t st) {
  using S = typename E::S;
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  const int gv = a.group / VEC;
  const SplitKernel k8{fn(&k_rms_norm_group_quant_split<E, VEC, 8, FP8, RES>), 8, kSplitLanes,
                       gv};
  const SplitKernel k4{fn(&k_rms_norm_group_quant_split<E, VEC, 4, FP8, RES>), 4, kSplitLanes,
                       gv};
  return split_run(name, {k8, k4}, a.rows, a.hidden / VEC, nullptr, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    const int64_t off = r0 * (int64_t)a.hidden;
    uint8_t* o = static_cast<uint8_t*>(a.out) + off;
    float* sc = a.scales + r0 * a.srow;
    const S* xp = static_cast<const S*>(a.x) + off;
    const S* wp = static_cast<const S*>(a.w);
    const float* ub = a.scale_ub;
    S* rp = a.res == nullptr ? nullptr : static_cast<S*>(a.res) + off;
    int h = a.hidden, grp = a.group, slices = p.slices, slice_vecs = p.slice_vecs;
    float e = a.eps;
    int64_t srow = a.srow, sgrp = a.sgrp, timeout = p.timeout_ticks;
    void* args[] = {&o, &sc, &xp, &wp, &ub, &rp, &n, &h, &e, &grp, &srow, &sgrp, &slices,
                    &slice_vecs, &ws, &timeout};
    return launch(args);
  });
}

template <class E, bool FP8>
static int dispatch(const GqArgs& a, hipStream_t st) {
  const char* name = "rms_norm_per_block_quant";
  constexpr int V = E::VEC;
  const bool vec_ok = a.hidden % V == 0 && aligned(16, a.x, a.w, a.res) && aligned(V, a.out);
  const KernelOfNv kernels =
      vec_ok ? (a.res ? &kernel_of<E, V, FP8, true> : &kernel_of<E, V, FP8, false>)
             : (a.res ? &kernel_of<E, 1, FP8, true> : &kernel_of<E, 1, FP8, false>);
  if (!row_fits(a.hidden, vec_ok ? V : 1, kernels, 64)) {
    if (vec_ok && split_rows_enabled()) {
      const int rc = a.res ? launch_split<E, V, FP8, true>(name, a, st)
                           : launch_split<E, V, FP8, false>(name, a, st);
      if (rc != MCOP_E_UNSUPPORTED) return rc;
    }
    if (!wide_rows_ok(name, a.rows)) return MCOP_E_UNSUPPORTED;
    using S = typename E::S;
    auto* o = static_cast<uint8_t*>(a.out);
    auto* xp = static_cast<const S*>(a.x);
    auto* wp = static_cast<const S*>(a.w);
    auto* rp = static_cast<S*>(a.res);
    const dim3 grid((unsigned)a.rows), block(kWideLanes);
#define MCOP_WIDE(UU, VL, RR)                                                                 \
  hipLaunchKernelGGL((k_rms_norm_group_quant_wide<E, UU, VL, FP8, RR>), grid, block, 0, st, o, \
                     a.scales, xp, wp, a.scale_ub, rp, a.hidden, a.eps, a.group, a.srow, a.sgrp)
    if (vec_ok) {
      if (a.res) MCOP_WIDE(V, true, true); else MCOP_WIDE(V, true, false);
    } else {
      if (a.res) MCOP_WIDE(4, false, true); else MCOP_WIDE(4, false, false);
    }
#undef MCOP_WIDE
    return check_launch(name);
  }
  Geometry g;
  // whole waves per row: a group's lanes must lie inside one row slice of the lane mapping
  if (!choose_geometry(name, a.rows, a.hidden, vec_ok ? V : 1, kernels, &g, 64)) {
    return MCOP_E_UNSUPPORTED;
  }
  if (g.vec == 1) {
    if (a.res) launch_nv<E, 1, FP8, true>(g, a, st);
    else launch_nv<E, 1, FP8, false>(g, a, st);
  } else {
    if (a.res) launch_nv<E, V, FP8, true>(g, a, st);
    else launch_nv<E, V, FP8, false>(g, a, st);
  }
  return check_launch(name);
}

}  // namespace mcop

extern "C" int mcop_rms_norm_per_block_quant(void* out, mcop_dtype out_dtype, float* scales,
                                             const void* input, const void* weight,
                                             const float* scale_ub, void* residual,
                                             int64_t num_tokens, int64_t hidden_size,
                                             mcop_dtype in_dtype, float epsilon,
                                             int64_t group_size, int is_scale_transposed,
                                             void* stream) {
  using namespace mcop;
  const char* name = "rms_norm_per_block_quant";
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size > INT32_MAX) {
    return set_error(MCOP_E_INVALID, "%s: bad shape num_tokens=%lld hidden_size=%lld", name,
                     (long long)num_tokens, (long long)hidden_size);
  }
  if (group_size != 64 && group_size != 128) {
    return set_error(MCOP_E_INVALID, "%s: unsupported group size %lld (64 or 128)", name,
                     (long long)group_size);
  }
  if (hidden_size % group_size != 0) {
    return set_error(MCOP_E_INVALID, "%s: hidden_size %lld is not a multiple of group_size %lld",
                     name, (long long)hidden_size, (long long)group_size);
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !scales || !input || !weight) {
    return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  }
  if (out_dtype != MCOP_I8 && out_dtype != MCOP_FP8_E4M3FN) {
    return set_error(MCOP_E_INVALID, "%s: out dtype %d is not int8 or fp8_e4m3fn", name,
                     (int)out_dtype);
  }
  const int64_t groups = hidden_size / group_size;
  const GqArgs a{out, scales, input, weight, scale_ub, residual, num_tokens, (int)hidden_size,
                 epsilon, (int)group_size, is_scale_transposed ? 1 : groups,
                 is_scale_transposed ? num_tokens : 1};
  const bool fp8 = out_dtype == MCOP_FP8_E4M3FN;
  auto st = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case MCOP_BF16: return fp8 ? dispatch<BF16, true>(a, st) : dispatch<BF16, false>(a, st);
    case MCOP_F16: return fp8 ? dispatch<F16, true>(a, st) : dispatch<F16, false>(a, st);
    case MCOP_F32: return fp8 ? dispatch<F32, true>(a, st) : dispatch<F32, false>(a, st);
    default:
      return set_error(MCOP_E_INVALID, "%s: input dtype %d is not bf16/fp16/fp32", name,
                       (int)in_dtype);
  }
}
