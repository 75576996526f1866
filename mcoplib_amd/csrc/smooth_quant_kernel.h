// smooth_quant_kernel.h -- the SmoothQuant row kernel and its dispatch, shared by the
// translation units that instantiate it per input dtype (rms_norm_smooth_quant*.hip), so the
// instantiations compile in parallel.
// The kernel: SmoothQuant (residual add +) RMSNorm + dynamic per-token
// quantization (mcoplib.op.rms_norm_dynamic_per_token_quant, "fused_rms_norm_dq").
//
// Semantics (per row, b() = round to the input dtype), following op/fused_rms_norm_dq.cu of
// the reference:
//   a = x (+ r, read only);  after_res <- b(a)                       compute_rms :69-99
//   rho = 1/sqrt(sum(a^2)/H + eps) on the unrounded a                 :94 (fp64 sum here)
//   u = (b(a) / rho) * w     [literal form; (b(a) * rho) * w with MCOP_SQ_STANDARD_NORM]
//   after_norm <- b(u);  v = u * smooth                              norm_and_quant :163-186
//   A = max|v|;  int8: s = A/127, q = sat[-127,127](rne(v * (1/s)))  :125-161, :296-297
//   fp8: this library's extension, with no counterpart in the reference (its entry accepts int8
//        only, :658; ScaledQuant is defined for int8 only, :51-66; its scale is A/127, :154):
//        s = A/448, q = e4m3fn(clamp(v / s, +-448)), dividing as the path's fp8 quantizers do
//        (op/vllm/quantization/fused_kernels/quant_conversions.cuh:52-59)
//   A == 0: s = 0 and q = 0.
// One pass: the row stays in VGPRs between the two reductions, so HBM sees x (and residual)
// read once and after_res, after_norm, the codes and the scale written once.  The division by
// rho is the correctly rounded quotient, computed with the per-row reciprocal and one
// Markstein correction (mcop_fdiv_const).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

// Weight / smooth-scale vectors may be stored in the input dtype or in fp32.
template <class EW, int VEC>
struct WVec {
  Pack<typename EW::S, VEC> p;
  __device__ __forceinline__ float at(int e) const { return EW::to_f(p.v[e]); }
};

// fp8 codes of one vector of v: e4m3fn(clamp(v / s, +-448)), the correctly rounded quotient
// (fp8_quotient_codes; `bounded`: 2^-18 <= s <= 2^100, where the short form is exact); a row
// whose absmax is 0 has s = 0 and codes 0.
template <int VEC>
__device__ __forceinline__ Pack<uint8_t, VEC> sq_fp8_codes(const float* v, float amax, float s,
                                                           float inv, bool s_ok, bool bounded) {
  if (amax > 0.0f) return fp8_quotient_codes<VEC>(v, s, inv, s_ok, bounded);
  Pack<uint8_t, VEC> z;
#pragma unroll
  for (int e = 0; e < VEC; ++e) z.v[e] = 0;
  return z;
}

// The lane's streamed vectors of one row's slice [j0, j0 + jn) (the whole row: 0, nvec): x
// (and the residual); lanes past the slice end load its first vector.
template <class E, int VEC, int NV, bool RES, bool EX, bool UA = EX>
__device__ __forceinline__ void sq_load(const RowPos& p, int j0, int jn,
                                        const typename E::S* __restrict__ x,
                                        const typename E::S* __restrict__ res, int hidden,
                                        int tpr, Pack<typename E::S, VEC>* xv,
                                        Pack<typename E::S, VEC>* rv) {
  using S = typename E::S;
  const int64_t lbase = p.lrow * (int64_t)hidden;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int k = vec_index(v, tpr, p.lt);
    const int64_t lj = (int64_t)(j0 + (EX ? k : load_index(k, jn))) * VEC;
    xv[v] = ld_nt<S, VEC>(row_elem<UA>(x, lbase, lj));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(row_elem<UA>(res, lbase, lj));
  }
}

// The row reductions of the one-workgroup kernels: the row's waves combined through LDS.
template <bool EX>
struct WgRowReduce {
  double* red_sum;
  float* red_max;
  int tpr;
  __device__ __forceinline__ double sum(double v) { return row_reduce<EX>(v, red_sum, tpr, SumOp()); }
  __device__ __forceinline__ float max(float v) { return row_reduce<EX>(v, red_max, tpr, MaxOp()); }
};

// One row (or, for tpr < blockDim, one of the workgroup's rows; or one slice [j0, j0 + jn) of a
// row shared by several workgroups) given the lane's loaded vectors and its weight and smooth
// vectors.  `red` combines the row's partial sum of squares and absmax (WgRowReduce, or the
// split-row exchange).  UA: the row index is uniform and the row's element offsets fit 32 bits
// (scalar row base, one 32-bit offset per vector: row_elem<true>).
template <class E, class EW, class ES, int VEC, int NV, bool FP8, bool RES, bool EX, bool UA,
          class Red>
__device__ __forceinline__ void sq_row(const RowPos& p, int j0, int jn,
                                       const Pack<typename E::S, VEC>* xv,
                                       const Pack<typename E::S, VEC>* rv,
                                       const WVec<EW, VEC>* wv, const WVec<ES, VEC>* sv,
                                       uint8_t* __restrict__ out, float* __restrict__ scales,
                                       typename E::S* __restrict__ ares,
                                       typename E::S* __restrict__ anorm, int hidden, int tpr,
                                       float eps, uint32_t flags, Red& red) {
  using S = typename E::S;
  const int64_t base = p.row * (int64_t)hidden;

  float a[NV][VEC];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int k = vec_index(v, tpr, p.lt);
    const int j = j0 + k;
    const bool in = EX || k < jn;
    Pack<S, VEC> o;
    double vs = 0.0;  // lanes past the row end (a copy of vector 0) do not count
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float t = E::to_f(xv[v].v[e]);
      if constexpr (RES) t += E::to_f(rv[v].v[e]);
      o.v[e] = E::from_f(t);
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
      a[v][e] = E::to_f(o.v[e]);  // b(a): what the later passes of the reference re-read
    }
    ss += in ? vs : 0.0;
    if (ares != nullptr && p.live && in) st_nt<S, VEC>(row_elem<UA>(ares, base, (int64_t)j * VEC), o);
  }

  ss = red.sum(ss);
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float inv_rho = mcop_div_rn(1.0f, rho);
  const bool rho_ok = mcop_divisor_ok(rho);
  const bool standard = (flags & MCOP_SQ_STANDARD_NORM) != 0;
  // The literal form: the wave divides in the short form when every lane's elements are in its
  // domain (every b(a)^2 <= a^2 (1 + 2^-8)^2 <= ss (1 + 2^-6), for every b(a) that is finite).
  // Only fp16 can round a finite a to an infinite b(a) while ss stays small (|x + r| >= 65520);
  // for bf16 such an a makes ss/H overflow fp32 or the quotient bound fail, and fp32 does not
  // round.  So fp16 rows with a residual also check that every b(a) is finite.
  constexpr bool kRoundOverflows = RES && sizeof(S) == 2 && !__is_same(E, BF16);
  bool short_div = false;
  if (!standard) {
    float amin = __builtin_inff();
    float amx = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        amin = __builtin_fminf(amin, __builtin_fabsf(a[v][e]));
        if constexpr (kRoundOverflows) amx = __builtin_fmaxf(amx, __builtin_fabsf(a[v][e]));
      }
    }
    const bool in_domain = div_domain_ok(amin, ss * (1.0 + 0x1p-6), inv_rho, rho_ok) &&
                           (!kRoundOverflows || amx <= 0x1.fffffep127f);
    short_div = __builtin_amdgcn_ballot_w64(!in_domain) == 0;
  }

  float amax = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int k = vec_index(v, tpr, p.lt);
    const int j = j0 + k;
    Pack<S, VEC> o;
    float n[VEC];
    if (standard) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) n[e] = a[v][e] * rho;
    } else if (short_div) {
      div_in_domain<VEC>(n, a[v], rho, inv_rho);
    } else {
      div_by_const<VEC>(n, a[v], rho, inv_rho, rho_ok);
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float u = n[e] * wv[v].at(e);
      o.v[e] = E::from_f(u);
      const float vv = u * sv[v].at(e);
      a[v][e] = vv;
      amax = __builtin_fmaxf(amax, __builtin_fabsf(vv));
    }
    if (anorm != nullptr && p.live && (EX || k < jn)) {
      st_nt<S, VEC>(row_elem<UA>(anorm, base, (int64_t)j * VEC), o);
    }
  }
  amax = red.max(amax);

  const float s = mcop_div_rn(amax, FP8 ? 448.0f : 127.0f);
  if (p.live && p.lt == 0) scales[p.row] = s;
  const float inv = amax > 0.0f ? mcop_div_rn(1.0f, s) : 0.0f;
  const bool s_ok = mcop_divisor_ok(s);
  const bool bounded = s >= 0x1p-18f && s <= 0x1p100f;

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int k = vec_index(v, tpr, p.lt);
    const int j = j0 + k;
    if (p.live && (EX || k < jn)) {
      Pack<uint8_t, VEC> q;
      if constexpr (FP8) {
        q = sq_fp8_codes<VEC>(a[v], amax, s, inv, s_ok, bounded);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-127>(a[v][e] * inv);
      }
      st_nt<uint8_t, VEC>(row_elem<UA>(out, base, (int64_t)j * VEC), q);
    }
  }
}

// The weight and smooth vectors (L2-resident, shared by every row) are requested before the
// row's own streamed loads.
// EX (exact): one row per workgroup and every lane in the row (tpr == blockDim.x, NV * tpr ==
// hidden / VEC): uniform row index, scalar base addresses with 32-bit offsets, no bounds tests.
template <class E, class EW, class ES, int VEC, int NV, bool FP8, bool RES, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_rms_norm_smooth_quant(uint8_t* __restrict__ out, float* __restrict__ scales,
                        const typename E::S* __restrict__ x, const typename EW::S* __restrict__ w,
                        const typename ES::S* __restrict__ sm, typename E::S* __restrict__ ares,
                        typename E::S* __restrict__ anorm, const typename E::S* __restrict__ res,
                        int64_t rows, int hidden, int tpr, float eps, uint32_t flags) {
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  const int nvec = hidden / VEC;
  WVec<EW, VEC> wv[NV];
  WVec<ES, VEC> sv[NV];
  RowPos p;
  if constexpr (EX) {
    p = row_pos_one();
  } else {
    p = row_pos(rows, tpr);
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    const int64_t lj = (int64_t)(EX ? j : load_index(j, nvec)) * VEC;
    wv[v].p = ld<typename EW::S, VEC>(row_elem<EX>(w, 0, lj));
    sv[v].p = ld<typename ES::S, VEC>(row_elem<EX>(sm, 0, lj));
  }
  shared_loads_first();
  Pack<typename E::S, VEC> xv[NV], rv[NV];
  sq_load<E, VEC, NV, RES, EX>(p, 0, nvec, x, res, hidden, tpr, xv, rv);
  WgRowReduce<EX> red{red_sum, red_max, tpr};
  sq_row<E, EW, ES, VEC, NV, FP8, RES, EX, EX>(p, 0, nvec, xv, rv, wv, sv, out, scales, ares,
                                                anorm, hidden, tpr, eps, flags, red);
}

// Rows too wide for one workgroup's registers, read once (split_row.h): workgroup b takes slice
// b % slices of row b / slices -- `slice_vecs` vectors, NV a lane -- and runs sq_row on it, the
// row's partial sum of squares and absmax combined with the other slices' through the workspace
// `ws`.  Every slice writes the row's scale (the same value).
template <class E, class EW, class ES, int VEC, int NV, bool FP8, bool RES>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_rms_norm_smooth_quant_split(uint8_t* __restrict__ out, float* __restrict__ scales,
                              const typename E::S* __restrict__ x,
                              const typename EW::S* __restrict__ w,
                              const typename ES::S* __restrict__ sm,
                              typename E::S* __restrict__ ares,
                              typename E::S* __restrict__ anorm,
                              const typename E::S* __restrict__ res, int64_t rows, int hidden,
                              int slices, int slice_vecs, float eps, uint32_t flags,
                              uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  __shared__ double x_sum;
  __shared__ float x_max;
  __shared__ int x_fail;
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int sl = (int)(blockIdx.x % (unsigned)slices);
  RowPos p;
  p.row = blockIdx.x / (unsigned)slices;
  p.lrow = p.row;
  p.lt = (int)threadIdx.x;
  p.live = true;
  const int j0 = sl * slice_vecs;
  const int jn = min(slice_vecs, nvec - j0);
  WVec<EW, VEC> wv[NV];
  WVec<ES, VEC> sv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t lj = (int64_t)(j0 + load_index(vec_index(v, tpr, p.lt), jn)) * VEC;
    wv[v].p = ld<typename EW::S, VEC>(row_elem<true>(w, 0, lj));
    sv[v].p = ld<typename ES::S, VEC>(row_elem<true>(sm, 0, lj));
  }
  shared_loads_first();
  Pack<typename E::S, VEC> xv[NV], rv[NV];
  sq_load<E, VEC, NV, RES, false, true>(p, j0, jn, x, res, hidden, tpr, xv, rv);
  SplitRowReduce red{red_sum, red_max, tpr, ws, p.row, slices, sl,
                     ws + split_ws_words(rows, slices) - 1, timeout_ticks, &x_sum, &x_max,
                     &x_fail};
  sq_row<E, EW, ES, VEC, NV, FP8, RES, false, true>(p, j0, jn, xv, rv, wv, sv, out, scales, ares,
                                                     anorm, hidden, tpr, eps, flags, red);
  if (red.failed() && p.lt == 0) scales[p.row] = __builtin_nanf("");
}

// Rows too wide for the registers: one 1024-lane workgroup per row and three passes over it --
// sum of squares; absmax of v; after_res, after_norm and the codes.  The row head stays in
// registers and LDS; each pass re-reads the rest of x (and of the residual, which this operator only
// reads), and the weight and smooth vectors (shared by all rows).
template <class E, class EW, class ES, int VEC, bool FP8, bool RES>
__global__ void __launch_bounds__(kWideLanes)
k_rms_norm_smooth_quant_wide(uint8_t* __restrict__ out, float* __restrict__ scales,
                             const typename E::S* __restrict__ x,
                             const typename EW::S* __restrict__ w,
                             const typename ES::S* __restrict__ sm,
                             typename E::S* __restrict__ ares, typename E::S* __restrict__ anorm,
                             const typename E::S* __restrict__ res, int hidden, float eps,
                             uint32_t flags) {
  using S = typename E::S;
  // The row head (the lane's first NC vectors of x, and of the residual) is loaded once and
  // kept in registers across the three passes, the next NL in LDS; the passes re-read only the
  // rest of the row.
  // NC is the largest head that compiles without spills at 1024 lanes (128 VGPRs a lane); the
  // fp8 quotient's correction steps take one vector's worth of registers.
  constexpr int NC = VEC > 1 ? (RES ? 4 : (sizeof(typename EW::S) == 4 || FP8) ? 5 : 6) : 16;
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int64_t base = (int64_t)blockIdx.x * hidden;
  // A head slot past the row end holds a copy of the row's vector 0 (its sum-of-squares term
  // is dropped), so the head loads are unconditional: loads under a per-lane branch each wait
  // for completion where the branch rejoins, which serializes their latencies.
  const int tid = (int)threadIdx.x;
  auto hoff = [&](int c, int lt) { return (int64_t)load_index(c * tpr + lt, nvec) * VEC; };
  Pack<S, VEC> xc[NC], rc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    xc[c] = ld<S, VEC>(x + base + hoff(c, tid));
    if constexpr (RES) rc[c] = ld<S, VEC>(res + base + hoff(c, tid));
  }
  // The next NL vectors of every lane are held in LDS: lane-private slots (vector c of lane t
  // at [c][t]: consecutive lanes, consecutive 16-byte slots), so no barrier is needed.  The
  // workgroup already fills a CU's registers, so the 128 KB cost no occupancy.
  constexpr int NL = VEC > 1 ? (RES ? 4 : 8) : 0;
  constexpr int NLS = NL > 0 ? NL * (RES ? 2 : 1) : 1;
  __shared__ Pack<S, VEC> lds[NLS][kWideLanes];
#pragma unroll
  for (int c = 0; c < NL; ++c) {
    lds[c][tid] = ld<S, VEC>(x + base + hoff(NC + c, tid));
    if constexpr (RES) lds[NL + c][tid] = ld<S, VEC>(res + base + hoff(NC + c, tid));
  }
  auto t_head = [&](int c, float* t) {  // a = x (+ r), unrounded; c < NC + NL
    Pack<S, VEC> xv, rv;
    if (c < NC) {
      xv = xc[c];
      if constexpr (RES) rv = rc[c];
    } else {
      xv = lds[c - NC][tid];
      if constexpr (RES) rv = lds[NL + c - NC][tid];
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      t[e] = E::to_f(xv.v[e]);
      if constexpr (RES) t[e] += E::to_f(rv.v[e]);
    }
  };
  auto t_of = [&](int64_t o, float* t) {
    const Pack<S, VEC> xv = ld<S, VEC>(x + base + o);
    Pack<S, VEC> rv;
    if constexpr (RES) rv = ld<S, VEC>(res + base + o);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      t[e] = E::to_f(xv.v[e]);
      if constexpr (RES) t[e] += E::to_f(rv.v[e]);
    }
  };
  const int tail0 = (NC + NL) * tpr + (int)threadIdx.x;  // the lane's first re-read vector
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    float t[VEC];
    t_head(c, t);
    double vs = 0.0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) vs = __builtin_fma((double)t[e], (double)t[e], vs);
    ss += c * tpr + tid < nvec ? vs : 0.0;
  }
  for (int j = tail0; j < nvec; j += tpr) {
    float t[VEC];
    t_of((int64_t)j * VEC, t);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss = __builtin_fma((double)t[e], (double)t[e], ss);
  }
  ss = row_reduce(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float inv_rho = mcop_div_rn(1.0f, rho);
  const bool rho_ok = mcop_divisor_ok(rho);
  const bool standard = (flags & MCOP_SQ_STANDARD_NORM) != 0;
  // u = (b(a) / rho) * w (or (b(a) * rho) * w), v = u * smooth
  auto uv_of = [&](int64_t o, const float* t, float* u, float* v) {
    float a[VEC], n[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) a[e] = rnd<E>(t[e]);
    if (standard) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) n[e] = a[e] * rho;
    } else {
      div_by_const<VEC>(n, a, rho, inv_rho, rho_ok);
    }
    WVec<EW, VEC> wv;
    WVec<ES, VEC> sv;
    wv.p = ld<typename EW::S, VEC>(w + o);
    sv.p = ld<typename ES::S, VEC>(sm + o);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      u[e] = n[e] * wv.at(e);
      v[e] = u[e] * sv.at(e);
    }
  };
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + (int)threadIdx.x;
    if (j < nvec) {
      float t[VEC], u[VEC], v[VEC];
      t_head(c, t);
      uv_of((int64_t)j * VEC, t, u, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[e]));
    }
  }
  for (int j = tail0; j < nvec; j += tpr) {
    float t[VEC], u[VEC], v[VEC];
    t_of((int64_t)j * VEC, t);
    uv_of((int64_t)j * VEC, t, u, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[e]));
  }
  amax = row_reduce(amax, red_max, tpr, MaxOp());
  const float s = mcop_div_rn(amax, FP8 ? 448.0f : 127.0f);
  if (threadIdx.x == 0) scales[blockIdx.x] = s;
  const float inv = amax > 0.0f ? mcop_div_rn(1.0f, s) : 0.0f;
  const bool s_ok = mcop_divisor_ok(s);
  const bool bounded = s >= 0x1p-18f && s <= 0x1p100f;
  auto emit = [&](int64_t o, const float* t) {
    float u[VEC], v[VEC];
    uv_of(o, t, u, v);
    Pack<S, VEC> ar, an;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      ar.v[e] = E::from_f(t[e]);
      an.v[e] = E::from_f(u[e]);
    }
    if (ares != nullptr) st<S, VEC>(ares + base + o, ar);
    if (anorm != nullptr) st<S, VEC>(anorm + base + o, an);
    Pack<uint8_t, VEC> q;
    if constexpr (FP8) {
      q = sq_fp8_codes<VEC>(v, amax, s, inv, s_ok, bounded);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-127>(v[e] * inv);
    }
    st<uint8_t, VEC>(out + base + o, q);
  };
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + (int)threadIdx.x;
    if (j < nvec) {
      float t[VEC];
      t_head(c, t);
      emit((int64_t)j * VEC, t);
    }
  }
  for (int j = tail0; j < nvec; j += tpr) {
    float t[VEC];
    t_of((int64_t)j * VEC, t);
    emit((int64_t)j * VEC, t);
  }
}

struct Args {
  void* out;
  float* scales;
  const void* x;
  const void* w;
  const void* sm;
  void* ares;
  void* anorm;
  const void* res;
  int64_t rows;
  int hidden;
  float eps;
  uint32_t flags;
};

template <class E, class EW, class ES, int VEC, bool FP8, bool RES>
static void launch_nv(const Geometry& g, const Args& a, hipStream_t st) {
  using S = typename E::S;
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* o = static_cast<uint8_t*>(a.out);
  auto* xp = static_cast<const S*>(a.x);
  auto* wp = static_cast<const typename EW::S*>(a.w);
  auto* sp = static_cast<const typename ES::S*>(a.sm);
  auto* arp = static_cast<S*>(a.ares);
  auto* anp = static_cast<S*>(a.anorm);
  auto* rp = static_cast<const S*>(a.res);
#define MCOP_LAUNCH(NVV, EXX)                                                                   \
  hipLaunchKernelGGL((k_rms_norm_smooth_quant<E, EW, ES, VEC, NVV, FP8, RES, EXX>), grid,      \
                     block, 0, st, o, a.scales, xp, wp, sp, arp, anp, rp, a.rows, a.hidden,      \
                     g.tpr, a.eps, a.flags)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it) on the latency path (at most 256
    // rows) take the EX form; bandwidth-bound shapes keep the generic one (a uniform-row form
    // measured slower at cfg 4's width)
    // (and only when the EX form keeps its registers)
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == a.hidden / VEC && a.rows <= 256;
#define MCOP_EX(NVV)                                                                           \
  (ex && exact_form_ok(reinterpret_cast<const void*>(                                          \
             &k_rms_norm_smooth_quant<E, EW, ES, VEC, NVV, FP8, RES, true>)))
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

template <class E, class EW, class ES, int VEC, bool FP8, bool RES>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4
               ? reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, 1, 4, FP8, RES>)
               : reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, 1, 16, FP8, RES>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, VEC, 1, FP8, RES>);
      case 2: return reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, VEC, 2, FP8, RES>);
      case 4: return reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, VEC, 4, FP8, RES>);
      case 8: return reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, VEC, 8, FP8, RES>);
      default: return reinterpret_cast<const void*>(&k_rms_norm_smooth_quant<E, EW, ES, VEC, 16, FP8, RES>);
    }
  }
}

// Rows too wide for the register kernels, vector path: the split-row kernel when it applies, its
// workspace from the stream-ordered allocator; MCOP_E_UNSUPPORTED when it does not.
template <class E, class EW, class ES, int VEC, bool FP8, bool RES>
static int launch_split(const char* name, const Args& a, hipStream_t st) {
  using S = typename E::S;
  // 512-lane workgroups (half the slices, so half the exchanges per row for the same resident
  // vectors per CU): 450 us against 469 us at 256 lanes for 2048 x 131072 bf16 fp8
  const SplitKernel k4{reinterpret_cast<const void*>(
                           &k_rms_norm_smooth_quant_split<E, EW, ES, VEC, 4, FP8, RES>), 4, 512};
  return split_run(name, {k4}, a.rows, a.hidden / VEC, nullptr, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    const int64_t off = r0 * (int64_t)a.hidden;
    auto* o = static_cast<uint8_t*>(a.out) + off;
    float* sc = a.scales + r0;
    auto* xp = static_cast<const S*>(a.x) + off;
    auto* wp = static_cast<const typename EW::S*>(a.w);
    auto* sp = static_cast<const typename ES::S*>(a.sm);
    auto* arp = a.ares == nullptr ? nullptr : static_cast<S*>(a.ares) + off;
    auto* anp = a.anorm == nullptr ? nullptr : static_cast<S*>(a.anorm) + off;
    auto* rp = a.res == nullptr ? nullptr : static_cast<const S*>(a.res) + off;
    int h = a.hidden, slices = p.slices, slice_vecs = p.slice_vecs;
    float e = a.eps;
    uint32_t f = a.flags;
    int64_t timeout = p.timeout_ticks;
    void* args[] = {&o, &sc, &xp, &wp, &sp, &arp, &anp, &rp, &n, &h, &slices, &slice_vecs, &e,
                    &f, &ws, &timeout};
    return launch(args);
  });
}

template <class E, class EW, class ES, bool FP8>
static int dispatch(const Args& a, hipStream_t st) {
  constexpr int V = E::VEC;
  constexpr int WB = (int)sizeof(typename EW::S) * V, SB = (int)sizeof(typename ES::S) * V;
  const bool vec_ok = a.hidden % V == 0 && aligned(16, a.x, a.ares, a.anorm, a.res) &&
                      aligned(WB, a.w) && aligned(SB, a.sm) && aligned(V, a.out);
  const bool r = a.res != nullptr;
  const KernelOfNv kernels =
      vec_ok ? (r ? &kernel_of<E, EW, ES, V, FP8, true> : &kernel_of<E, EW, ES, V, FP8, false>)
             : (r ? &kernel_of<E, EW, ES, 1, FP8, true> : &kernel_of<E, EW, ES, 1, FP8, false>);
  if (!row_fits(a.hidden, vec_ok ? V : 1, kernels)) {
    const char* name = "rms_norm_dynamic_per_token_quant (smooth)";
    if (vec_ok && split_rows_enabled()) {
      const int rc = r ? launch_split<E, EW, ES, V, FP8, true>(name, a, st)
                       : launch_split<E, EW, ES, V, FP8, false>(name, a, st);
      if (rc != MCOP_E_UNSUPPORTED) return rc;
    }
    if (!wide_rows_ok(name, a.rows)) return MCOP_E_UNSUPPORTED;
    using S = typename E::S;
    auto* o = static_cast<uint8_t*>(a.out);
    auto* xp = static_cast<const S*>(a.x);
    auto* wp = static_cast<const typename EW::S*>(a.w);
    auto* sp = static_cast<const typename ES::S*>(a.sm);
    auto* arp = static_cast<S*>(a.ares);
    auto* anp = static_cast<S*>(a.anorm);
    auto* rp = static_cast<const S*>(a.res);
    const dim3 grid((unsigned)a.rows), block(kWideLanes);
#define MCOP_WIDE(VV, RR)                                                                      \
  hipLaunchKernelGGL((k_rms_norm_smooth_quant_wide<E, EW, ES, VV, FP8, RR>), grid, block, 0,   \
                     st, o, a.scales, xp, wp, sp, arp, anp, rp, a.hidden, a.eps, a.flags)
    if (vec_ok) {
      if (r) MCOP_WIDE(V, true); else MCOP_WIDE(V, false);
    } else {
      if (r) MCOP_WIDE(1, true); else MCOP_WIDE(1, false);
    }
#undef MCOP_WIDE
    return check_launch(name);
  }
  Geometry g;
  if (!choose_geometry("rms_norm_dynamic_per_token_quant (smooth)", a.rows, a.hidden,
                       vec_ok ? V : 1, kernels, &g)) {
    return MCOP_E_UNSUPPORTED;
  }
  const bool has_res = a.res != nullptr;
  if (g.vec == 1) {
    if (has_res) launch_nv<E, EW, ES, 1, FP8, true>(g, a, st);
    else launch_nv<E, EW, ES, 1, FP8, false>(g, a, st);
  } else {
    if (has_res) launch_nv<E, EW, ES, V, FP8, true>(g, a, st);
    else launch_nv<E, EW, ES, V, FP8, false>(g, a, st);
  }
  return check_launch("rms_norm_dynamic_per_token_quant (smooth)");
}

template <class E, class EW, class ES>
static int dispatch_out(const Args& a, bool fp8, hipStream_t st) {
  return fp8 ? dispatch<E, EW, ES, true>(a, st) : dispatch<E, EW, ES, false>(a, st);
}

// Weight and smooth dtypes: each is the input dtype or fp32.
template <class E>
int dispatch_ws(const Args& a, mcop_dtype wdt, mcop_dtype sdt, mcop_dtype in_dt, bool fp8,
                       hipStream_t st) {
  const bool w32 = wdt == MCOP_F32, s32 = sdt == MCOP_F32;
  if ((!w32 && wdt != in_dt) || (!s32 && sdt != in_dt)) {
    return set_error(MCOP_E_INVALID,
                     "rms_norm_dynamic_per_token_quant (smooth): weight dtype %d / smooth dtype "
                     "%d must each be the input dtype %d or fp32",
                     (int)wdt, (int)sdt, (int)in_dt);
  }
  if (w32 && s32) return dispatch_out<E, F32, F32>(a, fp8, st);
  if (w32) return dispatch_out<E, F32, E>(a, fp8, st);
  if (s32) return dispatch_out<E, E, F32>(a, fp8, st);
  return dispatch_out<E, E, E>(a, fp8, st);
}


int dispatch_smooth_bf16(const Args& a, mcop_dtype wdt, mcop_dtype sdt, bool fp8, hipStream_t st);
int dispatch_smooth_f16(const Args& a, mcop_dtype wdt, mcop_dtype sdt, bool fp8, hipStream_t st);

}  // namespace mcop
