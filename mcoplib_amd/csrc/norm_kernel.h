// norm_kernel.h -- the RMSNorm row kernel without quantization and its dispatch, shared by the
// translation units that instantiate it per input dtype (rms_norm*.hip).
//
// One kernel serves three reference operators whose rounding chains differ (b() = round to the
// input dtype, a = x [+ r] in fp32, rho = 1/sqrt(sum(a^2)/H + eps), fp64 row sum here):
//   NORM_VLLM  vLLM _C::rms_norm (op/vllm/layernorm_kernels.cu:15-86):
//              y = b(b(x * rho) * w)
//   NORM_MC    mcoplib.op.rms_norm / head_rms_norm, their vectorized kernels
//              (op/fused_rms_norm_dq.cu:305-382, 493-557):
//              y = b((a * d) * w), d = rms_div ? RN(1/rho) : rho, a unrounded
//   NORM_MC_GENERIC  the same operators' element-wise kernels (:389-420, 559-578 with
//              compute_rms :69-99, norm_without_smooth :189-209, do_head_norm :212-224), which
//              the reference runs when the row is not a whole number of its vectors or longer
//              than three vectors per thread of a 1024-thread block:
//              y = b((a~ / rho) * w) if rms_div else b((a~ * rho) * w), a~ = b(a) with a
//              residual (it re-reads after_res), the input otherwise
// With a residual (mcoplib.op.rms_norm only) after_res <- b(a); the residual is not updated.
//
// Rows are addressed through a three-level index so that one kernel covers contiguous rows,
// vLLM's 3-D / 4-D strided inputs and head_rms_norm's selected heads with per-head weights:
//   row r = (i0 * n1 + i1) * n2 + i2;  input row at i0*s0 + i1*s1 + i2*s2, output row at
//   i0*o0 + i1*o1 + i2*o2, weight at i2*w2; residual and after_res rows at r * H.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

enum NormMode { NORM_VLLM = 0, NORM_MC = 1, NORM_MC_GENERIC = 2 };

struct RowMap {
  int64_t n1, n2;      // extents of the two inner indices (1 when unused)
  int64_t s0, s1, s2;  // input element strides
  int64_t o0, o1, o2;  // output element strides
  int64_t w2;          // weight element stride per inner index (0: one weight row)
};

struct RowOffsets {
  int64_t in, out, w;
};

// q = r / n, r % n for a row index r >= 0 and an extent n >= 1 that is the same for every lane:
// a shift for powers of two (head counts usually are), 32-bit division when both fit, else
// 64-bit division.
__device__ __forceinline__ int64_t div_extent(int64_t r, int64_t n, int64_t* rem) {
  if ((n & (n - 1)) == 0) {
    *rem = r & (n - 1);
    return r >> __builtin_ctzll((uint64_t)n);
  }
  if (((uint64_t)r | (uint64_t)n) <= 0xffffffffull) {
    const uint32_t q = (uint32_t)r / (uint32_t)n;
    *rem = (int64_t)((uint32_t)r - q * (uint32_t)n);
    return q;
  }
  *rem = r % n;
  return r / n;
}

__device__ __forceinline__ RowOffsets row_offsets(const RowMap& m, int64_t r) {
  int64_t i0 = r, i1 = 0, i2 = 0;
  if (m.n2 != 1) i0 = div_extent(r, m.n2, &i2);
  if (m.n1 != 1) i0 = div_extent(i0, m.n1, &i1);
  return {i0 * m.s0 + i1 * m.s1 + i2 * m.s2, i0 * m.o0 + i1 * m.o1 + i2 * m.o2, i2 * m.w2};
}

template <class EW, int VEC>
struct NormW {
  Pack<typename EW::S, VEC> p;
  __device__ __forceinline__ float at(int e) const { return EW::to_f(p.v[e]); }
};

// The normalized output of one vector from a (x [+ r], or b(x + r) for the element-wise chain
// with a residual), as the register-resident kernel computes it inline.
template <class E, class EW, int VEC>
__device__ __forceinline__ Pack<typename E::S, VEC> norm_out(const float* a,
                                                             const NormW<EW, VEC>& w, float rho,
                                                             float inv_rho, int mode,
                                                             int rms_div) {
  Pack<typename E::S, VEC> o;
  if (mode == NORM_VLLM) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(rnd<E>(a[e] * rho) * w.at(e));
  } else if (mode == NORM_MC || !rms_div) {
    const float d = (mode == NORM_MC && rms_div) ? inv_rho : rho;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f((a[e] * d) * w.at(e));
  } else {
    float n[VEC];
    div_by_const<VEC>(n, a, rho, inv_rho, mcop_divisor_ok(rho));
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(n[e] * w.at(e));
  }
  return o;
}

// EX (exact): one row per workgroup and every lane in the row (tpr == blockDim.x, NV * tpr ==
// hidden / VEC): uniform row index, scalar base addresses with 32-bit offsets, no bounds tests.
template <class E, class EW, int VEC, int NV, bool RES, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_rms_norm(typename E::S* __restrict__ out, typename E::S* __restrict__ ares,
           const typename E::S* __restrict__ x, const typename EW::S* __restrict__ w,
           const typename E::S* __restrict__ res, RowMap map, int64_t rows, int hidden, int tpr,
           float eps, int mode, int rms_div) {
  using S = typename E::S;
  __shared__ double red_sum[16];
  RowPos p;
  if constexpr (EX) {
    p = row_pos_one();
  } else {
    p = row_pos(rows, tpr);
  }
  const int nvec = hidden / VEC;
  const RowOffsets lo = row_offsets(map, p.lrow);
  const int64_t out_base = p.row == p.lrow ? lo.out : 0;
  const int64_t rbase = p.row * (int64_t)hidden;
  const int64_t lrbase = p.lrow * (int64_t)hidden;
  auto lj_of = [&](int v) {
    const int j = vec_index(v, tpr, p.lt);
    return (int64_t)(EX ? j : load_index(j, nvec)) * VEC;
  };

  Pack<S, VEC> xv[NV], rv[NV];
  NormW<EW, VEC> wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    wv[v].p = ld<typename EW::S, VEC>(row_elem<EX>(w, lo.w, lj_of(v)));
  }
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t lj = lj_of(v);
    xv[v] = ld_nt<S, VEC>(row_elem<EX>(x, lo.in, lj));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(row_elem<EX>(res, lrbase, lj));
  }

  float a[NV][VEC];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    const bool in = EX || j < nvec;
    double vs = 0.0;  // lanes past the row end (a copy of vector 0) do not count
    Pack<S, VEC> o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float t = E::to_f(xv[v].v[e]);
      if constexpr (RES) t += E::to_f(rv[v].v[e]);
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
      if constexpr (RES) {
        o.v[e] = E::from_f(t);
        // the element-wise kernels re-read the rounded after_res
        if (mode == NORM_MC_GENERIC) t = E::to_f(o.v[e]);
      }
      a[v][e] = t;
    }
    ss += in ? vs : 0.0;
    if constexpr (RES) {
      if (p.live && in) st_nt<S, VEC>(row_elem<EX>(ares, rbase, (int64_t)j * VEC), o);
    }
  }
  ss = row_reduce<EX>(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float inv_rho = mcop_div_rn(1.0f, rho);
  // The division form: the wave divides in the short form when every lane's elements are in its
  // domain (every a^2 <= ss (1 + 2^-6), rounded or not, for every a that is finite).  Only an
  // fp16 rounding of the residual sum can turn a finite sum (|x + r| >= 65520) into an infinite
  // a while ss stays small (bf16: ss/H overflows fp32 or the quotient bound fails; fp32 does not
  // round), so fp16 rows with a residual also check that every a is finite.
  constexpr bool kRoundOverflows = RES && sizeof(S) == 2 && !__is_same(E, BF16);
  bool short_div = false;
  if (mode != NORM_VLLM && mode != NORM_MC && rms_div) {
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
    const bool in_domain = div_domain_ok(amin, ss * (1.0 + 0x1p-6), inv_rho,
                                         mcop_divisor_ok(rho)) &&
                           (!kRoundOverflows || amx <= 0x1.fffffep127f);
    short_div = __builtin_amdgcn_ballot_w64(!in_domain) == 0;
  }

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    if (!(p.live && (EX || j < nvec))) continue;
    // kept inline (norm_out computes the same): through the helper the compiler issued this
    // kernel's streamed load before the shared weight load
    Pack<S, VEC> o;
    if (mode == NORM_VLLM) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(rnd<E>(a[v][e] * rho) * wv[v].at(e));
    } else if (mode == NORM_MC || !rms_div) {
      const float d = (mode == NORM_MC && rms_div) ? inv_rho : rho;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f((a[v][e] * d) * wv[v].at(e));
    } else {
      float n[VEC];
      if (short_div) {
        div_in_domain<VEC>(n, a[v], rho, inv_rho);
      } else {
        div_by_const<VEC>(n, a[v], rho, inv_rho, mcop_divisor_ok(rho));
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(n[e] * wv[v].at(e));
    }
    st_nt<S, VEC>(row_elem<EX>(out, out_base, (int64_t)j * VEC), o);
  }
}

// Rows too wide for one workgroup's registers, read once (split_row.h): workgroup b takes slice
// b % slices of row b / slices -- `slice_vecs` vectors, NV a lane -- and combines the row's sum
// of squares with the other slices' through the workspace `ws` (split_sum, in slice order);
// every other step is the register kernel's, element by element.  The launch covers rows
// [row0, row0 + rows) of the row map.  The row index is uniform: scalar row bases, 32-bit offsets
// within the row.
template <class E, class EW, int VEC, int NV, bool RES>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_rms_norm_split(typename E::S* __restrict__ out, typename E::S* __restrict__ ares,
                 const typename E::S* __restrict__ x, const typename EW::S* __restrict__ w,
                 const typename E::S* __restrict__ res, RowMap map, int64_t row0, int64_t rows,
                 int hidden, float eps, int mode, int rms_div, int slices, int slice_vecs,
                 uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  using S = typename E::S;
  __shared__ double red_sum[16];
  __shared__ double x_sum;
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int lt = (int)threadIdx.x;
  const int sl = (int)(blockIdx.x % (unsigned)slices);
  const int64_t row = blockIdx.x / (unsigned)slices;
  const int j0 = sl * slice_vecs;
  const int jn = min(slice_vecs, nvec - j0);
  const RowOffsets lo = row_offsets(map, row0 + row);
  const int64_t rbase = (row0 + row) * (int64_t)hidden;
  // Lanes past the slice end re-read the slice's first vector, which does not count.
  auto in_of = [&](int v) { return vec_index(v, tpr, lt) < jn; };
  auto lj_of = [&](int v) {
    return (int64_t)(j0 + (in_of(v) ? vec_index(v, tpr, lt) : 0)) * VEC;
  };
  Pack<S, VEC> xv[NV], rv[NV];
  NormW<EW, VEC> wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    wv[v].p = ld<typename EW::S, VEC>(row_elem<true>(w, lo.w, lj_of(v)));
  }
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    xv[v] = ld_nt<S, VEC>(row_elem<true>(x, lo.in, lj_of(v)));
    if constexpr (RES) rv[v] = ld_nt<S, VEC>(row_elem<true>(res, rbase, lj_of(v)));
  }
  // a, held in the dtype: x without a residual, b(x + r) with one (the element-wise chain's
  // a~; the host sends the vectorized chain with a residual, whose a is unrounded, elsewhere)
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    double vs = 0.0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float t = E::to_f(xv[v].v[e]);
      if constexpr (RES) {
        t += E::to_f(rv[v].v[e]);
        xv[v].v[e] = E::from_f(t);
      }
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
    }
    ss += in_of(v) ? vs : 0.0;
    if constexpr (RES) {
      if (in_of(v)) st_nt<S, VEC>(row_elem<true>(ares, rbase, lj_of(v)), xv[v]);
    }
  }
  SplitRowReduce red{red_sum, nullptr, tpr, ws, row, slices, sl,
                     ws + split_ws_words(rows, slices) - 1, timeout_ticks, &x_sum, nullptr};
  ss = red.sum(ss);
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float inv_rho = mcop_div_rn(1.0f, rho);
  // the register kernel's choice of division form, per wave (both forms give the correctly
  // rounded quotient)
  constexpr bool kRoundOverflows = RES && sizeof(S) == 2 && !__is_same(E, BF16);
  bool short_div = false;
  if (mode != NORM_VLLM && mode != NORM_MC && rms_div) {
    float amin = __builtin_inff();
    float amx = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float t = __builtin_fabsf(E::to_f(xv[v].v[e]));
        amin = __builtin_fminf(amin, t);
        if constexpr (kRoundOverflows) amx = __builtin_fmaxf(amx, t);
      }
    }
    const bool in_domain = div_domain_ok(amin, ss * (1.0 + 0x1p-6), inv_rho,
                                         mcop_divisor_ok(rho)) &&
                           (!kRoundOverflows || amx <= 0x1.fffffep127f);
    short_div = __builtin_amdgcn_ballot_w64(!in_domain) == 0;
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (!in_of(v)) continue;
    float av[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) av[e] = E::to_f(xv[v].v[e]);
    Pack<S, VEC> o;
    if (mode == NORM_VLLM) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(rnd<E>(av[e] * rho) * wv[v].at(e));
    } else if (mode == NORM_MC || !rms_div) {
      const float d = (mode == NORM_MC && rms_div) ? inv_rho : rho;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f((av[e] * d) * wv[v].at(e));
    } else {
      float n[VEC];
      if (short_div) {
        div_in_domain<VEC>(n, av, rho, inv_rho);
      } else {
        div_by_const<VEC>(n, av, rho, inv_rho, mcop_divisor_ok(rho));
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) o.v[e] = E::from_f(n[e] * wv[v].at(e));
    }
    st_nt<S, VEC>(row_elem<true>(out, lo.out, lj_of(v)), o);
  }
}

// Rows too wide for the registers: one 1024-lane workgroup per row, two passes (sum of squares;
// after_res and the output).  The row's head stays on chip between the passes -- the first NC
// vectors of x (and residual) of every lane in registers, the next NL in lane-private LDS slots
// (vector c of lane t at [c][t], so no barrier is needed; the workgroup already fills a CU's
// registers, so the 128 KB cost no occupancy) -- and the second pass re-reads the rest of the
// row, and the weight.
template <class E, class EW, int VEC, bool RES>
__global__ void __launch_bounds__(kWideLanes)
k_rms_norm_wide(typename E::S* __restrict__ out, typename E::S* __restrict__ ares,
                const typename E::S* __restrict__ x, const typename EW::S* __restrict__ w,
                const typename E::S* __restrict__ res, RowMap map, int hidden, float eps,
                int mode, int rms_div) {
  using S = typename E::S;
  // NC: the largest register head that compiles without spills at 1024 lanes (fp16 conversions
  // take more registers)
  constexpr int NC = VEC > 1 ? (RES ? 4 : std::is_same<E, F16>::value ? 4 : 8) : 16;
  constexpr int NL = VEC > 1 ? (RES ? 4 : 8) : 0;
  constexpr int NLS = NL > 0 ? NL * (RES ? 2 : 1) : 1;
  __shared__ double red_sum[16];
  __shared__ Pack<S, VEC> lds[NLS][kWideLanes];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x, tid = (int)threadIdx.x;
  const RowOffsets lo = row_offsets(map, blockIdx.x);
  const int64_t rbase = (int64_t)blockIdx.x * hidden;
  auto t_from = [&](const Pack<S, VEC>& xv, const Pack<S, VEC>& rv, float* t) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      t[e] = E::to_f(xv.v[e]);
      if constexpr (RES) t[e] += E::to_f(rv.v[e]);
    }
  };
  auto t_of = [&](int64_t o, float* t) {
    const Pack<S, VEC> xv = ld<S, VEC>(x + lo.in + o);
    Pack<S, VEC> rv;
    if constexpr (RES) rv = ld<S, VEC>(res + rbase + o);
    t_from(xv, rv, t);
  };
  Pack<S, VEC> xc[NC], rc[NC];
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + tid;
    if (j < nvec) {
      const Pack<S, VEC> xv = ld<S, VEC>(x + lo.in + (int64_t)j * VEC);
      Pack<S, VEC> rv;
      if constexpr (RES) rv = ld<S, VEC>(res + rbase + (int64_t)j * VEC);
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
      Pack<S, VEC> rv;
      if constexpr (RES) rv = lds[NL + c - NC][tid];
      t_from(lds[c - NC][tid], rv, t);
    }
  };
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    if (c * tpr + tid < nvec) {
      float t[VEC];
      t_head(c, t);
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss = __builtin_fma((double)t[e], (double)t[e], ss);
    }
  }
  const int tail0 = (NC + NL) * tpr + tid;
  for (int j = tail0; j < nvec; j += tpr) {
    float t[VEC];
    t_of((int64_t)j * VEC, t);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss = __builtin_fma((double)t[e], (double)t[e], ss);
  }
  ss = row_reduce(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float inv_rho = mcop_div_rn(1.0f, rho);
  auto emit = [&](int64_t o, float* t) {
    if constexpr (RES) {
      Pack<S, VEC> r;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        r.v[e] = E::from_f(t[e]);
        // the element-wise kernels re-read the rounded after_res
        if (mode == NORM_MC_GENERIC) t[e] = E::to_f(r.v[e]);
      }
      st<S, VEC>(ares + rbase + o, r);
    }
    NormW<EW, VEC> wv;
    wv.p = ld<typename EW::S, VEC>(w + lo.w + o);
    st<S, VEC>(out + lo.out + o, norm_out<E, EW, VEC>(t, wv, rho, inv_rho, mode, rms_div));
  };
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + tid;
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

struct NormArgs {
  void* out;
  void* ares;
  const void* x;
  const void* w;
  const void* res;
  RowMap map;
  int64_t rows;
  int hidden;
  float eps;
  int mode;
  int rms_div;
};

template <class E, class EW, int VEC, bool RES>
static void norm_launch_nv(const Geometry& g, const NormArgs& a, hipStream_t st) {
  using S = typename E::S;
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* o = static_cast<S*>(a.out);
  auto* arp = static_cast<S*>(a.ares);
  auto* xp = static_cast<const S*>(a.x);
  auto* wp = static_cast<const typename EW::S*>(a.w);
  auto* rp = static_cast<const S*>(a.res);
#define MCOP_LAUNCH(NVV, EXX)                                                                  \
  hipLaunchKernelGGL((k_rms_norm<E, EW, VEC, NVV, RES, EXX>), grid, block, 0, st, o, arp, xp, wp, \
                     rp, a.map, a.rows, a.hidden, g.tpr, a.eps, a.mode, a.rms_div)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it): the EX form at two vectors a lane,
    // and at four or eight on the latency path (at most 256 rows), when it keeps its registers
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == a.hidden / VEC &&
                    (g.nv == 2 || a.rows <= 256);
#define MCOP_EX(NVV)                                                                           \
  (ex && exact_form_ok(reinterpret_cast<const void*>(&k_rms_norm<E, EW, VEC, NVV, RES, true>)))
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

template <class E, class EW, int VEC, bool RES>
static const void* norm_kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_rms_norm<E, EW, 1, 4, RES>)
                   : reinterpret_cast<const void*>(&k_rms_norm<E, EW, 1, 16, RES>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_rms_norm<E, EW, VEC, 1, RES>);
      case 2: return reinterpret_cast<const void*>(&k_rms_norm<E, EW, VEC, 2, RES>);
      case 4: return reinterpret_cast<const void*>(&k_rms_norm<E, EW, VEC, 4, RES>);
      case 8: return reinterpret_cast<const void*>(&k_rms_norm<E, EW, VEC, 8, RES>);
      default: return reinterpret_cast<const void*>(&k_rms_norm<E, EW, VEC, 16, RES>);
    }
  }
}

// Vectors are usable when every row start and the weight rows stay 16-byte aligned.
template <class E, class EW>
static bool norm_vec_ok(const NormArgs& a) {
  constexpr int V = E::VEC;
  constexpr int WB = (int)sizeof(typename EW::S) * V;
  const RowMap& m = a.map;
  const bool strides = m.s0 % V == 0 && m.s1 % V == 0 && m.s2 % V == 0 && m.o0 % V == 0 &&
                       m.o1 % V == 0 && m.o2 % V == 0 && m.w2 % V == 0;
  return a.hidden % V == 0 && strides && aligned(16, a.x, a.out, a.res, a.ares) &&
         aligned(WB, a.w);
}

// Rows too wide for the register kernels, vector path: the split-row kernel when it applies, its
// workspace from the stream-ordered allocator; MCOP_E_UNSUPPORTED (no message) when it does not.
template <class E, class EW, int VEC, bool RES>
static int norm_launch_split(const char* name, const NormArgs& a, hipStream_t st) {
  using S = typename E::S;
  // the kernel holds a in the dtype, which the vectorized chain's unrounded x + r is not (that
  // chain only runs on rows narrow enough for the register kernels)
  if (RES && a.mode != NORM_MC_GENERIC) return MCOP_E_UNSUPPORTED;
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  const SplitKernel k8{fn(&k_rms_norm_split<E, EW, VEC, 8, RES>), 8};
  const SplitKernel k4{fn(&k_rms_norm_split<E, EW, VEC, 4, RES>), 4};
  return split_run(name, {k8, k4}, a.rows, a.hidden / VEC, nullptr, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    S* o = static_cast<S*>(a.out);
    S* arp = static_cast<S*>(a.ares);
    const S* xp = static_cast<const S*>(a.x);
    const typename EW::S* wp = static_cast<const typename EW::S*>(a.w);
    const S* rp = static_cast<const S*>(a.res);
    RowMap m = a.map;
    int64_t row0 = r0;
    int h = a.hidden, mode = a.mode, rms_div = a.rms_div, slices = p.slices,
        slice_vecs = p.slice_vecs;
    float e = a.eps;
    int64_t timeout = p.timeout_ticks;
    void* args[] = {&o, &arp, &xp, &wp, &rp, &m, &row0, &n, &h, &e, &mode, &rms_div, &slices,
                    &slice_vecs, &ws, &timeout};
    return launch(args);
  });
}

template <class E, class EW>
static int norm_dispatch(const char* name, const NormArgs& a, hipStream_t st) {
  constexpr int V = E::VEC;
  const bool vec_ok = norm_vec_ok<E, EW>(a);
  const bool r = a.res != nullptr;
  const KernelOfNv kernels =
      vec_ok ? (r ? &norm_kernel_of<E, EW, V, true> : &norm_kernel_of<E, EW, V, false>)
             : (r ? &norm_kernel_of<E, EW, 1, true> : &norm_kernel_of<E, EW, 1, false>);
  if (!row_fits(a.hidden, vec_ok ? V : 1, kernels)) {
    if (vec_ok && split_rows_enabled()) {
      const int rc = r ? norm_launch_split<E, EW, V, true>(name, a, st)
                       : norm_launch_split<E, EW, V, false>(name, a, st);
      if (rc != MCOP_E_UNSUPPORTED) return rc;
    }
    if (!wide_rows_ok(name, a.rows)) return MCOP_E_UNSUPPORTED;
    using S = typename E::S;
    auto* o = static_cast<S*>(a.out);
    auto* arp = static_cast<S*>(a.ares);
    auto* xp = static_cast<const S*>(a.x);
    auto* wp = static_cast<const typename EW::S*>(a.w);
    auto* rp = static_cast<const S*>(a.res);
    const dim3 grid((unsigned)a.rows), block(kWideLanes);
#define MCOP_WIDE(VV, RR)                                                                  \
  hipLaunchKernelGGL((k_rms_norm_wide<E, EW, VV, RR>), grid, block, 0, st, o, arp, xp, wp, rp, \
                     a.map, a.hidden, a.eps, a.mode, a.rms_div)
    if (vec_ok) {
      if (r) MCOP_WIDE(V, true); else MCOP_WIDE(V, false);
    } else {
      if (r) MCOP_WIDE(1, true); else MCOP_WIDE(1, false);
    }
#undef MCOP_WIDE
    return check_launch(name);
  }
  Geometry g;
  if (!choose_geometry(name, a.rows, a.hidden, vec_ok ? V : 1, kernels, &g)) {
    return MCOP_E_UNSUPPORTED;
  }
  if (g.vec == 1) {
    if (r) norm_launch_nv<E, EW, 1, true>(g, a, st);
    else norm_launch_nv<E, EW, 1, false>(g, a, st);
  } else {
    if (r) norm_launch_nv<E, EW, V, true>(g, a, st);
    else norm_launch_nv<E, EW, V, false>(g, a, st);
  }
  return check_launch(name);
}

// Weight dtype: the input dtype, fp32 or (head_rms_norm) bf16.
template <class E>
int norm_dispatch_w(const char* name, const NormArgs& a, mcop_dtype wdt, hipStream_t st) {
  switch (wdt) {
    case MCOP_F32: return norm_dispatch<E, F32>(name, a, st);
    case MCOP_BF16: return norm_dispatch<E, BF16>(name, a, st);
    case MCOP_F16:
      if constexpr (std::is_same_v<E, F16>) return norm_dispatch<E, F16>(name, a, st);
      [[fallthrough]];
    default:
      return set_error(MCOP_E_INVALID, "%s: weight dtype %d is not supported for this input",
                       name, (int)wdt);
  }
}

int norm_dispatch_bf16(const char* name, const NormArgs& a, mcop_dtype wdt, hipStream_t st);
int norm_dispatch_f16(const char* name, const NormArgs& a, mcop_dtype wdt, hipStream_t st);

}  // namespace mcop
