// fused_add_rms_norm.hip -- in-place residual add + RMSNorm (vLLM `_C::fused_add_rms_norm`).
//
// Semantics (per row, b() = round to the dtype), following op/vllm/layernorm_kernels.cu:92-144
// and op/vllm/type_convert.cuh:104-165 of the reference:
//   z = b(x + r);  residual <- z                     (packed add, :118-125)
//   rho = 1/sqrt(sum(z^2)/H + eps)  on the rounded z  (:122, :127-133; fp64 sum here)
//   x <- b(b(z * rho) * w)                            (:136-143: scale then weight multiply)
// One pass over HBM: x, residual and weight are loaded once into VGPRs, residual is written
// from registers before the reduction, x after it (8*H bytes per bf16 row, plus the weight).
// Rows too wide for the registers take k_fused_add_rms_norm_split (the row split over several
// workgroups, read once) or, under graph capture, on the scalar path and past 64 slices,
// k_fused_add_rms_norm_wide: one 1024-lane workgroup per row, the row's first 8 vectors a lane
// held in registers and (bf16, fp32) the next 8 in LDS (one read of rows up to 131072 bf16
// elements); beyond them two passes (sum of squares; then residual and output), the second
// re-reading x and residual, which each lane then overwrites at the same addresses.
#include <hip/hip_runtime.h>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

// With eight vectors a lane the kernel asks for four waves per SIMD (at most 128 VGPRs, met
// without spilling; 138 and three waves left free): rows of 20480-24576 bf16 elements ran 5-9%
// faster.  fp16 would spill under that bound and keeps the default.
// EX (exact): one row per workgroup and every lane in the row (tpr == blockDim.x, NV * tpr ==
// hidden / VEC): uniform row index, scalar base addresses with 32-bit offsets, no bounds tests.
template <class E, int VEC, int NV, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
__attribute__((amdgpu_waves_per_eu(NV == 8 && !std::is_same<E, F16>::value ? 4 : 1)))
k_fused_add_rms_norm(typename E::S* __restrict__ x, int64_t x_stride,
                     typename E::S* __restrict__ res, const typename E::S* __restrict__ w,
                     int64_t rows, int hidden, int tpr, float eps) {
  using S = typename E::S;
  __shared__ double red_sum[16];
  RowPos p;
  if constexpr (EX) {
    p = row_pos_one();
  } else {
    p = row_pos(rows, tpr);
  }
  const int nvec = hidden / VEC;
  const int64_t xbase = p.row * x_stride, xlbase = p.lrow * x_stride;
  const int64_t rbase = p.row * (int64_t)hidden, rlbase = p.lrow * (int64_t)hidden;
  auto lj_of = [&](int v) {
    const int j = vec_index(v, tpr, p.lt);
    return (int64_t)(EX ? j : load_index(j, nvec)) * VEC;
  };

  Pack<S, VEC> xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = ld<S, VEC>(row_elem<EX>(w, 0, lj_of(v)));
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t lj = lj_of(v);
    xv[v] = ld_nt<S, VEC>(row_elem<EX>(x, xlbase, lj));
    rv[v] = ld_nt<S, VEC>(row_elem<EX>(res, rlbase, lj));
  }

  float z[NV][VEC];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    const bool in = EX || j < nvec;
    Pack<S, VEC> o;
    double vs = 0.0;  // lanes past the row end (a copy of vector 0) do not count
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      o.v[e] = E::from_f(E::to_f(xv[v].v[e]) + E::to_f(rv[v].v[e]));
      const float t = E::to_f(o.v[e]);
      z[v][e] = t;
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
    }
    ss += in ? vs : 0.0;
    if (p.live && in) st_nt<S, VEC>(row_elem<EX>(res, rbase, (int64_t)j * VEC), o);
  }

  ss = row_reduce<EX>(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    if (p.live && (EX || j < nvec)) {
      Pack<S, VEC> o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        o.v[e] = E::from_f(rnd<E>(z[v][e] * rho) * E::to_f(wv[v].v[e]));
      }
      st_nt<S, VEC>(row_elem<EX>(x, xbase, (int64_t)j * VEC), o);
    }
  }
}

// Rows too wide for one workgroup's registers, read once (split_row.h): workgroup b takes slice
// b % slices of row b / slices -- `slice_vecs` vectors, NV a lane -- holds its rounded sums z
// in the dtype (packed) and its weight vectors, writes the residual, and combines the row's
// sum of squares with the other slices' through the workspace `ws` (split_sum, in slice order)
// before writing x.  The row index is uniform: scalar row bases, 32-bit offsets.
template <class E, int VEC, int NV>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_fused_add_rms_norm_split(typename E::S* __restrict__ x, int64_t x_stride,
                           typename E::S* __restrict__ res, const typename E::S* __restrict__ w,
                           int64_t rows, int hidden, int slices, int slice_vecs, float eps,
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
  const int64_t xbase = row * x_stride, rbase = row * (int64_t)hidden;
  // Lanes past the slice end re-read the slice's first vector, which does not count.
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
    xv[v] = ld_nt<S, VEC>(row_elem<true>(x, xbase, lj_of(v)));
    rv[v] = ld_nt<S, VEC>(row_elem<true>(res, rbase, lj_of(v)));
  }
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    double vs = 0.0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      xv[v].v[e] = E::from_f(E::to_f(xv[v].v[e]) + E::to_f(rv[v].v[e]));  // z
      const double d = (double)E::to_f(xv[v].v[e]);
      vs = __builtin_fma(d, d, vs);
    }
    ss += in_of(v) ? vs : 0.0;
    if (in_of(v)) st_nt<S, VEC>(row_elem<true>(res, rbase, lj_of(v)), xv[v]);
  }
  SplitRowReduce red{red_sum, nullptr, tpr, ws, row, slices, sl,
                     ws + split_ws_words(rows, slices) - 1, timeout_ticks, &x_sum, nullptr};
  ss = red.sum(ss);
  const float rho = mcop_inv_rms(ss, hidden, eps);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (in_of(v)) {
      Pack<S, VEC> o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        o.v[e] = E::from_f(rnd<E>(E::to_f(xv[v].v[e]) * rho) * E::to_f(wv[v].v[e]));
      }
      st_nt<S, VEC>(row_elem<true>(x, xbase, lj_of(v)), o);
    }
  }
}

template <class E, int VEC>
__global__ void __launch_bounds__(kWideLanes)
k_fused_add_rms_norm_wide(typename E::S* __restrict__ x, int64_t x_stride,
                          typename E::S* __restrict__ res, const typename E::S* __restrict__ w,
                          int hidden, float eps) {
  using S = typename E::S;
  // The row head (the lane's first NC vectors) stays in registers as the rounded sum z, and
  // the next NL in LDS, so rows up to (NC + NL) * 1024 vectors are read once.  Head loads are
  // unconditional (a lane past the row end re-reads the row's last vector and does not count
  // it) and issued G vectors at a time; the residual of the head is written in the first pass,
  // that of the re-read tail in the second, after its last read.  NC (with NL below) is the
  // largest head that compiles without spills at 1024 lanes (128 VGPRs a lane).
  constexpr int NC = 8, G = 4;
  __shared__ double red_sum[16];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x, tid = (int)threadIdx.x;
  S* xr = x + (int64_t)blockIdx.x * x_stride;
  S* rr = res + (int64_t)blockIdx.x * hidden;
  // element offsets within the row fit 32 bits (hidden <= INT32_MAX)
  auto z_of = [&](int o) {
    const Pack<S, VEC> xv = ld<S, VEC>(xr + o);
    const Pack<S, VEC> rv = ld<S, VEC>(rr + o);
    Pack<S, VEC> z;
#pragma unroll
    for (int e = 0; e < VEC; ++e) z.v[e] = E::from_f(E::to_f(xv.v[e]) + E::to_f(rv.v[e]));
    return z;
  };
  auto sum_sq = [&](const Pack<S, VEC>& z) {
    double vs = 0.0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const double d = (double)E::to_f(z.v[e]);
      vs = __builtin_fma(d, d, vs);
    }
    return vs;
  };
  // offset of head vector c of lane t, clamped into the row (lanes past its end re-read the
  // last vector and neither count nor store it)
  auto head_off = [&](int c, int t) { return min(c * tpr + t, nvec - 1) * VEC; };

  Pack<S, VEC> zc[NC];
  double ss = 0.0;
#pragma unroll
  for (int g = 0; g < NC; g += G) {
    Pack<S, VEC> xv[G], rv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
      xv[k] = ld<S, VEC>(xr + head_off(g + k, tid));
      rv[k] = ld<S, VEC>(rr + head_off(g + k, tid));
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        zc[g + k].v[e] = E::from_f(E::to_f(xv[k].v[e]) + E::to_f(rv[k].v[e]));
      }
      const double vs = sum_sq(zc[g + k]);
      ss += (g + k) * tpr + tid < nvec ? vs : 0.0;
      if constexpr (sizeof(Pack<S, VEC>) == 16) {  // keep z packed (4 VGPRs), not as floats
        u32x4 u = __builtin_bit_cast(u32x4, zc[g + k]);
        asm volatile("" : "+v"(u));
        zc[g + k] = __builtin_bit_cast(Pack<S, VEC>, u);
      }
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
      if ((g + k) * tpr + tid < nvec) st<S, VEC>(rr + head_off(g + k, tid), zc[g + k]);
    }
    __builtin_amdgcn_sched_barrier(0);  // at most G vectors' loads in flight
  }
  // The next NL vectors of every lane are held in LDS: lane-private slots (vector c of lane t
  // at [c][t]), so no barrier is needed; the workgroup already fills a CU's registers, so the
  // 128 KB cost no occupancy.  With them a 131072-wide bf16 row is read once.  (Not for fp16,
  // whose conversions leave no registers for the LDS traffic.)
  constexpr int NL = VEC > 1 && !std::is_same<E, F16>::value ? 8 : 0;
  __shared__ Pack<S, VEC> lds[NL > 0 ? NL : 1][kWideLanes];
  int tid1 = tid;  // opaque copies of the lane index: each loop computes its own addresses
  asm volatile("" : "+v"(tid1));
#pragma unroll
  for (int g = NC; g < NC + NL; g += G) {
    Pack<S, VEC> xv[G], rv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
      xv[k] = ld<S, VEC>(xr + head_off(g + k, tid1));
      rv[k] = ld<S, VEC>(rr + head_off(g + k, tid1));
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
      Pack<S, VEC> z;
#pragma unroll
      for (int e = 0; e < VEC; ++e) z.v[e] = E::from_f(E::to_f(xv[k].v[e]) + E::to_f(rv[k].v[e]));
      const double vs = sum_sq(z);
      ss += (g + k) * tpr + tid1 < nvec ? vs : 0.0;
      lds[g + k - NC][tid] = z;
      if ((g + k) * tpr + tid1 < nvec) st<S, VEC>(rr + head_off(g + k, tid1), z);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const int tail0 = (NC + NL) * tpr + tid;
  for (int j = tail0; j < nvec; j += tpr) ss += sum_sq(z_of(j * VEC));
  ss = row_reduce(ss, red_sum, tpr, SumOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  // the lane index again, opaque to the compiler: the second pass recomputes its addresses
  // instead of holding the first pass's in registers across the reduction
  int tid2 = tid;
  asm volatile("" : "+v"(tid2));
  auto y_of = [&](const Pack<S, VEC>& z, const Pack<S, VEC>& wv) {
    Pack<S, VEC> y;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      y.v[e] = E::from_f(rnd<E>(E::to_f(z.v[e]) * rho) * E::to_f(wv.v[e]));
    }
    return y;
  };
#pragma unroll
  for (int g = 0; g < NC; g += G) {
    Pack<S, VEC> wv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) wv[k] = ld<S, VEC>(w + head_off(g + k, tid2));
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const Pack<S, VEC> y = y_of(zc[g + k], wv[k]);
      if ((g + k) * tpr + tid2 < nvec) st<S, VEC>(xr + head_off(g + k, tid2), y);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  int tid3 = tid;
  asm volatile("" : "+v"(tid3));
#pragma unroll
  for (int g = NC; g < NC + NL; g += G) {
    Pack<S, VEC> wv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) wv[k] = ld<S, VEC>(w + head_off(g + k, tid3));
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const Pack<S, VEC> y = y_of(lds[g + k - NC][tid], wv[k]);
      if ((g + k) * tpr + tid3 < nvec) st<S, VEC>(xr + head_off(g + k, tid3), y);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int j = tail0; j < nvec; j += tpr) {
    const int o = j * VEC;
    const Pack<S, VEC> z = z_of(o);
    st<S, VEC>(rr + o, z);
    st<S, VEC>(xr + o, y_of(z, ld<S, VEC>(w + o)));
  }
}

template <class E, int VEC>
static void launch_nv(const Geometry& g, void* x, int64_t xs, void* res, const void* w,
                      int64_t rows, int hidden, float eps, hipStream_t st) {
  using S = typename E::S;
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* xp = static_cast<S*>(x);
  auto* rp = static_cast<S*>(res);
  auto* wp = static_cast<const S*>(w);
#define MCOP_LAUNCH(NVV, EXX)                                                                   \
  hipLaunchKernelGGL((k_fused_add_rms_norm<E, VEC, NVV, EXX>), grid, block, 0, st, xp, xs, rp, wp, \
                     rows, hidden, g.tpr, eps)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it): the EX form at two vectors a lane,
    // and at four or eight on the latency path (at most 256 rows)
    // (and only when that form keeps its registers)
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == hidden / VEC &&
                    (g.nv == 2 || rows <= 256);
#define MCOP_EX(NVV) \
  (ex && exact_form_ok(reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, VEC, NVV, true>)))
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

template <class E, int VEC>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, 1, 4>)
                   : reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, 1, 16>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, VEC, 1>);
      case 2: return reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, VEC, 2>);
      case 4: return reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, VEC, 4>);
      case 8: return reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, VEC, 8>);
      default: return reinterpret_cast<const void*>(&k_fused_add_rms_norm<E, VEC, 16>);
    }
  }
}

// Rows too wide for the register kernels, vector path: the split-row kernel when it applies, its
// workspace from the stream-ordered allocator; MCOP_E_UNSUPPORTED (no message) when it does not.
template <class E, int VEC>
static int launch_split(void* x, int64_t xs, void* res, const void* w, int64_t rows,
                        int hidden, float eps, hipStream_t st) {
  using S = typename E::S;
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  const SplitKernel k8{fn(&k_fused_add_rms_norm_split<E, VEC, 8>), 8};
  const SplitKernel k4{fn(&k_fused_add_rms_norm_split<E, VEC, 4>), 4};
  return split_run("fused_add_rms_norm", {k8, k4}, rows, hidden / VEC, nullptr, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    S* xp = static_cast<S*>(x) + r0 * xs;
    S* rp = static_cast<S*>(res) + r0 * (int64_t)hidden;
    const S* wp = static_cast<const S*>(w);
    int64_t stride = xs;
    int h = hidden, slices = p.slices, slice_vecs = p.slice_vecs;
    float e = eps;
    int64_t timeout = p.timeout_ticks;
    void* args[] = {&xp, &stride, &rp, &wp, &n, &h, &slices, &slice_vecs, &e, &ws, &timeout};
    return launch(args);
  });
}

template <class E>
static int dispatch(void* x, int64_t xs, void* res, const void* w, int64_t rows, int64_t hidden,
                    float eps, hipStream_t st) {
  constexpr int V = E::VEC;
  const bool vec_ok = hidden % V == 0 && xs % V == 0 && aligned(16, x, res, w);
  const KernelOfNv kernels = vec_ok ? &kernel_of<E, V> : &kernel_of<E, 1>;
  if (!row_fits(hidden, vec_ok ? V : 1, kernels)) {
    if (vec_ok && split_rows_enabled()) {
      const int rc = launch_split<E, V>(x, xs, res, w, rows, (int)hidden, eps, st);
      if (rc != MCOP_E_UNSUPPORTED) return rc;
    }
    if (!wide_rows_ok("fused_add_rms_norm", rows)) return MCOP_E_UNSUPPORTED;
    using S = typename E::S;
    auto* xp = static_cast<S*>(x);
    auto* rp = static_cast<S*>(res);
    auto* wp = static_cast<const S*>(w);
    if (vec_ok) {
      hipLaunchKernelGGL((k_fused_add_rms_norm_wide<E, V>), dim3((unsigned)rows),
                         dim3(kWideLanes), 0, st, xp, xs, rp, wp, (int)hidden, eps);
    } else {
      hipLaunchKernelGGL((k_fused_add_rms_norm_wide<E, 1>), dim3((unsigned)rows),
                         dim3(kWideLanes), 0, st, xp, xs, rp, wp, (int)hidden, eps);
    }
    return check_launch("fused_add_rms_norm");
  }
  Geometry g;
  if (!choose_geometry("fused_add_rms_norm", rows, hidden, vec_ok ? V : 1, kernels, &g)) {
    return MCOP_E_UNSUPPORTED;
  }
  if (g.vec == 1) {
    launch_nv<E, 1>(g, x, xs, res, w, rows, (int)hidden, eps, st);
  } else {
    launch_nv<E, V>(g, x, xs, res, w, rows, (int)hidden, eps, st);
  }
  return check_launch("fused_add_rms_norm");
}

}  // namespace mcop

extern "C" int mcop_fused_add_rms_norm(void* input, int64_t input_row_stride, void* residual,
                                       const void* weight, int64_t num_tokens,
                                       int64_t hidden_size, mcop_dtype dtype, float epsilon,
                                       void* stream) {
  using namespace mcop;
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size > INT32_MAX ||
      input_row_stride < hidden_size) {
    return set_error(MCOP_E_INVALID,
                     "fused_add_rms_norm: bad shape num_tokens=%lld hidden_size=%lld "
                     "input_row_stride=%lld",
                     (long long)num_tokens, (long long)hidden_size, (long long)input_row_stride);
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!input || !residual || !weight) {
    return set_error(MCOP_E_INVALID, "fused_add_rms_norm: null pointer");
  }
  auto st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MCOP_BF16:
      return dispatch<BF16>(input, input_row_stride, residual, weight, num_tokens, hidden_size,
                            epsilon, st);
    case MCOP_F16:
      return dispatch<F16>(input, input_row_stride, residual, weight, num_tokens, hidden_size,
                           epsilon, st);
    case MCOP_F32:
      return dispatch<F32>(input, input_row_stride, residual, weight, num_tokens, hidden_size,
                           epsilon, st);
    default:
      return set_error(MCOP_E_INVALID, "fused_add_rms_norm: dtype %d is not bf16/fp16/fp32",
                       (int)dtype);
  }
}
