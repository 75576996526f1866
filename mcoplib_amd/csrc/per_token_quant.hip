// per_token_quant.hip -- standalone dynamic per-token quantizers (vLLM `_C` ops): int8
// symmetric, int8 asymmetric (zero point) and fp8-e4m3fn, one pass over HBM.
//
// Semantics (per row, v = f(x) widened exactly):
//   int8 symmetric   op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:94-132
//     A = max|v|; scale = A / 127; q = sat[-127,127](rne(v * (A > 0 ? 127 / A : 0)))
//   int8 zero point  :370-422
//     s = (max v - min v) / 255; zp = rne(-128 - min v / s);
//     q = sat[-128,127](float_to_int32_rn(v * (1/s)) + zp), NaN products coding 127
//     (a constant row, s == 0, has no finite zero point: zp = -128 and q = -128 here)
//   fp8 e4m3fn       op/vllm/quantization/fp8/common.cu:142-180
//     A = max|v| (min with *scale_ub); s = max(A / 448, 1/(448*512)); q = e4m3fn(clamp(v / s))
// The row is loaded once into VGPRs; one max reduction (two for the zero point form).  Rows too
// wide for the registers take k_per_token_quant_split (the row split over several workgroups,
// read once) or, under graph capture, on the scalar path and past 64 slices,
// k_per_token_quant_wide (two passes, the row's head held on chip).
#include <hip/hip_runtime.h>

#include <cfloat>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

enum PtqMode { PTQ_INT8 = 0, PTQ_INT8_AZP = 1, PTQ_FP8 = 2 };

// Per-row quantization parameters from the row's max (|v| max, or v max with the zero point)
// and, for the zero point, the max of -v.
struct PtqRow {
  float s;      // the stored scale
  float inv;    // the multiplier of the codes
  int zp;       // zero point (PTQ_INT8_AZP)
  bool narrow;  // |zp| <= 2^29 and inv finite: the zero point sum fits int32 (PTQ_INT8_AZP)
  bool s_ok;    // s inside the fast-quotient domain (PTQ_FP8)
  bool bounded; // no scale bound cut the row's absmax (PTQ_FP8)
  bool in_range;  // inv is finite, so every |v * inv| <= 127 * (1 + 2^-23) (PTQ_INT8)
};

template <int MODE>
__device__ __forceinline__ PtqRow ptq_row(float mx, float nmn, const float* scale_ub) {
  PtqRow r{};
  if constexpr (MODE == PTQ_INT8_AZP) {
    const float mn = -nmn;
    r.s = mcop_div_rn(mx - mn, 255.0f);
    const bool degenerate = !(r.s > 0.0f);
    // zp = rne(-128 - mn / s) converted with saturation (it lies in [-128, 127] for s > 0)
    r.zp = degenerate ? -128 : cvt_rne_i32(-128.0f - mcop_div_rn(mn, r.s));
    r.inv = degenerate ? 0.0f : mcop_div_rn(1.0f, r.s);
    // a subnormal s (a row of tiny values) makes inv infinite, and the products infinite: the
    // 64-bit sum then keeps -inf at -128 where an int32 sum would wrap
    r.narrow = r.zp >= -(1 << 29) && r.zp <= (1 << 29) && r.inv <= FLT_MAX;
  } else if constexpr (MODE == PTQ_INT8) {
    r.s = mcop_div_rn(mx, 127.0f);
    r.inv = mx > 0.0f ? mcop_div_rn(127.0f, mx) : 0.0f;
    // an absmax below 127 / FLT_MAX (tiny bf16 rows) makes inv infinite: the products of the
    // row's nonzero values are then infinite and saturate, and 0 * inf = NaN codes 0
    r.in_range = r.inv <= FLT_MAX;
  } else {
    float A = mx;
    if (scale_ub != nullptr) A = __builtin_fminf(A, *scale_ub);
    r.s = __builtin_fmaxf(mcop_div_rn(A, 448.0f), 1.0f / 229376.0f);
    r.inv = mcop_div_rn(1.0f, r.s);
    r.s_ok = mcop_divisor_ok(r.s);
    r.bounded = A == mx && r.s <= 0x1p100f;
  }
  return r;
}

// Codes of one vector of v.
template <class E, int VEC, int MODE>
__device__ __forceinline__ Pack<uint8_t, VEC> ptq_codes(const float* a, const PtqRow& r) {
  Pack<uint8_t, VEC> q;
  if constexpr (MODE == PTQ_INT8_AZP) {
    // float_to_int32_rn of the reference clamps with fmin/fmax before the saturating
    // conversion, so a NaN product becomes 2^31 -> INT32_MAX and codes 127.  Every finite v lies
    // in [mn, mx], so |v * inv| <= |mn / s| + 255 (to a relative 2^-21), and |zp| >= |mn / s| -
    // 129.  With |zp| <= 2^29 and a finite inv (uniform over the row) the products stay below
    // 2^30 in magnitude:
    // clamping NaN to 2^30 instead still codes 127, and the int32 sum with zp cannot overflow.
    // Otherwise the sum is formed in 64 bits.  The sum saturates to int8.
    if (r.narrow) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int t = cvt_rne_i32(__builtin_fminf(a[e] * r.inv, 0x1p30f)) + r.zp;
        q.v[e] = (uint8_t)(int8_t)(t < -128 ? -128 : (t > 127 ? 127 : t));
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int64_t t = (int64_t)cvt_rne_i32(__builtin_fminf(a[e] * r.inv, 0x1p31f)) + r.zp;
        q.v[e] = (uint8_t)(int8_t)(t < -128 ? -128 : (t > 127 ? 127 : t));
      }
    }
  } else if constexpr (MODE == PTQ_INT8) {
    if (std::is_same_v<E, F32> || !r.in_range) {
      // fp32 inputs can carry NaN payloads in the low byte, and an infinite inv gives infinite
      // products: round, convert and saturate
#pragma unroll
      for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-127>(a[e] * r.inv);
    } else {
      // |v * inv| <= 127 * (1 + 2^-23) < 127.5, so the code never saturates
#pragma unroll
      for (int e = 0; e < VEC; ++e) q.v[e] = q_i8_in_range(a[e], r.inv);
    }
  } else {
    q = fp8_quotient_codes<VEC>(a, r.s, r.inv, r.s_ok, r.bounded);
  }
  return q;
}

template <int MODE>
__device__ __forceinline__ void ptq_fold(float t, float& mx, float& nmn) {
  if constexpr (MODE == PTQ_INT8_AZP) {
    mx = __builtin_fmaxf(mx, t);
    nmn = __builtin_fmaxf(nmn, -t);
  } else {
    mx = __builtin_fmaxf(mx, __builtin_fabsf(t));
  }
}

// EX (exact): one row per workgroup and every lane in the row (tpr == blockDim.x, NV * tpr ==
// hidden / VEC): uniform row index, scalar base addresses with 32-bit offsets, no bounds tests.
template <class E, int VEC, int NV, int MODE, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_per_token_quant(uint8_t* __restrict__ out, float* __restrict__ scales, int32_t* __restrict__ azp,
                  const typename E::S* __restrict__ x, const float* __restrict__ scale_ub,
                  int64_t rows, int hidden, int64_t in_stride, int64_t out_stride, int tpr) {
  using S = typename E::S;
  __shared__ float red_a[16];
  __shared__ float red_b[16];
  RowPos p;
  if constexpr (EX) {
    p = row_pos_one();
  } else {
    p = row_pos(rows, tpr);
  }
  const int nvec = hidden / VEC;
  const int64_t lbase = p.lrow * in_stride;
  const int64_t obase = p.row * out_stride;

  Pack<S, VEC> xv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    xv[v] = ld_nt<S, VEC>(row_elem<EX>(x, lbase, (int64_t)(EX ? j : load_index(j, nvec)) * VEC));
  }
  // Lanes past the row end hold a copy of vector 0 (read only: no effect on max or min).
  float a[NV][VEC];
  float mx = MODE == PTQ_INT8_AZP ? -__builtin_inff() : 0.0f;
  float nmn = -__builtin_inff();  // max of -v, i.e. -(min v)
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      a[v][e] = E::to_f(xv[v].v[e]);
      ptq_fold<MODE>(a[v][e], mx, nmn);
    }
  }
  mx = row_reduce<EX>(mx, red_a, tpr, MaxOp());
  if constexpr (MODE == PTQ_INT8_AZP) nmn = row_reduce<EX>(nmn, red_b, tpr, MaxOp());
  const PtqRow r = ptq_row<MODE>(mx, nmn, scale_ub);
  if (p.live && p.lt == 0) {
    scales[p.row] = r.s;
    if constexpr (MODE == PTQ_INT8_AZP) azp[p.row] = r.zp;
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    if (p.live && (EX || j < nvec)) {
      st_nt<uint8_t, VEC>(row_elem<EX>(out, obase, (int64_t)j * VEC), ptq_codes<E, VEC, MODE>(a[v], r));
    }
  }
}

// Rows too wide for one workgroup's registers, read once (split_row.h): workgroup b takes slice
// b % slices of row b / slices -- `slice_vecs` vectors, NV a lane, held in the input dtype --
// and combines the row's max (and, with the zero point, the max of -v) with the other slices'
// through the workspace `ws` in one exchange; every other step is the register kernel's.  The
// row index is uniform: scalar row bases, 32-bit offsets within the row.
template <class E, int VEC, int NV, int MODE>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_per_token_quant_split(uint8_t* __restrict__ out, float* __restrict__ scales,
                        int32_t* __restrict__ azp, const typename E::S* __restrict__ x,
                        const float* __restrict__ scale_ub, int64_t rows, int hidden,
                        int64_t in_stride, int64_t out_stride, int slices, int slice_vecs,
                        uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  using S = typename E::S;
  __shared__ float red_a[16];
  __shared__ float red_b[16];
  __shared__ float x_max[2];
  __shared__ int x_fail;
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int lt = (int)threadIdx.x;
  const int sl = (int)(blockIdx.x % (unsigned)slices);
  const int64_t row = blockIdx.x / (unsigned)slices;
  const int j0 = sl * slice_vecs;
  const int jn = min(slice_vecs, nvec - j0);
  // Lanes past the slice end re-read the slice's first vector (no effect on max or min).
  auto in_of = [&](int v) { return vec_index(v, tpr, lt) < jn; };
  auto lj_of = [&](int v) {
    return (int64_t)(j0 + (in_of(v) ? vec_index(v, tpr, lt) : 0)) * VEC;
  };
  Pack<S, VEC> xv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    xv[v] = ld_nt<S, VEC>(row_elem<true>(x, row * in_stride, lj_of(v)));
  }
  float mx = MODE == PTQ_INT8_AZP ? -__builtin_inff() : 0.0f;
  float nmn = -__builtin_inff();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) ptq_fold<MODE>(E::to_f(xv[v].v[e]), mx, nmn);
  }
  uint64_t* err = ws + split_ws_words(rows, slices) - 1;
  if constexpr (MODE == PTQ_INT8_AZP) {
    mx = row_reduce<true>(mx, red_a, tpr, MaxOp());
    nmn = row_reduce<true>(nmn, red_b, tpr, MaxOp());
    split_max2(split_slots(ws, row, slices, 0), slices, sl, kSplitTag, &mx, &nmn, err,
               timeout_ticks, x_max, &x_fail);
  } else {
    SplitRowReduce red{nullptr, red_a, tpr, ws, row, slices, sl, err, timeout_ticks, nullptr,
                       x_max, &x_fail};
    mx = red.max(mx);
  }
  const PtqRow r = ptq_row<MODE>(mx, nmn, scale_ub);
  // slice 0 stores the scale; a slice whose exchange failed stores NaN (split_row.h)
  if (lt == 0 && (sl == 0 || x_fail != 0)) {
    scales[row] = x_fail != 0 ? __builtin_nanf("") : r.s;
    if constexpr (MODE == PTQ_INT8_AZP) azp[row] = r.zp;
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (!in_of(v)) continue;
    float a[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) a[e] = E::to_f(xv[v].v[e]);
    st_nt<uint8_t, VEC>(row_elem<true>(out, row * out_stride, lj_of(v)),
                        ptq_codes<E, VEC, MODE>(a, r));
  }
}

// Rows too wide for the registers: one 1024-lane workgroup per row, two passes (max / min;
// codes).  The row's head stays on chip between the passes -- the first NC vectors of every
// lane in registers, the next NL in lane-private LDS slots (vector c of lane t at [c][t], so no
// barrier is needed; the workgroup already fills a CU's registers, so the 128 KB cost no
// occupancy) -- and the second pass re-reads only the rest.
template <class E, int VEC, int MODE>
__global__ void __launch_bounds__(kWideLanes)
k_per_token_quant_wide(uint8_t* __restrict__ out, float* __restrict__ scales,
                       int32_t* __restrict__ azp, const typename E::S* __restrict__ x,
                       const float* __restrict__ scale_ub, int hidden, int64_t in_stride,
                       int64_t out_stride) {
  using S = typename E::S;
  constexpr int NC = VEC > 1 ? 8 : 16, NL = VEC > 1 ? 8 : 0;
  __shared__ float red_a[16];
  __shared__ float red_b[16];
  __shared__ Pack<S, VEC> lds[NL > 0 ? NL : 1][kWideLanes];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x, tid = (int)threadIdx.x;
  const S* xr = x + (int64_t)blockIdx.x * in_stride;
  uint8_t* orow = out + (int64_t)blockIdx.x * out_stride;
  // A head slot past the row end holds a copy of the row's vector 0 (which leaves the max and
  // min unchanged; nothing is stored from it), so every load is unconditional: loads under a
  // per-lane branch each wait for completion where the branch rejoins, which serializes their
  // latencies.
  auto hoff = [&](int c, int lt) { return (int64_t)load_index(c * tpr + lt, nvec) * VEC; };
  Pack<S, VEC> xc[NC];
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const Pack<S, VEC> xv = ld<S, VEC>(xr + hoff(c, tid));
    if (c < NC) xc[c] = xv; else lds[c - NC][tid] = xv;
  }
  auto head = [&](int c) -> Pack<S, VEC> { return c < NC ? xc[c] : lds[c - NC][tid]; };
  float mx = MODE == PTQ_INT8_AZP ? -__builtin_inff() : 0.0f;
  float nmn = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const Pack<S, VEC> xv = head(c);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ptq_fold<MODE>(E::to_f(xv.v[e]), mx, nmn);
  }
  const int tail0 = (NC + NL) * tpr + tid;
  for (int j = tail0; j < nvec; j += tpr) {
    const Pack<S, VEC> xv = ld<S, VEC>(xr + (int64_t)j * VEC);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ptq_fold<MODE>(E::to_f(xv.v[e]), mx, nmn);
  }
  mx = row_reduce(mx, red_a, tpr, MaxOp());
  if constexpr (MODE == PTQ_INT8_AZP) nmn = row_reduce(nmn, red_b, tpr, MaxOp());
  const PtqRow r = ptq_row<MODE>(mx, nmn, scale_ub);
  if (threadIdx.x == 0) {
    scales[blockIdx.x] = r.s;
    if constexpr (MODE == PTQ_INT8_AZP) azp[blockIdx.x] = r.zp;
  }
  auto emit = [&](const Pack<S, VEC>& xv, int64_t o, bool in) {
    float a[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) a[e] = E::to_f(xv.v[e]);
    const Pack<uint8_t, VEC> q = ptq_codes<E, VEC, MODE>(a, r);
    if (in) st<uint8_t, VEC>(orow + o, q);
  };
  // The lane index, opaque to the compiler: the codes pass recomputes its vectors' offsets
  // instead of holding them from the loads.
  int lt = tid;
  __asm__ volatile("" : "+v"(lt));
  if ((NC + NL) * tpr <= nvec) {  // the head is whole: no store needs a lane test
#pragma unroll
    for (int c = 0; c < NC + NL; ++c) emit(head(c), (int64_t)(c * tpr + lt) * VEC, true);
  } else {
#pragma unroll
    for (int c = 0; c < NC + NL; ++c) emit(head(c), hoff(c, lt), c * tpr + lt < nvec);
  }
  for (int j = tail0; j < nvec; j += tpr) {
    emit(ld<S, VEC>(xr + (int64_t)j * VEC), (int64_t)j * VEC, true);
  }
}

template <class E, int VEC, int MODE>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_per_token_quant<E, 1, 4, MODE>)
                   : reinterpret_cast<const void*>(&k_per_token_quant<E, 1, 16, MODE>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_per_token_quant<E, VEC, 1, MODE>);
      case 2: return reinterpret_cast<const void*>(&k_per_token_quant<E, VEC, 2, MODE>);
      case 4: return reinterpret_cast<const void*>(&k_per_token_quant<E, VEC, 4, MODE>);
      case 8: return reinterpret_cast<const void*>(&k_per_token_quant<E, VEC, 8, MODE>);
      default: return reinterpret_cast<const void*>(&k_per_token_quant<E, VEC, 16, MODE>);
    }
  }
}

struct PtqArgs {
  void* out;
  float* scales;
  int32_t* azp;
  const void* x;
  const float* scale_ub;
  int64_t rows;
  int hidden;
  int64_t in_stride;
  int64_t out_stride;
};

template <class E, int VEC, int MODE>
static void launch_nv(const Geometry& g, const PtqArgs& a, hipStream_t st) {
  using S = typename E::S;
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* o = static_cast<uint8_t*>(a.out);
  auto* xp = static_cast<const S*>(a.x);
#define MCOP_LAUNCH(NVV, EXX)                                                                   \
  hipLaunchKernelGGL((k_per_token_quant<E, VEC, NVV, MODE, EXX>), grid, block, 0, st, o, a.scales, \
                     a.azp, xp, a.scale_ub, a.rows, a.hidden, a.in_stride, a.out_stride, g.tpr)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it): the EX form at two vectors a lane,
    // and at four or eight on the latency path (at most 256 rows), when it keeps its registers
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == a.hidden / VEC &&
                    (g.nv == 2 || a.rows <= 256);
#define MCOP_EX(NVV)                                                                           \
  (ex && exact_form_ok(reinterpret_cast<const void*>(&k_per_token_quant<E, VEC, NVV, MODE, true>)))
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

// Rows too wide for the register kernels, vector path: the split-row kernel when it applies, its
// workspace from the stream-ordered allocator; MCOP_E_UNSUPPORTED (no message) when it does not.
template <class E, int VEC, int MODE>
static int launch_split(const char* name, const PtqArgs& a, hipStream_t st) {
  using S = typename E::S;
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  // (a sixteen-vector candidate, chosen by residency at three waves per SIMD, ran slower: 134.3
  // against 129.2 us for int8 and 154.8 against 133.8 us for fp8 at 2048 x 131072 bf16)
  const SplitKernel k8{fn(&k_per_token_quant_split<E, VEC, 8, MODE>), 8};
  const SplitKernel k4{fn(&k_per_token_quant_split<E, VEC, 4, MODE>), 4};
  return split_run(name, {k8, k4}, a.rows, a.hidden / VEC, nullptr, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    uint8_t* o = static_cast<uint8_t*>(a.out) + r0 * a.out_stride;
    float* sc = a.scales + r0;
    int32_t* zp = a.azp == nullptr ? nullptr : a.azp + r0;
    const S* xp = static_cast<const S*>(a.x) + r0 * a.in_stride;
    const float* ub = a.scale_ub;
    int h = a.hidden, slices = p.slices, slice_vecs = p.slice_vecs;
    int64_t is = a.in_stride, os = a.out_stride, timeout = p.timeout_ticks;
    void* args[] = {&o, &sc, &zp, &xp, &ub, &n, &h, &is, &os, &slices, &slice_vecs, &ws,
                    &timeout};
    return launch(args);
  });
}

template <class E, int MODE>
static int dispatch(const char* name, const PtqArgs& a, hipStream_t st) {
  constexpr int V = E::VEC;
  const bool vec_ok = a.hidden % V == 0 && a.in_stride % V == 0 && a.out_stride % V == 0 &&
                      aligned(16, a.x) && aligned(V, a.out);
  const KernelOfNv kernels = vec_ok ? &kernel_of<E, V, MODE> : &kernel_of<E, 1, MODE>;
  if (!row_fits(a.hidden, vec_ok ? V : 1, kernels)) {
    if (vec_ok && split_rows_enabled()) {
      const int rc = launch_split<E, V, MODE>(name, a, st);
      if (rc != MCOP_E_UNSUPPORTED) return rc;
    }
    if (!wide_rows_ok(name, a.rows)) return MCOP_E_UNSUPPORTED;
    using S = typename E::S;
    auto* o = static_cast<uint8_t*>(a.out);
    auto* xp = static_cast<const S*>(a.x);
    const dim3 grid((unsigned)a.rows), block(kWideLanes);
    if (vec_ok) {
      hipLaunchKernelGGL((k_per_token_quant_wide<E, V, MODE>), grid, block, 0, st, o, a.scales,
                         a.azp, xp, a.scale_ub, a.hidden, a.in_stride, a.out_stride);
    } else {
      hipLaunchKernelGGL((k_per_token_quant_wide<E, 1, MODE>), grid, block, 0, st, o, a.scales,
                         a.azp, xp, a.scale_ub, a.hidden, a.in_stride, a.out_stride);
    }
    return check_launch(name);
  }
  Geometry g;
  if (!choose_geometry(name, a.rows, a.hidden, vec_ok ? V : 1, kernels, &g)) {
    return MCOP_E_UNSUPPORTED;
  }
  if (g.vec == 1) launch_nv<E, 1, MODE>(g, a, st);
  else launch_nv<E, V, MODE>(g, a, st);
  return check_launch(name);
}

template <int MODE>
static int dispatch_dtype(const char* name, const PtqArgs& a, mcop_dtype dt, hipStream_t st) {
  switch (dt) {
    case MCOP_BF16: return dispatch<BF16, MODE>(name, a, st);
    case MCOP_F16: return dispatch<F16, MODE>(name, a, st);
    case MCOP_F32: return dispatch<F32, MODE>(name, a, st);
    default:
      return set_error(MCOP_E_INVALID, "%s: input dtype %d is not bf16/fp16/fp32", name, (int)dt);
  }
}

static int check_shape(const char* name, int64_t rows, int64_t hidden, int64_t in_stride,
                       int64_t out_stride) {
  if (rows < 0 || hidden <= 0 || hidden > INT32_MAX || in_stride < hidden ||
      out_stride < hidden) {
    return set_error(MCOP_E_INVALID,
                     "%s: bad shape num_tokens=%lld hidden_size=%lld strides=%lld/%lld", name,
                     (long long)rows, (long long)hidden, (long long)in_stride,
                     (long long)out_stride);
  }
  return MCOP_OK;
}

}  // namespace mcop

extern "C" int mcop_dynamic_scaled_int8_quant(int8_t* out, float* scales, int32_t* azp,
                                              const void* input, int64_t num_tokens,
                                              int64_t hidden_size, mcop_dtype in_dtype,
                                              void* stream) {
  using namespace mcop;
  const char* name = "dynamic_scaled_int8_quant";
  if (int rc = check_shape(name, num_tokens, hidden_size, hidden_size, hidden_size)) return rc;
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !scales || !input) return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  const PtqArgs a{out, scales, azp, input, nullptr, num_tokens, (int)hidden_size, hidden_size,
                  hidden_size};
  auto st = static_cast<hipStream_t>(stream);
  return azp ? dispatch_dtype<PTQ_INT8_AZP>(name, a, in_dtype, st)
             : dispatch_dtype<PTQ_INT8>(name, a, in_dtype, st);
}

extern "C" int mcop_dynamic_per_token_scaled_fp8_quant(uint8_t* out, float* scales,
                                                       const void* input, const float* scale_ub,
                                                       int64_t num_tokens, int64_t hidden_size,
                                                       int64_t input_row_stride,
                                                       int64_t output_row_stride,
                                                       mcop_dtype in_dtype, void* stream) {
  using namespace mcop;
  const char* name = "dynamic_per_token_scaled_fp8_quant";
  if (int rc = check_shape(name, num_tokens, hidden_size, input_row_stride, output_row_stride)) {
    return rc;
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !scales || !input) return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  const PtqArgs a{out, scales, nullptr, input, scale_ub, num_tokens, (int)hidden_size,
                  input_row_stride, output_row_stride};
  return dispatch_dtype<PTQ_FP8>(name, a, in_dtype, static_cast<hipStream_t>(stream));
}
