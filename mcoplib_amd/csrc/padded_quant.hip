// padded_quant.hip -- residual add + RMSNorm + per-token int8 quantization into a padded
// per-row wire layout (mcoplib.op.fused_add_rms_norm_dynamic_per_token_quant_padding_output),
// one pass over HBM.
//
// Layout of `padded` (row stride pad_bytes = 2 * pad_size bytes): row t holds its H int8 codes
// at bytes [0, H) and its fp32 scale at bytes [H, H + 4); the remaining bytes are not written
// (op/fused_add_layernorm_per_token_quant_padding_output.cu:216, 246, 255, 320).
//
// The reference dispatches two kernels with different rounding chains (entry :344-395):
//   H == 7168 ("opt" kernel, :181-283), a = x + r in fp32, never rounded in between:
//     r <- b(a); p = a * w; A = max|p|; rho = 1/sqrt(sum a^2 / H + eps);
//     s = max((A * rho) / 127, FLT_EPSILON); u = p * rho;
//     rms <- b(u); q = sat[-127,127](rne(u * (1/s)))
//   any other H ("generic" kernel, :287-340), with bf16 products rounded to bf16:
//     r <- b(a); A = max|b(b(a) * w)|; rho as above; s as above;
//     y = b(b(b(a) * rho) * w); q = sat[-127,127](rne(y * (1/s)))
//     The generic kernel writes only `padded` and the residual; here it also writes rms <- y,
//     the unpacked codes and scales[t], so every output is defined for every H.
// Both write q to `padded` and to the unpacked int8 output, s to `padded` and (opt) scales[t].
// b() = round to bf16 (RNE); the row sum is the fp64 sum rounded once (order-independent).
#include <hip/hip_runtime.h>

#include <cfloat>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

// EX (exact): one row per workgroup and every lane in the row (tpr == blockDim.x, NV * tpr ==
// hidden / VEC): uniform row index, scalar base addresses with 32-bit offsets, no bounds tests.
template <int VEC, int NV, bool OPT, bool EX = false>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_add_rms_norm_quant_padded(uint8_t* __restrict__ padded, uint16_t* __restrict__ rms,
                            uint8_t* __restrict__ q_out, float* __restrict__ scales,
                            const uint16_t* __restrict__ x, uint16_t* __restrict__ res,
                            const uint16_t* __restrict__ w, int64_t rows, int hidden,
                            int64_t pad_bytes, int tpr, float eps) {
  using E = BF16;
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
  const int64_t pbase = p.row * pad_bytes;
  auto lj_of = [&](int v) {
    const int j = vec_index(v, tpr, p.lt);
    return (int64_t)(EX ? j : load_index(j, nvec)) * VEC;
  };

  Pack<uint16_t, VEC> xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = ld<uint16_t, VEC>(row_elem<EX>(w, 0, lj_of(v)));
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int64_t lj = lj_of(v);
    xv[v] = ld_nt<uint16_t, VEC>(row_elem<EX>(x, lbase, lj));
    rv[v] = ld_nt<uint16_t, VEC>(row_elem<EX>(res, lbase, lj));
  }

  // a: opt keeps p = a * w (fp32); generic keeps b(a) (the residual value it re-reads)
  const bool full = EX || (int64_t)NV * tpr == nvec;
  float a[NV][VEC];
  double ss = 0.0;
  float amax = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    const bool in = EX || j < nvec;
    double vs = 0.0;
    Pack<uint16_t, VEC> o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = E::to_f(xv[v].v[e]) + E::to_f(rv[v].v[e]);
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
      o.v[e] = E::from_f(t);
      const float wf = E::to_f(wv[v].v[e]);
      float m;
      if constexpr (OPT) {
        a[v][e] = t * wf;
        m = a[v][e];
      } else {
        a[v][e] = E::to_f(o.v[e]);
        m = rnd<E>(a[v][e] * wf);
      }
      // lanes past the row end hold a copy of vector 0, possibly of the updated residual
      amax = __builtin_fmaxf(amax, (full || in) ? __builtin_fabsf(m) : 0.0f);
    }
    ss += in ? vs : 0.0;
    if (p.live && in) st_nt<uint16_t, VEC>(row_elem<EX>(res, base, (int64_t)j * VEC), o);
  }
  ss = row_reduce<EX>(ss, red_sum, tpr, SumOp());
  amax = row_reduce<EX>(amax, red_max, tpr, MaxOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float s = __builtin_fmaxf(mcop_div_rn(amax * rho, 127.0f), FLT_EPSILON);
  const float inv = mcop_div_rn(1.0f, s);
  if (p.live && p.lt == 0) {
    scales[p.row] = s;
    uint8_t* sp = padded + pbase + hidden;
    if ((reinterpret_cast<uintptr_t>(sp) & 3) == 0) {
      *reinterpret_cast<float*>(sp) = s;
    } else {
      const uint32_t b = __builtin_bit_cast(uint32_t, s);
#pragma unroll
      for (int k = 0; k < 4; ++k) sp[k] = (uint8_t)(b >> (8 * k));
    }
  }

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    if (p.live && (EX || j < nvec)) {
      Pack<uint16_t, VEC> o;
      Pack<uint8_t, VEC> q;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float y;
        if constexpr (OPT) {
          y = a[v][e] * rho;
          o.v[e] = E::from_f(y);
        } else {
          o.v[e] = E::from_f(rnd<E>(a[v][e] * rho) * E::to_f(wv[v].v[e]));
          y = E::to_f(o.v[e]);
        }
        q.v[e] = q_i8<-127>(y * inv);
      }
      st_nt<uint16_t, VEC>(row_elem<EX>(rms, base, (int64_t)j * VEC), o);
      st_nt<uint8_t, VEC>(row_elem<EX>(q_out, base, (int64_t)j * VEC), q);
      st_nt<uint8_t, VEC>(row_elem<EX>(padded, pbase, (int64_t)j * VEC), q);
    }
  }
}

// Rows too wide for one workgroup's registers (the generic chain: 7168-wide rows always fit),
// read once (split_row.h): workgroup b takes slice b % slices of row b / slices --
// `slice_vecs` vectors, NV a lane -- holds z = b(x + r) and the weight in bf16, and combines
// the row's sum of squares and absmax (which does not need rho) with the other slices' in one
// exchange (split_sum_max); every other step is the register kernel's.  Slice 0 stores the
// scale.  The row index is uniform: scalar row bases, 32-bit offsets within the row.
template <int NV>
__global__ void __launch_bounds__(max_tpr(8, NV))
k_add_rms_norm_quant_padded_split(uint8_t* __restrict__ padded, uint16_t* __restrict__ rms,
                                  uint8_t* __restrict__ q_out, float* __restrict__ scales,
                                  const uint16_t* __restrict__ x, uint16_t* __restrict__ res,
                                  const uint16_t* __restrict__ w, int64_t rows, int hidden,
                                  int64_t pad_bytes, float eps, int slices, int slice_vecs,
                                  uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  using E = BF16;
  constexpr int VEC = 8;
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
  const int j0 = sl * slice_vecs;
  const int jn = min(slice_vecs, nvec - j0);
  const int64_t base = row * (int64_t)hidden;
  const int64_t pbase = row * pad_bytes;
  // Lanes past the slice end re-read the slice's first vector, which does not count.
  auto in_of = [&](int v) { return vec_index(v, tpr, lt) < jn; };
  auto lj_of = [&](int v) {
    return (int64_t)(j0 + (in_of(v) ? vec_index(v, tpr, lt) : 0)) * VEC;
  };
  Pack<uint16_t, VEC> xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = ld<uint16_t, VEC>(row_elem<true>(w, 0, lj_of(v)));
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    xv[v] = ld_nt<uint16_t, VEC>(row_elem<true>(x, base, lj_of(v)));
    rv[v] = ld_nt<uint16_t, VEC>(row_elem<true>(res, base, lj_of(v)));
  }
  double ss = 0.0;
  float amax = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    double vs = 0.0;
    float vm = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = E::to_f(xv[v].v[e]) + E::to_f(rv[v].v[e]);
      const double d = (double)t;
      vs = __builtin_fma(d, d, vs);
      xv[v].v[e] = E::from_f(t);  // z = b(a), the residual value the generic chain re-reads
      vm = __builtin_fmaxf(vm, __builtin_fabsf(rnd<E>(E::to_f(xv[v].v[e]) *
                                                      E::to_f(wv[v].v[e]))));
    }
    ss += in_of(v) ? vs : 0.0;
    amax = __builtin_fmaxf(amax, in_of(v) ? vm : 0.0f);
    if (in_of(v)) st_nt<uint16_t, VEC>(row_elem<true>(res, base, lj_of(v)), xv[v]);
  }
  ss = row_reduce<true>(ss, red_sum, tpr, SumOp());
  amax = row_reduce<true>(amax, red_max, tpr, MaxOp());
  split_sum_max(ws, row, slices, sl, kSplitTag, &ss, &amax, ws + split_ws_words(rows, slices) - 1,
                timeout_ticks, &x_sum, &x_max, &x_fail);
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float s = __builtin_fmaxf(mcop_div_rn(amax * rho, 127.0f), FLT_EPSILON);
  const float inv = mcop_div_rn(1.0f, s);
  // slice 0 stores the scale; a slice whose exchange failed stores NaN (split_row.h)
  if (lt == 0 && (sl == 0 || x_fail != 0)) {
    const float s_out = x_fail != 0 ? __builtin_nanf("") : s;
    scales[row] = s_out;
    uint8_t* sp = padded + pbase + hidden;
    if ((reinterpret_cast<uintptr_t>(sp) & 3) == 0) {
      *reinterpret_cast<float*>(sp) = s_out;
    } else {
      const uint32_t b = __builtin_bit_cast(uint32_t, s_out);
#pragma unroll
      for (int k = 0; k < 4; ++k) sp[k] = (uint8_t)(b >> (8 * k));
    }
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (!in_of(v)) continue;
    Pack<uint16_t, VEC> o;
    Pack<uint8_t, VEC> q;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      o.v[e] = E::from_f(rnd<E>(E::to_f(xv[v].v[e]) * rho) * E::to_f(wv[v].v[e]));
      q.v[e] = q_i8<-127>(E::to_f(o.v[e]) * inv);
    }
    const int64_t lj = lj_of(v);
    st_nt<uint16_t, VEC>(row_elem<true>(rms, base, lj), o);
    st_nt<uint8_t, VEC>(row_elem<true>(q_out, base, lj), q);
    st_nt<uint8_t, VEC>(row_elem<true>(padded, pbase, lj), q);
  }
}

// Rows too wide for the registers (the generic chain: 7168-wide rows always fit): one 1024-lane
// workgroup per row, two passes (sum of squares and absmax, which does not need rho; then the
// residual, rms, codes, padded codes and scale).  The row's head stays on chip as the rounded
// sums z = b(x + r) -- the first NC vectors of every lane in registers, the next NL in
// lane-private LDS slots (vector c of lane t at [c][t], so no barrier is needed; the workgroup
// already fills a CU's registers, so the 128 KB cost no occupancy) -- and its residual is
// written in the first pass.  The second pass re-reads the rest of x and residual, and the
// weight; the residual of that rest is written in the last pass only, by the lane that read it.
template <int VEC>
__global__ void __launch_bounds__(kWideLanes)
k_add_rms_norm_quant_padded_wide(uint8_t* __restrict__ padded, uint16_t* __restrict__ rms,
                                 uint8_t* __restrict__ q_out, float* __restrict__ scales,
                                 const uint16_t* __restrict__ x, uint16_t* __restrict__ res,
                                 const uint16_t* __restrict__ w, int hidden, int64_t pad_bytes,
                                 float eps) {
  using E = BF16;
  constexpr int NC = VEC > 1 ? 8 : 16, NL = VEC > 1 ? 8 : 0;
  __shared__ double red_sum[16];
  __shared__ float red_max[16];
  __shared__ Pack<uint16_t, VEC> lds[NL > 0 ? NL : 1][kWideLanes];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * hidden;
  const int64_t pbase = (int64_t)blockIdx.x * pad_bytes;
  double ss = 0.0;
  float amax = 0.0f;
  // sum of squares (on the unrounded sums) and absmax of one vector; returns z = b(x + r)
  auto fold = [&](int64_t o) {
    const Pack<uint16_t, VEC> xv = ld<uint16_t, VEC>(x + base + o);
    const Pack<uint16_t, VEC> rv = ld<uint16_t, VEC>(res + base + o);
    const Pack<uint16_t, VEC> wv = ld<uint16_t, VEC>(w + o);
    Pack<uint16_t, VEC> z;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = E::to_f(xv.v[e]) + E::to_f(rv.v[e]);
      ss = __builtin_fma((double)t, (double)t, ss);
      z.v[e] = E::from_f(t);
      amax = __builtin_fmaxf(amax, __builtin_fabsf(rnd<E>(E::to_f(z.v[e]) * E::to_f(wv.v[e]))));
    }
    return z;
  };
  Pack<uint16_t, VEC> zc[NC];
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + tid;
    if (j < nvec) {
      const Pack<uint16_t, VEC> z = fold((int64_t)j * VEC);
      if (c < NC) zc[c] = z; else lds[c - NC][tid] = z;
      st<uint16_t, VEC>(res + base + (int64_t)j * VEC, z);
    }
  }
  const int tail0 = (NC + NL) * tpr + tid;
  for (int j = tail0; j < nvec; j += tpr) (void)fold((int64_t)j * VEC);
  ss = row_reduce(ss, red_sum, tpr, SumOp());
  amax = row_reduce(amax, red_max, tpr, MaxOp());
  const float rho = mcop_inv_rms(ss, hidden, eps);
  const float s = __builtin_fmaxf(mcop_div_rn(amax * rho, 127.0f), FLT_EPSILON);
  const float inv = mcop_div_rn(1.0f, s);
  if (threadIdx.x == 0) {
    scales[blockIdx.x] = s;
    uint8_t* sp = padded + pbase + hidden;
    if ((reinterpret_cast<uintptr_t>(sp) & 3) == 0) {
      *reinterpret_cast<float*>(sp) = s;
    } else {
      const uint32_t b = __builtin_bit_cast(uint32_t, s);
#pragma unroll
      for (int k = 0; k < 4; ++k) sp[k] = (uint8_t)(b >> (8 * k));
    }
  }
  auto emit = [&](const Pack<uint16_t, VEC>& z, int64_t o) {
    const Pack<uint16_t, VEC> wv = ld<uint16_t, VEC>(w + o);
    Pack<uint16_t, VEC> ro;
    Pack<uint8_t, VEC> q;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      ro.v[e] = E::from_f(rnd<E>(E::to_f(z.v[e]) * rho) * E::to_f(wv.v[e]));
      q.v[e] = q_i8<-127>(E::to_f(ro.v[e]) * inv);
    }
    st<uint16_t, VEC>(rms + base + o, ro);
    st<uint8_t, VEC>(q_out + base + o, q);
    st<uint8_t, VEC>(padded + pbase + o, q);
  };
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int j = c * tpr + tid;
    if (j < nvec) emit(c < NC ? zc[c] : lds[c - NC][tid], (int64_t)j * VEC);
  }
  for (int j = tail0; j < nvec; j += tpr) {
    const int64_t o = (int64_t)j * VEC;
    const Pack<uint16_t, VEC> xv = ld<uint16_t, VEC>(x + base + o);
    const Pack<uint16_t, VEC> rv = ld<uint16_t, VEC>(res + base + o);
    Pack<uint16_t, VEC> z;
#pragma unroll
    for (int e = 0; e < VEC; ++e) z.v[e] = E::from_f(E::to_f(xv.v[e]) + E::to_f(rv.v[e]));
    st<uint16_t, VEC>(res + base + o, z);
    emit(z, o);
  }
}

template <int VEC, bool OPT>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<1, 4, OPT>)
                   : reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<1, 16, OPT>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<VEC, 1, OPT>);
      case 2: return reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<VEC, 2, OPT>);
      case 4: return reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<VEC, 4, OPT>);
      case 8: return reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<VEC, 8, OPT>);
      default: return reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<VEC, 16, OPT>);
    }
  }
}

struct PadArgs {
  uint8_t* padded;
  uint16_t* rms;
  uint8_t* q;
  float* scales;
  const uint16_t* x;
  uint16_t* res;
  const uint16_t* w;
  int64_t rows;
  int hidden;
  int64_t pad_bytes;
  float eps;
};

template <int VEC, bool OPT>
static void launch_nv(const Geometry& g, const PadArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
#define MCOP_LAUNCH(NVV, EXX)                                                                  \
  hipLaunchKernelGGL((k_add_rms_norm_quant_padded<VEC, NVV, OPT, EXX>), grid, block, 0, st,     \
                     a.padded, a.rms, a.q, a.scales, a.x, a.res, a.w, a.rows, a.hidden,       \
                     a.pad_bytes, g.tpr, a.eps)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4, false); else MCOP_LAUNCH(16, false);
  } else {
    // exact rows (one row per workgroup, every lane in it) on the latency path (at most 256
    // rows) take the EX form, when it keeps its registers
    const bool ex = g.rpb == 1 && (int64_t)g.nv * g.tpr == a.hidden / VEC && a.rows <= 256;
#define MCOP_EX(NVV)                                                                           \
  (ex && exact_form_ok(                                                                        \
             reinterpret_cast<const void*>(&k_add_rms_norm_quant_padded<VEC, NVV, OPT, true>)))
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
static int launch_split(const char* name, const PadArgs& a, hipStream_t st) {
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  const SplitKernel k8{fn(&k_add_rms_norm_quant_padded_split<8>), 8};
  const SplitKernel k4{fn(&k_add_rms_norm_quant_padded_split<4>), 4};
  return split_run(name, {k8, k4}, a.rows, a.hidden / 8, nullptr, st,
                   [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    const int64_t off = r0 * (int64_t)a.hidden;
    uint8_t* pd = a.padded + r0 * a.pad_bytes;
    uint16_t* rm = a.rms + off;
    uint8_t* q = a.q + off;
    float* sc = a.scales + r0;
    const uint16_t* xp = a.x + off;
    uint16_t* rp = a.res + off;
    const uint16_t* wp = a.w;
    int h = a.hidden, slices = p.slices, slice_vecs = p.slice_vecs;
    int64_t pb = a.pad_bytes, timeout = p.timeout_ticks;
    float e = a.eps;
    void* args[] = {&pd, &rm, &q, &sc, &xp, &rp, &wp, &n, &h, &pb, &e, &slices, &slice_vecs,
                    &ws, &timeout};
    return launch(args);
  });
}

template <bool OPT>
static int dispatch(const PadArgs& a, hipStream_t st) {
  const char* name = "fused_add_rms_norm_dynamic_per_token_quant_padding_output";
  const bool vec_ok = a.hidden % 8 == 0 && a.pad_bytes % 8 == 0 &&
                      aligned(16, a.x, a.res, a.w, a.rms) && aligned(8, a.q, a.padded);
  if constexpr (!OPT) {
    if (!row_fits(a.hidden, vec_ok ? 8 : 1, vec_ok ? &kernel_of<8, OPT> : &kernel_of<1, OPT>)) {
      if (vec_ok && split_rows_enabled()) {
        const int rc = launch_split(name, a, st);
        if (rc != MCOP_E_UNSUPPORTED) return rc;
      }
      if (!wide_rows_ok(name, a.rows)) return MCOP_E_UNSUPPORTED;
      const dim3 grid((unsigned)a.rows), block(kWideLanes);
      if (vec_ok) {
        hipLaunchKernelGGL((k_add_rms_norm_quant_padded_wide<8>), grid, block, 0, st, a.padded,
                           a.rms, a.q, a.scales, a.x, a.res, a.w, a.hidden, a.pad_bytes, a.eps);
      } else {
        hipLaunchKernelGGL((k_add_rms_norm_quant_padded_wide<1>), grid, block, 0, st, a.padded,
                           a.rms, a.q, a.scales, a.x, a.res, a.w, a.hidden, a.pad_bytes, a.eps);
      }
      return check_launch(name);
    }
  }
  Geometry g;
  if (!choose_geometry(name, a.rows, a.hidden, vec_ok ? 8 : 1,
                       vec_ok ? &kernel_of<8, OPT> : &kernel_of<1, OPT>, &g)) {
    return MCOP_E_UNSUPPORTED;
  }
  if (g.vec == 1) launch_nv<1, OPT>(g, a, st);
  else launch_nv<8, OPT>(g, a, st);
  return check_launch(name);
}

}  // namespace mcop

extern "C" int mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output(
    int8_t* output, void* output_rms, int8_t* output_quant_int8, float* out_scales,
    const void* input, void* residual, const void* weight, int64_t num_tokens,
    int64_t hidden_size, int64_t pad_size, float epsilon, void* stream) {
  using namespace mcop;
  const char* name = "fused_add_rms_norm_dynamic_per_token_quant_padding_output";
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size > INT32_MAX || pad_size <= 0 ||
      2 * pad_size < hidden_size + 4) {
    return set_error(MCOP_E_INVALID,
                     "%s: bad shape num_tokens=%lld hidden_size=%lld pad_size=%lld (a padded "
                     "row of 2*pad_size bytes must hold hidden_size codes and a 4-byte scale)",
                     name, (long long)num_tokens, (long long)hidden_size, (long long)pad_size);
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!output || !output_rms || !output_quant_int8 || !out_scales || !input || !residual ||
      !weight) {
    return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  }
  const PadArgs a{reinterpret_cast<uint8_t*>(output),
                  static_cast<uint16_t*>(output_rms),
                  reinterpret_cast<uint8_t*>(output_quant_int8),
                  out_scales,
                  static_cast<const uint16_t*>(input),
                  static_cast<uint16_t*>(residual),
                  static_cast<const uint16_t*>(weight),
                  num_tokens,
                  (int)hidden_size,
                  2 * pad_size,
                  epsilon};
  auto st = static_cast<hipStream_t>(stream);
  // the reference's dispatch: the "opt" rounding chain for H == 7168, the generic one otherwise
  return hidden_size == 7168 ? dispatch<true>(a, st) : dispatch<false>(a, st);
}
