// scale_dynamic_quant.hip -- smooth-scale multiply + dynamic per-token int8 quantization
// without normalisation (mcoplib.op.scale_dynamic_quant).
//
// Semantics (per row), following op/scale_dynamic_quant.cu:40-104 of the reference:
//   v = f(h) * smooth (fp32);  A = max|v|
//   scales[t] = A * 0.00787401574803f     (:75, a multiplication, not A/127)
//   q = sat[-128,127](rne(v * (127/A)))   (:79, :88-91);  A == 0 gives q = 0
// One pass: the row is loaded once into VGPRs, one max reduction, codes from registers.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/mcop_norm.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

// Rows a split-row workgroup takes when the call has at least two.
constexpr int kSdqSplitRows = 2;

// R rows per lane (1, or 2 for many rows): the lane's smooth vectors, loaded once, serve R rows.
// The smooth scales are fp32, two loads per 16-byte input vector; even as cache hits they took
// 20% of the kernel's time in a compute-free model of this access pattern at 16384 x 7168, and
// sharing them between two rows recovers about half of that.
template <int VEC, int NV, int R>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_scale_dynamic_quant(uint8_t* __restrict__ out, float* __restrict__ scales,
                      const uint16_t* __restrict__ x, const float* __restrict__ sm, int64_t rows,
                      int hidden, int tpr) {
  __shared__ float red_max[16 * R];
  const int nvec = hidden / VEC;
  RowPos p[R];
#pragma unroll
  for (int k = 0; k < R; ++k) p[k] = row_pos_of(rows, tpr, k, R);

  Pack<float, VEC> sv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    sv[v] = ld<float, VEC>(sm + (int64_t)load_index(vec_index(v, tpr, p[0].lt), nvec) * VEC);
  }
  shared_loads_first();
  Pack<uint16_t, VEC> xv[R][NV];
#pragma unroll
  for (int k = 0; k < R; ++k) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      xv[k][v] = ld_nt<uint16_t, VEC>(x + p[k].lrow * (int64_t)hidden +
                                      (int64_t)load_index(vec_index(v, tpr, p[k].lt), nvec) * VEC);
    }
  }

  float a[R][NV][VEC];
  float amax[R];
  // Lanes past the row end hold a copy of vector 0, which does not change the max.
#pragma unroll
  for (int k = 0; k < R; ++k) {
    amax[k] = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float t = BF16::to_f(xv[k][v].v[e]) * sv[v].v[e];
        a[k][v][e] = t;
        amax[k] = __builtin_fmaxf(amax[k], __builtin_fabsf(t));
      }
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) amax[k] = row_reduce(amax[k], red_max + 16 * k, tpr, MaxOp());

#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (p[k].live && p[k].lt == 0) scales[p[k].row] = amax[k] * 0.00787401574803f;
    const float inv = amax[k] > 0.0f ? mcop_div_rn(127.0f, amax[k]) : 0.0f;
    const int64_t base = p[k].row * (int64_t)hidden;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int j = vec_index(v, tpr, p[k].lt);
      if (p[k].live && j < nvec) {
        Pack<uint8_t, VEC> q;
#pragma unroll
        for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-128>(a[k][v][e] * inv);
        st_nt<uint8_t, VEC>(out + base + (int64_t)j * VEC, q);
      }
    }
  }
}

// Rows too wide for one workgroup's registers, read once (split_row.h): workgroup b takes slice
// b % slices of the R rows of group b / slices -- `slice_vecs` vectors of each, NV a lane -- and
// holds their products v in registers; the slice's smooth vectors, loaded once, serve the R rows
// (they are fp32, twice the bytes of x).  The slices' absmax values are combined through the
// workspace `ws` in one exchange (split_max, or split_max2 for two rows); every other step is
// the register kernel's, element by element.  `rows` rows of the launch form `groups` groups;
// a group's row past the end computes on a copy of its first row and stores nothing.
template <int VEC, int NV, int R>
__global__ void __launch_bounds__(max_tpr(VEC, NV * R))
k_scale_dynamic_quant_split(uint8_t* __restrict__ out, float* __restrict__ scales,
                            const uint16_t* __restrict__ x, const float* __restrict__ sm,
                            int64_t groups, int64_t rows, int hidden, int slices, int slice_vecs,
                            uint64_t* __restrict__ ws, int64_t timeout_ticks) {
  static_assert(R == 1 || R == 2, "one or two rows a workgroup");
  __shared__ float red_max[16 * R];
  __shared__ float x_max[2];
  __shared__ int x_fail;
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x;
  const int lt = (int)threadIdx.x;
  const int sl = (int)(blockIdx.x % (unsigned)slices);
  const int64_t g = blockIdx.x / (unsigned)slices;
  const int j0 = sl * slice_vecs;
  const int jn = min(slice_vecs, nvec - j0);
  int64_t row[R];
  bool live[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    live[k] = g * R + k < rows;
    row[k] = live[k] ? g * R + k : g * R;
  }
  // Lanes past the slice end re-read the slice's first vector, which leaves the absmax unchanged.
  auto in_of = [&](int v) { return vec_index(v, tpr, lt) < jn; };
  auto lj_of = [&](int v) {
    return (int64_t)(j0 + (in_of(v) ? vec_index(v, tpr, lt) : 0)) * VEC;
  };
  Pack<float, VEC> sv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) sv[v] = ld<float, VEC>(sm + lj_of(v));
  shared_loads_first();
  Pack<uint16_t, VEC> xv[R][NV];
#pragma unroll
  for (int k = 0; k < R; ++k) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      xv[k][v] = ld_nt<uint16_t, VEC>(x + row[k] * (int64_t)hidden + lj_of(v));
    }
  }
  float a[R][NV][VEC];
  float amax[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    amax[k] = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float t = BF16::to_f(xv[k][v].v[e]) * sv[v].v[e];
        a[k][v][e] = t;
        amax[k] = __builtin_fmaxf(amax[k], __builtin_fabsf(t));
      }
    }
  }
  uint64_t* err = ws + split_ws_words(groups, slices) - 1;
  if constexpr (R == 1) {
    SplitRowReduce red{nullptr, red_max, tpr, ws, g, slices, sl, err, timeout_ticks, nullptr,
                       x_max, &x_fail};
    amax[0] = red.max(amax[0]);
  } else {
    amax[0] = row_reduce<true>(amax[0], red_max, tpr, MaxOp());
    amax[1] = row_reduce<true>(amax[1], red_max + 16, tpr, MaxOp());
    split_max2(split_slots(ws, g, slices, 0), slices, sl, kSplitTag, &amax[0], &amax[1], err,
               timeout_ticks, x_max, &x_fail);
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (!live[k]) continue;
    // slice 0 stores the scale; a slice whose exchange failed stores it too (NaN: split_row.h)
    if (lt == 0 && (sl == 0 || x_fail != 0)) scales[row[k]] = amax[k] * 0.00787401574803f;
    const float inv = amax[k] > 0.0f ? mcop_div_rn(127.0f, amax[k]) : 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (in_of(v)) {
        Pack<uint8_t, VEC> q;
#pragma unroll
        for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-128>(a[k][v][e] * inv);
        st_nt<uint8_t, VEC>(out + row[k] * (int64_t)hidden + lj_of(v), q);
      }
    }
  }
}

// Rows too wide for the registers: one 1024-lane workgroup per row and two passes over it
// (absmax; codes).  The row's head stays on chip between the passes -- the first NC vectors of
// every lane in registers, the next NL in lane-private LDS slots (vector c of lane t at [c][t],
// so no barrier is needed; the workgroup already fills a CU's registers, so the 128 KB cost no
// occupancy) -- and the second pass re-reads the rest of the row and the smooth scales.
template <int VEC>
__global__ void __launch_bounds__(kWideLanes)
k_scale_dynamic_quant_wide(uint8_t* __restrict__ out, float* __restrict__ scales,
                           const uint16_t* __restrict__ x, const float* __restrict__ sm,
                           int hidden) {
  constexpr int NC = VEC > 1 ? 8 : 16, NL = VEC > 1 ? 8 : 0;
  __shared__ float red_max[16];
  __shared__ Pack<uint16_t, VEC> lds[NL > 0 ? NL : 1][kWideLanes];
  const int nvec = hidden / VEC;
  const int tpr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * hidden;
  auto v_from = [&](const Pack<uint16_t, VEC>& xv, int64_t o, float* v) {
    const Pack<float, VEC> sv = ld<float, VEC>(sm + o);
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = BF16::to_f(xv.v[e]) * sv.v[e];
  };
  // Head slots past the row end hold a copy of the row's vector 0 (which leaves the absmax
  // unchanged), so every load is unconditional: loads under a per-lane branch each wait for
  // completion where the branch rejoins, which serializes their latencies.
  Pack<uint16_t, VEC> xc[NC];
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    const int64_t o = (int64_t)load_index(c * tpr + tid, nvec) * VEC;
    const Pack<uint16_t, VEC> xv = ld<uint16_t, VEC>(x + base + o);
    if (c < NC) xc[c] = xv; else lds[c - NC][tid] = xv;
  }
  auto head = [&](int c) -> Pack<uint16_t, VEC> { return c < NC ? xc[c] : lds[c - NC][tid]; };
  // The lane index, opaque to the compiler per pass: each pass recomputes its vectors' offsets
  // instead of holding 16 address pairs from the loads above.
  int lt = tid;
  __asm__ volatile("" : "+v"(lt));
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC + NL; ++c) {
    float v[VEC];
    v_from(head(c), (int64_t)load_index(c * tpr + lt, nvec) * VEC, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[e]));
  }
  const int tail0 = (NC + NL) * tpr + tid;
  for (int j = tail0; j < nvec; j += tpr) {
    float v[VEC];
    v_from(ld<uint16_t, VEC>(x + base + (int64_t)j * VEC), (int64_t)j * VEC, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[e]));
  }
  amax = row_reduce(amax, red_max, tpr, MaxOp());
  if (threadIdx.x == 0) scales[blockIdx.x] = amax * 0.00787401574803f;
  const float inv = amax > 0.0f ? mcop_div_rn(127.0f, amax) : 0.0f;
  auto emit = [&](const Pack<uint16_t, VEC>& xv, int64_t o, bool in) {
    float v[VEC];
    v_from(xv, o, v);
    Pack<uint8_t, VEC> q;
#pragma unroll
    for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-128>(v[e] * inv);
    if (in) st<uint8_t, VEC>(out + base + o, q);
  };
  __asm__ volatile("" : "+v"(lt));
  if ((NC + NL) * tpr <= nvec) {  // the head is whole: no store needs a lane test
#pragma unroll
    for (int c = 0; c < NC + NL; ++c) emit(head(c), (int64_t)(c * tpr + lt) * VEC, true);
  } else {
#pragma unroll
    for (int c = 0; c < NC + NL; ++c) {
      const int j = c * tpr + lt;
      emit(head(c), (int64_t)load_index(j, nvec) * VEC, j < nvec);
    }
  }
  for (int j = tail0; j < nvec; j += tpr) {
    emit(ld<uint16_t, VEC>(x + base + (int64_t)j * VEC), (int64_t)j * VEC, true);
  }
}

// Two rows per lane when the vector path has at least 2048 rows and at most four vectors per
// lane (more would spill); one otherwise (fewer rows: every row is already in flight).
static int rows_per_lane(const Geometry& g, int64_t rows) {
  return g.vec > 1 && g.nv <= 4 && rows >= 2048 ? 2 : 1;
}

template <int VEC>
static void launch_nv(const Geometry& g, int8_t* out, float* scales, const void* x,
                      const float* sm, int64_t rows, int hidden, hipStream_t st) {
  const dim3 block((unsigned)(g.tpr * g.rpb));
  auto* o = reinterpret_cast<uint8_t*>(out);
  auto* xp = static_cast<const uint16_t*>(x);
  if constexpr (VEC > 1) {
    if (rows_per_lane(g, rows) == 2) {
      const dim3 grid((unsigned)((rows + 2 * g.rpb - 1) / (2 * g.rpb)));
#define MCOP_LAUNCH(NVV)                                                                       \
  hipLaunchKernelGGL((k_scale_dynamic_quant<VEC, NVV, 2>), grid, block, 0, st, o, scales, xp,   \
                     sm, rows, hidden, g.tpr)
      switch (g.nv) {
        case 1: MCOP_LAUNCH(1); break;
        case 2: MCOP_LAUNCH(2); break;
        default: MCOP_LAUNCH(4); break;
      }
#undef MCOP_LAUNCH
      return;
    }
  }
  const dim3 grid((unsigned)g.blocks);
#define MCOP_LAUNCH(NVV)                                                                       \
  hipLaunchKernelGGL((k_scale_dynamic_quant<VEC, NVV, 1>), grid, block, 0, st, o, scales, xp,   \
                     sm, rows, hidden, g.tpr)
  if constexpr (VEC == 1) {
    if (g.nv == 4) MCOP_LAUNCH(4); else MCOP_LAUNCH(16);
  } else {
    switch (g.nv) {
      case 1: MCOP_LAUNCH(1); break;
      case 2: MCOP_LAUNCH(2); break;
      case 4: MCOP_LAUNCH(4); break;
      case 8: MCOP_LAUNCH(8); break;
      default: MCOP_LAUNCH(16); break;
    }
  }
#undef MCOP_LAUNCH
}

template <int VEC>
static const void* kernel_of(int nv) {
  if constexpr (VEC == 1) {
    return nv == 4 ? reinterpret_cast<const void*>(&k_scale_dynamic_quant<1, 4, 1>)
                   : reinterpret_cast<const void*>(&k_scale_dynamic_quant<1, 16, 1>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 1, 1>);
      case 2: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 2, 1>);
      case 4: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 4, 1>);
      case 8: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 8, 1>);
      default: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 16, 1>);
    }
  }
}

// Rows too wide for the register kernels, vector path: the split-row kernel when it applies, its
// workspace from the stream-ordered allocator; MCOP_E_UNSUPPORTED (no message) when it does not.
// With at least two rows a workgroup takes two rows at four vectors a lane, sharing the smooth
// vectors; a single row takes eight vectors a lane (or four).
static int launch_split(uint8_t* out, float* scales, const uint16_t* x, const float* sm,
                        int64_t rows, int hidden, hipStream_t st) {
  constexpr int V = BF16::VEC;
  auto fn = [](auto k) { return reinterpret_cast<const void*>(k); };
  const int R = rows >= 2 ? kSdqSplitRows : 1;
  const SplitKernel k8{fn(&k_scale_dynamic_quant_split<V, 8, 1>), 8};
  const SplitKernel k4{fn(&k_scale_dynamic_quant_split<V, 4, 1>), 4};
  const SplitKernel k4r2{fn(&k_scale_dynamic_quant_split<V, 4, 2>), 4};
  auto chunk = [&](int64_t r0, int64_t n, uint64_t* ws, const SplitPlan& p, auto launch) {
    // r0, n count groups of R rows
    const int64_t row0 = r0 * R;
    int64_t nrows = std::min<int64_t>(n * R, rows - row0);
    uint8_t* o = out + row0 * (int64_t)hidden;
    float* sc = scales + row0;
    const uint16_t* xp = x + row0 * (int64_t)hidden;
    const float* sp = sm;
    int h = hidden, slices = p.slices, slice_vecs = p.slice_vecs;
    int64_t timeout = p.timeout_ticks;
    void* args[] = {&o, &sc, &xp, &sp, &n, &nrows, &h, &slices, &slice_vecs, &ws, &timeout};
    return launch(args);
  };
  const char* name = "scale_dynamic_quant";
  const int64_t groups = (rows + R - 1) / R;
  if (R == 2) return split_run(name, {k4r2}, groups, hidden / V, nullptr, st, chunk);
  return split_run(name, {k8, k4}, groups, hidden / V, nullptr, st, chunk);
}

}  // namespace mcop

extern "C" int mcop_scale_dynamic_quant(int8_t* out, float* scales, const void* input,
                                        const float* smooth, int64_t num_tokens,
                                        int64_t hidden_size, void* stream) {
  using namespace mcop;
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size > INT32_MAX) {
    return set_error(MCOP_E_INVALID,
                     "scale_dynamic_quant: bad shape num_tokens=%lld hidden_size=%lld",
                     (long long)num_tokens, (long long)hidden_size);
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !scales || !input || !smooth) {
    return set_error(MCOP_E_INVALID, "scale_dynamic_quant: null pointer");
  }
  constexpr int V = BF16::VEC;
  const bool vec_ok = hidden_size % V == 0 && aligned(16, input, smooth) && aligned(V, out);
  auto st = static_cast<hipStream_t>(stream);
  const KernelOfNv kernels = vec_ok ? &kernel_of<V> : &kernel_of<1>;
  if (!row_fits(hidden_size, vec_ok ? V : 1, kernels)) {
    auto* o = reinterpret_cast<uint8_t*>(out);
    auto* xp = static_cast<const uint16_t*>(input);
    if (vec_ok && split_rows_enabled()) {
      const int rc = launch_split(o, scales, xp, smooth, num_tokens, (int)hidden_size, st);
      if (rc != MCOP_E_UNSUPPORTED) return rc;
    }
    if (!wide_rows_ok("scale_dynamic_quant", num_tokens)) return MCOP_E_UNSUPPORTED;
    if (vec_ok) {
      hipLaunchKernelGGL((k_scale_dynamic_quant_wide<V>), dim3((unsigned)num_tokens),
                         dim3(kWideLanes), 0, st, o, scales, xp, smooth, (int)hidden_size);
    } else {
      hipLaunchKernelGGL((k_scale_dynamic_quant_wide<1>), dim3((unsigned)num_tokens),
                         dim3(kWideLanes), 0, st, o, scales, xp, smooth, (int)hidden_size);
    }
    return check_launch("scale_dynamic_quant");
  }
  Geometry g;
  if (!choose_geometry("scale_dynamic_quant", num_tokens, hidden_size, vec_ok ? V : 1, kernels,
                       &g)) {
    return MCOP_E_UNSUPPORTED;
  }
  if (g.vec == 1) {
    launch_nv<1>(g, out, scales, input, smooth, num_tokens, (int)hidden_size, st);
  } else {
    launch_nv<V>(g, out, scales, input, smooth, num_tokens, (int)hidden_size, st);
  }
  return check_launch("scale_dynamic_quant");
}
