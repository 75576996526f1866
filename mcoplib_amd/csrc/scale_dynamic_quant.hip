// scale_dynamic_quant.hip -- smooth-scale multiply + dynamic per-token int8 quantization
// without normalisation (mcoplib.op.scale_dynamic_quant).
//
// Semantics (per row), following op/scale_dynamic_quant.cu:40-104 of the reference:
//   v = f(h) * smooth (fp32);  A = max|v|
//   scales[t] = A * 0.00787401574803f     (:75, a multiplication, not A/127)
//   q = sat[-128,127](rne(v * (127/A)))   (:79, :88-91);  A == 0 gives q = 0
// One pass: the row is loaded once into VGPRs, one max reduction, codes from registers.
#include <hip/hip_runtime.h>

#include "../../include/mcop_norm.h"
#include "rowkern.h"

namespace mcop {

template <int VEC, int NV>
__global__ void __launch_bounds__(max_tpr(VEC, NV))
k_scale_dynamic_quant(uint8_t* __restrict__ out, float* __restrict__ scales,
                      const uint16_t* __restrict__ x, const float* __restrict__ sm, int64_t rows,
                      int hidden, int tpr) {
  __shared__ float red_max[16];
  const RowPos p = row_pos(rows, tpr);
  const int nvec = hidden / VEC;
  const int64_t base = p.row * (int64_t)hidden;
  const int64_t lbase = p.lrow * (int64_t)hidden;

  Pack<uint16_t, VEC> xv[NV];
  Pack<float, VEC> sv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    sv[v] = ld<float, VEC>(sm + (int64_t)load_index(vec_index(v, tpr, p.lt), nvec) * VEC);
  }
  shared_loads_first();
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    xv[v] = ld_nt<uint16_t, VEC>(x + lbase +
                                 (int64_t)load_index(vec_index(v, tpr, p.lt), nvec) * VEC);
  }

  float a[NV][VEC];
  float amax = 0.0f;
  // Lanes past the row end hold a copy of vector 0, which does not change the max.
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float t = BF16::to_f(xv[v].v[e]) * sv[v].v[e];
      a[v][e] = t;
      amax = __builtin_fmaxf(amax, __builtin_fabsf(t));
    }
  }
  amax = row_reduce(amax, red_max, tpr, MaxOp());

  if (p.live && p.lt == 0) scales[p.row] = amax * 0.00787401574803f;
  const float inv = amax > 0.0f ? mcop_div_rn(127.0f, amax) : 0.0f;

#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int j = vec_index(v, tpr, p.lt);
    if (p.live && j < nvec) {
      Pack<uint8_t, VEC> q;
#pragma unroll
      for (int e = 0; e < VEC; ++e) q.v[e] = q_i8<-128>(a[v][e] * inv);
      st_nt<uint8_t, VEC>(out + base + (int64_t)j * VEC, q);
    }
  }
}

template <int VEC>
static void launch_nv(const Geometry& g, int8_t* out, float* scales, const void* x,
                      const float* sm, int64_t rows, int hidden, hipStream_t st) {
  const dim3 grid((unsigned)g.blocks), block((unsigned)(g.tpr * g.rpb));
  auto* o = reinterpret_cast<uint8_t*>(out);
  auto* xp = static_cast<const uint16_t*>(x);
#define MCOP_LAUNCH(NVV)                                                                     \
  hipLaunchKernelGGL((k_scale_dynamic_quant<VEC, NVV>), grid, block, 0, st, o, scales, xp, sm, \
                     rows, hidden, g.tpr)
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
    return nv == 4 ? reinterpret_cast<const void*>(&k_scale_dynamic_quant<1, 4>)
                   : reinterpret_cast<const void*>(&k_scale_dynamic_quant<1, 16>);
  } else {
    switch (nv) {
      case 1: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 1>);
      case 2: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 2>);
      case 4: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 4>);
      case 8: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 8>);
      default: return reinterpret_cast<const void*>(&k_scale_dynamic_quant<VEC, 16>);
    }
  }
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
  Geometry g;
  if (!choose_geometry("scale_dynamic_quant", num_tokens, hidden_size, vec_ok ? V : 1,
                       vec_ok ? &kernel_of<V> : &kernel_of<1>, &g)) {
    return set_error(MCOP_E_UNSUPPORTED,
                     "scale_dynamic_quant: hidden_size %lld is larger than the register-resident "
                     "kernels support",
                     (long long)hidden_size);
  }
  auto st = static_cast<hipStream_t>(stream);
  if (g.vec == 1) {
    launch_nv<1>(g, out, scales, input, smooth, num_tokens, (int)hidden_size, st);
  } else {
    launch_nv<V>(g, out, scales, input, smooth, num_tokens, (int)hidden_size, st);
  }
  return check_launch("scale_dynamic_quant");
}
