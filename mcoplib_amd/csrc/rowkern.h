// rowkern.h -- building blocks of the gfx950 row kernels (device code) and their launch
// geometry (host code).
//
// Layout model: a row of `hidden` elements is split into vectors of VEC elements (16 bytes on
// the vector path, one element on the scalar path).  Lane `lt` of a row owns vectors
// lt, lt + tpr, lt + 2*tpr, ... (NV of them), so every load/store instruction of a wave covers
// 64 consecutive vectors (1 KiB of bf16 for 16-byte vectors).  A workgroup holds
// `blockDim.x / tpr` rows; tpr (lanes per row) is a multiple of 64, so a row is a whole number
// of waves and the row reductions never mix rows inside a wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "numerics.h"

namespace mcop {

// ---------------------------------------------------------------------------------------------
// Element types.  S is the storage type; to_f widens exactly; from_f rounds to nearest even.
struct BF16 {
  using S = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f(S s) {
    return __builtin_bit_cast(float, (uint32_t)s << 16);
  }
  static __device__ __forceinline__ S from_f(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);  // v_cvt_pk_bf16_f32, RNE
  }
};
struct F16 {
  using S = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float to_f(S s) {
    return (float)__builtin_bit_cast(_Float16, s);
  }
  static __device__ __forceinline__ S from_f(float f) {
    // The empty asm pins f as a rounded fp32 value: without it the compiler folds a producing
    // fp32 multiply and this conversion into one v_fma_mixlo_f16, which rounds the exact
    // product to fp16 once instead of rounding it to fp32 first (different results when the
    // operands are not fp16 values).
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
  }
};
struct F32 {
  using S = float;
  static constexpr int VEC = 4;
  static __device__ __forceinline__ float to_f(S s) { return s; }
  static __device__ __forceinline__ S from_f(float f) { return f; }
};

// Round an fp32 value to the storage type and widen it back.
template <class E>
__device__ __forceinline__ float rnd(float f) {
  return E::to_f(E::from_f(f));
}

// N elements of type T as one aligned register block, so that a 4-, 8- or 16-byte block is one
// global load or store instruction (blocks of 32 bytes become two).
template <class T, int N>
struct alignas(sizeof(T) * N) Pack {
  T v[N];
};

template <class T, int N>
__device__ __forceinline__ Pack<T, N> ld(const T* p) {
  return *reinterpret_cast<const Pack<T, N>*>(p);
}
template <class T, int N>
__device__ __forceinline__ void st(T* p, const Pack<T, N>& v) {
  *reinterpret_cast<Pack<T, N>*>(p) = v;
}

// Register type of a B-byte block, for the non-temporal builtins (which take scalars/vectors).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <int B> struct RawOf;
template <> struct RawOf<1> { using T = uint8_t; };
template <> struct RawOf<2> { using T = uint16_t; };
template <> struct RawOf<4> { using T = uint32_t; };
template <> struct RawOf<8> { using T = u32x2; };
template <> struct RawOf<16> { using T = u32x4; };

// Streaming (non-temporal) load / store of a Pack: data touched once per call (the rows of x,
// residual and the outputs) is marked so it does not displace reused data (the weight vector)
// in the caches.  Measured on MI355X: +10% HBM throughput for the row kernels.
// Build-time switches of the streaming hints (both on by default; the tuning sweeps build
// variants with them off).
#ifndef MCOP_NT_LOADS
#define MCOP_NT_LOADS 1
#endif
#ifndef MCOP_NT_STORES
#define MCOP_NT_STORES 1
#endif

template <class T, int N>
__device__ __forceinline__ Pack<T, N> ld_nt(const T* p) {
  constexpr int B = (int)sizeof(T) * N;
  if constexpr (!MCOP_NT_LOADS) {
    return ld<T, N>(p);
  } else if constexpr (B == 32) {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + 1);
    struct Two { u32x4 a, b; };
    return __builtin_bit_cast(Pack<T, N>, Two{a, b});
  } else {
    using R = typename RawOf<B>::T;
    return __builtin_bit_cast(Pack<T, N>, __builtin_nontemporal_load(reinterpret_cast<const R*>(p)));
  }
}
template <class T, int N>
__device__ __forceinline__ void st_nt(T* p, const Pack<T, N>& v) {
  constexpr int B = (int)sizeof(T) * N;
  if constexpr (!MCOP_NT_STORES) {
    st<T, N>(p, v);
  } else {
    using R = typename RawOf<B>::T;
    __builtin_nontemporal_store(__builtin_bit_cast(R, v), reinterpret_cast<R*>(p));
  }
}

// ---------------------------------------------------------------------------------------------
// Quantizers.

// rne(v) converted to int32 by the hardware conversion, whose results are defined for every
// input: NaN -> 0, out-of-range values saturate.  Inline VALU asm keeps that definition (a C++
// cast of NaN is undefined behaviour the compiler may exploit).
__device__ __forceinline__ int cvt_rne_i32(float v) {
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(__builtin_rintf(v)));
  return r;
}

// int8 code of v: saturate(rne(v)) to [LO, 127]; NaN -> 0.
template <int LO>
__device__ __forceinline__ uint8_t q_i8(float v) {
  const int i = cvt_rne_i32(v);
  return (uint8_t)(i < LO ? LO : (i > 127 ? 127 : i));
}

// int8 code of t = y * inv when |t| <= 127.5 is guaranteed (absmax scaling, no scale bound):
// RN(t + 1.5 * 2^23) holds rne(t) in the low mantissa bits (exact for |t| < 2^22), so its low
// byte is the two's-complement code.  Two operations instead of round / convert / clamp; the
// empty asm keeps the product rounded on its own (no fused multiply-add).  A NaN t keeps the
// payload of y, whose low 13 bits are zero for bf16 / fp16 values, so NaN codes 0 as in q_i8.
__device__ __forceinline__ uint8_t q_i8_in_range(float y, float inv) {
  float t = y * inv;
  asm("" : "+v"(t));
  return (uint8_t)__builtin_bit_cast(uint32_t, t + 12582912.0f);
}

// OCP fp8 e4m3fn codes of N values in [-448 - 2^-15, 448] (v_cvt_pk_fp8_f32: RNE, so a value
// one ulp beyond -448 codes -448).
template <int N>
__device__ __forceinline__ Pack<uint8_t, N> cvt_fp8(const float* c) {
  Pack<uint8_t, N> p;
  if constexpr (N == 1) {
    const int r = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[0], 0, false);
    p.v[0] = (uint8_t)(r & 0xff);
  } else {
    static_assert(N % 4 == 0, "fp8 packs are built 4 codes per dword");
#pragma unroll
    for (int d = 0; d < N / 4; ++d) {
      int r = __builtin_amdgcn_cvt_pk_fp8_f32(c[4 * d + 0], c[4 * d + 1], 0, false);
      r = __builtin_amdgcn_cvt_pk_fp8_f32(c[4 * d + 2], c[4 * d + 3], r, true);
#pragma unroll
      for (int k = 0; k < 4; ++k) p.v[4 * d + k] = (uint8_t)((uint32_t)r >> (8 * k));
    }
  }
  return p;
}

// q[e] = a[e] / b correctly rounded for the N values of one vector (b fixed for the row,
// inv == RN(1/b), b_ok == mcop_divisor_ok(b)).  Every element takes the 3-operation Markstein
// form of mcop_fdiv_const; if any lane of the wave has an element outside that form's domain
// (|a| or |q| outside [2^-100, 2^100], a zero, a non-finite value, or a divisor outside the
// domain) the wave recomputes the vector with mcop_fdiv_const, whose fallback is the full IEEE
// division.  The recomputation sits behind a wave-uniform branch, so rows of ordinary values do
// not pay for the full division.
template <int N>
__device__ __forceinline__ void div_by_const(float* q, const float* a, float b, float inv,
                                             bool b_ok) {
  bool slow = !b_ok;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float q0 = a[e] * inv;
    const float r = __builtin_fmaf(-q0, b, a[e]);
    const float qq = __builtin_fmaf(r, inv, q0);
    q[e] = qq;
    const float aa = __builtin_fabsf(a[e]), aq = __builtin_fabsf(qq);
    slow |= !(aa >= 0x1p-100f && aq >= 0x1p-100f && aq <= 0x1p100f);
  }
  if (__builtin_amdgcn_ballot_w64(slow) != 0) {
#pragma unroll
    for (int e = 0; e < N; ++e) q[e] = mcop_fdiv_const(a[e], b, inv, b_ok);
  }
}

// Whether every element a lane divides by the row's b > 0 lies in the domain of the 3-operation
// form of div_by_const (|a| and |a/b| in [2^-100, 2^100], b_ok), from bounds the row already has,
// so that the per-element tests can be skipped: `amin` <= every |a| of the lane (0 for a lane
// holding a zero, which then fails: the form would drop the sign of -0), `amax_sq` >= every
// a^2 of the row (non-finite for a row holding NaN or infinity, which then fails).  The computed
// quotient is within one ulp of a/b and inv = RN(1/b) within half an ulp of 1/b, so the tests
// below on amin * inv and on amax_sq * inv^2 against 2^200 (in binary64, with margins of 2^-20
// and 2^-17; no square root) imply the per-element ones; div_by_const then takes its
// 3-operation form for every element, so skipping its tests changes no result.
__device__ __forceinline__ bool div_domain_ok(float amin, double amax_sq, float inv, bool b_ok) {
  const double lo = (double)amin * (double)inv * (1.0 - 0x1p-20);
  const double hi_sq = amax_sq * ((double)inv * (double)inv) * (1.0 + 0x1p-17);
  return b_ok && amin >= 0x1p-100f && lo >= 0x1p-100 && hi_sq <= 0x1p200;
}

// q[e] = a[e] / b for one vector in the 3-operation form; only for elements div_domain_ok
// admits (else div_by_const).
template <int N>
__device__ __forceinline__ void div_in_domain(float* q, const float* a, float b, float inv) {
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float q0 = a[e] * inv;
    q[e] = __builtin_fmaf(__builtin_fmaf(-q0, b, a[e]), inv, q0);
  }
}

// clamp(v, -448, 448) with fmin/fmax semantics (a NaN operand yields the other operand), as
// the reference's float_to_fp8 does before its conversion.
__device__ __forceinline__ float clamp_fp8(float v) {
  return __builtin_fmaxf(-448.0f, __builtin_fminf(v, 448.0f));
}

// fp8-e4m3fn codes of clamp(RN(a[e] / b)) for the N values of one vector.
// `bounded` (uniform over the row) states that every |a| of the row is at most 448 * b * (1 +
// 2^-22) (the row's absmax was not cut by a scale bound) and that 2^-18 <= b <= 2^100.  Then the
// Markstein form q0 = a*inv, r = fma(-q0, b, a), q = fma(r, inv, q0) is exact for every element
// with |a| >= 2^-100 and |a/b| >= 2^-100 (|q| <= 449: no intermediate overflow or underflow);
// every other element has |a/b| < 2^-82, the form then yields some |q| < 2^-80, and any such
// value codes to a zero.  copysign gives that zero a's sign (the correction step turns -0 into
// +0).  In a bounded row every quotient that is not NaN lies within [-448 - u, 448 + u] (u =
// 2^-15, one ulp of 448), where the clamp to [-448, 448] and the conversion's round-to-nearest
// give the same code, so only the upper clamp is applied: it sends NaN to +448 as the two-sided
// clamp does.  Rows that are not bounded take div_by_const and the two-sided clamp.
template <int N>
__device__ __forceinline__ Pack<uint8_t, N> fp8_quotient_codes(const float* a, float b, float inv,
                                                               bool b_ok, bool bounded) {
  float c[N];
  if (bounded) {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float q0 = a[e] * inv;
      const float r = __builtin_fmaf(-q0, b, a[e]);
      c[e] = __builtin_fminf(__builtin_copysignf(__builtin_fmaf(r, inv, q0), a[e]), 448.0f);
    }
  } else {
    div_by_const<N>(c, a, b, inv, b_ok);
#pragma unroll
    for (int e = 0; e < N; ++e) c[e] = clamp_fp8(c[e]);
  }
  return cvt_fp8<N>(c);
}

// ---------------------------------------------------------------------------------------------
// Row reductions.  Every thread of the workgroup must call them (they may contain a barrier).
// `lds` holds one slot per wave of the workgroup (at most 16).  The sum is of fp64 partials;
// its result is independent of the order up to fp64 rounding, which the single rounding to
// fp32 afterwards absorbs.

struct SumOp {
  __device__ __forceinline__ double operator()(double a, double b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return __builtin_fmaxf(a, b);
  }
};

// A lane's partner value under a DPP lane pattern (a register move inside each 16-lane row,
// no LDS round trip), for 32- and 64-bit values.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ double dpp_mov(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, true);
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <- 15 - i within each 16 lanes

// All-reduce within each aligned 16-lane segment: after the quad steps every lane holds its
// quad's value, the half-row mirror pairs quad 0 with 1 and 2 with 3, the row mirror pairs the
// two halves.
template <class T, class Op>
__device__ __forceinline__ T reduce16(T v, Op op) {
  v = op(v, dpp_mov<kDppXor1>(v));
  v = op(v, dpp_mov<kDppXor2>(v));
  v = op(v, dpp_mov<kDppHalfMirror>(v));
  return op(v, dpp_mov<kDppMirror>(v));
}

// The value lane `lane` holds, read into scalar registers (v_readlane_b32: no LDS round trip).
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ double lane_value(double v, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// All-reduce over the wave: after reduce16 every lane of a 16-lane segment holds that
// segment's value (bit for bit: each step combines the same two operands in both lanes), so the
// wave's value combines lanes 0, 16, 32 and 48, in that fixed order, and is uniform.
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  v = reduce16(v, op);
  return op(op(lane_value(v, 0), lane_value(v, 16)), op(lane_value(v, 32), lane_value(v, 48)));
}

// ONE: the workgroup holds exactly one row (tpr == blockDim.x), so its first wave is wave 0.
template <bool ONE = false, class T, class Op>
__device__ __forceinline__ T row_reduce(T v, T* lds, int tpr, Op op) {
  if (!ONE && tpr < 64) {  // several rows per wave: all-reduce within each row's aligned segment
    v = reduce16(v, op);
    if (tpr == 32) v = op(v, __shfl_xor(v, 16, 64));
    return v;
  }
  v = wave_reduce(v, op);
  if (tpr == 64) return v;  // the row is one wave
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds[wave] = v;
  __syncthreads();
  const int wpr = tpr >> 6;
  const int first = ONE ? 0 : (wave / wpr) * wpr;
  T t = lds[first];
  for (int i = 1; i < wpr; ++i) t = op(t, lds[first + i]);
  return t;
}

// Issue order of a lane's loads: the vectors every row shares (weights, smooth scales; L2
// hits) go out before the row's own streamed vectors.  The scheduling barrier keeps the
// compiler from interleaving the two groups; on MI355X that order measured faster (the
// SmoothQuant kernel at 16384 x 7168: 148 us against 181 us interleaved).
#ifndef MCOP_SHARED_FIRST
#define MCOP_SHARED_FIRST 1
#endif
__device__ __forceinline__ void shared_loads_first() {
#if MCOP_SHARED_FIRST
  __builtin_amdgcn_sched_barrier(0);
#endif
}

// Position of this thread: its row and its lane within the row.  `lrow` is the row its loads
// use: the last row for lanes of a workgroup's trailing rows past the end, so that every load
// of the kernel is unconditional (no branch, hence no wait, between the loads of a lane); such
// lanes store nothing.
struct RowPos {
  int64_t row;
  int64_t lrow;
  int lt;
  bool live;
};
// Workgroups hold several rows only when tpr is 16, 32, 64 or 128 (a power of two), so the row
// within the workgroup is a shift (tpr is a kernel argument: the shift amount is scalar work).
__device__ __forceinline__ RowPos row_pos(int64_t num_rows, int tpr) {
  RowPos p;
  if ((int)blockDim.x == tpr) {
    p.row = blockIdx.x;
    p.lt = threadIdx.x;
  } else {
    const int sh = 31 - __builtin_clz((unsigned)tpr);
    p.row = ((int64_t)blockIdx.x << (31 - __builtin_clz(blockDim.x >> sh))) + (threadIdx.x >> sh);
    p.lt = threadIdx.x & (tpr - 1);
  }
  p.live = p.row < num_rows;
  p.lrow = p.live ? p.row : num_rows - 1;
  return p;
}

// Position of this thread when its workgroup holds exactly one row (tpr == blockDim.x, the grid
// one workgroup per row): the row index is uniform, so row base addresses are scalar.
__device__ __forceinline__ RowPos row_pos_one() {
  RowPos p;
  p.row = blockIdx.x;
  p.lrow = p.row;
  p.lt = threadIdx.x;
  p.live = true;
  return p;
}

// Element j of a row that starts at element `row` of tensor t.  In the exact-row form of a kernel
// (EX: the workgroup holds one row, so `row` is uniform) a row pointer plus a 32-bit offset (j <
// hidden, an int), which keeps the row base in scalar registers and lets one offset serve every
// tensor; otherwise one 64-bit address per lane, as the generic form has always computed it.
template <bool EX, class T>
__device__ __forceinline__ T* row_elem(T* t, int64_t row, int64_t j) {
  if constexpr (EX) {
    return (t + row) + (uint32_t)j;
  } else {
    return t + row + j;
  }
}

// Position of the k-th of R rows that each lane handles: workgroup b covers R runs of rpb
// adjacent rows (run k = rows [(b*R + k) * rpb, +rpb)), so each load instruction of a wave reads
// rows that sit next to each other.  row_pos_of(n, tpr, 0, 1) == row_pos(n, tpr).
__device__ __forceinline__ RowPos row_pos_of(int64_t num_rows, int tpr, int k, int R) {
  RowPos p;
  if ((int)blockDim.x == tpr) {
    p.row = (int64_t)blockIdx.x * R + k;
    p.lt = threadIdx.x;
  } else {
    const int sh = 31 - __builtin_clz((unsigned)tpr);
    const int lg_rpb = 31 - __builtin_clz(blockDim.x >> sh);
    p.row = (((int64_t)blockIdx.x * R + k) << lg_rpb) + (threadIdx.x >> sh);
    p.lt = threadIdx.x & (tpr - 1);
  }
  p.live = p.row < num_rows;
  p.lrow = p.live ? p.row : num_rows - 1;
  return p;
}

// Vector index of a lane's v-th vector, and the index its loads use (0 when past the row end,
// so the load stays inside the row and is discarded).
__device__ __forceinline__ int vec_index(int v, int tpr, int lt) { return v * tpr + lt; }
__device__ __forceinline__ int load_index(int j, int nvec) { return j < nvec ? j : 0; }

// Largest lanes-per-row a kernel with NV vectors of VEC elements per lane is compiled for:
// 1024 keeps at most 128 VGPRs per lane, which rows of 4 or 8 16-byte vectors per lane exceed,
// so those are compiled for 512 lanes (256 VGPRs).
__host__ __device__ constexpr int max_tpr(int vec, int nv) { return (vec > 1 && nv >= 4) ? 512 : 1024; }

}  // namespace mcop

// ---------------------------------------------------------------------------------------------
// Host side: launch geometry and error reporting shared by the entry points.
namespace mcop {

struct Geometry {
  int vec;     // elements per vector (1 = scalar path)
  int nv;      // vectors per lane
  int tpr;     // lanes per row (16, 32 or a multiple of 64, <= 1024)
  int rpb;     // rows per workgroup
  int64_t blocks;
};

// The kernel instantiation used for a given number of vectors per lane (for occupancy queries).
using KernelOfNv = const void* (*)(int nv);

// Picks the launch shape of a row kernel. `vec` is 1 or the 16-byte vector width.  Returns false,
// with the message set (mcop_last_error), when the row does not fit the register-resident
// kernels or the rows need more workgroups than one launch allows.  Rows of at
// most 32 lanes may take 16 or 32 lanes (several rows per wave) unless `min_tpr` is 64.
// `wide_nv4`: take four vectors per lane as soon as the row fills a 4-wave workgroup with them
// (the default; the per-token norm-quant kernel measured faster at two for 8192-wide rows).
bool choose_geometry(const char* op, int64_t rows, int64_t hidden, int vec, KernelOfNv kernels,
                     Geometry* g, int min_tpr = 16, bool wide_nv4 = true);

// True when a row of `hidden` elements fits the register-resident kernels at vector width `vec`:
// some vectors-per-lane candidate holds it within its lanes-per-row limit, and that candidate's
// kernel compiled without spilling registers.  Other rows take the operator's multi-pass kernel.
bool row_fits(int64_t hidden, int vec, KernelOfNv kernels, int min_tpr = 16);

// True when the exact-row (EX) instantiation `ex_kernel` may replace the generic one the launch
// shape was chosen for: it compiled without spilling registers.  Otherwise the launch keeps the
// generic form, which choose_geometry has already checked.
bool exact_form_ok(const void* ex_kernel);

// Whether rows too wide for the register-resident kernels may take a split-row kernel (rows
// shared by several workgroups, split_row.h): on unless the calling thread switched it off with
// mcop_debug_set_split_rows (then they take the multi-pass kernels, as graph captures do).
bool split_rows_enabled();

// Launch check of the multi-pass kernels for rows too wide for the register-resident ones
// (one 1024-lane workgroup per row): false, with the message set, beyond 2^31 - 1 rows.
bool wide_rows_ok(const char* op, int64_t rows);
constexpr int kWideLanes = 1024;

// True when every non-null pointer is aligned to `bytes`.
bool aligned(int bytes, const void* p0, const void* p1 = nullptr, const void* p2 = nullptr,
             const void* p3 = nullptr, const void* p4 = nullptr, const void* p5 = nullptr);

int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

}  // namespace mcop
