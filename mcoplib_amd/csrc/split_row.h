// split_row.h -- rows split over several workgroups: the device-side exchange of per-row
// partial results between the workgroups that share a row, and the host-side plan of such a
// launch.
//
// A row too wide for one workgroup's registers is cut into S slices of at most nv * kSplitLanes
// 16-byte vectors; S consecutive workgroups (a "group") hold one slice each in registers, so the
// row is read from HBM once, as in the register-resident kernels.  Workgroup b takes slice b % S
// of row b / S of the launch's rows.  Where the one-workgroup kernels reduce across the row's
// waves through LDS, the group reduces across its workgroups through a small device workspace:
//   - each workgroup reduces its slice (row_reduce) and publishes the result in tagged 64-bit
//     words: the high half carries a tag, the low half 32 data bits; an fp64 partial takes two
//     words.  Each word is written and read with one relaxed atomic access at agent scope
//     (coherent across the XCDs' L2 caches), so a reader that sees the tag also sees the data in
//     the same word, and no fence or cache write-back is needed;
//   - one wave per workgroup polls the S words of its row until every tag is set, then combines
//     them in slice order (so every workgroup of the row, and every launch shape, gets the same
//     bits) and shares the result through LDS;
//   - every row has its own slots, and the workspace is zeroed before each launch, so stale
//     words never carry a tag; a launch covers at most as many rows as the workspace has slots
//     for (kSplitWsWords), longer calls take several launches;
//   - progress needs no co-residency of the grid: workgroups are dispatched in index order, so
//     every workgroup of the lowest unfinished row has been dispatched, and a row's workgroups
//     wait only for each other -- at most S - 1 waiting workgroups per launch hold resources
//     (also with other kernels on the device);
//   - every wait is bounded by the wall clock all the same: a wait that exceeds it sets the
//     workspace's error word, and every later wait of the launch returns at once, so the grid
//     always drains.  A row whose exchange failed this way gets NaN for the exchanged sum or
//     maximum, so its scale (or, for the norms, its output) is NaN: the failure is visible in
//     the results instead of leaving partial sums in them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/mcop_norm.h"
#include "rowkern.h"

namespace mcop {

// Slices are held by workgroups of at most 256 lanes by default (four waves: the resident
// workgroups of a CU then fill its wave slots in steps of four), four or eight 16-byte vectors
// a lane.
constexpr int kSplitLanes = 256;
// Most slices per row (one polling lane each).
constexpr int kSplitMaxSlices = 64;

// Workspace layout (64-bit words): for the launch's row r, phase f (0: the sum of squares, 1:
// the absmax), slice s, word k: index ((r * 2 + f) * S + s) * 2 + k; the last word is the error
// flag.  kSplitWsWords bounds a launch's workspace (2 MiB; the rows of one launch follow).
constexpr int64_t kSplitWsWords = (int64_t)1 << 18;
constexpr uint32_t kSplitTag = 1;

__host__ __device__ constexpr int64_t split_ws_words(int64_t rows, int slices) {
  return rows * 2 * slices * 2 + 1;
}

__device__ __forceinline__ uint64_t* split_slots(uint64_t* ws, int64_t row, int slices,
                                                 int phase) {
  return ws + ((row * 2 + phase) * slices) * 2;
}

__device__ __forceinline__ void ws_put(uint64_t* p, uint32_t tag, uint32_t data) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | data, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ws_get(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 of the workgroup: waits until the `words` tagged words of each of the group's S slices
// (at slots[s * 2 + k], k < words) carry `tag`; lane s < S returns its slice's words in w0, w1.
// False when the wait timed out or another wait of the launch did before (error word set): the
// error word is read with every poll of the slots and decides first, so once it is set every
// later exchange of the launch fails, also one whose slots are complete.
__device__ __forceinline__ bool split_wait(const uint64_t* slots, int slices, int words,
                                           uint32_t tag, uint64_t* err, int64_t timeout_ticks,
                                           uint64_t* w0, uint64_t* w1) {
  const int lane = (int)threadIdx.x & 63;
  const int64_t t0 = wall_clock64();
  while (true) {
    bool ok = true;
    if (lane < slices) {
      *w0 = ws_get(slots + lane * 2);
      *w1 = words > 1 ? ws_get(slots + lane * 2 + 1) : ((uint64_t)tag << 32);
    }
    const uint64_t e = ws_get(err);  // requested with the slot words, not after them
    if (lane < slices) ok = (uint32_t)(*w0 >> 32) == tag && (uint32_t)(*w1 >> 32) == tag;
    if (e != 0) return false;
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
    if (wall_clock64() - t0 > timeout_ticks) {
      if (lane == 0) ws_put(err, 1, 1);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Wave 0, after split_wait of a two-word fp64 exchange: the sum of the S slices' partials (lane
// s holds slice s's low word in w0, its high word in w1), in slice order.
__device__ __forceinline__ double slice_sum(uint64_t w0, uint64_t w1, int slices) {
  const uint32_t lo = (uint32_t)w0, hi = (uint32_t)w1;
  double total = 0.0;
  for (int s = 0; s < slices; ++s) {
    const uint64_t b = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)hi, s) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)lo, s);
    total += __builtin_bit_cast(double, b);
  }
  return total;
}

// The group's sum of the slices' fp64 partials, in slice order; `part` is this workgroup's
// partial (uniform), `sl` its slice.  Every thread of the workgroup calls it.  After a failed
// wait the sum is NaN and *lds_fail (when given) is 1, else 0; the same holds for the maxima of
// split_max, split_sum_max and split_max2 below.
__device__ __forceinline__ double split_sum(uint64_t* slots, int slices, int sl, uint32_t tag,
                                            double part, uint64_t* err, int64_t timeout_ticks,
                                            double* lds, int* lds_fail) {
  if (threadIdx.x == 0) {
    const uint64_t b = __builtin_bit_cast(uint64_t, part);
    ws_put(slots + sl * 2, tag, (uint32_t)b);
    ws_put(slots + sl * 2 + 1, tag, (uint32_t)(b >> 32));
  }
  if (threadIdx.x < 64) {
    uint64_t w0 = 0, w1 = 0;
    const bool ok = split_wait(slots, slices, 2, tag, err, timeout_ticks, &w0, &w1);
    const double total = ok ? slice_sum(w0, w1, slices) : __builtin_nan("");
    if (threadIdx.x == 0) {
      *lds = total;
      if (lds_fail != nullptr) *lds_fail = ok ? 0 : 1;
    }
  }
  __syncthreads();
  return *lds;
}

// The group's largest of the slices' (non-negative or NaN-free) fp32 maxima.
__device__ __forceinline__ float split_max(uint64_t* slots, int slices, int sl, uint32_t tag,
                                           float part, uint64_t* err, int64_t timeout_ticks,
                                           float* lds, int* lds_fail) {
  if (threadIdx.x == 0) ws_put(slots + sl * 2, tag, __builtin_bit_cast(uint32_t, part));
  if (threadIdx.x < 64) {
    uint64_t w0 = 0, w1 = 0;
    const bool ok = split_wait(slots, slices, 1, tag, err, timeout_ticks, &w0, &w1);
    float m = (int)(threadIdx.x & 63) < slices ? __builtin_bit_cast(float, (uint32_t)w0) : 0.0f;
    m = wave_reduce(m, MaxOp());
    if (threadIdx.x == 0) {
      *lds = ok ? m : __builtin_nanf("");
      if (lds_fail != nullptr) *lds_fail = ok ? 0 : 1;
    }
  }
  __syncthreads();
  return *lds;
}

// The group's fp64 sum (in slice order) and fp32 maximum of the slices' partials, in one round:
// both are published before either wait (the sum in the phase-0 slots, the maximum in the
// phase-1 slots).  lds holds one double and one float.
__device__ __forceinline__ void split_sum_max(uint64_t* ws, int64_t row, int slices, int sl,
                                              uint32_t tag, double* sum, float* mx,
                                              uint64_t* err, int64_t timeout_ticks,
                                              double* lds_sum, float* lds_max, int* lds_fail) {
  uint64_t* s0 = split_slots(ws, row, slices, 0);
  uint64_t* s1 = split_slots(ws, row, slices, 1);
  if (threadIdx.x == 0) {
    const uint64_t b = __builtin_bit_cast(uint64_t, *sum);
    ws_put(s0 + sl * 2, tag, (uint32_t)b);
    ws_put(s0 + sl * 2 + 1, tag, (uint32_t)(b >> 32));
    ws_put(s1 + sl * 2, tag, __builtin_bit_cast(uint32_t, *mx));
  }
  if (threadIdx.x < 64) {
    uint64_t w0 = 0, w1 = 0, m0 = 0, m1 = 0;
    bool ok = split_wait(s0, slices, 2, tag, err, timeout_ticks, &w0, &w1);
    ok = split_wait(s1, slices, 1, tag, err, timeout_ticks, &m0, &m1) && ok;
    const double total = ok ? slice_sum(w0, w1, slices) : __builtin_nan("");
    float m = (int)(threadIdx.x & 63) < slices ? __builtin_bit_cast(float, (uint32_t)m0) : 0.0f;
    m = wave_reduce(m, MaxOp());
    if (threadIdx.x == 0) {
      *lds_sum = total;
      *lds_max = ok ? m : __builtin_nanf("");
      *lds_fail = ok ? 0 : 1;
    }
  }
  __syncthreads();
  *sum = *lds_sum;
  *mx = *lds_max;
}

// The group's largest of the slices' pairs of fp32 maxima (a, b), in one exchange: phase-0 slots,
// one word each.  lds holds two floats.
__device__ __forceinline__ void split_max2(uint64_t* slots, int slices, int sl, uint32_t tag,
                                           float* a, float* b, uint64_t* err,
                                           int64_t timeout_ticks, float* lds, int* lds_fail) {
  if (threadIdx.x == 0) {
    ws_put(slots + sl * 2, tag, __builtin_bit_cast(uint32_t, *a));
    ws_put(slots + sl * 2 + 1, tag, __builtin_bit_cast(uint32_t, *b));
  }
  if (threadIdx.x < 64) {
    uint64_t w0 = 0, w1 = 0;
    const bool ok = split_wait(slots, slices, 2, tag, err, timeout_ticks, &w0, &w1);
    const bool mine = (int)(threadIdx.x & 63) < slices;
    float ma = mine ? __builtin_bit_cast(float, (uint32_t)w0) : -__builtin_inff();
    float mb = mine ? __builtin_bit_cast(float, (uint32_t)w1) : -__builtin_inff();
    ma = wave_reduce(ma, MaxOp());
    mb = wave_reduce(mb, MaxOp());
    if (threadIdx.x == 0) {
      lds[0] = ok ? ma : __builtin_nanf("");
      lds[1] = ok ? mb : __builtin_nanf("");
      *lds_fail = ok ? 0 : 1;
    }
  }
  __syncthreads();
  *a = lds[0];
  *b = lds[1];
}

// The row reductions of a split-row kernel: the workgroup's waves through LDS (row_reduce),
// then the row's workgroups through the workspace (split_sum, split_max).
struct SplitRowReduce {
  double* red_sum;
  float* red_max;
  int tpr;
  uint64_t* ws;
  int64_t row;
  int slices;
  int sl;
  uint64_t* err;
  int64_t timeout_ticks;
  double* x_sum;
  float* x_max;
  int* x_fail = nullptr;  // LDS: 1 after an exchange that failed (nullptr: not recorded)
  __device__ __forceinline__ double sum(double v) {
    v = row_reduce<true>(v, red_sum, tpr, SumOp());
    return split_sum(split_slots(ws, row, slices, 0), slices, sl, kSplitTag, v, err,
                     timeout_ticks, x_sum, x_fail);
  }
  __device__ __forceinline__ float max(float v) {
    v = row_reduce<true>(v, red_max, tpr, MaxOp());
    return split_max(split_slots(ws, row, slices, 1), slices, sl, kSplitTag, v, err,
                     timeout_ticks, x_max, x_fail);
  }
  // After the row's last exchange, in every thread: whether it failed (then every later
  // exchange of the launch failed too; the kernel writes NaN scales for the row).
  __device__ __forceinline__ bool failed() const { return x_fail != nullptr && *x_fail != 0; }
};

// Zeroes the n words of a launch's workspace and writes `last` into its last word (the error
// word: 0, or nonzero to fail every wait of the launch at once, a test hook's forced failure).
__global__ void k_fill_u64(uint64_t* __restrict__ p, int64_t n, uint64_t last);

// Host side -------------------------------------------------------------------------------------

// The launches of a split-row kernel: S slices of `slice_vecs` vectors (the last may be
// shorter) over `lanes` lanes each, at most `chunk_rows` rows (chunk_rows * S workgroups) per
// launch, a workspace of `ws_words` words.
struct SplitPlan {
  const void* kernel;
  int nv;
  int slices;
  int slice_vecs;
  int lanes;
  int64_t chunk_rows;
  int64_t ws_words;
  int64_t timeout_ticks;
};

// A split-row kernel instantiation, the vectors a lane it holds, its most lanes per workgroup
// (at most its launch bound) and the multiple of vectors every slice but the last holds (slices
// start on it: whole quantization groups).
struct SplitKernel {
  const void* fn;
  int nv;
  int lanes = kSplitLanes;
  int align = 1;
};

// Plans the split-row launches (one slice per workgroup) for `rows` rows of `nvec` vectors, over
// the candidate kernels `cands`: the one that keeps the most row vectors resident per CU (its workgroups per CU x lanes x nv, from its register use; the
// workgroup's lifetime is mostly the exchanges' latency, so bytes resident set the bandwidth),
// the earlier on a tie.  False (no message set) when none applies (the row fits fewer than two
// slices or needs more than kSplitMaxSlices, the kernel spills, or the stream is being captured
// into a graph), in which case the caller runs its multi-pass kernel instead.
bool split_plan(const SplitKernel* cands, int ncand, int64_t rows, int64_t nvec, hipStream_t st,
                SplitPlan* p);

// Zeroes the launch's workspace (`rows` rows of the plan) with a fill kernel and launches the
// plan's kernel with `args` (its parameter list, as hipLaunchKernel takes it) over rows * S
// workgroups; `static_ws` (the no-allocation scratch) only changes the trace line.
int split_launch(const char* op, void** args, const SplitPlan& p, int64_t rows, uint64_t* ws,
                 bool static_ws, hipStream_t st);

// Runs a split-row kernel (the planned one of `cands`) over `rows` rows of `nvec` vectors: plans it, takes its workspace
// (`scratch`, the no-allocation entry point's array, or else the stream-ordered allocator,
// released on the same stream after the launches), and launches it over chunks of at most
// plan.chunk_rows rows.  For each chunk, launch_chunk(r0, n, ws, plan, launch) builds the
// kernel's parameter list for rows [r0, r0 + n) and returns launch(args).  MCOP_E_UNSUPPORTED
// (no message) when the split does not apply: the caller runs its multi-pass kernel.
template <class LaunchChunk>
int split_run(const char* op, std::initializer_list<SplitKernel> cands, int64_t rows,
              int64_t nvec, uint64_t* scratch, hipStream_t st, LaunchChunk&& launch_chunk) {
  SplitPlan p;
  if (!split_plan(cands.begin(), (int)cands.size(), rows, nvec, st, &p)) {
    return MCOP_E_UNSUPPORTED;
  }
  uint64_t* ws = scratch;
  if (scratch != nullptr && p.ws_words > kSplitWsWords) {  // launches are sized to fit it
    return set_error(MCOP_E_UNSUPPORTED, "%s: a launch needs %lld workspace words, more than "
                     "the %lld of the no-allocation scratch", op, (long long)p.ws_words,
                     (long long)kSplitWsWords);
  }
  if (scratch == nullptr &&
      hipMallocAsync(reinterpret_cast<void**>(&ws), (size_t)p.ws_words * 8, st) != hipSuccess) {
    (void)hipGetLastError();
    return MCOP_E_UNSUPPORTED;
  }
  int rc = MCOP_OK;
  for (int64_t r0 = 0; r0 < rows && rc == MCOP_OK; r0 += p.chunk_rows) {
    const int64_t n = rows - r0 < p.chunk_rows ? rows - r0 : p.chunk_rows;
    rc = launch_chunk(r0, n, ws, p, [&](void** args) {
      return split_launch(op, args, p, n, ws, scratch != nullptr, st);
    });
  }
  if (scratch == nullptr && hipFreeAsync(ws, st) != hipSuccess) {
    (void)hipGetLastError();
    return rc != MCOP_OK ? rc : set_error(MCOP_E_LAUNCH, "%s: hipFreeAsync failed", op);
  }
  return rc;
}

}  // namespace mcop
