// abi.hip -- host-side pieces shared by every entry point of libmcop_norm.so: error state,
// launch geometry, the (debug) launch-shape override.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "../../include/mcop_norm.h"
#include "mcop_testing.h"
#include "rowkern.h"
#include "split_row.h"

namespace mcop {

namespace {
thread_local char g_err[512] = "";
// launch-shape override of the calling thread (mcop_debug_set_launch_override)
thread_local int g_over_nv = 0;
thread_local int g_over_tpr = 0;
// split-row kernels switched off for the calling thread (mcop_debug_set_split_rows)
thread_local int g_no_split = 0;
// split-row launches of the calling thread start with their error word set, so every exchange
// fails at once (mcop_debug_fail_split_waits)
thread_local int g_fail_split_waits = 0;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t round64(int64_t a) { return ceil_div(a, 64) * 64; }
}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(MCOP_E_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return MCOP_OK;
}

bool aligned(int bytes, const void* p0, const void* p1, const void* p2, const void* p3,
             const void* p4, const void* p5) {
  const void* ps[6] = {p0, p1, p2, p3, p4, p5};
  for (const void* p : ps) {
    if (p != nullptr && (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) != 0) return false;
  }
  return true;
}

namespace {
// MCOP_DEBUG_TRACE=1|ON prints every launch decision to stdout (the reference's env switch of
// the same name prints every operator's arguments).
bool trace_enabled() {
  static const bool on = [] {
    const char* v = getenv("MCOP_DEBUG_TRACE");
    return v != nullptr && (strcmp(v, "1") == 0 || strcmp(v, "ON") == 0 || strcmp(v, "on") == 0);
  }();
  return on;
}

// Attributes of one kernel (hipFuncGetAttributes, cached; the answer depends only on the code
// object).  `spills`: the kernel keeps registers in private (scratch) memory, whose per-lane
// traffic would compete with the streamed rows.
struct KernelInfo {
  bool ok;
  bool spills;
};
KernelInfo kernel_info(const void* kernel) {
  static std::mutex mu;
  static std::unordered_map<const void*, KernelInfo> cache;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(kernel);
    if (it != cache.end()) return it->second;
  }
  KernelInfo k{false, false};
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, kernel) != hipSuccess) {
    (void)hipGetLastError();
    return k;  // not cached: no device yet, or a transient failure
  }
  k.ok = true;
  k.spills = attr.localSizeBytes > 0;
  std::lock_guard<std::mutex> lk(mu);
  cache[kernel] = k;
  return k;
}

// Resident workgroups per CU of one kernel at one workgroup size (hipOccupancy..., cached).
// Kernels that spill count as 0.
int blocks_per_cu(const void* kernel, int block) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> cache;
  const uint64_t key = (uint64_t)reinterpret_cast<uintptr_t>(kernel) * 4099u + (uint64_t)block;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int n = 0;
  const KernelInfo k = kernel_info(kernel);
  if (!k.ok || k.spills ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, 0) != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  std::lock_guard<std::mutex> lk(mu);
  cache[key] = n;
  return n;
}
}  // namespace

// Launch shape of a row kernel.  A lane holds nv vectors of each streamed tensor, a row spans
// tpr = nvec / nv lanes rounded up to whole waves (or, for rows of at most 32 lanes, to 16 or
// 32 lanes: several rows per wave), and rows narrower than 256 lanes are packed several per
// workgroup.  Rules, from measurements on MI355X (bf16 rows of 4096-16384):
//   - at most 256 rows (decode): row latency matters; the smallest nv >= 2 whose row fits
//     (1 for rows of at most 64 vectors);
//   - otherwise nv = 4 when the row fills a 4-wave workgroup with it (bf16 rows of >= 8192:
//     fewer waves per row share the per-row work of the reductions and scale computations;
//     2-35% faster than nv = 2, most for the kernels with the heaviest per-row work); else
//     nv = 2 when its workgroups have at most 512 lanes and fill the CU (32 resident waves,
//     from the kernel's occupancy); else nv = 4 (e.g. 7-wave workgroups leave a third of the
//     wave slots empty); 8 or 16 only for rows that do not fit otherwise.  Kernels that spill
//     registers are skipped while another shape fits.
// Scalar path (hidden not a multiple of the vector width, or misaligned pointers): nv in {4,16}.
// Lanes per row for n lanes of work: whole waves, or 16 / 32 lanes when the row is that short.
static int64_t row_lanes(int64_t n, int min_tpr) {
  if (n <= 32 && min_tpr <= 32) return n <= 16 && min_tpr <= 16 ? 16 : 32;
  return round64(n);
}

static bool valid_tpr(int64_t t, int min_tpr) {
  return (t >= min_tpr && (t == 16 || t == 32)) || (t > 0 && t % 64 == 0);
}

bool row_fits(int64_t hidden, int vec, KernelOfNv kernels, int min_tpr) {
  static const int kVecNv[] = {1, 2, 4, 8, 16};
  static const int kScalarNv[] = {4, 16};
  const int64_t nvec = hidden / vec;
  const int* cands = vec > 1 ? kVecNv : kScalarNv;
  const int ncand = vec > 1 ? 5 : 2;
  for (int c = 0; c < ncand; ++c) {
    if (row_lanes(ceil_div(nvec, cands[c]), min_tpr) > max_tpr(vec, cands[c])) continue;
    if (!kernel_info(kernels(cands[c])).spills) return true;
  }
  return false;
}

bool split_rows_enabled() { return g_no_split == 0; }

bool exact_form_ok(const void* ex_kernel) {
  const KernelInfo k = kernel_info(ex_kernel);
  if (k.ok && !k.spills) return true;
  if (trace_enabled()) {
    fprintf(stdout, "[mcop]   exact-row form %s: generic form\n",
            k.ok ? "spills registers" : "has no attributes");
    fflush(stdout);
  }
  return false;
}

__global__ void __launch_bounds__(256) k_fill_u64(uint64_t* __restrict__ p, int64_t n,
                                                   uint64_t last) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = i == n - 1 ? last : 0;
}

namespace {
// The wall clock's rate of a device in kHz (cached), for the split-row kernels' wait bound.
int wall_clock_khz(int dev) {
  static std::mutex mu;
  static int cache[64];
  if (dev < 0 || dev >= 64) return 0;
  {
    std::lock_guard<std::mutex> lk(mu);
    if (cache[dev] > 0) return cache[dev];
  }
  int clk = 0;
  if (hipDeviceGetAttribute(&clk, hipDeviceAttributeWallClockRate, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lk(mu);
  cache[dev] = clk;
  return clk;
}
}  // namespace

bool split_plan(const SplitKernel* cands, int ncand, int64_t rows, int64_t nvec, hipStream_t st,
                SplitPlan* p) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (cs != hipStreamCaptureStatusNone) return false;  // graphs take the multi-pass kernel
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const int clk = wall_clock_khz(dev);
  if (clk <= 0) return false;
  int64_t best = 0;
  for (int c = 0; c < ncand; ++c) {
    const int nv = cands[c].nv;
    const int64_t align = std::max(cands[c].align, 1);
    // nv * lanes is a multiple of align (both powers of two), so the rounded slice still fits
    const int64_t slice_vecs =
        ceil_div(ceil_div(nvec, ceil_div(nvec, (int64_t)nv * cands[c].lanes)), align) * align;
    const int64_t slices = ceil_div(nvec, slice_vecs);
    if (slices < 2 || slices > kSplitMaxSlices) continue;
    const int64_t lanes = round64(ceil_div(slice_vecs, nv));
    const int64_t resident = blocks_per_cu(cands[c].fn, (int)lanes) * lanes * nv;
    if (resident <= best) continue;  // spills (or cannot launch), or keeps less resident
    best = resident;
    p->kernel = cands[c].fn;
    p->nv = nv;
    p->slices = (int)slices;
    p->slice_vecs = (int)slice_vecs;
    p->lanes = (int)lanes;
  }
  if (best == 0) return false;
  p->chunk_rows = std::min<int64_t>(rows, (kSplitWsWords - 1) / (4 * p->slices));
  p->ws_words = split_ws_words(p->chunk_rows, p->slices);
  // 2 s of the wall clock: the dispatch order already guarantees progress (split_row.h), so the
  // bound only ends waits stalled from outside (the queue preempted for that long)
  p->timeout_ticks = (int64_t)clk * 2000;
  return true;
}

int split_launch(const char* op, void** args, const SplitPlan& p, int64_t rows, uint64_t* ws,
                 bool static_ws, hipStream_t st) {
  const int64_t words = split_ws_words(rows, p.slices);
  hipLaunchKernelGGL(k_fill_u64, dim3((unsigned)ceil_div(words, 256)), dim3(256), 0, st, ws,
                     words, (uint64_t)(g_fail_split_waits ? 1 : 0));
  if (int rc = check_launch(op)) return rc;
  const hipError_t e = hipLaunchKernel(p.kernel, dim3((unsigned)(rows * p.slices)),
                                       dim3((unsigned)p.lanes), args, 0, st);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return set_error(MCOP_E_LAUNCH, "%s: kernel launch failed: %s", op, hipGetErrorString(e));
  }
  if (trace_enabled()) {
    fprintf(stdout, "[mcop] %s rows=%lld: split-row kernel, %d slices of %d vectors over %d "
            "lanes, workspace %s\n", op, (long long)rows, p.slices, p.slice_vecs, p.lanes,
            static_ws ? "in the no-allocation scratch" : "from the stream-ordered allocator");
    fflush(stdout);
  }
  return MCOP_OK;
}

bool wide_rows_ok(const char* op, int64_t rows) {
  if (rows > 0x7fffffffLL) {
    set_error(MCOP_E_UNSUPPORTED, "%s: %lld rows need more than the 2147483647 workgroups one "
              "launch allows", op, (long long)rows);
    return false;
  }
  if (trace_enabled()) {
    fprintf(stdout, "[mcop] %s rows=%lld: multi-pass kernel, one %d-lane workgroup per row\n",
            op, (long long)rows, kWideLanes);
    fflush(stdout);
  }
  return true;
}

bool choose_geometry(const char* op, int64_t rows, int64_t hidden, int vec, KernelOfNv kernels,
                     Geometry* g, int min_tpr, bool wide_nv4) {
  const int64_t nvec = hidden / vec;
  int nv = 0;
  int64_t tpr = 0;
  const int onv = g_over_nv;
  const int otpr = g_over_tpr;
  const bool nv_allowed = vec > 1 ? (onv == 1 || onv == 2 || onv == 4 || onv == 8 || onv == 16)
                                  : (onv == 4 || onv == 16);
  if (nv_allowed) {
    const int64_t t = otpr > 0 ? otpr : row_lanes(ceil_div(nvec, onv), min_tpr);
    if (valid_tpr(t, min_tpr) && t <= max_tpr(vec, onv) && (int64_t)onv * t >= nvec) {
      nv = onv;
      tpr = t;
    }
  }
  if (nv == 0) {
    static const int kVecNv[] = {1, 2, 4, 8, 16};
    static const int kScalarNv[] = {4, 16};
    const int* cands = vec > 1 ? kVecNv : kScalarNv;
    const int ncand = vec > 1 ? 5 : 2;
    const bool latency = rows <= 256;
    int fallback_nv = 0;
    int64_t fallback_tpr = 0;
    for (int c = 0; c < ncand && nv == 0; ++c) {
      const int cand = cands[c];
      const int64_t t = row_lanes(ceil_div(nvec, cand), min_tpr);
      if (t > max_tpr(vec, cand)) continue;
      if (vec > 1 && cand == 1 && nvec > 64) continue;
      if (kernel_info(kernels(cand)).spills) continue;
      if (fallback_nv == 0) {
        fallback_nv = cand;
        fallback_tpr = t;
      }
      if (latency || (vec > 1 && cand == 1)) {
        nv = cand;
        tpr = t;
        break;
      }
      const int rpb = t < 256 ? (int)(256 / t) : 1;
      const int block = (int)t * rpb;
      const int nb = blocks_per_cu(kernels(cand), block);
      const int waves = nb * block / 64;
      if (trace_enabled()) {
        fprintf(stdout, "[mcop]   %s candidate nv=%d tpr=%lld wg=%d resident_wgs/CU=%d\n", op,
                cand, (long long)t, block, nb);
      }
      if (nb == 0) continue;  // spills (or cannot launch at this size)
      // two vectors per lane only for rows that would not fill a 4-wave workgroup at four
      if (vec > 1 && cand == 2 &&
          (t > 512 || waves < 32 ||
           (wide_nv4 && row_lanes(ceil_div(nvec, 4), min_tpr) >= 256))) {
        continue;
      }
      nv = cand;
      tpr = t;
    }
    if (nv == 0) {
      nv = fallback_nv;
      tpr = fallback_tpr;
    }
  }
  if (nv == 0) {
    set_error(MCOP_E_UNSUPPORTED,
              "%s: hidden_size %lld is larger than the register-resident kernels support",
              op, (long long)hidden);
    return false;
  }
  g->vec = vec;
  g->nv = nv;
  g->tpr = (int)tpr;
  g->rpb = tpr < 256 ? (int)(256 / tpr) : 1;
  g->blocks = ceil_div(rows, g->rpb);
  if (g->blocks > 0x7fffffffLL) {  // a launch's grid holds at most 2^31 - 1 workgroups
    set_error(MCOP_E_UNSUPPORTED,
              "%s: %lld rows need %lld workgroups, more than the 2147483647 one launch allows",
              op, (long long)rows, (long long)g->blocks);
    return false;
  }
  if (trace_enabled()) {
    fprintf(stdout, "[mcop] %s rows=%lld hidden=%lld vec=%d nv=%d tpr=%d rows/wg=%d wgs=%lld\n",
            op, (long long)rows, (long long)hidden, g->vec, g->nv, g->tpr, g->rpb,
            (long long)g->blocks);
    fflush(stdout);
  }
  return true;
}

}  // namespace mcop

extern "C" {

const char* mcop_last_error(void) { return mcop::g_err; }

int mcop_abi_version(void) { return MCOP_ABI_VERSION; }

int mcop_debug_set_launch_override(int vectors_per_lane, int lanes_per_row) {
  if (vectors_per_lane < 0 || lanes_per_row < 0 || lanes_per_row > 1024 ||
      (lanes_per_row % 64 != 0 && lanes_per_row != 16 && lanes_per_row != 32)) {
    return mcop::set_error(MCOP_E_INVALID, "mcop_debug_set_launch_override: bad shape (%d, %d)",
                           vectors_per_lane, lanes_per_row);
  }
  mcop::g_over_nv = vectors_per_lane;
  mcop::g_over_tpr = lanes_per_row;
  return MCOP_OK;
}

int mcop_debug_set_split_rows(int enabled) {
  mcop::g_no_split = enabled ? 0 : 1;
  return MCOP_OK;
}

int mcop_debug_fail_split_waits(int on) {
  mcop::g_fail_split_waits = on ? 1 : 0;
  return MCOP_OK;
}

}  // extern "C"
