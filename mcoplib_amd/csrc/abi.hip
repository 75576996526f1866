// abi.hip -- host-side pieces shared by every entry point of libmcop_norm.so: error state,
// launch geometry, the launch-shape override.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "../../include/mcop_norm.h"
#include "rowkern.h"

namespace mcop {

namespace {
thread_local char g_err[512] = "";
std::atomic<int> g_over_nv{0};
std::atomic<int> g_over_tpr{0};

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

// Vector path: vectors per lane nv in {1,2,4,8,16}; the default is two 16-byte vectors per tensor
// per lane (enough loads in flight per wave while keeping VGPR use near 64), one for rows of at
// most 64 vectors.  Scalar path (hidden not a multiple of the vector width, or misaligned
// pointers): nv in {4,16}.  Rows narrower than 256 lanes are packed several per workgroup.
bool choose_geometry(int64_t rows, int64_t hidden, int vec, Geometry* g) {
  const int64_t nvec = hidden / vec;
  int nv = 0;
  int64_t tpr = 0;
  const int onv = g_over_nv.load(std::memory_order_relaxed);
  const int otpr = g_over_tpr.load(std::memory_order_relaxed);
  const bool nv_allowed = vec > 1 ? (onv == 1 || onv == 2 || onv == 4 || onv == 8 || onv == 16)
                                  : (onv == 4 || onv == 16);
  if (nv_allowed) {
    const int64_t t = otpr > 0 ? otpr : round64(ceil_div(nvec, onv));
    if (t % 64 == 0 && t <= max_tpr(vec, onv) && (int64_t)onv * t >= nvec) {
      nv = onv;
      tpr = t;
    }
  }
  if (nv == 0) {
    if (vec > 1) {
      for (int cand : {1, 2, 4, 8, 16}) {
        if (cand == 1 && nvec > 64) continue;
        const int64_t t = round64(ceil_div(nvec, cand));
        if (t <= max_tpr(vec, cand)) {
          nv = cand;
          tpr = t;
          break;
        }
      }
    } else {
      for (int cand : {4, 16}) {
        const int64_t t = round64(ceil_div(nvec, cand));
        if (t <= max_tpr(vec, cand)) {
          nv = cand;
          tpr = t;
          break;
        }
      }
    }
  }
  if (nv == 0) return false;
  g->vec = vec;
  g->nv = nv;
  g->tpr = (int)tpr;
  g->rpb = tpr < 256 ? (int)(256 / tpr) : 1;
  g->blocks = ceil_div(rows, g->rpb);
  return true;
}

}  // namespace mcop

extern "C" {

const char* mcop_last_error(void) { return mcop::g_err; }

int mcop_abi_version(void) { return MCOP_ABI_VERSION; }

int mcop_set_launch_override(int vectors_per_lane, int lanes_per_row) {
  if (vectors_per_lane < 0 || lanes_per_row < 0 || lanes_per_row > 1024 ||
      lanes_per_row % 64 != 0) {
    return mcop::set_error(MCOP_E_INVALID, "mcop_set_launch_override: bad shape (%d, %d)",
                           vectors_per_lane, lanes_per_row);
  }
  mcop::g_over_nv.store(vectors_per_lane, std::memory_order_relaxed);
  mcop::g_over_tpr.store(lanes_per_row, std::memory_order_relaxed);
  return MCOP_OK;
}

}  // extern "C"
