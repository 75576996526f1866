// Host-side check of libmcop_norm's C ABI under AddressSanitizer and UndefinedBehaviorSanitizer.
//
// Built by this folder's Makefile from a host-only compile of every mcoplib_amd/csrc/*.hip file
// (no device code, no code objects registered), so it runs on a machine without a GPU and never
// touches one. Every entry point is called over a
// grid of shapes (empty, one row, ragged and maximal widths, row counts past the launch limit),
// dtypes, flags and pointer alignments, with device-pointer arguments that host code never
// dereferences. Each call must end in a documented status: 0 for an empty call, MCOP_E_INVALID
// or MCOP_E_UNSUPPORTED from the argument checks, or MCOP_E_LAUNCH once argument checking and
// launch-shape selection are done and the launch itself fails for want of a device; every
// failure leaves a non-empty message. With MCOP_DEBUG_TRACE=1 the launch-decision printing runs
// too. Any sanitizer report ends the run with a non-zero status.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/mcop_norm.h"
#include "../../mcoplib_amd/csrc/mcop_testing.h"

namespace {

int g_calls = 0;
int g_fail = 0;
int g_status[4] = {0, 0, 0, 0};  // counts of 0, -1, -2, -3

// Stand-ins for device buffers: distinct, 256-byte aligned addresses (plus `mis` bytes) that the
// host code only compares and passes on.
void* dev(int slot, int mis = 0) {
  return reinterpret_cast<void*>(static_cast<uintptr_t>(0x7f0000000000ull) +
                                 static_cast<uintptr_t>(slot) * 0x100000000ull +
                                 static_cast<uintptr_t>(mis));
}

void expect(int rc, const char* what, int64_t rows, int64_t hidden) {
  ++g_calls;
  const char* msg = mcop_last_error();
  const size_t len = strnlen(msg, 512);
  const bool known = rc == MCOP_OK || rc == MCOP_E_INVALID || rc == MCOP_E_UNSUPPORTED ||
                     rc == MCOP_E_LAUNCH;
  if (!known || len >= 512 || (rc != MCOP_OK && len == 0) || (rc == MCOP_OK && rows > 0)) {
    ++g_fail;
    fprintf(stderr, "unexpected: %s rows=%lld hidden=%lld rc=%d msg='%.*s'\n", what,
            (long long)rows, (long long)hidden, rc, (int)(len < 200 ? len : 200), msg);
    return;
  }
  g_status[-rc] += 1;
}

const int64_t kRows[] = {0, 1, 3, 64, 256, 257, 8192, (int64_t)1 << 31, (int64_t)1 << 36};
const int64_t kHidden[] = {0,    1,     7,     8,     16,     64,     100,    512,
                           2048, 4096,  5120,  7168,  7176,   8192,   16384,  16392,
                           32768, 65536, 65544, 131072, 131073, (int64_t)1 << 24};
const mcop_dtype kFloat[] = {MCOP_BF16, MCOP_F16, MCOP_F32};
const mcop_dtype kAll[] = {MCOP_BF16, MCOP_F16, MCOP_F32, MCOP_I8, MCOP_FP8_E4M3FN};

}  // namespace

int main() {
  for (int64_t T : kRows) {
    for (int64_t H : kHidden) {
      for (int mis : {0, 2}) {
        for (mcop_dtype in : kAll) {
          expect(mcop_fused_add_rms_norm(dev(0, mis), H + (mis ? 8 : 0), dev(1), dev(2), T, H, in,
                                         1e-6f, nullptr),
                 "fused_add_rms_norm", T, H);
          for (mcop_dtype out : kAll) {
            for (int res = 0; res < 2; ++res) {
              expect(mcop_rms_norm_dynamic_per_token_quant(
                         dev(0), out, (float*)dev(1), dev(2, mis), dev(3), res ? nullptr
                                                                               : (float*)dev(4),
                         res ? dev(5) : nullptr, T, H, in, 1e-6f, nullptr),
                     "rms_norm_dynamic_per_token_quant", T, H);
              expect(mcop_rms_norm_dynamic_per_token_quant_noalloc(
                         dev(0), out, (float*)dev(1), dev(2, mis), dev(3), res ? nullptr
                                                                               : (float*)dev(4),
                         res ? dev(5) : nullptr, T, H, in, 1e-6f, nullptr),
                     "rms_norm_dynamic_per_token_quant_noalloc", T, H);
              for (mcop_dtype wd : kFloat) {
                for (mcop_dtype sd : kFloat) {
                  expect(mcop_rms_norm_smooth_quant(
                             dev(0), out, (float*)dev(1), dev(2, mis), dev(3), wd, dev(4), sd,
                             res ? dev(5) : nullptr, res ? dev(6) : nullptr,
                             res ? dev(7) : nullptr, T, H, in, 1e-6f, (uint32_t)res, nullptr),
                         "rms_norm_smooth_quant", T, H);
                }
              }
              for (int64_t g : {(int64_t)0, (int64_t)64, (int64_t)128, (int64_t)100}) {
                expect(mcop_rms_norm_per_block_quant(dev(0), out, (float*)dev(1), dev(2, mis),
                                                     dev(3), res ? nullptr : (float*)dev(4),
                                                     res ? dev(5) : nullptr, T, H, in, 1e-6f, g,
                                                     res, nullptr),
                       "rms_norm_per_block_quant", T, H);
              }
            }
          }
          for (int azp = 0; azp < 2; ++azp) {
            expect(mcop_dynamic_scaled_int8_quant((int8_t*)dev(0), (float*)dev(1),
                                                  azp ? (int32_t*)dev(2) : nullptr, dev(3, mis),
                                                  T, H, in, nullptr),
                   "dynamic_scaled_int8_quant", T, H);
          }
          for (int64_t stride : {H, H + 8, H - 1}) {
            expect(mcop_dynamic_per_token_scaled_fp8_quant((uint8_t*)dev(0), (float*)dev(1),
                                                           dev(2, mis), nullptr, T, H, stride,
                                                           stride, in, nullptr),
                   "dynamic_per_token_scaled_fp8_quant", T, H);
          }
          expect(mcop_rms_norm_dynamic_per_token_quant_custom(
                     (int8_t*)dev(0), (float*)dev(1), dev(2, mis), dev(3), nullptr, dev(4), T, H,
                     in, 1e-6f, nullptr),
                 "rms_norm_dynamic_per_token_quant_custom", T, H);
          for (mcop_dtype wd : kFloat) {
            for (int div = 0; div < 2; ++div) {
              expect(mcop_rms_norm(dev(0), dev(1, mis), dev(2), wd, div ? dev(3) : nullptr,
                                   div ? dev(4) : nullptr, T, H, in, 1e-6f, div, nullptr),
                     "rms_norm", T, H);
            }
            for (int64_t heads : {(int64_t)1, (int64_t)8}) {
              expect(mcop_head_rms_norm(dev(0), dev(1, mis), dev(2), wd, T, heads, H,
                                        heads - 1, 1, in, 1e-6f, nullptr),
                     "head_rms_norm", T, H);
              expect(mcop_head_rms_norm(dev(0), dev(1), dev(2), wd, T, heads, H, 0, heads + 1,
                                        in, 1e-6f, nullptr),
                     "head_rms_norm (too many heads)", T, H);
            }
          }
          for (int dims = 1; dims <= 5; ++dims) {
            expect(mcop_vllm_rms_norm(dev(0), dev(1, mis), dev(2), T, H, dims, H + 8,
                                      (H + 8) * 4, (H + 8) * 16, 4, 4, in, 1e-6f, nullptr),
                   "vllm_rms_norm", T, H);
          }
        }
        expect(mcop_scale_dynamic_quant((int8_t*)dev(0), (float*)dev(1), dev(2, mis),
                                        (float*)dev(3), T, H, nullptr),
               "scale_dynamic_quant", T, H);
        for (int64_t pad : {H, H + 2, H + 64, (int64_t)0}) {
          expect(mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output(
                     (int8_t*)dev(0), dev(1), (int8_t*)dev(2), (float*)dev(3), dev(4, mis),
                     dev(5), dev(6), T, H, pad, 1e-6f, nullptr),
                 "padding_output", T, H);
        }
        expect(mcop_fp8_e4m3fn_from_f32((uint8_t*)dev(0), (float*)dev(1, mis), T * H, 1.0f,
                                        nullptr),
               "fp8_e4m3fn_from_f32", T * H, 1);
      }
    }
  }
  // null pointers on every entry point
  expect(mcop_fused_add_rms_norm(nullptr, 64, nullptr, nullptr, 4, 64, MCOP_BF16, 1e-6f, nullptr),
         "fused_add_rms_norm (null)", 4, 64);
  expect(mcop_scale_dynamic_quant(nullptr, nullptr, nullptr, nullptr, 4, 64, nullptr),
         "scale_dynamic_quant (null)", 4, 64);
  expect(mcop_fp8_e4m3fn_from_f32(nullptr, nullptr, 4, 1.0f, nullptr), "fp8 (null)", 4, 1);
  // launch-shape overrides of this thread, valid and invalid, then the automatic choice again
  const int nvs[] = {-1, 0, 1, 2, 3, 4, 8, 16, 32};
  const int tprs[] = {-64, 0, 16, 32, 48, 64, 128, 1024, 1088};
  for (int nv : nvs) {
    for (int tpr : tprs) {
      const int rc = mcop_debug_set_launch_override(nv, tpr);
      expect(rc, "debug_set_launch_override", 0, 0);
      expect(mcop_rms_norm_dynamic_per_token_quant(dev(0), MCOP_I8, (float*)dev(1), dev(2),
                                                   dev(3), nullptr, nullptr, 4096, 8192,
                                                   MCOP_BF16, 1e-6f, nullptr),
             "rms_norm_dynamic_per_token_quant (override)", 4096, 8192);
    }
  }
  mcop_debug_set_launch_override(0, 0);
  printf("calls %d: ok %d, invalid %d, unsupported %d, launch %d; unexpected %d; abi %d\n",
         g_calls, g_status[0], g_status[1], g_status[2], g_status[3], g_fail,
         mcop_abi_version());
  return g_fail == 0 ? 0 : 1;
}
