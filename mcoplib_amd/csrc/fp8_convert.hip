// fp8_convert.hip -- the clamp-and-convert step of the fp8 epilogues as a standalone entry
// point, so the hardware conversion (v_cvt_pk_fp8_f32) can be checked bit for bit against the
// OCP fp8-e4m3fn definition over any set of fp32 inputs.
#include <hip/hip_runtime.h>

#include "../../include/mcop_norm.h"
#include "mcop_testing.h"
#include "rowkern.h"

namespace mcop {

__global__ void __launch_bounds__(256)
k_fp8_from_f32(uint8_t* __restrict__ out, const float* __restrict__ in, int64_t n, float mul) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float c = clamp_fp8(in[i] * mul);
    out[i] = cvt_fp8<1>(&c).v[0];
  }
}

}  // namespace mcop

extern "C" int mcop_fp8_e4m3fn_from_f32(uint8_t* out, const float* in, int64_t n, float mul,
                                        void* stream) {
  using namespace mcop;
  if (n < 0) return set_error(MCOP_E_INVALID, "fp8_e4m3fn_from_f32: n=%lld", (long long)n);
  if (n == 0) return MCOP_OK;
  if (!out || !in) return set_error(MCOP_E_INVALID, "fp8_e4m3fn_from_f32: null pointer");
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_fp8_from_f32, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, in, n, mul);
  return check_launch("fp8_e4m3fn_from_f32");
}
