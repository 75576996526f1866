// rms_norm_smooth_quant_bf16.hip -- bf16 input instantiations of the SmoothQuant row kernel
// (smooth_quant_kernel.h).
#include "smooth_quant_kernel.h"

namespace mcop {

int dispatch_smooth_bf16(const Args& a, mcop_dtype wdt, mcop_dtype sdt, bool fp8, hipStream_t st) {
  return dispatch_ws<BF16>(a, wdt, sdt, MCOP_BF16, fp8, st);
}

}  // namespace mcop
