// rms_norm_smooth_quant_f16.hip -- f16 input instantiations of the SmoothQuant row kernel
// (smooth_quant_kernel.h).
#include "smooth_quant_kernel.h"

namespace mcop {

int dispatch_smooth_f16(const Args& a, mcop_dtype wdt, mcop_dtype sdt, bool fp8, hipStream_t st) {
  return dispatch_ws<F16>(a, wdt, sdt, MCOP_F16, fp8, st);
}

}  // namespace mcop
