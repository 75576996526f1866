// rms_norm_f16.hip -- fp16 input instantiations of the RMSNorm row kernel (norm_kernel.h).
#include "norm_kernel.h"

namespace mcop {

int norm_dispatch_f16(const char* name, const NormArgs& a, mcop_dtype wdt, hipStream_t st) {
  return norm_dispatch_w<F16>(name, a, wdt, st);
}

}  // namespace mcop
