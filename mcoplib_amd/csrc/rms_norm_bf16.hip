// rms_norm_bf16.hip -- bf16 input instantiations of the RMSNorm row kernel (norm_kernel.h).
#include "norm_kernel.h"

namespace mcop {

int norm_dispatch_bf16(const char* name, const NormArgs& a, mcop_dtype wdt, hipStream_t st) {
  return norm_dispatch_w<BF16>(name, a, wdt, st);
}

}  // namespace mcop
