// rms_norm_smooth_quant.hip -- entry point of the SmoothQuant (residual add +) RMSNorm + dynamic
// per-token quantization (mcoplib.op.rms_norm_dynamic_per_token_quant, "fused_rms_norm_dq");
// the kernel and its semantics are in smooth_quant_kernel.h.  This unit instantiates the fp32
// input kernels; the bf16 and fp16 ones are in rms_norm_smooth_quant_{bf16,f16}.hip.
#include "smooth_quant_kernel.h"

extern "C" int mcop_rms_norm_smooth_quant(void* out, mcop_dtype out_dtype, float* scales,
                                          const void* input, const void* weight,
                                          mcop_dtype weight_dtype, const void* smooth,
                                          mcop_dtype smooth_dtype, void* after_res,
                                          void* after_norm, const void* residual,
                                          int64_t num_tokens, int64_t hidden_size,
                                          mcop_dtype in_dtype, float epsilon, uint32_t flags,
                                          void* stream) {
  using namespace mcop;
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size > INT32_MAX) {
    return set_error(MCOP_E_INVALID,
                     "rms_norm_dynamic_per_token_quant (smooth): bad shape num_tokens=%lld "
                     "hidden_size=%lld",
                     (long long)num_tokens, (long long)hidden_size);
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !scales || !input || !weight || !smooth) {
    return set_error(MCOP_E_INVALID, "rms_norm_dynamic_per_token_quant (smooth): null pointer");
  }
  if (out_dtype != MCOP_I8 && out_dtype != MCOP_FP8_E4M3FN) {
    return set_error(MCOP_E_INVALID,
                     "rms_norm_dynamic_per_token_quant (smooth): out dtype %d is not int8 or "
                     "fp8_e4m3fn",
                     (int)out_dtype);
  }
  const Args a{out,       scales,    input,      weight,          smooth, after_res,
               after_norm, residual, num_tokens, (int)hidden_size, epsilon, flags};
  const bool fp8 = out_dtype == MCOP_FP8_E4M3FN;
  auto st = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case MCOP_BF16: return dispatch_smooth_bf16(a, weight_dtype, smooth_dtype, fp8, st);
    case MCOP_F16: return dispatch_smooth_f16(a, weight_dtype, smooth_dtype, fp8, st);
    case MCOP_F32:
      if (weight_dtype != MCOP_F32 || smooth_dtype != MCOP_F32) {
        return set_error(MCOP_E_INVALID,
                         "rms_norm_dynamic_per_token_quant (smooth): fp32 input needs fp32 "
                         "weight and smooth scales");
      }
      return dispatch_out<F32, F32, F32>(a, fp8, st);
    default:
      return set_error(MCOP_E_INVALID,
                       "rms_norm_dynamic_per_token_quant (smooth): input dtype %d is not "
                       "bf16/fp16/fp32",
                       (int)in_dtype);
  }
}
