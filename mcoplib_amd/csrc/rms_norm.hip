// rms_norm.hip -- entry points of the RMSNorm operators without quantization:
//   mcop_rms_norm        mcoplib.op.rms_norm (optional residual -> after_res, rms_div)
//   mcop_head_rms_norm   mcoplib.op.head_rms_norm (selected heads, per-head weights)
//   mcop_vllm_rms_norm   vLLM _C::rms_norm (2-D / 3-D / 4-D strided input)
// The kernel and the three rounding chains are in norm_kernel.h.  This unit instantiates the
// fp32 input kernels; the bf16 and fp16 ones are in rms_norm_{bf16,f16}.hip.
#include "norm_kernel.h"

namespace mcop {

static int elem_bytes(mcop_dtype dt) { return dt == MCOP_F32 ? 4 : 2; }

static int dispatch_in(const char* name, const NormArgs& a, mcop_dtype in_dt, mcop_dtype wdt,
                       hipStream_t st) {
  switch (in_dt) {
    case MCOP_BF16: return norm_dispatch_bf16(name, a, wdt, st);
    case MCOP_F16: return norm_dispatch_f16(name, a, wdt, st);
    case MCOP_F32:
      if (wdt == MCOP_F32) return norm_dispatch<F32, F32>(name, a, st);
      if (wdt == MCOP_BF16) return norm_dispatch<F32, BF16>(name, a, st);
      return set_error(MCOP_E_INVALID, "%s: weight dtype %d is not supported for fp32 input",
                       name, (int)wdt);
    default:
      return set_error(MCOP_E_INVALID, "%s: input dtype %d is not bf16/fp16/fp32", name,
                       (int)in_dt);
  }
}

// The reference runs its vectorized kernel when the row is a whole number of vectors of n
// elements (16 bytes of the input, or 4 elements when either the input or the weight is fp32)
// and at most three vectors per thread of a 1024-thread block; otherwise its element-wise one.
static int mc_mode(int64_t hidden, mcop_dtype in_dt, mcop_dtype wdt) {
  const int64_t n = (in_dt == MCOP_F32 || wdt == MCOP_F32) ? 4 : 8;
  return (hidden % n == 0 && hidden <= 3 * 1024 * n) ? NORM_MC : NORM_MC_GENERIC;
}

static bool bad_shape(const char* name, int64_t rows, int64_t hidden) {
  if (rows < 0 || hidden <= 0 || hidden > INT32_MAX) {
    set_error(MCOP_E_INVALID, "%s: bad shape rows=%lld hidden_size=%lld", name, (long long)rows,
              (long long)hidden);
    return true;
  }
  return false;
}

}  // namespace mcop

extern "C" int mcop_rms_norm(void* out, const void* input, const void* weight,
                             mcop_dtype weight_dtype, void* after_res, const void* residual,
                             int64_t num_tokens, int64_t hidden_size, mcop_dtype in_dtype,
                             float epsilon, int rms_div, void* stream) {
  using namespace mcop;
  const char* name = "rms_norm";
  if (bad_shape(name, num_tokens, hidden_size)) return MCOP_E_INVALID;
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !input || !weight) return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  if (residual && !after_res) {
    return set_error(MCOP_E_INVALID, "%s: a residual needs an after_res output", name);
  }
  NormArgs a{};
  a.out = out;
  a.ares = residual ? after_res : nullptr;
  a.x = input;
  a.w = weight;
  a.res = residual;
  a.map = RowMap{1, 1, hidden_size, 0, 0, hidden_size, 0, 0, 0};
  a.rows = num_tokens;
  a.hidden = (int)hidden_size;
  a.eps = epsilon;
  a.mode = mc_mode(hidden_size, in_dtype, weight_dtype);
  a.rms_div = rms_div ? 1 : 0;
  return dispatch_in(name, a, in_dtype, weight_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int mcop_head_rms_norm(void* out, const void* input, const void* weight,
                                  mcop_dtype weight_dtype, int64_t num_tokens,
                                  int64_t num_heads, int64_t head_size, int64_t head_offset,
                                  int64_t head_norm, mcop_dtype in_dtype, float epsilon,
                                  void* stream) {
  using namespace mcop;
  const char* name = "head_rms_norm";
  if (bad_shape(name, num_tokens, head_size)) return MCOP_E_INVALID;
  if (num_heads <= 0 || head_offset < 0 || head_norm < 0 || head_offset + head_norm > num_heads) {
    return set_error(MCOP_E_INVALID,
                     "%s: heads [%lld, %lld) are not inside the %lld heads of a token", name,
                     (long long)head_offset, (long long)(head_offset + head_norm),
                     (long long)num_heads);
  }
  if (num_tokens == 0 || head_norm == 0) return MCOP_OK;
  if (!out || !input || !weight) return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  const int64_t off = head_offset * head_size;
  const int ib = elem_bytes(in_dtype), wb = elem_bytes(weight_dtype);
  NormArgs a{};
  a.out = static_cast<char*>(out) + off * ib;
  a.ares = nullptr;
  a.x = static_cast<const char*>(input) + off * ib;
  a.w = static_cast<const char*>(weight) + off * wb;
  a.res = nullptr;
  const int64_t tok = num_heads * head_size;
  a.map = RowMap{1, head_norm, tok, 0, head_size, tok, 0, head_size, head_size};
  a.rows = num_tokens * head_norm;
  a.hidden = (int)head_size;
  a.eps = epsilon;
  a.mode = mc_mode(head_size, in_dtype, weight_dtype);
  a.rms_div = 1;
  return dispatch_in(name, a, in_dtype, weight_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int mcop_vllm_rms_norm(void* out, const void* input, const void* weight,
                                  int64_t num_tokens, int64_t hidden_size, int num_dims,
                                  int64_t input_stride_d2, int64_t input_stride_d3,
                                  int64_t input_stride_d4, int64_t input_shape_d2,
                                  int64_t input_shape_d3, mcop_dtype dtype, float epsilon,
                                  void* stream) {
  using namespace mcop;
  const char* name = "vllm rms_norm";
  if (bad_shape(name, num_tokens, hidden_size)) return MCOP_E_INVALID;
  if (num_dims < 1 || num_dims > 4) {
    return set_error(MCOP_E_INVALID, "%s: %d dimensions (1 to 4 supported)", name, num_dims);
  }
  if (num_tokens == 0) return MCOP_OK;
  if (!out || !input || !weight) return set_error(MCOP_E_INVALID, "%s: null pointer", name);
  const int64_t H = hidden_size;
  RowMap m{1, 1, H, 0, 0, H, 0, 0, 0};
  if (num_dims == 2) {
    m.s0 = input_stride_d2;
  } else if (num_dims == 3) {
    if (input_shape_d2 <= 0) return set_error(MCOP_E_INVALID, "%s: bad 3-D shape", name);
    m = RowMap{1, input_shape_d2, input_stride_d3, 0, input_stride_d2, input_shape_d2 * H, 0, H,
               0};
  } else if (num_dims == 4) {
    if (input_shape_d2 <= 0 || input_shape_d3 <= 0) {
      return set_error(MCOP_E_INVALID, "%s: bad 4-D shape", name);
    }
    m = RowMap{input_shape_d3, input_shape_d2, input_stride_d4, input_stride_d3,
               input_stride_d2, input_shape_d3 * input_shape_d2 * H, input_shape_d2 * H, H, 0};
  }
  NormArgs a{};
  a.out = out;
  a.ares = nullptr;
  a.x = input;
  a.w = weight;
  a.res = nullptr;
  a.map = m;
  a.rows = num_tokens;
  a.hidden = (int)H;
  a.eps = epsilon;
  a.mode = NORM_VLLM;
  a.rms_div = 0;
  return dispatch_in(name, a, dtype, dtype, static_cast<hipStream_t>(stream));
}
