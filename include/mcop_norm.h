/*
 * mcop_norm.h -- C ABI of libmcop_norm.so, the gfx950 (MI355X) implementation of the fused
 * RMSNorm + per-token quantization operators of MetaX-MACA/mcoplib.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are raw device pointers (HIP global memory on the calling device).
 *     Rows are `hidden_size` elements long and contiguous unless a row stride is given.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream). Every call
 *     is asynchronous: it only enqueues kernels on `stream` and never synchronizes.
 *   - The device is the one current on the calling host thread (hipSetDevice); callers that
 *     hold tensors on another device make it current first.
 *   - Return value: MCOP_OK (0) or a negative MCOP_E_* code. The message of the last failure on
 *     the calling thread is returned by mcop_last_error(). No state is kept between calls
 *     (apart from the calling thread's test hooks, mcoplib_amd/csrc/mcop_testing.h) and calls
 *     are re-entrant. Nothing is allocated, with one exception: on the 16-byte vector path,
 *     rows too wide for one workgroup's registers (more than 65536 bf16/fp16 or 32768 fp32
 *     elements for most operators, fewer where a kernel would spill) run split over several
 *     workgroups, which exchange per-row partial results through a device workspace of at most
 *     2 MiB taken from the stream-ordered allocator (hipMallocAsync and hipFreeAsync on
 *     `stream`); under graph capture those rows take a multi-pass kernel that needs none.
 *   - Floating-point inputs may be bf16, fp16 or fp32 (mcop_dtype). Quantized outputs are int8
 *     or OCP fp8-e4m3fn. Per-token scales are fp32, one per row.
 *   - Results do not depend on the launch configuration: the row sum of squares is accumulated
 *     in fp64 and rounded once to fp32, and every other step is a correctly rounded fp32
 *     operation, so any split of a row over lanes gives the same bits.
 */
#ifndef MCOP_NORM_H
#define MCOP_NORM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MCOP_BF16 = 0,
  MCOP_F16 = 1,
  MCOP_F32 = 2,
  MCOP_I8 = 3,
  MCOP_FP8_E4M3FN = 4
} mcop_dtype;

enum {
  MCOP_OK = 0,
  MCOP_E_INVALID = -1,  /* bad argument: null pointer, size, dtype combination */
  MCOP_E_UNSUPPORTED = -2, /* valid request beyond a launch limit (more than 2^31 - 1 workgroups) */
  MCOP_E_LAUNCH = -3    /* the HIP runtime rejected the kernel launch */
};

/* Flags of mcop_rms_norm_smooth_quant. */
enum {
  /* Default (bit clear): the reference's literal normalisation u = (a / rho) * w with
     rho = 1/sqrt(mean(a^2)+eps), i.e. multiplication by sqrt(mean(a^2)+eps)
     (op/fused_rms_norm_dq.cu:94,139,179). Bit set: the textbook u = (a * rho) * w. */
  MCOP_SQ_STANDARD_NORM = 1u << 0
};

/* H1. In-place residual add + RMSNorm (vLLM `_C::fused_add_rms_norm`).
 *   residual[t,:] <- z = round(input + residual);  input[t,:] <- round(round(z * rho) * weight)
 *   with rho = 1/sqrt(sum(z^2)/H + eps) computed on the rounded z.
 * `input_row_stride` is the element stride between rows of `input` (>= hidden_size);
 * `residual` is contiguous. input, residual and weight share `dtype`.
 * Replaces fused_add_rms_norm(), op/vllm/layernorm_kernels.cu:243-292
 * (schema op/vllm/torch_bindings.cpp:161-164). */
int mcop_fused_add_rms_norm(void* input, int64_t input_row_stride, void* residual,
                            const void* weight, int64_t num_tokens, int64_t hidden_size,
                            mcop_dtype dtype, float epsilon, void* stream);

/* H2 / H3. (Residual add +) RMSNorm + dynamic per-token quantization.
 *   a = input (+ residual); if residual: residual <- round(a)
 *   rho = 1/sqrt(sum(a^2)/H + eps);  y = round(round(a * rho) * weight)
 *   A = max|y| (A = min(A, *scale_ub) when scale_ub != NULL)
 *   int8: s = max(A/127, FLT_EPSILON), q = sat[-128,127](rne(y * (1/s)))
 *   fp8 : s = max(A/448, 1/(448*512)), q = e4m3fn(clamp(y / s, -448, 448))
 *   scales[t] = s
 * `out_dtype` is MCOP_I8 or MCOP_FP8_E4M3FN; input, weight and residual share `in_dtype`;
 * `scale_ub` is a device pointer to one fp32 value or NULL; `residual` may be NULL.
 * Replaces rms_norm_dynamic_per_token_quant(),
 * op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:163-192
 * (schema op/vllm/torch_bindings.cpp:216-221), and
 * rms_norm_dynamic_per_token_quant_custom(), op/rms_norm_dynamic_per_token_quant.cu:266-285
 * (pybind op/pybind.cpp:55, declaration include/rms_norm_dynamic_per_token_quant.h:2-8). */
int mcop_rms_norm_dynamic_per_token_quant(void* out, mcop_dtype out_dtype, float* scales,
                                          const void* input, const void* weight,
                                          const float* scale_ub, void* residual,
                                          int64_t num_tokens, int64_t hidden_size,
                                          mcop_dtype in_dtype, float epsilon, void* stream);

/* mcop_rms_norm_dynamic_per_token_quant that allocates nothing, with the same arguments and
 * results. It has no counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Where the allocating entry takes a stream-ordered workspace (rows too wide for
 * one workgroup's registers, run split over several workgroups), this one uses a scratch array
 * of 2 MiB that the library holds on each GPU it runs on until the process ends; long calls are
 * cut into launches that fit it, and a launch that would not fit is refused with
 * MCOP_E_UNSUPPORTED and a message. Every call on a GPU shares that GPU's array (zeroed by the
 * call before use), so calls of this entry point that overlap on one GPU (other streams, other
 * threads) race: serialize them. The first call on a device resolves the array's address there. */
int mcop_rms_norm_dynamic_per_token_quant_noalloc(void* out, mcop_dtype out_dtype, float* scales,
                                                  const void* input, const void* weight,
                                                  const float* scale_ub, void* residual,
                                                  int64_t num_tokens, int64_t hidden_size,
                                                  mcop_dtype in_dtype, float epsilon,
                                                  void* stream);

/* H4. SmoothQuant (residual add +) RMSNorm + dynamic per-token quantization
 * (mcoplib.op.rms_norm_dynamic_per_token_quant, "fused_rms_norm_dq").
 *   a = input (+ residual, read only); after_res <- round(a)
 *   rho = 1/sqrt(sum(a^2)/H + eps) on the unrounded a;  a~ = round(a)
 *   u = (a~ / rho) * w   (or (a~ * rho) * w with MCOP_SQ_STANDARD_NORM); after_norm <- round(u)
 *   v = u * smooth;  A = max|v|
 *   int8: s = A/127, q = sat[-127,127](rne(v * (1/s)));
 *   fp8 (this library's extension; the reference's operator is int8 only): s = A/448,
 *   q = e4m3fn(clamp(v / s, -448, 448));  A == 0 gives s = 0 and q = 0.
 * `weight_dtype` and `smooth_dtype` are each `in_dtype` or MCOP_F32. after_res, after_norm and
 * residual may be NULL.
 * Replaces rms_norm_dynamic_per_token_quant(), op/fused_rms_norm_dq.cu:646-667
 * (pybind op/pybind.cpp:42, declaration include/fused_rms_norm_dq.h:3-12). */
int mcop_rms_norm_smooth_quant(void* out, mcop_dtype out_dtype, float* scales,
                               const void* input, const void* weight, mcop_dtype weight_dtype,
                               const void* smooth, mcop_dtype smooth_dtype, void* after_res,
                               void* after_norm, const void* residual, int64_t num_tokens,
                               int64_t hidden_size, mcop_dtype in_dtype, float epsilon,
                               uint32_t flags, void* stream);

/* H5. Smooth-scale multiply + dynamic per-token int8 quantization, no normalisation.
 *   v = input * smooth;  A = max|v|;  scales[t] = A * 0.00787401574803f
 *   q = sat[-128,127](rne(v * (127/A)));  A == 0 gives q = 0.
 * input is bf16, smooth fp32 [hidden_size], out int8, scales fp32 [num_tokens].
 * Replaces scale_dynamic_quant(), op/scale_dynamic_quant.cu:127-153
 * (pybind op/pybind.cpp:51, declaration include/scale_dynamic_quant.h:6-10). */
int mcop_scale_dynamic_quant(int8_t* out, float* scales, const void* input, const float* smooth,
                             int64_t num_tokens, int64_t hidden_size, void* stream);

/* Dynamic per-token int8 quantization without normalisation (vLLM `_C::dynamic_scaled_int8_quant`).
 *   azp == NULL (symmetric): A = max|x|; scales[t] = A/127; q = sat[-127,127](rne(x * (127/A)))
 *     (A == 0 gives q = 0);
 *   azp != NULL (asymmetric): s = (max x - min x)/255; azp[t] = rne(-128 - min x / s);
 *     q = sat[-128,127](rne(x * (1/s)) + azp[t]) (a NaN element codes 127, as the reference's
 *     fmin clamp before its conversion gives); a constant row (s == 0) gives azp = q = -128.
 * input bf16/fp16/fp32 [T,H] contiguous; out int8 [T,H]; scales fp32 [T]; azp int32 [T].
 * Replaces dynamic_scaled_int8_quant(),
 * op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:459-527 (kernels :94-132,
 * :370-422; schema op/vllm/torch_bindings.cpp:374-379). */
int mcop_dynamic_scaled_int8_quant(int8_t* out, float* scales, int32_t* azp, const void* input,
                                   int64_t num_tokens, int64_t hidden_size, mcop_dtype in_dtype,
                                   void* stream);

/* Dynamic per-token fp8-e4m3fn quantization without normalisation
 * (vLLM `_C::dynamic_per_token_scaled_fp8_quant`):
 *   A = max|x| (min with *scale_ub); s = max(A/448, 1/(448*512)); q = e4m3fn(clamp(x/s, +-448)).
 * Rows of input and out may be strided (element strides >= hidden_size).
 * Replaces dynamic_per_token_scaled_fp8_quant(), op/vllm/quantization/fp8/common.cu:375-411
 * (kernel :142-180; schema op/vllm/torch_bindings.cpp:359-364). */
int mcop_dynamic_per_token_scaled_fp8_quant(uint8_t* out, float* scales, const void* input,
                                            const float* scale_ub, int64_t num_tokens,
                                            int64_t hidden_size, int64_t input_row_stride,
                                            int64_t output_row_stride, mcop_dtype in_dtype,
                                            void* stream);

/* mcoplib's own (residual add +) RMSNorm + per-token int8 quantization
 * (mcoplib.op.rms_norm_dynamic_per_token_quant_custom), int8 only, with the reference's two
 * kernels' arithmetic:
 *   H != 7168: as mcop_rms_norm_dynamic_per_token_quant with int8 out, except
 *     s = max(A/127, 1.5e-6) and q = sat[-127,127](rne(y * (1/s)));
 *   H == 7168: p = a * w in fp32 (no bf16 rounding), A = max|p|,
 *     s = max((A * rho)/127, FLT_EPSILON), q = sat[-127,127](rne((p * rho) * (1/s)));
 *     scale_ub is not used.
 * residual (if given) <- b(input + residual).
 * Replaces rms_norm_dynamic_per_token_quant_custom(), op/rms_norm_dynamic_per_token_quant.cu:
 * 266-285 (kernels :52-92 with kernel/rms_norm_vllm.cuh:330-454, and :94-186; pybind
 * op/pybind.cpp:55; Python wrapper mcoplib/custom_ops.py:29-45). */
int mcop_rms_norm_dynamic_per_token_quant_custom(int8_t* out, float* scales, const void* input,
                                                 const void* weight, const float* scale_ub,
                                                 void* residual, int64_t num_tokens,
                                                 int64_t hidden_size, mcop_dtype in_dtype,
                                                 float epsilon, void* stream);

/* (Residual add +) RMSNorm without quantization (mcoplib.op.rms_norm):
 *   a = x (+ residual, read only); after_res <- b(a) when a residual is given;
 *   out <- b((a * d) * w), d = rms_div ? RN(1/rho) : rho   (the reference's vectorized kernel,
 *   taken when H is a multiple of n and H <= 3072*n, n = 4 if the input or the weight is fp32,
 *   else 8); otherwise its element-wise chain: out <- b((a~ / rho) * w) (rms_div) or
 *   b((a~ * rho) * w), a~ = b(a) with a residual, x without.  rho = 1/sqrt(sum(a^2)/H + eps).
 * input, out, residual, after_res: [T,H] contiguous in_dtype; weight [H] in_dtype or fp32.
 * Replaces rms_norm(), op/fused_rms_norm_dq.cu:980-998 (dispatch :814-978, kernels :305-420;
 * pybind op/pybind.cpp:44). */
int mcop_rms_norm(void* out, const void* input, const void* weight, mcop_dtype weight_dtype,
                  void* after_res, const void* residual, int64_t num_tokens, int64_t hidden_size,
                  mcop_dtype in_dtype, float epsilon, int rms_div, void* stream);

/* Per-head RMSNorm of heads [head_offset, head_offset + head_norm) of every token
 * (mcoplib.op.head_rms_norm): input / out [T, num_heads, head_size] contiguous, weight
 * [num_heads, head_size] (bf16 or fp32; row h normalizes head h); other heads of out are not
 * written.  out <- b((x * RN(1/rho)) * w) for the reference's vectorized sizes (as for
 * mcop_rms_norm), else b((x / rho) * w).
 * Replaces head_rms_norm(), op/fused_rms_norm_dq.cu:804-812 (dispatch :669-802, kernels
 * :493-578; pybind op/pybind.cpp:43). */
int mcop_head_rms_norm(void* out, const void* input, const void* weight, mcop_dtype weight_dtype,
                       int64_t num_tokens, int64_t num_heads, int64_t head_size,
                       int64_t head_offset, int64_t head_norm, mcop_dtype in_dtype,
                       float epsilon, void* stream);

/* vLLM `_C::rms_norm`: out[r] <- b(b(x_r * rho) * w) for the num_tokens rows of a 2-D, 3-D or
 * 4-D input addressed with the given strides (as the reference kernel's arguments:
 * input.stride(-2), -3, -4 and input.size(-2), -3); out [num_tokens, H] contiguous; weight
 * [H] in the input dtype.
 * Replaces rms_norm(), op/vllm/layernorm_kernels.cu:186-231 (kernel :15-86; schema
 * op/vllm/torch_bindings.cpp:155-158). */
int mcop_vllm_rms_norm(void* out, const void* input, const void* weight, int64_t num_tokens,
                       int64_t hidden_size, int num_dims, int64_t input_stride_d2,
                       int64_t input_stride_d3, int64_t input_stride_d4, int64_t input_shape_d2,
                       int64_t input_shape_d3, mcop_dtype dtype, float epsilon, void* stream);

/* (Residual add +) RMSNorm + dynamic per-group quantization (vLLM `_C::rms_norm_per_block_quant`):
 * as mcop_rms_norm_dynamic_per_token_quant, but with one scale per group of group_size (64 or
 * 128) consecutive elements of a row: A_g = max|y| over the group (min with *scale_ub, fp8
 * only), s_g = max(A_g/127, FLT_EPSILON) (int8) or max(A_g/448, 1/(448*512)) (fp8).
 * scales: fp32 [T, H/group_size], or [H/group_size, T] when is_scale_transposed != 0.
 * hidden_size must be a multiple of group_size.
 * Replaces rms_norm_per_block_quant(),
 * op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:238-270
 * (dispatch :194-236, kernel :92-126, layernorm_utils.cuh:283-393, 455-535; schema
 * op/vllm/torch_bindings.cpp:224-229). */
int mcop_rms_norm_per_block_quant(void* out, mcop_dtype out_dtype, float* scales,
                                  const void* input, const void* weight, const float* scale_ub,
                                  void* residual, int64_t num_tokens, int64_t hidden_size,
                                  mcop_dtype in_dtype, float epsilon, int64_t group_size,
                                  int is_scale_transposed, void* stream);

/* Residual add + RMSNorm + per-token int8 quantization into a padded per-row wire layout
 * (mcoplib.op.fused_add_rms_norm_dynamic_per_token_quant_padding_output).
 *   output: int8 [T, 2*pad_size] bytes; row t holds its H codes at bytes [0, H) and its fp32
 *     scale at bytes [H, H+4); the rest of the row is not written (2*pad_size >= H + 4);
 *   output_rms: bf16 [T,H] normalized values; output_quant_int8: int8 [T,H] the same codes;
 *   out_scales: fp32 [T]; input, residual (updated in place: input + residual), weight: bf16.
 * Two rounding chains, as the reference dispatches them: H == 7168 keeps a = x + r in fp32
 * (rms = b((a*w)*rho), q = sat[-127,127](rne((a*w)*rho / s))), other H round bf16 products
 * (q from y = b(b(b(a)*rho)*w)); s = max(absmax*rho/127, FLT_EPSILON) with absmax taken over
 * a*w (H == 7168) or b(b(a)*w).
 * Replaces add_rms_norm_dynamic_per_token_quant_padding_output(),
 * op/fused_add_layernorm_per_token_quant_padding_output.cu:397-416 (kernels :181-283 and
 * :287-340, dispatch :344-395; pybind op/pybind.cpp:54; Python wrapper
 * mcoplib/custom_ops.py:7-27). */
int mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output(
    int8_t* output, void* output_rms, int8_t* output_quant_int8, float* out_scales,
    const void* input, void* residual, const void* weight, int64_t num_tokens,
    int64_t hidden_size, int64_t pad_size, float epsilon, void* stream);

/* Message of the last failed call on this host thread ("" if none). Stands in for the
 * reference's TORCH_CHECK messages (c10::Error text), which its entry points raise directly. */
const char* mcop_last_error(void);

/* ABI version of this header (bumped on any signature change). The reference's extension has
 * no such query; callers over a C ABI use it to refuse a library built from another header. */
int mcop_abi_version(void);
#define MCOP_ABI_VERSION 2

#ifdef __cplusplus
}
#endif

#endif /* MCOP_NORM_H */
