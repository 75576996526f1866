// torch_ops.cpp -- the operator surfaces of the fused norm/quant path as a C++ torch extension
// (module mcoplib_amd._torch_ops) over the C ABI of libmcop_norm.so (include/mcop_norm.h).
//
// Two surfaces, as the reference builds them in C++:
//   - mcoplib.op (pybind, op/pybind.cpp:42-44, 51, 54, 55): rms_norm_dynamic_per_token_quant
//     (fused_rms_norm_dq), rms_norm_dynamic_per_token_quant_custom, scale_dynamic_quant,
//     fused_add_rms_norm_dynamic_per_token_quant_padding_output, rms_norm, head_rms_norm;
//   - torch.ops._C (TORCH_LIBRARY, op/vllm/torch_bindings.cpp:155-164, 216-229, 359-364,
//     374-379): rms_norm, fused_add_rms_norm, rms_norm_dynamic_per_token_quant,
//     rms_norm_per_block_quant, dynamic_scaled_int8_quant, dynamic_per_token_scaled_fp8_quant,
//     registered by register_vllm_ops() for the CUDA (HIP) key, plus a no-op Meta kernel.
// Every function checks its arguments as the reference does (TORCH_CHECK with the reference's
// condition text) and, beyond the reference, that every tensor is on the device and that element
// counts match (the kernels trust them); then it makes the input's device current and enqueues
// one kernel on torch's current stream of that device.  Nothing synchronizes.
#include <torch/extension.h>

#include <ATen/hip/HIPContext.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <memory>
#include <optional>
#include <string>

#include "../../include/mcop_norm.h"

namespace {

using at::Tensor;
using OptTensor = std::optional<Tensor>;

mcop_dtype code_of(at::ScalarType t) {
  switch (t) {
    case at::kBFloat16: return MCOP_BF16;
    case at::kHalf: return MCOP_F16;
    case at::kFloat: return MCOP_F32;
    case at::kChar: return MCOP_I8;
    case at::kFloat8_e4m3fn: return MCOP_FP8_E4M3FN;
    default: TORCH_CHECK(false, "libmcop_norm: unsupported dtype ", t);
  }
}

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check_rc(int rc) {
  if (rc != MCOP_OK) TORCH_CHECK(false, mcop_last_error());
}

bool is_float_type(at::ScalarType t) {
  return t == at::kFloat || t == at::kHalf || t == at::kBFloat16;
}

// The error AT_DISPATCH_* raises for a dtype outside its list.
void dispatch_check(at::ScalarType t, const char* name) {
  TORCH_CHECK(is_float_type(t), '"', name, "\" not implemented for '", c10::toString(t), "'");
}

void on_device(const char* name, std::initializer_list<const Tensor*> ts) {
  const Tensor* first = nullptr;
  for (const Tensor* t : ts) {
    if (t == nullptr || !t->defined()) continue;
    TORCH_CHECK(t->is_cuda(), name, ": all tensors must be on a CUDA (HIP) device, got ",
                t->device());
    if (first == nullptr) {
      first = t;
    } else {
      TORCH_CHECK(t->device() == first->device(), name, ": tensors on different devices (",
                  first->device(), " and ", t->device(), ")");
    }
  }
}

const Tensor* opt(const OptTensor& t) { return t.has_value() ? &*t : nullptr; }

void numel_check(const char* name, const char* what, const Tensor& t, int64_t n) {
  TORCH_CHECK(t.numel() == n, name, ": ", what, " has ", t.numel(), " elements, expected ", n);
}

void contiguous_check(const char* name, const char* what, const Tensor& t) {
  TORCH_CHECK(t.is_contiguous(), name, ": ", what, " must be contiguous");
}

// (num_tokens, hidden_size) of a [..., hidden_size] tensor (numel / size(-1), as the reference)
std::pair<int64_t, int64_t> rows_of(const Tensor& t) {
  TORCH_CHECK(t.dim() > 0, "expected a tensor with at least one dimension");
  const int64_t h = t.size(-1);
  TORCH_CHECK(h > 0, "hidden_size (the last dimension) must be positive");
  return {t.numel() / h, h};
}

// Element stride between the rows of t, for tensors whose rows are uniformly strided.
int64_t row_stride(const char* name, const Tensor& t, int64_t T, int64_t H) {
  if (t.dim() < 2 || T <= 1) return H;
  for (int64_t d = 0; d + 2 < t.dim(); ++d) {
    TORCH_CHECK(t.size(d) <= 1 || t.stride(d) == t.stride(d + 1) * t.size(d + 1), name,
                ": rows must be uniformly strided");
  }
  return t.stride(-2);
}

const float* ub_ptr(const char* name, const OptTensor& scale_ub) {
  if (!scale_ub.has_value()) return nullptr;
  TORCH_CHECK(scale_ub->scalar_type() == at::kFloat && scale_ub->numel() >= 1, name,
              ": scale_ub must be a float32 tensor with one element");
  return scale_ub->data_ptr<float>();
}

using DeviceGuard = c10::hip::OptionalHIPGuardMasqueradingAsCUDA;

// ------------------------------------------------------------------------ mcoplib.op surface

// Shared launcher of the (residual add +) RMSNorm + per-token quant kernel, vLLM's arithmetic or
// mcoplib's own (`custom`).
void norm_quant(const char* name, Tensor& out, const Tensor& input, const Tensor& weight,
                Tensor& scales, double eps, const OptTensor& scale_ub, const OptTensor& residual,
                bool custom) {
  on_device(name, {&out, &input, &weight, &scales, opt(scale_ub), opt(residual)});
  const auto [T, H] = rows_of(input);
  numel_check(name, "out", out, T * H);
  numel_check(name, "weight", weight, H);
  numel_check(name, "scales", scales, T);
  contiguous_check(name, "weight", weight);
  contiguous_check(name, "scales", scales);
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(), name,
              ": weight must have the input dtype ", input.scalar_type());
  if (residual.has_value()) {
    TORCH_CHECK(residual->scalar_type() == input.scalar_type(), name,
                ": residual must have the input dtype ", input.scalar_type());
    contiguous_check(name, "residual", *residual);
    numel_check(name, "residual", *residual, T * H);
  }
  const float* ub = ub_ptr(name, scale_ub);
  void* rp = residual.has_value() ? residual->data_ptr() : nullptr;
  const DeviceGuard guard(input.device());
  if (custom) {
    check_rc(mcop_rms_norm_dynamic_per_token_quant_custom(
        static_cast<int8_t*>(out.data_ptr()), scales.data_ptr<float>(), input.data_ptr(),
        weight.data_ptr(), ub, rp, T, H, code_of(input.scalar_type()), (float)eps,
        stream_of(input)));
  } else {
    check_rc(mcop_rms_norm_dynamic_per_token_quant(
        out.data_ptr(), code_of(out.scalar_type()), scales.data_ptr<float>(), input.data_ptr(),
        weight.data_ptr(), ub, rp, T, H, code_of(input.scalar_type()), (float)eps,
        stream_of(input)));
  }
}

// op/fused_rms_norm_dq.cu:646-667 (pybind op/pybind.cpp:42)
void op_smooth_quant(Tensor& out, const Tensor& input, const Tensor& weight,
                     const Tensor& smooth_scale, Tensor& scales, double var_epsilon,
                     Tensor& after_res, Tensor& after_norm, const OptTensor& residual,
                     bool standard_norm) {
  const char* name = "rms_norm_dynamic_per_token_quant";
  TORCH_CHECK(out.scalar_type() == at::kChar || out.scalar_type() == at::kFloat8_e4m3fn,
              "Expected out.dtype() == torch::kInt8 || out.dtype() == torch::kFloat8_e4m3fn to "
              "be true, but got false.");
  TORCH_CHECK(out.is_contiguous() && input.is_contiguous(),
              "Expected out.is_contiguous() && input.is_contiguous() to be true, but got false.");
  TORCH_CHECK(scales.scalar_type() == at::kFloat,
              "Expected scales.dtype() == torch::kFloat32 to be true, but got false.");
  dispatch_check(input.scalar_type(), "rms_norm_dynamic_per_token_quant_dispatch");
  on_device(name, {&out, &input, &weight, &smooth_scale, &scales, &after_res, &after_norm,
                   opt(residual)});
  const auto [T, H] = rows_of(input);
  numel_check(name, "out", out, T * H);
  numel_check(name, "weight", weight, H);
  numel_check(name, "smooth_scale", smooth_scale, H);
  numel_check(name, "scales", scales, T);
  contiguous_check(name, "weight", weight);
  contiguous_check(name, "smooth_scale", smooth_scale);
  contiguous_check(name, "scales", scales);
  for (const auto& [what, t] : {std::pair<const char*, const Tensor*>{"after_res", &after_res},
                                {"after_norm", &after_norm}}) {
    contiguous_check(name, what, *t);
    numel_check(name, what, *t, T * H);
    TORCH_CHECK(t->scalar_type() == input.scalar_type(), name, ": ", what,
                " must have the input dtype ", input.scalar_type());
  }
  if (residual.has_value()) {
    TORCH_CHECK(residual->scalar_type() == input.scalar_type(), name,
                ": residual must have the input dtype ", input.scalar_type());
    contiguous_check(name, "residual", *residual);
    numel_check(name, "residual", *residual, T * H);
  }
  for (const auto& [what, t] : {std::pair<const char*, const Tensor*>{"weight", &weight},
                                {"smooth_scale", &smooth_scale}}) {
    TORCH_CHECK(t->scalar_type() == input.scalar_type() || t->scalar_type() == at::kFloat, name,
                ": ", what, " must be ", input.scalar_type(), " or float32, got ",
                t->scalar_type());
  }
  const DeviceGuard guard(input.device());
  check_rc(mcop_rms_norm_smooth_quant(
      out.data_ptr(), code_of(out.scalar_type()), scales.data_ptr<float>(), input.data_ptr(),
      weight.data_ptr(), code_of(weight.scalar_type()), smooth_scale.data_ptr(),
      code_of(smooth_scale.scalar_type()), after_res.data_ptr(), after_norm.data_ptr(),
      residual.has_value() ? residual->data_ptr() : nullptr, T, H,
      code_of(input.scalar_type()), (float)var_epsilon,
      standard_norm ? (uint32_t)MCOP_SQ_STANDARD_NORM : 0u, stream_of(input)));
}

// op/rms_norm_dynamic_per_token_quant.cu:266-285 (pybind op/pybind.cpp:55)
void op_custom(Tensor& out, const Tensor& input, const Tensor& weight, Tensor& scales,
               double var_epsilon, const OptTensor& scale_ub, const OptTensor& residual) {
  TORCH_CHECK(out.scalar_type() == at::kChar,
              "Expected out.dtype() == torch::kInt8 to be true, but got false.");
  TORCH_CHECK(out.is_contiguous() && input.is_contiguous(),
              "Expected out.is_contiguous() && input.is_contiguous() to be true, but got false.");
  TORCH_CHECK(scales.scalar_type() == at::kFloat,
              "Expected scales.dtype() == torch::kFloat32 to be true, but got false.");
  dispatch_check(input.scalar_type(), " rms_norm_dynamic_per_token_quant_dispatch_");
  norm_quant("rms_norm_dynamic_per_token_quant_custom", out, input, weight, scales, var_epsilon,
             scale_ub, residual, true);
}

// op/scale_dynamic_quant.cu:127-153 (pybind op/pybind.cpp:51): returns new (codes, scales [T])
std::tuple<Tensor, Tensor> op_scale_dynamic_quant(const Tensor& hidden_states,
                                                  const Tensor& smooth_scales,
                                                  py::object dst_dtype) {
  const char* name = "scale_dynamic_quant";
  TORCH_CHECK(hidden_states.is_cuda(), "Expected hidden_states.is_cuda() to be true, but got "
                                       "false.");
  TORCH_CHECK(smooth_scales.is_cuda(), "Expected smooth_scales.is_cuda() to be true, but got "
                                       "false.");
  const at::ScalarType dt = dst_dtype.is_none()
                                ? at::kChar
                                : torch::python::detail::py_object_to_dtype(dst_dtype);
  const auto [T, H] = rows_of(hidden_states);
  Tensor output = at::empty_like(hidden_states, hidden_states.options().dtype(dt));
  Tensor scales = at::empty({T}, smooth_scales.options());
  TORCH_CHECK(hidden_states.scalar_type() == at::kBFloat16 && dt == at::kChar,
              "Only support bfloat16");
  on_device(name, {&hidden_states, &smooth_scales});
  contiguous_check(name, "hidden_states", hidden_states);
  contiguous_check(name, "smooth_scales", smooth_scales);
  numel_check(name, "smooth_scales", smooth_scales, H);
  TORCH_CHECK(smooth_scales.scalar_type() == at::kFloat, name,
              ": smooth_scales must be float32");
  const DeviceGuard guard(hidden_states.device());
  check_rc(mcop_scale_dynamic_quant(static_cast<int8_t*>(output.data_ptr()),
                                    scales.data_ptr<float>(), hidden_states.data_ptr(),
                                    smooth_scales.data_ptr<float>(), T, H,
                                    stream_of(hidden_states)));
  return {output, scales};
}

// op/fused_add_layernorm_per_token_quant_padding_output.cu:397-416 (pybind op/pybind.cpp:54)
void op_padded(Tensor& output, Tensor& output_rms, Tensor& output_quant_int8, Tensor& out_scales,
               const Tensor& input, Tensor& residual, const Tensor& weight, int64_t pad_size,
               double epsilon) {
  const char* name = "fused_add_rms_norm_dynamic_per_token_quant_padding_output";
  TORCH_CHECK(output.scalar_type() == at::kChar,
              "Expected output.dtype() == torch::kInt8 to be true, but got false.");
  TORCH_CHECK(input.scalar_type() == at::kBFloat16,
              "Expected input.dtype() == at::ScalarType::BFloat16 to be true, but got false.");
  TORCH_CHECK(output.is_contiguous() && input.is_contiguous(),
              "Expected output.is_contiguous() && input.is_contiguous() to be true, but got "
              "false.");
  on_device(name, {&output, &output_rms, &output_quant_int8, &out_scales, &input, &residual,
                   &weight});
  const auto [T, H] = rows_of(input);
  TORCH_CHECK(2 * pad_size >= H + 4, name, ": a padded row of 2*pad_size = ", 2 * pad_size,
              " bytes cannot hold ", H, " codes and a 4-byte scale");
  numel_check(name, "output", output, T * 2 * pad_size);
  const std::tuple<const char*, const Tensor*, at::ScalarType> outs[] = {
      {"output_rms", &output_rms, at::kBFloat16},
      {"output_quant_int8", &output_quant_int8, at::kChar},
      {"residual", &residual, at::kBFloat16},
      {"weight", &weight, at::kBFloat16},
      {"out_scales", &out_scales, at::kFloat}};
  for (const auto& [what, t, want] : outs) {
    TORCH_CHECK(t->scalar_type() == want, name, ": ", what, " must be ", want, ", got ",
                t->scalar_type());
    contiguous_check(name, what, *t);
  }
  numel_check(name, "output_rms", output_rms, T * H);
  numel_check(name, "output_quant_int8", output_quant_int8, T * H);
  numel_check(name, "residual", residual, T * H);
  numel_check(name, "weight", weight, H);
  numel_check(name, "out_scales", out_scales, T);
  const DeviceGuard guard(input.device());
  check_rc(mcop_fused_add_rms_norm_dynamic_per_token_quant_padding_output(
      static_cast<int8_t*>(output.data_ptr()), output_rms.data_ptr(),
      static_cast<int8_t*>(output_quant_int8.data_ptr()), out_scales.data_ptr<float>(),
      input.data_ptr(), residual.data_ptr(), weight.data_ptr(), T, H, pad_size, (float)epsilon,
      stream_of(input)));
}

// op/fused_rms_norm_dq.cu:980-998 (pybind op/pybind.cpp:44)
void op_rms_norm(Tensor& out, const Tensor& input, const Tensor& weight, double var_epsilon,
                 const OptTensor& after_res, const OptTensor& residual, bool rms_div) {
  const char* name = "rms_norm";
  TORCH_CHECK(out.is_contiguous() && input.is_contiguous(),
              "Expected out.is_contiguous() && input.is_contiguous() to be true, but got false.");
  TORCH_CHECK(weight.is_contiguous(), "Expected weight.is_contiguous() to be true, but got "
                                      "false.");
  dispatch_check(input.scalar_type(), "rms_norm_per_token_dispatch");
  on_device(name, {&out, &input, &weight, opt(after_res), opt(residual)});
  const auto [T, H] = rows_of(input);
  TORCH_CHECK(out.scalar_type() == input.scalar_type(), name,
              ": out must have the input dtype ", input.scalar_type());
  TORCH_CHECK(weight.scalar_type() == input.scalar_type() || weight.scalar_type() == at::kFloat,
              name, ": weight must be ", input.scalar_type(), " or float32, got ",
              weight.scalar_type());
  numel_check(name, "out", out, T * H);
  numel_check(name, "weight", weight, H);
  if (residual.has_value()) {
    TORCH_CHECK(after_res.has_value(), name, ": a residual needs an after_res output");
    for (const auto& [what, t] : {std::pair<const char*, const Tensor*>{"residual", &*residual},
                                  {"after_res", &*after_res}}) {
      TORCH_CHECK(t->scalar_type() == input.scalar_type(), name, ": ", what,
                  " must have the input dtype ", input.scalar_type());
      contiguous_check(name, what, *t);
      numel_check(name, what, *t, T * H);
    }
  }
  const DeviceGuard guard(input.device());
  check_rc(mcop_rms_norm(out.data_ptr(), input.data_ptr(), weight.data_ptr(),
                         code_of(weight.scalar_type()),
                         residual.has_value() ? after_res->data_ptr() : nullptr,
                         residual.has_value() ? residual->data_ptr() : nullptr, T, H,
                         code_of(input.scalar_type()), (float)var_epsilon, rms_div ? 1 : 0,
                         stream_of(input)));
}

// op/fused_rms_norm_dq.cu:804-812 (pybind op/pybind.cpp:43)
void op_head_rms_norm(Tensor& out, const Tensor& hidden_states, const Tensor& weight,
                      double var_epsilon, int64_t head_offset, int64_t head_norm) {
  const char* name = "head_rms_norm";
  TORCH_CHECK(out.is_contiguous() && weight.is_contiguous() && hidden_states.is_contiguous(),
              "Expected out.is_contiguous() && weight.is_contiguous() && "
              "hidden_states.is_contiguous() to be true, but got false.");
  dispatch_check(hidden_states.scalar_type(), "head_rms_norm_dispatch");
  on_device(name, {&out, &hidden_states, &weight});
  TORCH_CHECK(hidden_states.dim() == 3, name,
              ": hidden_states must be [num_tokens, num_heads, head_size]");
  const int64_t T = hidden_states.size(0), NH = hidden_states.size(1),
                D = hidden_states.size(2);
  TORCH_CHECK(out.sizes() == hidden_states.sizes() &&
                  out.scalar_type() == hidden_states.scalar_type(),
              name, ": out must match hidden_states in shape and dtype");
  TORCH_CHECK(weight.scalar_type() == at::kBFloat16 || weight.scalar_type() == at::kFloat, name,
              ": weight must be bfloat16 or float32, got ", weight.scalar_type());
  TORCH_CHECK(head_offset >= 0 && head_norm >= 0 && head_offset + head_norm <= NH, name,
              ": heads [", head_offset, ", ", head_offset + head_norm,
              ") are not inside the ", NH, " heads");
  TORCH_CHECK(weight.numel() >= (head_offset + head_norm) * D, name, ": weight holds ",
              weight.numel(), " elements, needs ", (head_offset + head_norm) * D);
  const DeviceGuard guard(hidden_states.device());
  check_rc(mcop_head_rms_norm(out.data_ptr(), hidden_states.data_ptr(), weight.data_ptr(),
                              code_of(weight.scalar_type()), T, NH, D, head_offset, head_norm,
                              code_of(hidden_states.scalar_type()), (float)var_epsilon,
                              stream_of(hidden_states)));
}

// ------------------------------------------------------------------------- torch.ops._C surface

// op/vllm/layernorm_kernels.cu:186-231
void c_rms_norm(Tensor& result, const Tensor& input_arg, const Tensor& weight, double epsilon) {
  const char* name = "rms_norm";
  TORCH_CHECK(result.is_contiguous(), "Expected out.is_contiguous() to be true, but got false.");
  const Tensor input = input_arg.stride(-1) == 1 ? input_arg : input_arg.contiguous();
  TORCH_CHECK(weight.is_contiguous(), "Expected weight.is_contiguous() to be true, but got "
                                      "false.");
  dispatch_check(input.scalar_type(), "rms_norm_kernel");
  const int64_t nd = input.dim();
  TORCH_CHECK(nd == 2 || nd == 3 || nd == 4, "Expects rank 2, 3 or 4 tensors but got ", nd);
  TORCH_CHECK(weight.scalar_type() == input.scalar_type() &&
                  result.scalar_type() == input.scalar_type(),
              name, ": result, input and weight must share one dtype");
  on_device(name, {&result, &input, &weight});
  const auto [T, H] = rows_of(input);
  numel_check(name, "result", result, T * H);
  numel_check(name, "weight", weight, H);
  const DeviceGuard guard(input.device());
  check_rc(mcop_vllm_rms_norm(result.data_ptr(), input.data_ptr(), weight.data_ptr(), T, H,
                              (int)nd, input.stride(-2), nd >= 3 ? input.stride(-3) : 0,
                              nd >= 4 ? input.stride(-4) : 0, nd >= 3 ? input.size(-2) : 0,
                              nd >= 4 ? input.size(-3) : 0, code_of(input.scalar_type()),
                              (float)epsilon, stream_of(input)));
}

// op/vllm/layernorm_kernels.cu:243-292
void c_fused_add_rms_norm(Tensor& input, Tensor& residual, const Tensor& weight, double epsilon) {
  const char* name = "fused_add_rms_norm";
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(),
              "Expected weight.scalar_type() == input.scalar_type() to be true, but got false.");
  TORCH_CHECK(input.scalar_type() == residual.scalar_type(),
              "Expected input.scalar_type() == residual.scalar_type() to be true, but got false.");
  TORCH_CHECK(residual.is_contiguous(), "Expected residual.is_contiguous() to be true, but got "
                                        "false.");
  TORCH_CHECK(weight.is_contiguous(), "Expected weight.is_contiguous() to be true, but got "
                                      "false.");
  dispatch_check(input.scalar_type(), "fused_add_rms_norm_kernel");
  on_device(name, {&input, &residual, &weight});
  const auto [T, H] = rows_of(input);
  numel_check(name, "residual", residual, T * H);
  numel_check(name, "weight", weight, H);
  // rows of `input` are addressed as row * stride(-2) (the reference's input_stride)
  int64_t stride = H;
  if (input.dim() >= 2 && T > 1) {
    TORCH_CHECK(input.stride(-1) == 1, name, ": input must be contiguous in its last dimension");
    for (int64_t d = 0; d + 2 < input.dim(); ++d) {
      TORCH_CHECK(input.size(d) <= 1 ||
                      input.stride(d) == input.stride(d + 1) * input.size(d + 1),
                  name, ": input rows must be uniformly strided");
    }
    stride = input.stride(-2);
  }
  const DeviceGuard guard(input.device());
  check_rc(mcop_fused_add_rms_norm(input.data_ptr(), stride, residual.data_ptr(),
                                   weight.data_ptr(), T, H, code_of(input.scalar_type()),
                                   (float)epsilon, stream_of(input)));
}

void quant_out_checks(const Tensor& result, const Tensor& input, const Tensor& weight,
                      const Tensor& scale, const OptTensor& scale_ub, const OptTensor& residual) {
  TORCH_CHECK(result.scalar_type() == at::kFloat8_e4m3fn || result.scalar_type() == at::kChar,
              "Expected out.dtype() == kFp8Type || out.dtype() == torch::kInt8 to be true, but "
              "got false.");
  TORCH_CHECK(result.is_contiguous() && input.is_contiguous(),
              "Expected out.is_contiguous() && input.is_contiguous() to be true, but got false.");
  if (scale_ub.has_value()) {
    TORCH_CHECK(result.scalar_type() == at::kFloat8_e4m3fn,
                "Expected out.dtype() == kFp8Type to be true, but got false.");
  }
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(),
              "Expected weight.dtype() == input.dtype() to be true, but got false.");
  TORCH_CHECK(scale.scalar_type() == at::kFloat,
              "Expected scales.dtype() == torch::kFloat32 to be true, but got false.");
  if (residual.has_value()) {
    TORCH_CHECK(residual->scalar_type() == input.scalar_type(),
                "Expected residual->scalar_type() == input.scalar_type() to be true, but got "
                "false.");
  }
}

// op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:163-192
void c_norm_quant(Tensor& result, const Tensor& input, const Tensor& weight, Tensor& scale,
                  double epsilon, const OptTensor& scale_ub, const OptTensor& residual) {
  quant_out_checks(result, input, weight, scale, scale_ub, residual);
  dispatch_check(input.scalar_type(), "rms_norm_dynamic_per_token_quant_dispatch");
  norm_quant("rms_norm_dynamic_per_token_quant", result, input, weight, scale, epsilon, scale_ub,
             residual, false);
}

// op/vllm/quantization/fused_kernels/fused_layernorm_dynamic_per_token_quant.cu:238-270
void c_per_block_quant(Tensor& result, const Tensor& input, const Tensor& weight, Tensor& scale,
                       double epsilon, const OptTensor& scale_ub, const OptTensor& residual,
                       int64_t group_size, bool is_scale_transposed) {
  const char* name = "rms_norm_per_block_quant";
  quant_out_checks(result, input, weight, scale, scale_ub, residual);
  TORCH_CHECK(group_size == 64 || group_size == 128, "Unsupported group size: ", group_size);
  dispatch_check(input.scalar_type(), "rms_norm_per_block_quant_fp_dispatch");
  on_device(name, {&result, &input, &weight, &scale, opt(scale_ub), opt(residual)});
  const auto [T, H] = rows_of(input);
  TORCH_CHECK(H % group_size == 0, name, ": hidden_size ", H,
              " is not a multiple of group_size ", group_size);
  numel_check(name, "result", result, T * H);
  numel_check(name, "weight", weight, H);
  numel_check(name, "scale", scale, T * (H / group_size));
  contiguous_check(name, "weight", weight);
  contiguous_check(name, "scale", scale);
  if (residual.has_value()) {
    contiguous_check(name, "residual", *residual);
    numel_check(name, "residual", *residual, T * H);
  }
  const float* ub = ub_ptr(name, scale_ub);
  const DeviceGuard guard(input.device());
  check_rc(mcop_rms_norm_per_block_quant(
      result.data_ptr(), code_of(result.scalar_type()), scale.data_ptr<float>(),
      input.data_ptr(), weight.data_ptr(), ub,
      residual.has_value() ? residual->data_ptr() : nullptr, T, H, code_of(input.scalar_type()),
      (float)epsilon, group_size, is_scale_transposed ? 1 : 0, stream_of(input)));
}

// op/vllm/quantization/compressed_tensors/int8_quant_kernels.cu:459-527
void c_int8_quant(Tensor& result, const Tensor& input, Tensor& scale, const OptTensor& azp) {
  const char* name = "dynamic_scaled_int8_quant";
  TORCH_CHECK(input.is_contiguous(), "Expected input.is_contiguous() to be true, but got false.");
  TORCH_CHECK(result.is_contiguous(), "Expected out.is_contiguous() to be true, but got false.");
  TORCH_CHECK(scale.is_contiguous(), "Expected scales.is_contiguous() to be true, but got "
                                     "false.");
  TORCH_CHECK(!azp.has_value() || azp->is_contiguous(),
              "Expected !azp || azp->is_contiguous() to be true, but got false.");
  dispatch_check(input.scalar_type(), "dynamic_scaled_int8_quant_kernel");
  TORCH_CHECK(result.scalar_type() == at::kChar, "expected scalar type Char but found ",
              result.scalar_type());
  TORCH_CHECK(scale.scalar_type() == at::kFloat, "expected scalar type Float but found ",
              scale.scalar_type());
  if (azp.has_value()) {
    TORCH_CHECK(azp->scalar_type() == at::kInt, "expected scalar type Int but found ",
                azp->scalar_type());
  }
  on_device(name, {&result, &input, &scale, opt(azp)});
  const auto [T, H] = rows_of(input);
  numel_check(name, "result", result, T * H);
  numel_check(name, "scale", scale, T);
  if (azp.has_value()) numel_check(name, "azp", *azp, T);
  const DeviceGuard guard(input.device());
  check_rc(mcop_dynamic_scaled_int8_quant(
      static_cast<int8_t*>(result.data_ptr()), scale.data_ptr<float>(),
      azp.has_value() ? azp->data_ptr<int32_t>() : nullptr, input.data_ptr(), T, H,
      code_of(input.scalar_type()), stream_of(input)));
}

// op/vllm/quantization/fp8/common.cu:375-411
void c_fp8_quant(Tensor& result, const Tensor& input, Tensor& scale, const OptTensor& scale_ub) {
  const char* name = "dynamic_per_token_scaled_fp8_quant";
  TORCH_CHECK(input.stride(-1) == 1, "last dimension of input must be contiguous");
  TORCH_CHECK(result.stride(-1) == 1, "last dimension of output must be contiguous");
  dispatch_check(input.scalar_type(), "dynamic_per_token_scaled_fp8_quant_kernel_scalar_type");
  TORCH_CHECK(result.scalar_type() == at::kFloat8_e4m3fn,
              "\"dynamic_per_token_scaled_fp8_quant_kernel_fp8_type\" not implemented for '",
              c10::toString(result.scalar_type()), "'");
  TORCH_CHECK(scale.scalar_type() == at::kFloat, "expected scalar type Float but found ",
              scale.scalar_type());
  on_device(name, {&result, &input, &scale, opt(scale_ub)});
  const auto [T, H] = rows_of(input);
  TORCH_CHECK(result.sizes() == input.sizes(), name, ": result shape ", result.sizes(),
              " != input shape ", input.sizes());
  numel_check(name, "scale", scale, T);
  contiguous_check(name, "scale", scale);
  const float* ub = ub_ptr(name, scale_ub);
  const int64_t in_stride = row_stride(name, input, T, H);
  const int64_t out_stride = row_stride(name, result, T, H);
  const DeviceGuard guard(input.device());
  check_rc(mcop_dynamic_per_token_scaled_fp8_quant(
      static_cast<uint8_t*>(result.data_ptr()), scale.data_ptr<float>(), input.data_ptr(), ub, T,
      H, in_stride, out_stride, code_of(input.scalar_type()), stream_of(input)));
}

// Meta kernel of the mutating _C ops (no outputs to describe): drop the arguments.
void meta_noop(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  torch::jit::drop(*stack, op.schema().arguments().size());
}

struct VllmOp {
  const char* name;
  const char* schema;
};
constexpr VllmOp kVllmOps[] = {
    {"rms_norm", "rms_norm(Tensor! result, Tensor input, Tensor weight, float epsilon) -> ()"},
    {"fused_add_rms_norm",
     "fused_add_rms_norm(Tensor! input, Tensor! residual, Tensor weight, float epsilon) -> ()"},
    {"rms_norm_dynamic_per_token_quant",
     "rms_norm_dynamic_per_token_quant(Tensor! result, Tensor input, Tensor weight, "
     "Tensor! scale, float epsilon, Tensor? scale_ub, Tensor!? residual) -> ()"},
    {"rms_norm_per_block_quant",
     "rms_norm_per_block_quant(Tensor! result, Tensor input, Tensor weight, Tensor! scale, "
     "float epsilon, Tensor? scale_ub, Tensor!? residual, int group_size, "
     "bool is_scale_transposed) -> ()"},
    {"dynamic_scaled_int8_quant",
     "dynamic_scaled_int8_quant(Tensor! result, Tensor input, Tensor! scale, Tensor!? azp) -> ()"},
    {"dynamic_per_token_scaled_fp8_quant",
     "dynamic_per_token_scaled_fp8_quant(Tensor! result, Tensor input, Tensor! scale, "
     "Tensor? scale_ub) -> ()"},
};

// Registers the _C schemas (each only if no other library, e.g. vLLM's own _C, defined it) with
// CUDA implementations here and a Meta kernel for the schemas defined here.  Idempotent.
void register_vllm_ops() {
  static bool done = false;
  if (done) return;
  static std::unique_ptr<torch::Library> defs, cuda, meta;
  defs = std::make_unique<torch::Library>(torch::Library::FRAGMENT, "_C", std::nullopt, __FILE__,
                                          __LINE__);
  meta = std::make_unique<torch::Library>(torch::Library::IMPL, "_C", c10::DispatchKey::Meta,
                                          __FILE__, __LINE__);
  for (const VllmOp& o : kVllmOps) {
    const std::string full = std::string("_C::") + o.name;
    if (!c10::Dispatcher::singleton().findSchema({full, ""}).has_value()) {
      defs->def(o.schema);
      meta->impl(o.name, torch::CppFunction::makeFromBoxedFunction<&meta_noop>());
    }
  }
  cuda = std::make_unique<torch::Library>(torch::Library::IMPL, "_C", c10::DispatchKey::CUDA,
                                          __FILE__, __LINE__);
  cuda->impl("rms_norm", TORCH_FN(c_rms_norm));
  cuda->impl("fused_add_rms_norm", TORCH_FN(c_fused_add_rms_norm));
  cuda->impl("rms_norm_dynamic_per_token_quant", TORCH_FN(c_norm_quant));
  cuda->impl("rms_norm_per_block_quant", TORCH_FN(c_per_block_quant));
  cuda->impl("dynamic_scaled_int8_quant", TORCH_FN(c_int8_quant));
  cuda->impl("dynamic_per_token_scaled_fp8_quant", TORCH_FN(c_fp8_quant));
  done = true;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "mcoplib.op and torch.ops._C surfaces of the fused RMSNorm + quantization path "
            "over libmcop_norm.so (gfx950)";
  // mcoplib.op
  m.def("rms_norm_dynamic_per_token_quant", &op_smooth_quant,
        "SmoothQuant (residual add +) RMSNorm + dynamic per-token quantization "
        "(fused_rms_norm_dq; reference op/fused_rms_norm_dq.cu:646-667).\n\n"
        "after_res <- input (+ residual); after_norm <- after_res / rsqrt(mean(after_res^2) + "
        "eps) * weight (the reference's literal form; standard_norm=True multiplies by the "
        "rsqrt instead); out <- per-token quantization of after_norm * smooth_scale; scales[t] "
        "<- absmax/127 (int8) or absmax/448 (fp8-e4m3fn, an extension: the reference accepts "
        "int8 only).  residual is read, not updated; weight and smooth_scale are each the "
        "input dtype or fp32.",
        py::arg("out"), py::arg("input"), py::arg("weight"), py::arg("smooth_scale"),
        py::arg("scales"), py::arg("var_epsilon"), py::arg("after_res"), py::arg("after_norm"),
        py::arg("residual") = py::none(), py::arg("standard_norm") = false);
  m.def("rms_norm_dynamic_per_token_quant_custom", &op_custom,
        "(Residual add +) RMSNorm + dynamic per-token int8 quantization with mcoplib's own "
        "arithmetic (reference op/rms_norm_dynamic_per_token_quant.cu:266-285): scale floor "
        "1.5e-6 and codes in [-127, 127]; at H == 7168 the reference's fp32 chain (codes from "
        "(x [+ r]) * w * rsqrt(...) without bf16 rounding, scale_ub unused).  residual is "
        "updated in place to input + residual; out and scales ([T] or [T, 1] fp32) are "
        "written.",
        py::arg("out"), py::arg("input"), py::arg("weight"), py::arg("scales"),
        py::arg("var_epsilon"), py::arg("scale_ub") = py::none(),
        py::arg("residual") = py::none());
  m.def("scale_dynamic_quant", &op_scale_dynamic_quant,
        "Smooth-scale multiply + dynamic per-token int8 quantization (reference "
        "op/scale_dynamic_quant.cu:127-153).  Returns new (codes shaped like hidden_states, "
        "scales [T] fp32).",
        py::arg("hidden_states"), py::arg("smooth_scales"), py::arg("dst_dtype") = py::none());
  m.def("fused_add_rms_norm_dynamic_per_token_quant_padding_output", &op_padded,
        "Residual add + RMSNorm + per-token int8 quantization with a padded per-row output "
        "(reference op/fused_add_layernorm_per_token_quant_padding_output.cu:397-416).\n\n"
        "output (int8, 2*pad_size bytes per row) receives each row's codes at bytes [0, H) and "
        "its fp32 scale at bytes [H, H+4); output_rms (bf16) the normalized row, "
        "output_quant_int8 the codes again, out_scales the scales; residual becomes input + "
        "residual.  H == 7168 uses the reference's fp32 chain (its \"opt\" kernel), other H its "
        "bf16-rounded chain; every output is written for every H.",
        py::arg("output"), py::arg("output_rms"), py::arg("output_quant_int8"),
        py::arg("out_scales"), py::arg("input"), py::arg("residual"), py::arg("weight"),
        py::arg("pad_size"), py::arg("epsilon"));
  m.def("rms_norm", &op_rms_norm,
        "(Residual add +) RMSNorm (reference op/fused_rms_norm_dq.cu:980-998): out <- (input [+ "
        "residual]) / rsqrt(mean(.^2) + eps) * weight when rms_div (the reference's "
        "convention), or * rsqrt(...) * weight otherwise; with a residual, after_res <- input "
        "+ residual (the residual itself is not updated).  weight is the input dtype or fp32.",
        py::arg("out"), py::arg("input"), py::arg("weight"), py::arg("var_epsilon"),
        py::arg("after_res") = py::none(), py::arg("residual") = py::none(),
        py::arg("rms_div") = true);
  m.def("head_rms_norm", &op_head_rms_norm,
        "Per-head RMSNorm of heads [head_offset, head_offset + head_norm) of hidden_states "
        "[num_tokens, num_heads, head_size] with per-head weights [num_heads, head_size] (bf16 "
        "or fp32); out (same shape) is written for those heads only (reference "
        "op/fused_rms_norm_dq.cu:804-812), as x / rsqrt(mean(x^2) + eps) * weight.",
        py::arg("out"), py::arg("hidden_states"), py::arg("weight"), py::arg("var_epsilon"),
        py::arg("head_offset"), py::arg("head_norm"));
  // torch.ops._C
  m.def("register_vllm_ops", &register_vllm_ops,
        "Register the torch.ops._C schemas and their CUDA (HIP) implementations (idempotent).");
  m.def("c_rms_norm", &c_rms_norm, py::arg("result"), py::arg("input"), py::arg("weight"),
        py::arg("epsilon"));
  m.def("c_fused_add_rms_norm", &c_fused_add_rms_norm, py::arg("input"), py::arg("residual"),
        py::arg("weight"), py::arg("epsilon"));
  m.def("c_rms_norm_dynamic_per_token_quant", &c_norm_quant, py::arg("result"),
        py::arg("input"), py::arg("weight"), py::arg("scale"), py::arg("epsilon"),
        py::arg("scale_ub") = py::none(), py::arg("residual") = py::none());
  m.def("c_rms_norm_per_block_quant", &c_per_block_quant, py::arg("result"), py::arg("input"),
        py::arg("weight"), py::arg("scale"), py::arg("epsilon"), py::arg("scale_ub"),
        py::arg("residual"), py::arg("group_size"), py::arg("is_scale_transposed"));
  m.def("c_dynamic_scaled_int8_quant", &c_int8_quant, py::arg("result"), py::arg("input"),
        py::arg("scale"), py::arg("azp") = py::none());
  m.def("c_dynamic_per_token_scaled_fp8_quant", &c_fp8_quant, py::arg("result"),
        py::arg("input"), py::arg("scale"), py::arg("scale_ub") = py::none());
}
