// AOTInductor C shims (include/shim_cuda_zentorch.h): borrow the handles,
// call the op body, hand the result back as a new handle, and turn C++
// exceptions into AOTI_TORCH_FAILURE, as the reference's CPU shims do
// (src/cpu/cpp/shim_cpu_zentorch.cpp:367-513).
#include <torch/csrc/inductor/aoti_torch/utils.h>

#include "ops.hpp"
#include "shim_cuda_zentorch.h"

using torch::aot_inductor::new_tensor_handle;
using torch::aot_inductor::pointer_to_optional;
using torch::aot_inductor::tensor_handle_to_tensor_pointer;

#define ZT_T(h) (*tensor_handle_to_tensor_pointer(h))
#define ZT_OPT(h) pointer_to_optional<at::Tensor>(h)

#define ZT_UNARY_SHIM(suffix, ID)                                             \
  AOTITorchError aoti_torch_cuda_zentorch_woq_linear##suffix(                 \
      AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales, \
      AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,              \
      const char *zentorch_op_name, AtenTensorHandle *ret0) {                 \
    AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({                              \
      auto r = zentorch_hip::woq_linear_unary<ID>(                            \
          ZT_T(X), ZT_T(W), ZT_T(weight_scales), ZT_OPT(weight_zero_points),  \
          ZT_OPT(B), zentorch_op_name);                                       \
      *ret0 = new_tensor_handle(std::move(r));                                \
    });                                                                       \
  }

extern "C" {

ZT_UNARY_SHIM(, ZT_PO_NONE)
ZT_UNARY_SHIM(_relu, ZT_PO_RELU)
ZT_UNARY_SHIM(_sigmoid, ZT_PO_SIGMOID)
ZT_UNARY_SHIM(_gelu_tanh, ZT_PO_GELU_TANH)
ZT_UNARY_SHIM(_gelu_erf, ZT_PO_GELU_ERF)

AOTITorchError aoti_torch_cuda_zentorch_woq_linear_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle add_input,
    AtenTensorHandle *B, const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::woq_linear_add(
        ZT_T(X), ZT_T(W), ZT_T(weight_scales), ZT_OPT(weight_zero_points),
        ZT_T(add_input), ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_woq_linear_mul_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle mul_input,
    AtenTensorHandle add_input, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::woq_linear_mul_add(
        ZT_T(X), ZT_T(W), ZT_T(weight_scales), ZT_OPT(weight_zero_points),
        ZT_T(mul_input), ZT_T(add_input), ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_woq_linear_add_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle add_input,
    AtenTensorHandle add_input_2, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::woq_linear_add_add(
        ZT_T(X), ZT_T(W), ZT_T(weight_scales), ZT_OPT(weight_zero_points),
        ZT_T(add_input), ZT_T(add_input_2), ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_woq_linear_silu_mul(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle mul_input,
    AtenTensorHandle *B, const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::woq_linear_silu_mul(
        ZT_T(X), ZT_T(W), ZT_T(weight_scales), ZT_OPT(weight_zero_points),
        ZT_T(mul_input), ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_woq_linear_gate_up_silu_mul(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B, const char *zentorch_op_name,
    AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::woq_linear_gate_up_silu_mul(
        ZT_T(X), ZT_T(W), ZT_T(weight_scales), ZT_OPT(weight_zero_points), ZT_OPT(B),
        zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_dynamic_qlinear(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *B, const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::dynamic_qlinear(ZT_T(X), ZT_T(W), ZT_T(weight_scales),
                                           ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_dynamic_qlinear_silu_mul(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle mul_input, AtenTensorHandle *B, const char *zentorch_op_name,
    AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::dynamic_qlinear_silu_mul(ZT_T(X), ZT_T(W), ZT_T(weight_scales),
                                                    ZT_T(mul_input), ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_dynamic_qlinear_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle add_input, AtenTensorHandle *B, const char *zentorch_op_name,
    AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::dynamic_qlinear_add(ZT_T(X), ZT_T(W), ZT_T(weight_scales),
                                               ZT_T(add_input), ZT_OPT(B), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

// static int8 qlinear (shim_cpu_zentorch.cpp:72-190 of the reference)
#define ZT_DTYPE_OPT(p)                                                         \
  ((p) ? c10::optional<c10::ScalarType>(static_cast<c10::ScalarType>(*(p)))      \
       : c10::optional<c10::ScalarType>())

#define ZT_QLINEAR_SHIM(NAME, PO)                                                           \
  AOTITorchError aoti_torch_cuda_zentorch_##NAME(                                           \
      AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,                    \
      AtenTensorHandle X_zero_points, AtenTensorHandle W_scales,                            \
      AtenTensorHandle W_zero_points, AtenTensorHandle *B, AtenTensorHandle *output_scales, \
      AtenTensorHandle *output_zero_points, const int32_t *output_dtype,                    \
      const char *zentorch_op_name, AtenTensorHandle *ret0) {                               \
    AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({                                            \
      auto r = zentorch_hip::qlinear_unary<PO>(                                             \
          ZT_T(X), ZT_T(W), ZT_T(X_scales), ZT_T(X_zero_points), ZT_T(W_scales),            \
          ZT_T(W_zero_points), ZT_OPT(B), ZT_OPT(output_scales), ZT_OPT(output_zero_points), \
          ZT_DTYPE_OPT(output_dtype), zentorch_op_name);                                    \
      *ret0 = new_tensor_handle(std::move(r));                                              \
    });                                                                                     \
  }                                                                                         \
  AOTITorchError aoti_torch_cuda_zentorch_##NAME##_out(                                     \
      AtenTensorHandle out, AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales, \
      AtenTensorHandle X_zero_points, AtenTensorHandle W_scales,                            \
      AtenTensorHandle W_zero_points, AtenTensorHandle *B, AtenTensorHandle *output_scales, \
      AtenTensorHandle *output_zero_points, const int32_t *output_dtype,                    \
      const char *zentorch_op_name) {                                                       \
    AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({                                            \
      zentorch_hip::qlinear_unary_out<PO>(                                                  \
          ZT_T(out), ZT_T(X), ZT_T(W), ZT_T(X_scales), ZT_T(X_zero_points), ZT_T(W_scales), \
          ZT_T(W_zero_points), ZT_OPT(B), ZT_OPT(output_scales), ZT_OPT(output_zero_points), \
          ZT_DTYPE_OPT(output_dtype), zentorch_op_name);                                    \
    });                                                                                     \
  }

ZT_QLINEAR_SHIM(qlinear, ZT_PO_NONE)
ZT_QLINEAR_SHIM(qlinear_relu, ZT_PO_RELU)
#undef ZT_QLINEAR_SHIM

AOTITorchError aoti_torch_cuda_zentorch_qlinear_sigmoid(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,
    AtenTensorHandle X_zero_points, AtenTensorHandle W_scales, AtenTensorHandle W_zero_points,
    AtenTensorHandle *B, AtenTensorHandle *output_scales, AtenTensorHandle *output_zero_points,
    const int32_t *output_dtype, const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::qlinear_unary<ZT_PO_SIGMOID>(
        ZT_T(X), ZT_T(W), ZT_T(X_scales), ZT_T(X_zero_points), ZT_T(W_scales),
        ZT_T(W_zero_points), ZT_OPT(B), ZT_OPT(output_scales), ZT_OPT(output_zero_points),
        ZT_DTYPE_OPT(output_dtype), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

AOTITorchError aoti_torch_cuda_zentorch_qlinear_mul_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,
    AtenTensorHandle X_zero_points, AtenTensorHandle W_scales, AtenTensorHandle W_zero_points,
    AtenTensorHandle mul_input, AtenTensorHandle add_input, AtenTensorHandle *B,
    AtenTensorHandle *output_scales, AtenTensorHandle *output_zero_points,
    const int32_t *output_dtype, const char *zentorch_op_name, AtenTensorHandle *ret0) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    auto r = zentorch_hip::qlinear_mul_add(
        ZT_T(X), ZT_T(W), ZT_T(X_scales), ZT_T(X_zero_points), ZT_T(W_scales),
        ZT_T(W_zero_points), ZT_T(mul_input), ZT_T(add_input), ZT_OPT(B), ZT_OPT(output_scales),
        ZT_OPT(output_zero_points), ZT_DTYPE_OPT(output_dtype), zentorch_op_name);
    *ret0 = new_tensor_handle(std::move(r));
  });
}

}  // extern "C"
