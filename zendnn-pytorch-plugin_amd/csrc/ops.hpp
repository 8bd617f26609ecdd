// Op bodies shared by the TORCH_LIBRARY registration (ops.cpp) and the
// AOTInductor C shims (shim_cuda_zentorch.cpp).
#pragma once

#include <ATen/ATen.h>

#include "zentorch_hip.h"

namespace zentorch_hip {

template <int32_t UNARY>
at::Tensor woq_linear_unary(const at::Tensor &input, const at::Tensor &weight,
                            const at::Tensor &weight_scales,
                            const c10::optional<at::Tensor> &weight_zero_points,
                            const c10::optional<at::Tensor> &bias,
                            c10::string_view zentorch_op_name);
extern template at::Tensor woq_linear_unary<ZT_PO_NONE>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
extern template at::Tensor woq_linear_unary<ZT_PO_RELU>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
extern template at::Tensor woq_linear_unary<ZT_PO_SIGMOID>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
extern template at::Tensor woq_linear_unary<ZT_PO_GELU_TANH>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
extern template at::Tensor woq_linear_unary<ZT_PO_GELU_ERF>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);

at::Tensor woq_linear_add(const at::Tensor &input, const at::Tensor &weight,
                          const at::Tensor &weight_scales,
                          const c10::optional<at::Tensor> &weight_zero_points,
                          const at::Tensor &add_input,
                          const c10::optional<at::Tensor> &bias,
                          c10::string_view zentorch_op_name);
at::Tensor woq_linear_mul_add(const at::Tensor &input, const at::Tensor &weight,
                              const at::Tensor &weight_scales,
                              const c10::optional<at::Tensor> &weight_zero_points,
                              const at::Tensor &mul_input,
                              const at::Tensor &add_input,
                              const c10::optional<at::Tensor> &bias,
                              c10::string_view zentorch_op_name);
at::Tensor woq_linear_add_add(const at::Tensor &input, const at::Tensor &weight,
                              const at::Tensor &weight_scales,
                              const c10::optional<at::Tensor> &weight_zero_points,
                              const at::Tensor &add_input,
                              const at::Tensor &add_input_2,
                              const c10::optional<at::Tensor> &bias,
                              c10::string_view zentorch_op_name);
at::Tensor woq_linear_gate_up_silu_mul(const at::Tensor &input, const at::Tensor &weight,
                                       const at::Tensor &weight_scales,
                                       const c10::optional<at::Tensor> &weight_zero_points,
                                       const c10::optional<at::Tensor> &bias,
                                       c10::string_view zentorch_op_name);
at::Tensor woq_linear_silu_mul(const at::Tensor &input, const at::Tensor &weight,
                               const at::Tensor &weight_scales,
                               const c10::optional<at::Tensor> &weight_zero_points,
                               const at::Tensor &mul_input,
                               const c10::optional<at::Tensor> &bias,
                               c10::string_view zentorch_op_name);
at::Tensor woq_repack_weight(const at::Tensor &unpacked_weight);
at::Tensor woq_repack_from_int4pack(const at::Tensor &packed_weight);
at::Tensor dynamic_qlinear(const at::Tensor &input, const at::Tensor &weight,
                           const at::Tensor &weight_scales,
                           const c10::optional<at::Tensor> &bias,
                           c10::string_view zentorch_op_name);
at::Tensor dynamic_qlinear_silu_mul(const at::Tensor &input, const at::Tensor &weight,
                                    const at::Tensor &weight_scales, const at::Tensor &mul_input,
                                    const c10::optional<at::Tensor> &bias,
                                    c10::string_view zentorch_op_name);
at::Tensor dynamic_qlinear_add(const at::Tensor &input, const at::Tensor &weight,
                               const at::Tensor &weight_scales, const at::Tensor &add_input,
                               const c10::optional<at::Tensor> &bias,
                               c10::string_view zentorch_op_name);
at::Tensor dynamic_qlinear_asym(const at::Tensor &input, const at::Tensor &weight,
                                const at::Tensor &weight_scales, const at::Tensor &weight_colsum,
                                const c10::optional<at::Tensor> &bias,
                                c10::string_view zentorch_op_name);
at::Tensor s8_weight_colsum(const at::Tensor &weight);

// static int8 qlinear (QLinear.cpp:367-573)
template <int32_t PO>
at::Tensor qlinear_unary(const at::Tensor &input, const at::Tensor &weight,
                         const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                         const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                         const c10::optional<at::Tensor> &bias,
                         const c10::optional<at::Tensor> &output_scales,
                         const c10::optional<at::Tensor> &output_zero_points,
                         c10::optional<c10::ScalarType> output_dtype,
                         c10::string_view zentorch_op_name);
template <int32_t PO>
void qlinear_unary_out(at::Tensor &out, const at::Tensor &input, const at::Tensor &weight,
                       const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                       const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                       const c10::optional<at::Tensor> &bias,
                       const c10::optional<at::Tensor> &output_scales,
                       const c10::optional<at::Tensor> &output_zero_points,
                       c10::optional<c10::ScalarType> output_dtype,
                       c10::string_view zentorch_op_name);
#define ZT_QLIN_EXTERN(PO_)                                                                     \
  extern template at::Tensor qlinear_unary<PO_>(                                                \
      const at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &,           \
      const at::Tensor &, const at::Tensor &, const c10::optional<at::Tensor> &,                \
      const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,                     \
      c10::optional<c10::ScalarType>, c10::string_view);                                        \
  extern template void qlinear_unary_out<PO_>(                                                  \
      at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &,                 \
      const at::Tensor &, const at::Tensor &, const at::Tensor &,                               \
      const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,                     \
      const c10::optional<at::Tensor> &, c10::optional<c10::ScalarType>, c10::string_view);
ZT_QLIN_EXTERN(ZT_PO_NONE)
ZT_QLIN_EXTERN(ZT_PO_RELU)
ZT_QLIN_EXTERN(ZT_PO_SIGMOID)
#undef ZT_QLIN_EXTERN
at::Tensor qlinear_mul_add(const at::Tensor &input, const at::Tensor &weight,
                           const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                           const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                           const at::Tensor &mul_input, const at::Tensor &add_input,
                           const c10::optional<at::Tensor> &bias,
                           const c10::optional<at::Tensor> &output_scales,
                           const c10::optional<at::Tensor> &output_zero_points,
                           c10::optional<c10::ScalarType> output_dtype,
                           c10::string_view zentorch_op_name);

}  // namespace zentorch_hip
