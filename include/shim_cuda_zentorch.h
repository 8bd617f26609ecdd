/*
 * shim_cuda_zentorch.h -- AOTInductor C shims for zentorch's quantized-linear
 * ops on the GPU (exported by zentorch/_C.so).
 *
 * Each function mirrors the reference's aoti_torch_cpu_zentorch_* shim of the
 * same suffix (src/cpu/cpp/shim_cpu_zentorch.hpp:150-197, bodies
 * shim_cpu_zentorch.cpp:367-513) with an identical argument list: tensors are
 * borrowed AtenTensorHandles, an optional tensor is an AtenTensorHandle*
 * (NULL = None), the result is a new handle owned by the caller, and C++
 * exceptions become AOTI_TORCH_FAILURE.  Only the device differs: "cuda" is
 * PyTorch-ROCm's name for the HIP device.
 */
#ifndef SHIM_CUDA_ZENTORCH_H
#define SHIM_CUDA_ZENTORCH_H

#include <torch/csrc/inductor/aoti_torch/c/shim.h>

#ifdef __cplusplus
extern "C" {
#endif

/* shim_cpu_zentorch.hpp:150-153 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:155-158 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_relu(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:160-163 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_sigmoid(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:165-168 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_gelu_tanh(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:170-173 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_gelu_erf(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:175-178 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle add_input,
    AtenTensorHandle *B, const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:180-184 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_mul_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle mul_input,
    AtenTensorHandle add_input, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:186-190 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_add_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle add_input,
    AtenTensorHandle add_input_2, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* No reference counterpart: shim of the zentorch_woq_linear_silu_mul
 * extension, shaped like the _add shim. */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_silu_mul(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle mul_input,
    AtenTensorHandle *B, const char *zentorch_op_name, AtenTensorHandle *ret0);

/* No reference counterpart: shim of the zentorch_woq_linear_gate_up_silu_mul
 * extension (merged gate_up weight, output silu(gate) * up). */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_woq_linear_gate_up_silu_mul(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *weight_zero_points, AtenTensorHandle *B,
    const char *zentorch_op_name, AtenTensorHandle *ret0);

/* shim_cpu_zentorch.hpp:195-197 */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_dynamic_qlinear(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle *B, const char *zentorch_op_name, AtenTensorHandle *ret0);

/* No reference counterpart: shims of the dynamic-qlinear extensions with a
 * fused silu * mul or residual add, shaped like the dynamic_qlinear shim with
 * the binary operand after the weight scales. */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_dynamic_qlinear_silu_mul(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle mul_input, AtenTensorHandle *B, const char *zentorch_op_name,
    AtenTensorHandle *ret0);

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_dynamic_qlinear_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle weight_scales,
    AtenTensorHandle add_input, AtenTensorHandle *B, const char *zentorch_op_name,
    AtenTensorHandle *ret0);

/* Static int8 qlinear: shim_cpu_zentorch.hpp:28-74.  X_zero_points and
 * W_zero_points may be uninitialized handles (None); output_dtype is a
 * c10::ScalarType code or NULL (None). */
AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_qlinear(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,
    AtenTensorHandle X_zero_points, AtenTensorHandle W_scales,
    AtenTensorHandle W_zero_points, AtenTensorHandle *B,
    AtenTensorHandle *output_scales, AtenTensorHandle *output_zero_points,
    const int32_t *output_dtype, const char *zentorch_op_name,
    AtenTensorHandle *ret0);

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_qlinear_relu(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,
    AtenTensorHandle X_zero_points, AtenTensorHandle W_scales,
    AtenTensorHandle W_zero_points, AtenTensorHandle *B,
    AtenTensorHandle *output_scales, AtenTensorHandle *output_zero_points,
    const int32_t *output_dtype, const char *zentorch_op_name,
    AtenTensorHandle *ret0);

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_qlinear_sigmoid(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,
    AtenTensorHandle X_zero_points, AtenTensorHandle W_scales,
    AtenTensorHandle W_zero_points, AtenTensorHandle *B,
    AtenTensorHandle *output_scales, AtenTensorHandle *output_zero_points,
    const int32_t *output_dtype, const char *zentorch_op_name,
    AtenTensorHandle *ret0);

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_qlinear_mul_add(
    AtenTensorHandle X, AtenTensorHandle W, AtenTensorHandle X_scales,
    AtenTensorHandle X_zero_points, AtenTensorHandle W_scales,
    AtenTensorHandle W_zero_points, AtenTensorHandle mul_input,
    AtenTensorHandle add_input, AtenTensorHandle *B,
    AtenTensorHandle *output_scales, AtenTensorHandle *output_zero_points,
    const int32_t *output_dtype, const char *zentorch_op_name,
    AtenTensorHandle *ret0);

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_qlinear_out(
    AtenTensorHandle out, AtenTensorHandle X, AtenTensorHandle W,
    AtenTensorHandle X_scales, AtenTensorHandle X_zero_points,
    AtenTensorHandle W_scales, AtenTensorHandle W_zero_points,
    AtenTensorHandle *B, AtenTensorHandle *output_scales,
    AtenTensorHandle *output_zero_points, const int32_t *output_dtype,
    const char *zentorch_op_name);

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_zentorch_qlinear_relu_out(
    AtenTensorHandle out, AtenTensorHandle X, AtenTensorHandle W,
    AtenTensorHandle X_scales, AtenTensorHandle X_zero_points,
    AtenTensorHandle W_scales, AtenTensorHandle W_zero_points,
    AtenTensorHandle *B, AtenTensorHandle *output_scales,
    AtenTensorHandle *output_zero_points, const int32_t *output_dtype,
    const char *zentorch_op_name);

#ifdef __cplusplus
}
#endif

#endif /* SHIM_CUDA_ZENTORCH_H */
