"""Meta (shape/dtype) kernels for the zentorch quantized-linear ops, so
FakeTensor tracing and Inductor see the output layout without running the GPU
kernels.  Shapes follow the reference's meta kernels
(src/cpu/python/zentorch/_meta_registrations.py:552-772).
"""
import functools

import torch


@functools.lru_cache(None)
def _meta_lib():
    return torch.library.Library("zentorch", "IMPL", "Meta")


def register_meta(op_name, overload_name="default"):
    def wrapper(fn):
        _meta_lib().impl(getattr(getattr(torch.ops.zentorch, op_name), overload_name), fn)
        return fn
    return wrapper


def _woq_out(input, weight):
    # [*, N] with N = weight.shape[1], input dtype (_meta_registrations.py:561-563)
    out = list(input.size())
    out[-1] = weight.shape[1]
    return input.new_empty(out, dtype=input.dtype)


@register_meta("zentorch_woq_linear")
def meta_zentorch_woq_linear(input, weight, weight_scales, weight_zero_points=None,
                             bias=None, zentorch_op_name="zentorch::zentorch_woq_linear"):
    return _woq_out(input, weight)


for _suffix in ("relu", "sigmoid", "gelu_tanh", "gelu_erf"):
    register_meta(f"zentorch_woq_linear_{_suffix}")(
        lambda input, weight, weight_scales, weight_zero_points=None, bias=None,
        zentorch_op_name="": _woq_out(input, weight))


@register_meta("zentorch_woq_linear_add")
def meta_zentorch_woq_linear_add(input, weight, weight_scales, weight_zero_points,
                                 add_input, bias=None, zentorch_op_name=""):
    return _woq_out(input, weight)


@register_meta("zentorch_woq_linear_mul_add")
def meta_zentorch_woq_linear_mul_add(input, weight, weight_scales, weight_zero_points,
                                     mul_input, add_input, bias=None, zentorch_op_name=""):
    return _woq_out(input, weight)


@register_meta("zentorch_woq_linear_add_add")
def meta_zentorch_woq_linear_add_add(input, weight, weight_scales, weight_zero_points,
                                     add_input, add_input_2, bias=None, zentorch_op_name=""):
    return _woq_out(input, weight)


@register_meta("zentorch_woq_linear_silu_mul")
def meta_zentorch_woq_linear_silu_mul(input, weight, weight_scales, weight_zero_points,
                                      mul_input, bias=None, zentorch_op_name=""):
    return _woq_out(input, weight)


@register_meta("zentorch_woq_linear_gate_up_silu_mul")
def meta_zentorch_woq_linear_gate_up_silu_mul(input, weight, weight_scales, weight_zero_points,
                                              bias=None, zentorch_op_name=""):
    # merged gate_up weight [K/8, 2I] -> output [*, I]
    out = list(input.size())
    out[-1] = weight.size(1) // 2
    return input.new_empty(out)


@register_meta("zentorch_dynamic_qlinear")
def meta_zentorch_dynamic_qlinear(input, weight, weight_scales, bias=None,
                                  zentorch_op_name="zentorch::zentorch_dynamic_qlinear"):
    out = list(input.size())
    out[-1] = weight.size(0)
    return input.new_empty(out)


@register_meta("zentorch_dynamic_qlinear_silu_mul")
def meta_zentorch_dynamic_qlinear_silu_mul(input, weight, weight_scales, mul_input, bias=None,
                                           zentorch_op_name=""):
    return meta_zentorch_dynamic_qlinear(input, weight, weight_scales, bias)


@register_meta("zentorch_dynamic_qlinear_add")
def meta_zentorch_dynamic_qlinear_add(input, weight, weight_scales, add_input, bias=None,
                                      zentorch_op_name=""):
    return meta_zentorch_dynamic_qlinear(input, weight, weight_scales, bias)


@register_meta("zentorch_dynamic_qlinear_asym")
def meta_zentorch_dynamic_qlinear_asym(input, weight, weight_scales, weight_colsum, bias=None,
                                       zentorch_op_name=""):
    return meta_zentorch_dynamic_qlinear(input, weight, weight_scales, bias)


@register_meta("zentorch_s8_weight_colsum")
def meta_zentorch_s8_weight_colsum(weight):
    return weight.new_empty((weight.size(0),), dtype=torch.int32)


def _qlinear_out(input, weight, output_dtype):
    out = list(input.size())
    out[-1] = weight.size(0)
    return input.new_empty(out, dtype=output_dtype or torch.float32)


@register_meta("zentorch_qlinear")
def meta_zentorch_qlinear(input, weight, input_scales, input_zero_points, weight_scales,
                          weight_zero_points, bias=None, output_scales=None,
                          output_zero_points=None, output_dtype=None, zentorch_op_name=""):
    return _qlinear_out(input, weight, output_dtype)


@register_meta("zentorch_qlinear_relu")
def meta_zentorch_qlinear_relu(input, weight, input_scales, input_zero_points, weight_scales,
                               weight_zero_points, bias=None, output_scales=None,
                               output_zero_points=None, output_dtype=None, zentorch_op_name=""):
    return _qlinear_out(input, weight, output_dtype)


@register_meta("zentorch_qlinear_sigmoid")
def meta_zentorch_qlinear_sigmoid(input, weight, input_scales, input_zero_points,
                                  weight_scales, weight_zero_points, bias=None,
                                  output_scales=None, output_zero_points=None,
                                  output_dtype=None, zentorch_op_name=""):
    return _qlinear_out(input, weight, output_dtype)


@register_meta("zentorch_qlinear_mul_add")
def meta_zentorch_qlinear_mul_add(input, weight, input_scales, input_zero_points,
                                  weight_scales, weight_zero_points, mul_input, add_input,
                                  bias=None, output_scales=None, output_zero_points=None,
                                  output_dtype=None, zentorch_op_name=""):
    return _qlinear_out(input, weight, output_dtype)


@register_meta("zentorch_qlinear", "out")
def meta_zentorch_qlinear_out(out, *args, **kwargs):
    return None


@register_meta("zentorch_qlinear_relu", "out")
def meta_zentorch_qlinear_relu_out(out, *args, **kwargs):
    return None


@register_meta("zentorch_woq_repack_weight")
def meta_zentorch_woq_repack_weight(unpacked_weight):
    # [N, K/8] int32 (the reference's meta returns the input dtype, int8, which
    # disagrees with its own CPU kernel; int32 is what the kernel returns)
    return unpacked_weight.new_empty(
        (unpacked_weight.size(0), unpacked_weight.size(1) // 8), dtype=torch.int32)


@register_meta("zentorch_woq_repack_from_int4pack")
def meta_zentorch_woq_repack_from_int4pack(packed_weight):
    K = packed_weight.size(1) * 2
    return packed_weight.new_empty((packed_weight.size(0), K // 8), dtype=torch.int32)


@register_meta("zentorch_fused_moe")
def meta_zentorch_fused_moe(output, input, w13, w2, w13_bias, w2_bias, topk_weights, topk_id,
                            skip_weighted, act, w13_scales=None, w2_scales=None,
                            zentorch_op_name="zentorch::zentorch_fused_moe"):
    # writes `output` in place and returns nothing (FusedMoE.cpp:728-736)
    return None
