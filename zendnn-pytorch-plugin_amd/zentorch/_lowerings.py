"""Inductor lowerings of the zentorch quantized-linear ops onto their C shims.

A graph that Inductor compiles (``torch.compile`` with the default backend on
a model that calls ``torch.ops.zentorch.*``, or AOTInductor on an exported
program holding them) lowers each zentorch op to one ``ExternKernelAlloc``.
With ``cpp_wrapper`` (and in AOTInductor) the generated C++ calls
``aoti_torch_cuda_zentorch_<op>`` from include/shim_cuda_zentorch.h
directly, so no Python runs between the kernels; the Python wrapper calls
the torch op.  This follows the reference's WOQ lowerings
(src/cpu/python/zentorch/_lowerings.py:1399-1951: one ExternKernelAlloc
class per op with ``cpp_kernel_name="aoti_torch_cpu_zentorch_<op>"``, the
shim header included by the wrapper, optional tensors interleaved in schema
order, ``register_lowering(..., type_promotion_kind=None)``).  Here a single
class serves every op: the argument order, the output layout and the
operand strides come from the op's schema and the FX node's example values.

Operands keep the stride order they had when traced (the ops are tagged
``needs_fixed_stride_order``); the output is the contiguous tensor the op's
Meta kernel describes.
"""
import os
from typing import Any, List, Optional, Sequence

import sympy
import torch
from torch._inductor import ir
from torch._inductor.lowering import register_lowering
from torch._inductor.virtualized import V

_HERE = os.path.dirname(os.path.abspath(__file__))
SHIM_HEADER = os.path.normpath(
    os.path.join(_HERE, "..", "..", "include", "shim_cuda_zentorch.h"))

# ops with a shim of the same suffix in include/shim_cuda_zentorch.h
SHIM_OPS = (
    "woq_linear", "woq_linear_relu", "woq_linear_sigmoid", "woq_linear_gelu_tanh",
    "woq_linear_gelu_erf", "woq_linear_add", "woq_linear_mul_add", "woq_linear_add_add",
    "woq_linear_silu_mul", "woq_linear_gate_up_silu_mul", "dynamic_qlinear",
    "dynamic_qlinear_silu_mul", "dynamic_qlinear_add",
    "qlinear", "qlinear_relu", "qlinear_sigmoid", "qlinear_mul_add",
)


def _expr(s):
    return s.node.expr if isinstance(s, torch.SymInt) else sympy.Integer(int(s))


def _schema_values(op, args, kwargs) -> List[Any]:
    """Values of the op's positional schema arguments, defaults filled in."""
    pos = [a for a in op._schema.arguments if not a.kwarg_only]
    out = []
    for i, a in enumerate(pos):
        if i < len(args):
            out.append(args[i])
        elif a.name in kwargs:
            out.append(kwargs[a.name])
        else:
            out.append(a.default_value if a.has_default_value() else None)
    return out


class ZentorchShimKernel(ir.ExternKernelAlloc):
    """One zentorch op, called through ``aoti_torch_cuda_zentorch_<op>``.

    ``slots[i]`` is the index in ``inputs`` of the i-th positional schema
    argument, None when that (optional) argument is absent, or ``("const",
    value)`` for a non-tensor argument (qlinear's output_dtype).
    """

    def __init__(self, layout, inputs: Sequence[ir.IRNode], slots: List[Any],
                 op_name: Optional[str], op, shim: str) -> None:
        # op_name is None when the schema takes the name positionally (it is
        # then one of the constant slots)
        kw = {} if op_name is None else {"zentorch_op_name": op_name}
        super().__init__(layout, inputs, (), kw,
                         python_kernel_name=f"torch.ops.zentorch.{op._schema.name.split('::')[1]}"
                                            ".default",
                         cpp_kernel_name=shim,
                         ordered_kwargs_for_cpp_kernel=list(kw),
                         op_overload=op)
        self.slots = slots

    def codegen(self, wrapper) -> None:
        if V.graph.cpp_wrapper:
            if not os.path.exists(SHIM_HEADER):
                raise RuntimeError(f"zentorch: shim header {SHIM_HEADER} is missing")
            wrapper.include_extra_header(SHIM_HEADER)
        super().codegen(wrapper)

    def codegen_args(self) -> List[str]:
        wrapper = V.graph.wrapper_code
        vals = [None if s is None else (s[1] if isinstance(s, tuple) else self.inputs[s])
                for s in self.slots]
        if V.graph.cpp_wrapper:
            pos = [a for a in self.op_overload._schema.arguments if not a.kwarg_only]
            out = []
            for v, a in zip(vals, pos):
                if isinstance(v, torch.dtype):
                    # the shims take a ScalarType as const int32_t *
                    # (shim_cpu_zentorch.hpp:33 of the reference)
                    var = f"var_{next(wrapper.arg_var_id)}"
                    wrapper.writeline(f"int32_t {var} = {wrapper.codegen_dtype(v)};")
                    out.append(f"&{var}")
                else:
                    out.append(wrapper.val_to_arg_str(v, a.type))
            return out
        return [wrapper.val_to_arg_str(v) for v in vals]

    def apply_constraint(self) -> None:
        pass

    @classmethod
    def create(cls, op, shim: str, args, kwargs) -> "ZentorchShimKernel":
        fx_node = V.graph.current_node
        values = _schema_values(op, args, kwargs)
        examples = _schema_values(op, fx_node.args, fx_node.kwargs)
        inputs, slots = [], []
        pos = [a for a in op._schema.arguments if not a.kwarg_only]
        for v, ex, arg in zip(values, examples, pos):
            if v is None:
                slots.append(None)
                continue
            if not isinstance(arg.type, (torch.TensorType, torch.OptionalType)) or (
                    isinstance(arg.type, torch.OptionalType)
                    and not isinstance(arg.type.getElementType(), torch.TensorType)):
                slots.append(("const", v))
                continue
            x = cls.realize_input(v)
            ev = ex.meta.get("val") if isinstance(ex, torch.fx.Node) else None
            if isinstance(ev, torch.Tensor) and ev.dim() > 0:
                x = cls.require_stride_order(x, ir.get_stride_order(ev.stride()))
            slots.append(len(inputs))
            inputs.append(x)
        out = fx_node.meta["val"]
        size = [_expr(s) for s in out.shape]
        layout = ir.FixedLayout(out.device, out.dtype, size,
                                ir.FlexibleLayout.contiguous_strides(size))
        name_arg = next(a for a in op._schema.arguments if a.name == "zentorch_op_name")
        op_name = (kwargs.get("zentorch_op_name", name_arg.default_value)
                   if name_arg.kwarg_only else None)
        return cls(layout, inputs, slots, op_name, op, shim)


def _register(name: str) -> None:
    op = getattr(torch.ops.zentorch, f"zentorch_{name}").default
    shim = f"aoti_torch_cuda_zentorch_{name}"

    def lowering(*args, **kwargs):
        return ir.TensorBox.create(ZentorchShimKernel.create(op, shim, args, kwargs))

    register_lowering(op, type_promotion_kind=None)(lowering)


for _name in SHIM_OPS:
    _register(_name)
