"""Inductor lowerings of the zentorch ops (zentorch/_lowerings.py) without a
GPU: Inductor's cpp_wrapper code for a zentorch op must call the op's shim
with the schema's argument order (NULL for an absent optional tensor, the
op name as a C string, the output handle last), compile and link against
zentorch/_C.so.  The call then fails inside the shim, because the ops run on
the GPU only, and the failure comes back as an error naming that call.
"""
import pytest
import torch

import zentorch  # noqa: F401
from oracle import oracle as O


@pytest.mark.timeout(600)
def test_cpp_wrapper_calls_the_shim():
    from zentorch._lowerings import SHIM_OPS, SHIM_HEADER
    import os
    assert os.path.exists(SHIM_HEADER)
    assert len(SHIM_OPS) == 17
    x = torch.randn(4, 256).bfloat16()
    wp = O.woq_repack_weight(torch.randint(-8, 8, (64, 256), dtype=torch.int8))
    s = torch.rand(2, 64).bfloat16()
    b = torch.randn(64).bfloat16()

    def f(x, w, s, b):
        return torch.ops.zentorch.zentorch_woq_linear_relu(x, w, s, None, b) + 1

    torch._dynamo.reset()
    fn = torch.compile(f, options={"cpp_wrapper": True})
    with pytest.raises(RuntimeError) as e:
        fn(x, wp.t(), s, b)
    msg = str(e.value)
    assert "aoti_torch_cuda_zentorch_woq_linear_relu(" in msg
    call = msg.split("aoti_torch_cuda_zentorch_woq_linear_relu(", 1)[1].split(") API", 1)[0]
    args = [a.strip() for a in call.split(",")]
    assert len(args) == 7, args
    assert args[3] == "nullptr"                       # weight_zero_points=None
    assert args[4].startswith("&temporary_reference")  # bias: AtenTensorHandle*
    assert args[5] == '"zentorch::zentorch_woq_linear_relu"'
    assert args[6].startswith("&") and args[6].endswith("_handle")


@pytest.mark.timeout(600)
def test_cpp_wrapper_calls_the_qlinear_shim():
    """zentorch_qlinear: zero points that are None become uninitialized
    tensor handles, output_dtype a pointer to its ScalarType code, and the
    op name (positional in this schema) a C string."""
    x = torch.randn(4, 64)
    w = torch.randint(-128, 128, (16, 64), dtype=torch.int8)
    xs, ws = torch.tensor([0.02]), torch.rand(16)

    def f(x, w, xs, ws):
        return torch.ops.zentorch.zentorch_qlinear(x, w, xs, None, ws, None, None, None, None,
                                                   torch.bfloat16) * 2

    torch._dynamo.reset()
    fn = torch.compile(f, options={"cpp_wrapper": True})
    with pytest.raises(RuntimeError) as e:
        fn(x, w, xs, ws)
    msg = str(e.value)
    call = msg.split("aoti_torch_cuda_zentorch_qlinear(", 1)[1].split(") API", 1)[0]
    args = [a.strip() for a in call.split(",")]
    assert len(args) == 12, args
    assert args[6] == args[7] == args[8] == "nullptr"        # bias, output scales / zp
    assert args[9].startswith("&")                           # output_dtype
    assert args[10] == '"zentorch::zentorch_qlinear"'
