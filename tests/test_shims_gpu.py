"""The AOTInductor C shims of zentorch/_C.so (include/shim_cuda_zentorch.h)
called as a cpp_wrapper / AOTInductor model calls them: real AtenTensorHandles
in, a new handle out (caller-owned), optional operands as AtenTensorHandle*
(NULL = None), failures as AOTI_TORCH_FAILURE instead of exceptions
(src/cpu/cpp/shim_cpu_zentorch.cpp:367-513 of the reference).  Each shim's
result must equal the torch op's bit for bit: both run the same op body.

Handles are made and consumed with torch's own AOTI helpers
(torch._C._aoti.unsafe_alloc_void_ptrs_from_tensors /
alloc_tensor_by_stealing_from_void_ptr).
"""
import ctypes
import os

import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C_SO = os.path.join(ROOT, "zendnn-pytorch-plugin_amd", "zentorch", "_C.so")

_get_ptr = ctypes.pythonapi.PyCapsule_GetPointer
_get_ptr.restype, _get_ptr.argtypes = ctypes.c_void_p, [ctypes.py_object, ctypes.c_char_p]
_new_cap = ctypes.pythonapi.PyCapsule_New
_new_cap.restype, _new_cap.argtypes = ctypes.py_object, [ctypes.c_void_p, ctypes.c_char_p,
                                                          ctypes.c_void_p]


@pytest.fixture(autouse=True)
def _announce(request):
    import zentorch  # noqa: F401
    print(f"\n[case] {request.node.name}", flush=True)


class Handles:
    """New AtenTensorHandles for tensors; released (stolen back) at exit."""

    def __init__(self):
        self.ptrs = []

    def __call__(self, t):
        cap = torch._C._aoti.unsafe_alloc_void_ptrs_from_tensors([t])[0]
        p = _get_ptr(cap, None)
        self.ptrs.append(p)
        return ctypes.c_void_p(p)

    def opt(self, t):
        """AtenTensorHandle* for an optional operand (None -> NULL)."""
        return None if t is None else ctypes.byref(self(t))

    def release(self):
        for p in self.ptrs:
            torch._C._aoti.alloc_tensor_by_stealing_from_void_ptr(_new_cap(p, None, None))
        self.ptrs = []


def shim(name):
    fn = getattr(ctypes.CDLL(C_SO), f"aoti_torch_cuda_zentorch_{name}")
    fn.restype = ctypes.c_int32
    return fn


def call(name, *args):
    """Call shim `name`; returns (status, result tensor or None)."""
    ret = ctypes.c_void_p()
    rc = shim(name)(*args, f"zentorch::zentorch_{name}".encode(), ctypes.byref(ret))
    out = None
    if rc == 0:
        out = torch._C._aoti.alloc_tensor_by_stealing_from_void_ptr(_new_cap(ret.value, None,
                                                                             None))
    return rc, out


def woq_case(M=8, N=128, K=512, G=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(G, N, generator=g) * 0.015 + 0.005).bfloat16()
    b = torch.randn(N, generator=g).bfloat16()
    bufs = [torch.randn(M, N, generator=g).bfloat16() for _ in range(2)]
    return ([t.to(DEV) for t in (x, O.woq_repack_weight(q), s, b)] +
            [[t.to(DEV) for t in bufs]])


@pytest.mark.parametrize("suffix", ["", "_relu", "_sigmoid", "_gelu_tanh", "_gelu_erf"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_woq_unary_shims(suffix, with_bias):
    x, wp, s, b, _ = woq_case(seed=len(suffix))
    h = Handles()
    try:
        bias = b if with_bias else None
        rc, y = call(f"woq_linear{suffix}", h(x), h(wp.t()), h(s), None, h.opt(bias))
        assert rc == 0
        ref = getattr(torch.ops.zentorch, f"zentorch_woq_linear{suffix}")(x, wp.t(), s, None, bias)
        assert torch.equal(y, ref)
    finally:
        h.release()


def test_woq_binary_shims():
    x, wp, s, b, (a1, a2) = woq_case(seed=3)
    ops = torch.ops.zentorch
    h = Handles()
    try:
        rc, y = call("woq_linear_add", h(x), h(wp.t()), h(s), None, h(a1), h.opt(b))
        assert rc == 0 and torch.equal(y, ops.zentorch_woq_linear_add(x, wp.t(), s, None, a1, b))
        rc, y = call("woq_linear_mul_add", h(x), h(wp.t()), h(s), None, h(a1), h(a2), h.opt(b))
        assert rc == 0 and torch.equal(
            y, ops.zentorch_woq_linear_mul_add(x, wp.t(), s, None, a1, a2, b))
        rc, y = call("woq_linear_add_add", h(x), h(wp.t()), h(s), None, h(a1), h(a2), None)
        assert rc == 0 and torch.equal(
            y, ops.zentorch_woq_linear_add_add(x, wp.t(), s, None, a1, a2))
        rc, y = call("woq_linear_silu_mul", h(x), h(wp.t()), h(s), None, h(a1), h.opt(b))
        assert rc == 0 and torch.equal(
            y, ops.zentorch_woq_linear_silu_mul(x, wp.t(), s, None, a1, b))
        rc, y = call("woq_linear_gate_up_silu_mul", h(x), h(wp.t()), h(s), None, h.opt(b))
        assert rc == 0 and y.shape == (x.shape[0], wp.shape[0] // 2)
        assert torch.equal(y, ops.zentorch_woq_linear_gate_up_silu_mul(x, wp.t(), s, None, b))
    finally:
        h.release()


def test_woq_zero_point_shim():
    g = torch.Generator().manual_seed(9)
    M, N, K, G = 4, 64, 256, 2
    x = torch.randn(M, K, generator=g).bfloat16().to(DEV)
    q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int8)
    wp = O.woq_repack_weight(q).to(DEV)
    s = (torch.rand(G, N, generator=g) * 0.02).bfloat16().to(DEV)
    zp = torch.randint(0, 16, (G, N), generator=g, dtype=torch.int32).to(DEV)
    h = Handles()
    try:
        rc, y = call("woq_linear", h(x), h(wp.t()), h(s), h.opt(zp), None)
        assert rc == 0
        assert torch.equal(y, torch.ops.zentorch.zentorch_woq_linear(x, wp.t(), s, zp))
    finally:
        h.release()


@pytest.mark.parametrize("name", ["dynamic_qlinear", "dynamic_qlinear_silu_mul",
                                  "dynamic_qlinear_add"])
def test_dynamic_qlinear_shims(name):
    g = torch.Generator().manual_seed(4)
    M, N, K = 33, 200, 512
    x = torch.randn(M, K, generator=g).bfloat16().to(DEV)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(DEV)
    sw = (torch.rand(N, generator=g) * 0.009 + 0.001).to(DEV)
    b = (torch.randn(N, generator=g) * 0.1).bfloat16().to(DEV)
    other = torch.randn(M, N, generator=g).bfloat16().to(DEV)
    fn = getattr(torch.ops.zentorch, f"zentorch_{name}")
    h = Handles()
    try:
        if name == "dynamic_qlinear":
            rc, y = call(name, h(x), h(w), h(sw), h.opt(b))
            ref = fn(x, w, sw, b)
        else:
            rc, y = call(name, h(x), h(w), h(sw), h(other), h.opt(b))
            ref = fn(x, w, sw, other, b)
        assert rc == 0 and torch.equal(y, ref)
    finally:
        h.release()


SCALAR_TYPE = {torch.uint8: 0, torch.int8: 1, torch.float32: 6, torch.bfloat16: 15}


@pytest.mark.parametrize("name,out_dtype", [("qlinear", torch.uint8),
                                            ("qlinear_relu", torch.bfloat16),
                                            ("qlinear_sigmoid", torch.float32),
                                            ("qlinear_mul_add", torch.float32)])
def test_qlinear_shims(name, out_dtype):
    g = torch.Generator().manual_seed(31)
    M, N, K = 6, 48, 128
    x = torch.randn(M, K, generator=g).to(DEV)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8).to(DEV)
    xs = torch.tensor([0.03], device=DEV)
    xz = torch.tensor([120], dtype=torch.int32, device=DEV)
    ws = (torch.rand(N, generator=g) * 0.01 + 0.001).to(DEV)
    wz = torch.zeros(1, dtype=torch.int32, device=DEV)
    b = torch.randn(N, generator=g).to(out_dtype if out_dtype.is_floating_point
                                       else torch.float32).to(DEV)
    ys = torch.tensor([0.05], device=DEV) if out_dtype == torch.uint8 else None
    yz = torch.tensor([9], dtype=torch.int32, device=DEV) if out_dtype == torch.uint8 else None
    mul, add = (torch.randn(M, N, generator=g).to(DEV) for _ in range(2))
    dt = ctypes.c_int32(SCALAR_TYPE[out_dtype])
    h = Handles()
    try:
        head = [h(x), h(w), h(xs), h(xz), h(ws), h(wz)]
        if name == "qlinear_mul_add":
            head += [h(mul), h(add)]
        rc, y = call(name, *head, h.opt(b), h.opt(ys), h.opt(yz), ctypes.byref(dt))
        assert rc == 0
        fn = getattr(torch.ops.zentorch, f"zentorch_{name}")
        extra = (mul, add) if name == "qlinear_mul_add" else ()
        ref = fn(x, w, xs, xz, ws, wz, *extra, b, ys, yz, out_dtype)
        assert y.dtype == out_dtype and torch.equal(y, ref)
        if name in ("qlinear", "qlinear_relu"):
            out = torch.empty_like(ref)
            shim_out = shim(f"{name}_out")
            rc = shim_out(h(out), *head, h.opt(b), h.opt(ys), h.opt(yz), ctypes.byref(dt),
                          f"zentorch::zentorch_{name}.out".encode())
            torch.cuda.synchronize()
            assert rc == 0 and torch.equal(out, ref)
    finally:
        h.release()


def test_shim_failure_is_an_error_code():
    # a CPU input makes the op raise; the shim turns that into
    # AOTI_TORCH_FAILURE and leaves the output handle unset
    x, wp, s, b, _ = woq_case(seed=5)
    h = Handles()
    try:
        rc, y = call("woq_linear", h(x.cpu()), h(wp.t()), h(s), None, None)
        assert rc != 0 and y is None
        rc, y = call("dynamic_qlinear", h(x), h(wp), h(s), None)  # int32 "weight"
        assert rc != 0 and y is None
    finally:
        h.release()


def _all_ops(x, wp, s, b, a1, a2, xq, wq, sq, bq, oq, zq):
    z = torch.ops.zentorch
    w = wp.t()
    return [
        z.zentorch_woq_linear(x, w, s, None, b),
        z.zentorch_woq_linear_relu(x, w, s, None),
        z.zentorch_woq_linear_sigmoid(x, w, s, None, b),
        z.zentorch_woq_linear_gelu_tanh(x, w, s, None, b),
        z.zentorch_woq_linear_gelu_erf(x, w, s, None, bias=b),
        z.zentorch_woq_linear_add(x, w, s, None, a1, b),
        z.zentorch_woq_linear_mul_add(x, w, s, None, a1, a2, b),
        z.zentorch_woq_linear_add_add(x, w, s, None, a1, a2),
        z.zentorch_woq_linear_silu_mul(x, w, s, None, a1, b),
        z.zentorch_woq_linear_gate_up_silu_mul(x, w, s, None, b),
        z.zentorch_dynamic_qlinear(xq, wq, sq, bq),
        z.zentorch_dynamic_qlinear_silu_mul(xq, wq, sq, oq, bq),
        z.zentorch_dynamic_qlinear_add(xq, wq, sq, oq),
        z.zentorch_qlinear(xq, wq, sq[:1], None, sq, None, bq, None, None, torch.bfloat16),
        z.zentorch_qlinear_relu(xq, wq, sq[:1], zq, sq, None, None, None, None),
        z.zentorch_qlinear_sigmoid(xq, wq, sq[:1], zq, sq[:1], None, None, sq[:1] * 4, zq,
                                   torch.uint8),
        z.zentorch_qlinear_mul_add(xq, wq, sq[:1], None, sq, None, oq, oq, None, None, None,
                                   torch.bfloat16),
    ]


@pytest.mark.timeout(900)
@pytest.mark.parametrize("cpp_wrapper", [True, False])
def test_inductor_lowerings_call_the_shims(cpp_wrapper):
    """Inductor lowers every zentorch op to an ExternKernelAlloc; with
    cpp_wrapper the generated C++ calls the op's shim directly."""
    from torch._inductor.utils import run_and_get_code
    from zentorch._lowerings import SHIM_OPS
    x, wp, s, b, (a1, a2) = woq_case(M=8, N=128, K=512, seed=11)
    g = torch.Generator().manual_seed(12)
    xq = torch.randn(8, 256, generator=g).bfloat16().to(DEV)
    wq = torch.randint(-127, 128, (96, 256), generator=g, dtype=torch.int8).to(DEV)
    sq = (torch.rand(96, generator=g) * 0.009 + 0.001).to(DEV)
    bq = torch.randn(96, generator=g).bfloat16().to(DEV)
    oq = torch.randn(8, 96, generator=g).bfloat16().to(DEV)
    zq = torch.tensor([100], dtype=torch.int32, device=DEV)
    args = (x, wp, s, b, a1, a2, xq, wq, sq, bq, oq, zq)
    ref = _all_ops(*args)
    torch._dynamo.reset()
    fn = torch.compile(_all_ops, options={"cpp_wrapper": cpp_wrapper})
    outs, codes = run_and_get_code(fn, *args)
    code = "\n".join(codes)
    for name in SHIM_OPS:
        key = f"aoti_torch_cuda_zentorch_{name}(" if cpp_wrapper else \
            f"torch.ops.zentorch.zentorch_{name}.default("
        assert key in code, name
    for name, y, r in zip(SHIM_OPS, outs, ref):
        assert torch.equal(y, r), name


class DynModel(torch.nn.Module):
    def __init__(self, w, sw, b):
        super().__init__()
        self.w, self.sw, self.b = w, sw, b

    def forward(self, x):
        return torch.ops.zentorch.zentorch_dynamic_qlinear(x, self.w, self.sw, self.b)


def _noncontiguous(t):
    """Same values, last-dim stride 2 (test_dynamic_qlinear.py:81-93 of the
    reference's model tests)."""
    wide = torch.zeros(*t.shape[:-1], 2 * t.shape[-1], dtype=t.dtype, device=t.device)
    wide[..., ::2] = t
    return wide[..., ::2]


@pytest.mark.timeout(900)
@pytest.mark.parametrize("noncontig", [False, True])
def test_dynamic_qlinear_model_backends(noncontig):
    """The reference's dynamic-qlinear model tests
    (test/unittests/model_tests/test_dynamic_qlinear.py:96-205): a module
    calling the op, compiled with Inductor (cpp_wrapper, so the shim runs)
    and with the "zentorch" backend, must match eager, also when weight,
    scales and bias are non-contiguous views.  Both run the same kernel, so
    the match is exact."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(2, 5, 256, generator=g).bfloat16().to(DEV)
    w = torch.randint(-127, 128, (72, 256), generator=g, dtype=torch.int8).to(DEV)
    sw = (torch.rand(72, generator=g) * 0.009 + 0.001).to(DEV)
    b = torch.randn(72, generator=g).bfloat16().to(DEV)
    if noncontig:
        w, sw, b = (_noncontiguous(t) for t in (w, sw, b))
        assert not any(t.is_contiguous() for t in (w, sw, b))
    m = DynModel(w, sw, b).eval()
    with torch.inference_mode():
        ref = m(x)
        torch._dynamo.reset()
        y_ind = torch.compile(m, options={"cpp_wrapper": True})(x)
        torch._dynamo.reset()
        y_zt = torch.compile(m, backend="zentorch")(x)
    assert y_ind.shape == (2, 5, 72) and y_ind.dtype == torch.bfloat16
    assert torch.equal(y_ind, ref)
    assert torch.equal(y_zt, ref)
