"""torch.compile(backend="zentorch") on the GPU: the WOQ patterns of the
reference's model tests (test/unittests/model_tests/test_woq_linear.py,
test_woq_linear_unary_fusion.py, test_woq_linear_binary_binary_fusion.py)
are replaced by the zentorch ops exactly once, and the compiled model
matches the eager model within the reference's rtol = atol = 1e-2.

The eager reference is the same module run by stock PyTorch with fp32
inputs: the weights are dequantised in bf16 exactly as the pattern does
(so they carry the same rounding the kernels apply) and everything after
that runs in fp32.  A bf16 eager run would round after every op of a chain
(addmm, add, add) and differ from the fused kernels' single rounding by
more than the tolerance on a few elements.  The compiled model takes the
bf16 inputs and runs the HIP kernels.
"""
import pytest
import torch
import torch._dynamo

import zentorch
from zentorch._utils import counters
from zentorch._weight_cache import cache_size, clear_weight_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = dict(rtol=1e-2, atol=1e-2)


@pytest.fixture(autouse=True)
def _fresh(request):
    print(f"\n[case] {request.node.name}", flush=True)
    torch._dynamo.reset()
    counters.clear()
    clear_weight_cache()
    yield
    torch._dynamo.reset()


def symmetric_int4(weight, group_size=None):
    """Symmetric int4 quantisation as the reference's woq_test_utils.py:23-59:
    scale = absmax / 8 (clamped at 1e-8), q = clamp(round(w / scale), -8, 7)."""
    N, K = weight.shape
    w = weight.float() if group_size is None else weight.float().view(N, K // group_size, group_size)
    amax = w.abs().amax(dim=-1, keepdim=True)
    scale = torch.clamp(amax / 8, min=1e-8)
    q = torch.clamp(torch.round(w / scale), -8, 7).to(torch.int8)
    return q, scale.to(torch.bfloat16), torch.zeros_like(scale, dtype=torch.int8)


class WoqLinear(torch.nn.Module):
    """Dequantise-then-matmul linear (woq_test_utils.py:62-105)."""

    def __init__(self, N, K, group_size=None, bias=False, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        # weights ~ N(0, 1/K) as in a trained layer, so outputs stay O(1)
        q, s, zp = symmetric_int4(torch.randn(N, K, generator=g) / K ** 0.5, group_size)
        self.register_buffer("weight", q)
        self.register_buffer("zero_points", zp)
        self.register_buffer("scale", s)
        self.register_buffer("bias", torch.randn(N, generator=g).bfloat16() if bias else None)
        self.view = (N, K) if group_size else None

    def forward(self, x):
        dq = (self.weight.to(torch.bfloat16) - self.zero_points.to(torch.bfloat16)) * self.scale
        if self.view is not None:
            dq = dq.view(self.view)
        # .to() is a no-op for bf16 inputs; fp32 inputs give the fp32 reference
        w = dq.permute(1, 0).to(x.dtype)
        if self.bias is not None:
            return torch.addmm(self.bias.to(x.dtype), x, w)
        return torch.mm(x, w)


def compiled_vs_eager(model, *inputs):
    """(fp32 eager reference, compiled output on the bf16 inputs)."""
    model = model.to(DEV).eval()
    inputs = [t.to(DEV) for t in inputs]
    with torch.no_grad():
        ref = model(*[t.float() for t in inputs])
        out = torch.compile(model, backend="zentorch")(*inputs)
    torch.cuda.synchronize()
    return ref, out


@pytest.mark.parametrize("M", [1, 4, 33])
@pytest.mark.parametrize("N,K", [(64, 256), (4096, 4096)])
@pytest.mark.parametrize("group_size", [None, 128])
@pytest.mark.parametrize("bias", [False, True])
def test_woq_linear_pattern_replaced(M, N, K, group_size, bias):
    x = torch.randn(M, K).bfloat16()
    eager, out = compiled_vs_eager(WoqLinear(N, K, group_size, bias), x)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    assert out.dtype == torch.bfloat16 and out.shape == eager.shape
    torch.testing.assert_close(out.float(), eager.float(), **TOL)


class Int4PackLinear(torch.nn.Module):
    """The graph torchao's Int4OpaqueTensor produces (aten._weight_int4pack_mm_for_cpu)."""

    def __init__(self, N, K, gs=128, bias=False, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
        self.register_buffer("packed", torch.ops.aten._convert_weight_to_int4pack_for_cpu(q, 1))
        s = (torch.rand(K // gs, N, generator=g) * 0.01 + 0.005)
        z = (torch.rand(K // gs, N, generator=g) - 0.5) * 0.02
        self.register_buffer("sz", torch.stack([s, z], dim=2).bfloat16())
        self.register_buffer("bias", torch.randn(N, generator=g).bfloat16() if bias else None)
        self.gs = gs

    def forward(self, x):
        y = torch.ops.aten._weight_int4pack_mm_for_cpu(x, self.packed, self.gs, self.sz)
        return y + self.bias if self.bias is not None else y


@pytest.mark.parametrize("bias", [False, True])
def test_int4pack_pattern_replaced(bias):
    # eager only exists on the CPU (tinygemm's CPU kernel); the compiled
    # model runs on the GPU
    m = Int4PackLinear(128, 512, bias=bias)
    x = torch.randn(4, 512).bfloat16()
    with torch.no_grad():
        eager = m(x)
        out = torch.compile(m.to(DEV), backend="zentorch")(x.to(DEV)).cpu()
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    torch.testing.assert_close(out.float(), eager.float(), **TOL)


class Unary(torch.nn.Module):
    def __init__(self, act, **kw):
        super().__init__()
        self.lin = WoqLinear(256, 512, 128, **kw)
        self.act = act

    def forward(self, x):
        return self.act(self.lin(x))


@pytest.mark.parametrize("act,key", [
    (torch.nn.functional.gelu, "gelu_erf"),
    (lambda y: torch.nn.functional.gelu(y, approximate="tanh"), "gelu_tanh"),
    (torch.relu, "relu"),
    (torch.sigmoid, "sigmoid"),
])
@pytest.mark.parametrize("bias", [False, True])
def test_unary_fusion(act, key, bias):
    eager, out = compiled_vs_eager(Unary(act, bias=bias), torch.randn(8, 512).bfloat16())
    assert counters["zentorch"][f"zentorch_woq_linear_{key}"] == 1
    torch.testing.assert_close(out.float(), eager.float(), **TOL)


class BinaryBinary(torch.nn.Module):
    def __init__(self, kind, order, bias):
        super().__init__()
        self.lin = WoqLinear(256, 512, 128, bias=bias)
        self.kind, self.order = kind, order

    def forward(self, x, a1, a2):
        y = self.lin(x)
        t = (y * a1 if self.kind == "mul_add" else y + a1) if self.order % 2 == 0 else \
            (a1 * y if self.kind == "mul_add" else a1 + y)
        return t + a2 if self.order < 2 else a2 + t


@pytest.mark.parametrize("kind", ["add_add", "mul_add"])
@pytest.mark.parametrize("order", range(4))
@pytest.mark.parametrize("bias", [False, True])
def test_binary_binary_fusion(kind, order, bias):
    x = torch.randn(8, 512).bfloat16()
    a1, a2 = torch.randn(8, 256).bfloat16(), torch.randn(8, 256).bfloat16()
    eager, out = compiled_vs_eager(BinaryBinary(kind, order, bias), x, a1, a2)
    assert counters["zentorch"][f"zentorch_woq_linear_{kind}"] == 1
    torch.testing.assert_close(out.float(), eager.float(), **TOL)


class LlamaMLP(torch.nn.Module):
    """down(silu(gate(x)) * up(x)) + x, every projection int4 group-128."""

    def __init__(self, hidden=512, inter=1024):
        super().__init__()
        self.gate = WoqLinear(inter, hidden, 128, seed=1)
        self.up = WoqLinear(inter, hidden, 128, seed=2)
        self.down = WoqLinear(hidden, inter, 128, seed=3)

    def forward(self, x):
        return self.down(torch.nn.functional.silu(self.gate(x)) * self.up(x)) + x


@pytest.mark.parametrize("M", [1, 16])
def test_llama_mlp_routes_to_fused_ops(M):
    eager, out = compiled_vs_eager(LlamaMLP(), torch.randn(M, 512).bfloat16())
    c = counters["zentorch"]
    assert c["zentorch_woq_linear"] == 3
    assert c["zentorch_woq_linear_silu_mul"] == 1 and c["zentorch_woq_linear_add"] == 1
    # the compiled MLP rounds silu(gate)*up to bf16 before the down
    # projection, the fp32 reference does not: 2e-2
    torch.testing.assert_close(out.float(), eager.float(), rtol=2e-2, atol=2e-2)


def test_weight_cache_reuses_and_invalidates():
    m = WoqLinear(256, 512, 128).to(DEV).eval()
    x = torch.randn(4, 512, device=DEV).bfloat16()
    with torch.no_grad():
        f = torch.compile(m, backend="zentorch")
        y1 = f(x)
        n = cache_size()
        assert n >= 1  # packed weight (and the [G, N] scales)
        y2 = f(x)
        assert cache_size() == n and torch.equal(y1, y2)
        # an in-place update of the weight is seen on the next call
        m.weight.copy_(-m.weight.clamp(min=-7))
        y3 = f(x)
        torch.testing.assert_close(y3.float(), m(x).float(), **TOL)
        assert not torch.equal(y3, y1)


# Zero points: with every zero point 0 at compile time the rewrite drops
# them (symmetric int4, as the reference's pattern does at
# _op_replacements_new.py:370,386), behind a run-time guard; integer zero
# points that are not all zero are kept and run on the op's unsigned int4
# path (u = w + 8 with zero points zp + 8; WOQ_Linear.cpp:44-49 selects u4
# whenever zero points are given).
@pytest.mark.parametrize("M", [1, 8, 33])
@pytest.mark.parametrize("group_size", [None, 128])
@pytest.mark.parametrize("bias", [False, True])
def test_nonzero_zero_points_take_the_u4_kernels(M, group_size, bias):
    N, K = 256, 512
    model = WoqLinear(N, K, group_size=group_size, bias=bias, seed=5)
    g = torch.Generator().manual_seed(6)
    model.zero_points.copy_(torch.randint(-8, 8, model.zero_points.shape, generator=g,
                                          dtype=torch.int8))
    assert bool(model.zero_points.any())
    x = torch.randn(M, K).bfloat16()
    ref, out = compiled_vs_eager(model, x)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    torch.testing.assert_close(out.float(), ref.float(), **TOL)


def test_nonzero_zero_points_cached_and_updated():
    # the u4 packing and the zero points + 8 are made once per weight
    # version; in-place updates of either are seen on the next call, and a
    # weight that leaves [-8, 7] is refused rather than truncated
    M, N, K = 4, 128, 256
    model = WoqLinear(N, K, group_size=128, seed=9).to(DEV).eval()
    model.zero_points.fill_(2)
    x = torch.randn(M, K).bfloat16().to(DEV)
    with torch.no_grad():
        fn = torch.compile(model, backend="zentorch")
        y1 = fn(x)
        assert counters["zentorch"]["zentorch_woq_linear"] == 1
        n = cache_size()
        assert fn(x).equal(y1) and cache_size() == n
        model.zero_points.fill_(-3)
        torch.testing.assert_close(fn(x).float(), model(x.float()).float(), **TOL)
        model.weight.copy_(-model.weight.clamp(min=-7))
        torch.testing.assert_close(fn(x).float(), model(x.float()).float(), **TOL)
        model.weight.fill_(9)
        with pytest.raises(RuntimeError, match="int4"):
            fn(x)


def test_zero_points_changed_after_compile_rejected():
    M, N, K = 4, 128, 256
    model = WoqLinear(N, K, seed=7).to(DEV).eval()
    x = torch.randn(M, K).bfloat16().to(DEV)
    with torch.no_grad():
        fn = torch.compile(model, backend="zentorch")
        fn(x)
        assert counters["zentorch"]["zentorch_woq_linear"] == 1
        model.zero_points.fill_(1)
        with pytest.raises(RuntimeError, match="zero points"):
            fn(x)


class GateUpMLP(torch.nn.Module):
    """vLLM-style merged gate_up + SiluAndMul over a dequantised int4 weight
    [2I, K] (gate rows first)."""

    def __init__(self, I, K, group_size=None, bias=False, split="split", seed=0):
        super().__init__()
        self.lin = WoqLinear(2 * I, K, group_size=group_size, bias=bias, seed=seed)
        self.I, self.split = I, split

    def forward(self, x):
        h = self.lin(x)
        if self.split == "slice":
            g, u = h[..., :self.I], h[..., self.I:]
        else:
            g, u = h.split(self.I, dim=-1)
        return torch.nn.functional.silu(g) * u


@pytest.mark.parametrize("M", [1, 16, 40])
@pytest.mark.parametrize("split", ["split", "slice"])
@pytest.mark.parametrize("group_size,bias", [(128, False), (None, True)])
def test_gate_up_silu_mul_fused(M, split, group_size, bias):
    I, K = 256, 512
    model = GateUpMLP(I, K, group_size=group_size, bias=bias, split=split, seed=M)
    x = torch.randn(M, K).bfloat16()
    ref, out = compiled_vs_eager(model, x)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    assert counters["zentorch"]["zentorch_woq_linear_gate_up_silu_mul"] == 1
    assert out.shape == (M, I) and out.dtype == torch.bfloat16
    torch.testing.assert_close(out.float(), ref.float(), **TOL)
