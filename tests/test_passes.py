"""Graph-pass tests on the CPU: the WOQ op replacement and the post-op
fusions rewrite the subgraphs the reference's passes rewrite
(src/cpu/python/zentorch/_op_replacements_new.py:316-799,
_woq_linear_unary_fusion.py, _woq_linear_binary_binary_fusion.py) and leave
everything else alone.

Graphs are traced with make_fx over Inductor's decomposition table on fake
tensors, which is the form the post-grad passes see; the zentorch ops only
run their Meta kernels here.  The passes rewrite GPU subgraphs only, so the
tests add "cpu" to the pass devices; one test checks that a CPU graph is
left alone by default.  Numerics of compiled models are GPU tests
(test_compile_gpu.py).
"""
import pytest
import torch
from torch._inductor.decomposition import select_decomp_table
from torch.fx.experimental.proxy_tensor import make_fx

import zentorch
from zentorch import _utils
from zentorch._optimize import optimize
from zentorch._utils import counters

aten = torch.ops.aten
zt = torch.ops.zentorch


@pytest.fixture
def cpu_passes(monkeypatch):
    monkeypatch.setattr(_utils, "PASS_DEVICE_TYPES", ("cuda", "cpu"))
    counters.clear()
    yield
    counters.clear()


def trace(fn, *args):
    gm = make_fx(fn, decomposition_table=select_decomp_table(), tracing_mode="fake")(*args)
    # Inductor removes dead nodes before its passes; the decompositions leave
    # some (unused dtype casts) that would add users to pattern nodes.
    gm.graph.eliminate_dead_code()
    gm.recompile()
    gm._real_inputs = args  # the values a compile would see for its weights
    return gm


def targets(gm):
    return [n.target for n in gm.graph.nodes if n.op == "call_function"]


def run_passes(gm):
    ph = [n for n in gm.graph.nodes if n.op == "placeholder"]
    static = {n: t for n, t in zip(ph, getattr(gm, "_real_inputs", ()))
              if isinstance(t, torch.Tensor)}
    optimize(gm.graph, static)
    gm.recompile()
    return targets(gm)


def quantized(N, K, gs=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    if gs is None:
        w = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
        zp = torch.zeros(N, 1, dtype=torch.int8)
        s = (torch.rand(N, 1, generator=g) * 0.01 + 0.005).bfloat16()
    else:
        w = torch.randint(-8, 8, (N, K // gs, gs), generator=g, dtype=torch.int8)
        zp = torch.zeros(N, K // gs, 1, dtype=torch.int8)
        s = (torch.rand(N, K // gs, 1, generator=g) * 0.01 + 0.005).bfloat16()
    return w, zp, s


def dequant_t(w, zp, s, view=None):
    # woq_test_utils.py:62-74 of the reference: (bf16(w) - bf16(zp)) * s [-> view] -> permute
    dq = (w.to(torch.bfloat16) - zp.to(torch.bfloat16)) * s
    if view is not None:
        dq = dq.view(view)
    return dq.permute(1, 0)


# ---------------------------------------------------------------- replacement
@pytest.mark.parametrize("gs", [None, 128])
@pytest.mark.parametrize("bias", [False, True])
def test_dequant_matmul_replaced(cpu_passes, gs, bias):
    N, K = 64, 256
    w, zp, s = quantized(N, K, gs)
    x = torch.randn(4, K).bfloat16()
    b = torch.randn(N).bfloat16()
    view = (N, K) if gs else None

    def f(x, w, zp, s, b):
        d = dequant_t(w, zp, s, view)
        return torch.addmm(b, x, d) if bias else torch.mm(x, d)

    gm = trace(f, x, w, zp, s, b)
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    assert zt.zentorch_woq_linear.default in t and zt.zentorch_woq_repack_weight.default in t
    assert aten.mm.default not in t and aten.addmm.default not in t
    node = next(n for n in gm.graph.nodes if n.target == zt.zentorch_woq_linear.default)
    # operands: x, [K/8, N] packed view, [G, N] scales, zp dropped, bias
    assert tuple(node.args[1].meta["val"].shape) == (K // 8, N)
    assert tuple(node.args[2].meta["val"].shape) == ((K // gs) if gs else 1, N)
    assert node.args[3] is None
    assert (len(node.args) > 4 and node.args[4] is not None) == bias


@pytest.mark.parametrize("case", ["unsigned_weights", "unknown_values", "zp_overflow"])
def test_dequant_matmul_left_alone_unless_int4(cpu_passes, case):
    # the rewrite packs int4: weights outside [-8, 7], values unknown at
    # compile time, or zero points whose + 8 overflows their dtype stay
    # stock PyTorch
    N, K = 64, 256
    w, zp, s = quantized(N, K)
    if case == "unsigned_weights":
        w = torch.randint(0, 16, (N, K), dtype=torch.int8)
    elif case == "zp_overflow":
        zp = torch.full_like(zp, 125)
    x = torch.randn(4, K).bfloat16()
    gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s)), x, w, zp, s)
    if case == "unknown_values":
        gm._real_inputs = ()
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear"] == 0
    assert aten.mm.default in t and zt.zentorch_woq_linear.default not in t


@pytest.mark.parametrize("gs", [None, 128])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("zp_dtype", [torch.int8, torch.int32])
def test_nonzero_zero_points_take_the_u4_path(cpu_passes, gs, bias, zp_dtype):
    # integer zero points that are not all zero are kept: the weight is
    # packed as u = w + 8 and the op gets zp + 8 ([G, N]), no guard
    from zentorch._optimize import zero_points_guard
    N, K = 64, 256
    w, zp, s = quantized(N, K, gs)
    g = torch.Generator().manual_seed(3)
    zp = torch.randint(-8, 8, zp.shape, generator=g).to(zp_dtype)
    x = torch.randn(4, K).bfloat16()
    b = torch.randn(N).bfloat16()
    view = (N, K) if gs else None
    if bias:
        f = lambda x, w, zp, s, b: torch.addmm(b, x, dequant_t(w, zp, s, view))
        gm = trace(f, x, w, zp, s, b)
    else:
        gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s, view)), x, w, zp, s)
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    assert aten.mm.default not in t and aten.addmm.default not in t
    assert zero_points_guard not in t
    node = next(n for n in gm.graph.nodes if n.target == zt.zentorch_woq_linear.default)
    zeros = node.args[3]
    assert zeros is not None and zeros.target is aten.add.Tensor and zeros.args[1] == 8
    assert tuple(zeros.meta["val"].shape) == ((K // gs) if gs else 1, N)
    assert zeros.meta["val"].dtype == zp_dtype
    packed = node.args[1]
    while packed.target != zt.zentorch_woq_repack_weight.default:
        packed = packed.args[0]
    assert packed.args[0].target is aten.add.Tensor and packed.args[0].args[1] == 8


@pytest.mark.parametrize("gs", [None, 64])
def test_u4_rewrite_equals_the_dequantised_graph(gs):
    # what the rewrite computes -- the op's unsigned int4 path on u = w + 8
    # with zero points zp + 8 (the oracle, which the GPU kernels match) --
    # against the graph it replaces, (bf16(w) - bf16(zp)) * s in bf16 and a
    # matmul, in fp32 here
    from oracle import oracle as O
    N, K = 48, 256
    w, zp, s = quantized(N, K, gs)
    g = torch.Generator().manual_seed(5)
    zp = torch.randint(-8, 8, zp.shape, generator=g, dtype=torch.int8)
    x = torch.randn(3, K, generator=g).bfloat16()
    dq = ((w.to(torch.bfloat16) - zp.to(torch.bfloat16)) * s).reshape(N, K)
    ref = x.float() @ dq.float().t()
    packed = O.woq_repack_weight((w.reshape(N, K) + 8).to(torch.int8))
    scales = s.reshape(N, -1).t().contiguous()
    zeros = (zp.reshape(N, -1) + 8).t().contiguous()
    y = O.woq_linear(x, packed, scales, zero_points=zeros)
    torch.testing.assert_close(y.float(), ref, rtol=1e-2, atol=1e-2)
    # the symmetric s4 packing of the same weight would differ whenever zp != 0
    y_s4 = O.woq_linear(x, O.woq_repack_weight(w.reshape(N, K)), scales)
    assert not torch.allclose(y_s4.float(), ref, rtol=1e-2, atol=1e-2)


def test_zero_point_guard_inserted_and_checked(cpu_passes):
    from zentorch._optimize import zero_points_guard
    N, K = 64, 256
    w, zp, s = quantized(N, K)
    x = torch.randn(4, K).bfloat16()
    gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s)), x, w, zp, s)
    run_passes(gm)
    guards = [n for n in gm.graph.nodes if n.target is zero_points_guard]
    assert len(guards) == 1 and guards[0].args[0].name == "zp_1"
    assert guards[0].args[1].name == "w_1"  # the weight it assumed in [-8, 7]
    gm.graph.eliminate_dead_code()  # the guard has no users and must survive
    assert any(n.target is zero_points_guard for n in gm.graph.nodes)
    zero_points_guard(zp, w)  # all zero, weight in range: passes
    zp.add_(1)
    with pytest.raises(RuntimeError, match="zero points"):
        zero_points_guard(zp, w)
    zp.zero_()
    zero_points_guard(zp, w)
    w[0, 0] = 9  # an in-place update out of the signed int4 range
    with pytest.raises(RuntimeError, match="int4"):
        zero_points_guard(zp, w)
    # a new tensor is checked even where an old one passed (no address key)
    fresh = torch.ones_like(zp)
    with pytest.raises(RuntimeError, match="zero points"):
        zero_points_guard(fresh)


def test_per_group_reshape_form_replaced(cpu_passes):
    # Inductor can turn the per-group view into reshape before the pass runs
    N, K = 64, 256
    w, zp, s = quantized(N, K, 128)
    x = torch.randn(2, K).bfloat16()
    gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s, (N, K))), x, w, zp, s)
    for n in gm.graph.nodes:
        if n.target == aten.view.default:
            n.target = aten.reshape.default
    gm.recompile()
    run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1


def test_cpu_graph_left_alone_by_default():
    counters.clear()
    w, zp, s = quantized(64, 256)
    x = torch.randn(4, 256).bfloat16()
    gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s)), x, w, zp, s)
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear"] == 0
    assert aten.mm.default in t


def test_not_a_transpose_or_bad_shapes_left_alone(cpu_passes):
    N, K = 64, 256
    w, zp, s = quantized(N, K)
    x = torch.randn(4, K).bfloat16()
    # scales per input column instead of per output row
    s_bad = (torch.rand(1, K) * 0.01).bfloat16()
    gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s)), x, w, zp, s_bad)
    run_passes(gm)
    # K not a multiple of 8
    w2, zp2, s2 = quantized(16, 12)
    gm2 = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s)),
                torch.randn(3, 12).bfloat16(), w2, zp2, s2)
    run_passes(gm2)
    # int32 "weights" are not the int8 pattern
    gm3 = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s)), torch.randn(4, K).bfloat16(),
                w.int(), zp, s)
    run_passes(gm3)
    assert counters["zentorch"]["zentorch_woq_linear"] == 0


@pytest.mark.parametrize("bias", [False, True])
def test_int4pack_mm_replaced(cpu_passes, bias):
    N, K, gs = 64, 256, 128
    q = torch.randint(0, 16, (N, K), dtype=torch.int32)
    packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(q, 1)
    sz = torch.rand(K // gs, N, 2).bfloat16()
    x = torch.randn(4, K).bfloat16()
    b = torch.randn(N).bfloat16()

    def f(x, packed, sz, b):
        y = torch.ops.aten._weight_int4pack_mm_for_cpu(x, packed, gs, sz)
        return y + b if bias else y

    gm = trace(f, x, packed, sz, b)
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    assert zt.zentorch_woq_repack_from_int4pack.default in t
    node = next(n for n in gm.graph.nodes if n.target == zt.zentorch_woq_linear.default)
    assert node.args[3] is not None  # tinygemm zero points passed through
    assert (len(node.args) > 4 and node.args[4] is not None) == bias
    assert aten.add.Tensor not in t


# ------------------------------------------------------------------ fusions
def woq_inputs(M=4, N=64, K=256, gs=128, dtype=torch.bfloat16):
    x = torch.randn(M, K).to(dtype)
    wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), dtype=torch.int32).t()
    s = torch.rand(K // gs, N).bfloat16()
    return x, wp, s


def _woq(x, wp, s, b=None):
    return zt.zentorch_woq_linear(x, wp, s, None, b)


@pytest.mark.parametrize("act,op", [
    (lambda y: torch.nn.functional.gelu(y), "gelu_erf"),
    (lambda y: torch.nn.functional.gelu(y, approximate="tanh"), "gelu_tanh"),
    (torch.relu, "relu"),
    (torch.sigmoid, "sigmoid"),
])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_unary_fusions(cpu_passes, act, op, bias, dtype):
    x, wp, s = woq_inputs(dtype=dtype)
    b = torch.randn(wp.shape[1]).to(dtype)
    gm = trace(lambda x, wp, s, b: act(_woq(x, wp, s, b if bias else None)), x, wp, s, b)
    t = run_passes(gm)
    key = f"zentorch_woq_linear_{op}"
    assert counters["zentorch"][key] == 1, dict(counters["zentorch"])
    assert getattr(zt, key).default in t and zt.zentorch_woq_linear.default not in t
    # nothing of the activation is left
    assert not {aten.erf.default, aten.tanh.default, aten.sigmoid.default,
                aten.relu.default, aten.gelu.default} & set(t)


def test_gelu_tanh_not_taken_for_erf(cpu_passes):
    x, wp, s = woq_inputs()
    gm = trace(lambda x, wp, s: torch.nn.functional.gelu(_woq(x, wp, s), approximate="tanh"), x, wp, s)
    run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear_gelu_erf"] == 0
    assert counters["zentorch"]["zentorch_woq_linear_gelu_tanh"] == 1


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_silu_mul_fusion(cpu_passes, order, dtype):
    x, wp, s = woq_inputs(dtype=dtype)
    up = torch.randn(x.shape[0], wp.shape[1]).to(dtype)

    def f(x, wp, s, up):
        g = torch.nn.functional.silu(_woq(x, wp, s))
        return g * up if order == 0 else up * g

    gm = trace(f, x, wp, s, up)
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear_silu_mul"] == 1
    node = next(n for n in gm.graph.nodes if n.target == zt.zentorch_woq_linear_silu_mul.default)
    assert node.args[4].name.startswith("up")
    assert aten.mul.Tensor not in t


def test_llama_mlp_gate_up_down(cpu_passes):
    # down(silu(gate(x)) * up(x)) + residual: silu_mul on gate, plain up,
    # residual add fused into down
    x, wg, s = woq_inputs(N=128)
    _, wu, _ = woq_inputs(N=128)
    wd = torch.randint(-2 ** 31, 2 ** 31 - 1, (64, 128 // 8), dtype=torch.int32).t()
    sd = torch.rand(1, 64).bfloat16()
    res = torch.randn(4, 64).bfloat16()

    def mlp(x, wg, wu, s, wd, sd, res):
        h = torch.nn.functional.silu(_woq(x, wg, s)) * _woq(x, wu, s)
        return _woq(h, wd, sd) + res

    gm = trace(mlp, x, wg, wu, s, wd, sd, res)
    t = run_passes(gm)
    c = counters["zentorch"]
    assert c["zentorch_woq_linear_silu_mul"] == 1 and c["zentorch_woq_linear_add"] == 1
    assert t.count(zt.zentorch_woq_linear.default) == 1  # the up projection


@pytest.mark.parametrize("inner,op", [("add", "add_add"), ("mul", "mul_add")])
@pytest.mark.parametrize("order", range(4))
@pytest.mark.parametrize("bias", [False, True])
def test_binary_binary_fusions(cpu_passes, inner, op, order, bias):
    x, wp, s = woq_inputs()
    b = torch.randn(wp.shape[1]).bfloat16()
    a1 = torch.randn(x.shape[0], wp.shape[1]).bfloat16()
    a2 = torch.randn(x.shape[0], wp.shape[1]).bfloat16()
    f_in = (lambda p, q: p + q) if inner == "add" else (lambda p, q: p * q)

    def f(x, wp, s, b, a1, a2):
        y = _woq(x, wp, s, b if bias else None)
        t = f_in(y, a1) if order in (0, 2) else f_in(a1, y)
        return t + a2 if order in (0, 1) else a2 + t

    gm = trace(f, x, wp, s, b, a1, a2)
    t = run_passes(gm)
    key = f"zentorch_woq_linear_{op}"
    assert counters["zentorch"][key] == 1, dict(counters["zentorch"])
    node = next(n for n in gm.graph.nodes if n.target == getattr(zt, key).default)
    # buffer order of the fused op: inner operand, then outer operand
    assert node.args[4].name.startswith("a1") and node.args[5].name.startswith("a2")
    assert (len(node.args) > 6 and node.args[6] is not None) == bias
    assert aten.add.Tensor not in t and aten.mul.Tensor not in t


def test_broadcast_or_promoting_operands_not_fused(cpu_passes):
    x, wp, s = woq_inputs()
    row = torch.randn(wp.shape[1]).bfloat16()            # broadcast
    full32 = torch.randn(x.shape[0], wp.shape[1])        # fp32 -> promotes
    gm = trace(lambda x, wp, s, r, f: (_woq(x, wp, s) + r, _woq(x, wp, s) + f),
               x, wp, s, row, full32)
    run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear_add"] == 0


def test_compile_backend_runs_the_passes(cpu_passes):
    # torch.compile(backend="zentorch") rewrites the graph; on the CPU the
    # rewritten graph then fails loudly (no CPU kernels), which shows that
    # nothing falls back to a CPU implementation.
    import torch._dynamo

    torch._dynamo.reset()
    N, K = 64, 256
    w, zp, s = quantized(N, K, 128)
    x = torch.randn(4, K).bfloat16()

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.register_buffer("w", w)
            self.register_buffer("zp", zp)
            self.register_buffer("s", s)

        def forward(self, x):
            return torch.mm(x, dequant_t(self.w, self.zp, self.s, (N, K)))

    with pytest.raises(Exception, match="zentorch|NotImplemented|CPU"):
        with torch.no_grad():
            torch.compile(M(), backend="zentorch")(x)
    assert counters["zentorch"]["zentorch_woq_linear"] == 1
    torch._dynamo.reset()


# ------------------------------------------------------- merged gate_up
def gate_up_inputs(M=4, I=64, K=256, gs=128):
    x = torch.randn(M, K).bfloat16()
    wp = torch.randint(-2 ** 31, 2 ** 31 - 1, (2 * I, K // 8), dtype=torch.int32).t()
    s = torch.rand(K // gs, 2 * I).bfloat16()
    b = torch.randn(2 * I).bfloat16()
    return x, wp, s, b


@pytest.mark.parametrize("form", ["split", "chunk", "slice", "view3d", "decomposed_silu",
                                  "up_first", "bias"])
def test_gate_up_silu_mul_fused(cpu_passes, form):
    I = 64
    x, wp, s, b = gate_up_inputs(I=I)
    silu = (lambda t: t * torch.sigmoid(t)) if form == "decomposed_silu" else \
        torch.nn.functional.silu

    def f(x, wp, s, b):
        h = zt.zentorch_woq_linear(x, wp, s, None, b if form == "bias" else None)
        if form == "view3d":
            h = h.view(2, 2, 2 * I)
        if form == "chunk":
            g, u = h.chunk(2, dim=-1)
        elif form == "slice":
            g, u = h[:, :I], h[:, I:]
        else:
            g, u = h.split(I, dim=-1)
        return u * silu(g) if form == "up_first" else silu(g) * u

    gm = trace(f, x, wp, s, b)
    t = run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear_gate_up_silu_mul"] == 1, (form, t)
    assert zt.zentorch_woq_linear_gate_up_silu_mul.default in t
    assert zt.zentorch_woq_linear.default not in t
    assert not {aten.mul.Tensor, aten.sigmoid.default, aten.silu.default} & set(t)
    node = next(n for n in gm.graph.nodes if n.target == zt.zentorch_woq_linear_gate_up_silu_mul.default)
    assert (node.args[4] is not None) == (form == "bias")
    out = [n for n in gm.graph.nodes if n.op == "output"][0].args[0]
    out = out[0] if isinstance(out, (list, tuple)) else out
    assert tuple(out.meta["val"].shape) == ((2, 2, I) if form == "view3d" else (4, I))


@pytest.mark.parametrize("case", ["uneven_split", "gate_reused", "not_silu", "up_reused"])
def test_gate_up_left_alone(cpu_passes, case):
    I = 64
    x, wp, s, b = gate_up_inputs(I=I)

    def f(x, wp, s, b):
        h = zt.zentorch_woq_linear(x, wp, s, None, None)
        if case == "uneven_split":
            g, u = h[:, :32], h[:, 32:64]
        else:
            g, u = h.split(I, dim=-1)
        act = torch.relu(g) if case == "not_silu" else torch.nn.functional.silu(g)
        out = act * u
        if case == "gate_reused":
            return out, g
        if case == "up_reused":
            return out, u
        return out

    gm = trace(f, x, wp, s, b)
    run_passes(gm)
    assert counters["zentorch"]["zentorch_woq_linear_gate_up_silu_mul"] == 0


def test_dynamic_token_count_compiles_once(monkeypatch):
    # A graph compiled with dynamic shapes must serve every token count from
    # one compile: reading the weights' compile-time values must not guard
    # on the activations' symbolic sizes.
    import torch._dynamo
    from zentorch import _compile_backend

    torch._dynamo.reset()
    compiles = []
    real = _compile_backend._compile_forward

    def counting(gm, ex, inputs=()):
        compiles.append(len(gm.graph.nodes))
        return real(gm, ex, inputs)

    monkeypatch.setattr(_compile_backend, "_compile_forward", counting)

    class Lin(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.w = torch.nn.Parameter(torch.randn(32, 64), requires_grad=False)

        def forward(self, x):
            return torch.nn.functional.linear(x, self.w).relu()

    m = Lin()
    f = torch.compile(m, backend="zentorch", dynamic=True)
    with torch.no_grad():
        for M in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29):
            x = torch.randn(M, 64)
            torch.testing.assert_close(f(x), torch.nn.functional.linear(x, m.w).relu())
    assert len(compiles) == 1
    torch._dynamo.reset()


def test_weight_cache_rewrites_offset_forms(cpu_passes):
    # repack(add(w, 8)) and add(clone(zp view), 8) of module weights become
    # single cached transforms carrying the offset
    from zentorch import _compile_backend as B
    from zentorch._weight_cache import cached_clone_offset, cached_repack_weight_offset
    N, K = 64, 256
    w, zp, s = quantized(N, K, 128)
    zp = torch.full_like(zp, 3)
    x = torch.randn(4, K).bfloat16()
    gm = trace(lambda x, w, zp, s: torch.mm(x, dequant_t(w, zp, s, (N, K))), x, w, zp, s)
    run_passes(gm)
    ph = [n for n in gm.graph.nodes if n.op == "placeholder"]
    assert B.use_weight_cache(gm.graph, set(ph[1:])) >= 3
    gm.graph.eliminate_dead_code()
    rep = [n for n in gm.graph.nodes if n.target is cached_repack_weight_offset]
    clo = [n for n in gm.graph.nodes if n.target is cached_clone_offset]
    assert len(rep) == 1 and rep[0].args[1] == 8
    assert len(clo) == 1 and clo[0].args[1] == 8
    assert not any(n.target in (aten.add.Tensor, aten.add.Scalar) for n in gm.graph.nodes)
