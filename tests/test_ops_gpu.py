"""The torch ops (zentorch/_C.so) on the GPU: argument forms the reference's
callers use, HIP-graph capture, and agreement with the C-ABI and the oracle.

Mirrors the reference's model tests for the dynamic int8 op
(test/unittests/model_tests/test_dynamic_qlinear.py:96-114, 172-205:
[1, N] scales, non-contiguous weight / scales / bias made as stride-2 views,
3-D input, compiled with backend="zentorch") and the vLLM torchao caller
(src/cpu/python/zentorch/vllm/_torchao_int8_patch.py:141-164: [N, 1] scales
made contiguous and squeezed to [N]).  Tolerance rtol = atol = 1e-2.
"""
import warnings

import pytest
import torch

import zt_capi as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = dict(rtol=1e-2, atol=1e-2)


@pytest.fixture(autouse=True)
def _announce(request):
    import zentorch  # noqa: F401
    print(f"\n[case] {request.node.name}", flush=True)


def noncontiguous(t):
    """t's values as a stride-2 view along the last dim (the reference
    test's _make_noncontiguous)."""
    wide = torch.zeros(*t.shape[:-1], 2 * t.shape[-1], dtype=t.dtype, device=t.device)
    wide[..., ::2] = t
    v = wide[..., ::2]
    assert not v.is_contiguous()
    return v


def dyn_case(M, N, K, seed, x_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(x_dtype)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.009 + 0.001
    b = (torch.randn(N, generator=g) * 0.1).to(x_dtype)
    return x, w, sw, b


def dyn_op(x, w, sw, b):
    return torch.ops.zentorch.zentorch_dynamic_qlinear(x, w, sw, b)


@pytest.mark.parametrize("scale_shape", ["n", "1n", "n1"])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_dynamic_qlinear_op_scale_shapes(scale_shape, x_dtype):
    M, N, K = 24, 200, 512
    x, w, sw, b = dyn_case(M, N, K, seed=3, x_dtype=x_dtype)
    ref = O.dynamic_qlinear(x, w, sw, b)
    s = {"n": sw, "1n": sw.unsqueeze(0), "n1": sw.unsqueeze(1)}[scale_shape]
    y = dyn_op(x.to(DEV), w.to(DEV), s.to(DEV), b.to(DEV))
    assert y.dtype == x_dtype and y.shape == (M, N)
    torch.testing.assert_close(y.cpu().float(), ref.float(), **TOL)


@pytest.mark.parametrize("M,N,K", [(7, 96, 256), (128, 11008, 4096), (300, 136, 1024)])
def test_dynamic_qlinear_op_noncontiguous_args(M, N, K):
    x, w, sw, b = dyn_case(M, N, K, seed=M + N)
    ref = O.dynamic_qlinear(x, w, sw, b)
    wd, sd, bd = noncontiguous(w.to(DEV)), noncontiguous(sw.unsqueeze(0).to(DEV)), \
        noncontiguous(b.to(DEV))
    y = dyn_op(x.to(DEV), wd, sd, bd)
    torch.testing.assert_close(y.cpu().float(), ref.float(), **TOL)
    # the same values, contiguous: the same result bit for bit
    y2 = dyn_op(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV))
    assert torch.equal(y, y2)


def test_dynamic_qlinear_op_3d_and_strided_input():
    B, S, N, K = 3, 11, 160, 768
    x, w, sw, b = dyn_case(B * S, N, K, seed=17)
    ref = O.dynamic_qlinear(x, w, sw, b).view(B, S, N)
    x3 = x.view(B, S, K).to(DEV)
    y = dyn_op(x3, w.to(DEV), sw.to(DEV), None if b is None else b.to(DEV))
    assert y.shape == (B, S, N)
    torch.testing.assert_close(y.cpu().float(), ref.float(), **TOL)
    # a transposed (non-contiguous) 3-D input
    xt = x.view(B, S, K).transpose(0, 1).contiguous().to(DEV).transpose(0, 1)
    assert not xt.is_contiguous()
    yt = dyn_op(xt, w.to(DEV), sw.to(DEV), b.to(DEV))
    assert torch.equal(yt, y)


def test_dynamic_qlinear_op_no_bias_matches_capi():
    M, N, K = 64, 256, 1024
    x, w, sw, _ = dyn_case(M, N, K, seed=5)
    y = dyn_op(x.to(DEV), w.to(DEV), sw.to(DEV), None)
    yc = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), None)
    assert torch.equal(y, yc)
    torch.testing.assert_close(y.cpu().float(), O.dynamic_qlinear(x, w, sw, None).float(), **TOL)


class DynModel(torch.nn.Module):
    """The reference's Custom_Model_DynamicQLinear: buffers, one op call."""

    def __init__(self, w, sw, b):
        super().__init__()
        self.register_buffer("weight_int8", w)
        self.register_buffer("weight_scales", sw)
        self.register_buffer("bias", b)

    def forward(self, x):
        return torch.ops.zentorch.zentorch_dynamic_qlinear(
            x, self.weight_int8, self.weight_scales, self.bias)


@pytest.mark.parametrize("contiguous", [True, False])
def test_dynamic_qlinear_model_compiled(contiguous):
    import torch._dynamo
    M, N, K = 16, 96, 256
    x, w, sw, b = dyn_case(M, N, K, seed=23)
    wd, sd, bd = w.to(DEV), sw.unsqueeze(0).to(DEV), b.to(DEV)
    if not contiguous:
        wd, sd, bd = noncontiguous(wd), noncontiguous(sd), noncontiguous(bd)
    model = DynModel(wd, sd, bd).eval()
    xd = x.view(2, 8, K).to(DEV)
    with torch.inference_mode():
        eager = model(xd)
        torch._dynamo.reset()
        compiled = torch.compile(model, backend="zentorch")(xd)
    assert compiled.dtype == eager.dtype
    torch.testing.assert_close(compiled, eager, atol=1e-3, rtol=1e-3)
    torch.testing.assert_close(eager.view(M, N).cpu().float(),
                               O.dynamic_qlinear(x, w, sw, b).float(), **TOL)


# --------------------------------------------------------------- int4 WOQ op
def woq_case(M, N, K, G, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(G, N, generator=g) * 0.015 + 0.005).bfloat16()
    return x, q, O.woq_repack_weight(q), s


@pytest.mark.parametrize("M", [1, 4, 24, 64])
def test_woq_op_strided_input_rows(M):
    # a column slice of a wider activation: the op passes the row stride to
    # the kernels instead of copying
    N, K, G = 512, 2048, 16
    x, q, wp, s = woq_case(M, N, K, G, seed=M)
    ref = O.woq_linear(x, wp, s)
    wide = torch.zeros(M, K + 256, dtype=torch.bfloat16)
    wide[:, 128:128 + K] = x
    xs = wide.to(DEV)[:, 128:128 + K]
    assert M == 1 or not xs.is_contiguous()
    y = torch.ops.zentorch.zentorch_woq_linear(xs, wp.to(DEV).t(), s.to(DEV), None)
    torch.testing.assert_close(y.cpu().float(), ref.float(), **TOL)
    yc = torch.ops.zentorch.zentorch_woq_linear(x.to(DEV), wp.to(DEV).t(), s.to(DEV), None)
    assert torch.equal(y, yc)


def test_woq_op_3d_input_and_strided_binary():
    B, S, N, K, G = 2, 5, 256, 1024, 8
    x, q, wp, s = woq_case(B * S, N, K, G, seed=4)
    g = torch.Generator().manual_seed(8)
    add = torch.randn(B * S, N, generator=g).bfloat16()
    ref = O.woq_linear(x, wp, s, post_ops=("add",), post_bufs=[add])
    wide = torch.zeros(B * S, 2 * N, dtype=torch.bfloat16)
    wide[:, N:] = add
    add_s = wide.to(DEV)[:, N:].view(B, S, N)
    y = torch.ops.zentorch.zentorch_woq_linear_add(x.view(B, S, K).to(DEV), wp.to(DEV).t(),
                                                    s.to(DEV), None, add_s)
    assert y.shape == (B, S, N)
    torch.testing.assert_close(y.view(B * S, N).cpu().float(), ref.float(), **TOL)


def test_woq_op_weight_not_a_transposed_view():
    # a [K/8, N] weight with contiguous storage is copied into the kernels'
    # layout (with a one-time warning) and gives the same result
    M, N, K, G = 4, 128, 512, 4
    x, q, wp, s = woq_case(M, N, K, G, seed=6)
    w_view = wp.to(DEV).t()
    w_copy = w_view.contiguous()
    y_ref = torch.ops.zentorch.zentorch_woq_linear(x.to(DEV), w_view, s.to(DEV), None)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        y = torch.ops.zentorch.zentorch_woq_linear(x.to(DEV), w_copy, s.to(DEV), None)
    assert torch.equal(y, y_ref)


# ----------------------------------------------------------- HIP graph capture
def test_woq_op_split_k_workspace_under_graph_capture():
    """A captured call keeps its own workspace: capture a 24-row call whose K
    is split over workgroups (fp32 partials in the workspace), run larger
    eager calls that need more workspace, then replay the graph several
    times with eager work in between; every replay equals the eager result
    and a tensor allocated after the capture is left untouched."""
    ops = torch.ops.zentorch
    M, N, K, G = 24, 512, 14336, 112
    x, q, wp, s = woq_case(M, N, K, G, seed=31)
    xd, wd, sd = x.to(DEV), wp.to(DEV).t(), s.to(DEV)
    eager = ops.zentorch_woq_linear(xd, wd, sd, None)
    torch.testing.assert_close(eager.cpu().float(), O.woq_linear(x, wp, s).float(), **TOL)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.zentorch_woq_linear(xd, wd, sd, None)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = ops.zentorch_woq_linear(xd, wd, sd, None)

    big = woq_case(64, 4096, K, G, seed=32)
    bx, bw, bs = big[0].to(DEV), big[2].to(DEV).t(), big[3].to(DEV)
    sentinel = torch.full((1 << 22,), 7.0, device=DEV)
    for _ in range(3):
        yb = ops.zentorch_woq_linear(bx, bw, bs, None)  # larger split-K workspace
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, eager)
        assert bool((sentinel == 7.0).all())
    torch.testing.assert_close(yb[:, :64].cpu().float(),
                               O.woq_linear(big[0], big[2][:64].contiguous(),
                                            big[3][:, :64].contiguous()).float(), **TOL)


def test_dynamic_qlinear_op_under_graph_capture():
    M, N, K = 128, 1024, 2048
    x, w, sw, b = dyn_case(M, N, K, seed=41)
    xd, wd, sd, bd = x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)
    eager = dyn_op(xd, wd, sd, bd)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dyn_op(xd, wd, sd, bd)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = dyn_op(xd, wd, sd, bd)
    x2 = dyn_case(2 * M, N, K, seed=42)
    # new activations in the captured input before each replay (M = 128 runs
    # the split-K kernel, whose tile counters the captured quantise kernel
    # clears on every replay): each replay equals an eager call on them
    for i in range(3):
        dyn_op(x2[0].to(DEV), wd, sd, bd)
        xi = x if i == 2 else dyn_case(M, N, K, seed=50 + i)[0]
        xd.copy_(xi.to(DEV))
        ref = dyn_op(xd.clone(), wd, sd, bd)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, ref)
    assert torch.equal(y_graph, eager)
    torch.testing.assert_close(eager.cpu().float(), O.dynamic_qlinear(x, w, sw, b).float(), **TOL)


# the prefill GEMM kernels under graph capture: int8 256 x 192 and 256 x 128
# load-wave tiles, int4 load-wave 256 x 192 / 256 x 128 and the two-workgroup
# 32x32 kernel; each replay runs on new activations copied into the captured
# input and must equal an eager call on them, with other eager calls between
@pytest.mark.parametrize("path,M,N,K", [("int8", 2100, 4608, 256), ("int8", 2048, 512, 1024),
                                        ("int4", 2100, 4608, 256), ("int4", 2048, 2048, 256),
                                        ("int4", 2100, 8192, 128)])
def test_prefill_kernels_under_graph_capture(path, M, N, K):
    if path == "int8":
        x, w, sw, b = dyn_case(M, N, K, seed=N + K)
        wd, sd, bd = w.to(DEV), sw.to(DEV), b.to(DEV)
        op = lambda xx: dyn_op(xx, wd, sd, bd)
        ref0 = O.dynamic_qlinear(x, w, sw, b)
    else:
        x, q, wp, s = woq_case(M, N, K, K // 128, seed=N + K)
        wd, sd = wp.to(DEV).t(), s.to(DEV)
        op = lambda xx: torch.ops.zentorch.zentorch_woq_linear(xx, wd, sd, None)
        ref0 = O.woq_linear(x, wp, s)
    xd = x.to(DEV)
    eager = op(xd)
    torch.testing.assert_close(eager.cpu().float(), ref0.float(), **TOL)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        op(xd)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = op(xd)
    for i in range(3):
        xi = torch.randn(M, K, generator=torch.Generator().manual_seed(60 + i)).bfloat16()
        xd.copy_(xi.to(DEV))
        ref = op(xd.clone())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, ref)


# extension ops: dynamic qlinear with a fused silu * mul or residual add
@pytest.mark.parametrize("M,N,K", [(4, 96, 256), (128, 11008, 4096), (300, 136, 1024),
                                   (2048, 512, 1024)])
@pytest.mark.parametrize("op", ["silu_mul", "add"])
def test_dynamic_qlinear_fused_epilogue_ops(M, N, K, op):
    x, w, sw, b = dyn_case(M, N, K, seed=M + N + K)
    g = torch.Generator().manual_seed(M)
    other = torch.randn(M, N, generator=g).bfloat16()
    post = ("silu", "mul") if op == "silu_mul" else ("add",)
    ref = O.dynamic_qlinear(x, w, sw, b, post_ops=post, post_bufs=[other])
    fn = getattr(torch.ops.zentorch, f"zentorch_dynamic_qlinear_{op}")
    y = fn(x.to(DEV), w.to(DEV), sw.to(DEV), other.to(DEV), b.to(DEV))
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    torch.testing.assert_close(y.cpu().float(), ref.float(), **TOL)
    # 3-D input and operand
    y3 = fn(x.view(1, M, K).to(DEV), w.to(DEV), sw.to(DEV), other.view(1, M, N).to(DEV),
            b.to(DEV))
    assert torch.equal(y3.view(M, N), y)
