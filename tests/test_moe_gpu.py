"""GPU parity of the grouped int4 MoE (zt_woq_moe / zentorch_fused_moe with
int4 experts) against the CPU oracle.  Outputs are bf16: rtol = atol = 1e-2
(the tolerance of test_dynamic_qlinear.py:103 and the WOQ model tests).
Full Mixtral-sized layers are checked on a subset of tokens against the
oracle (output rows are independent) and by permutation invariance, which
must hold bit for bit.
"""
import pytest
import torch

import zt_capi as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = dict(rtol=1e-2, atol=1e-2)


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[case] {request.node.name}", flush=True)


def make_experts(E, H, I, gs=128, seed=0, bias=False):
    """Random symmetric int4 experts, packed per expert; weights ~1/sqrt(K)
    so activations stay O(1) through both layers."""
    g = torch.Generator().manual_seed(seed)
    q13 = torch.randint(-8, 8, (E, 2 * I, H), generator=g, dtype=torch.int8)
    q2 = torch.randint(-8, 8, (E, H, I), generator=g, dtype=torch.int8)
    s13 = (torch.rand(E, H // gs, 2 * I, generator=g) * 0.02 + 0.01) / H ** 0.5
    s2 = (torch.rand(E, I // gs, H, generator=g) * 0.02 + 0.01) / I ** 0.5
    w13 = torch.stack([O.woq_repack_weight(q13[e]) for e in range(E)])
    w2 = torch.stack([O.woq_repack_weight(q2[e]) for e in range(E)])
    b13 = (torch.randn(E, 2 * I, generator=g) * 0.1).bfloat16() if bias else None
    b2 = (torch.randn(E, H, generator=g) * 0.1).bfloat16() if bias else None
    return w13, s13.bfloat16(), w2, s2.bfloat16(), b13, b2


def route(T, E, k, seed=0):
    """Mixtral routing: top-k of the router logits, softmax over the chosen."""
    g = torch.Generator().manual_seed(seed + 1)
    logits = torch.randn(T, E, generator=g)
    top, ids = torch.topk(logits, k)
    return ids.int(), torch.softmax(top, dim=-1)


def dev(*ts):
    return [t.to(DEV) if t is not None else None for t in ts]


def run_gpu(x, ids, wts, experts, act="silu", skip=False):
    w13, s13, w2, s2, b13, b2 = dev(*experts)
    return C.woq_moe(x.to(DEV), ids.to(DEV), wts.to(DEV), w13, s13, w2, s2, b13, b2,
                     act=act, skip_weighted=skip).cpu()


@pytest.mark.parametrize("T,H,I,E,k", [(8, 256, 128, 4, 2), (33, 512, 256, 8, 2),
                                       (64, 1024, 2048, 8, 2), (5, 256, 384, 3, 3)])
@pytest.mark.parametrize("act", ["silu", "gelu", "gelu_tanh"])
def test_moe_vs_oracle(T, H, I, E, k, act):
    experts = make_experts(E, H, I, seed=T + H)
    ids, wts = route(T, E, k, seed=T)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(7)).bfloat16()
    y = run_gpu(x, ids, wts, experts, act=act)
    ref = O.woq_moe(x, ids, wts, *experts[:4], act=act)
    torch.testing.assert_close(y.float(), ref.float(), **TOL)


def test_moe_bias_bf16_weights_dropped_ids():
    T, H, I, E, k = 40, 512, 256, 6, 2
    experts = make_experts(E, H, I, seed=3, bias=True)
    ids, wts = route(T, E, k, seed=3)
    ids[0, 1] = -1    # remote expert (expert parallel): dropped
    ids[5, 0] = E + 3  # outside [0, E): dropped
    wts = wts.bfloat16()
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(8)).bfloat16()
    y = run_gpu(x, ids, wts, experts)
    ref = O.woq_moe(x, ids, wts, *experts[:4], w13_bias=experts[4], w2_bias=experts[5])
    torch.testing.assert_close(y.float(), ref.float(), **TOL)


def test_moe_one_expert_takes_every_pair_and_idle_experts():
    # M_e = 200 > the 64-row tile: several row tiles of one expert; the
    # other experts get nothing
    T, H, I, E = 200, 256, 256, 5
    experts = make_experts(E, H, I, seed=4)
    ids = torch.full((T, 1), 2, dtype=torch.int32)
    wts = torch.ones(T, 1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9)).bfloat16()
    y = run_gpu(x, ids, wts, experts, skip=True)
    ref = O.woq_moe(x, ids, wts, *experts[:4], skip_weighted=True)
    torch.testing.assert_close(y.float(), ref.float(), **TOL)


# both tile widths of each GEMM (ZT_MOE_BN="gate_up,down"): 128 (four
# compute waves and an A producer wave) and 256 (the wide form: four waves
# of two tiles, A moved by the compute waves); H = 384 leaves the last
# 256-column down tile half empty
@pytest.mark.parametrize("bn", ["128,128", "256,256", "256,128", "128,256"])
@pytest.mark.parametrize("T,H,I,E,k", [(8, 256, 128, 4, 2), (70, 512, 256, 8, 2),
                                       (64, 1024, 2048, 8, 2), (5, 384, 384, 3, 3)])
def test_moe_tile_widths(T, H, I, E, k, bn, knobs):
    knobs.set("ZT_MOE_BN", bn)
    experts = make_experts(E, H, I, seed=T + H + 1, bias=T == 70)
    ids, wts = route(T, E, k, seed=T + 1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(15)).bfloat16()
    y = run_gpu(x, ids, wts, experts)
    ref = O.woq_moe(x, ids, wts, *experts[:4], w13_bias=experts[4], w2_bias=experts[5])
    torch.testing.assert_close(y.float(), ref.float(), **TOL)


# routing past one 1024-pair chunk, with many experts (up to 64 distinct
# ones in a wave) and with few: every pair must land on its own row
@pytest.mark.parametrize("T,E,k", [(700, 96, 2), (1500, 3, 1), (513, 1024, 2)])
def test_moe_routing_chunks_and_many_experts(T, E, k):
    H, I = 256, 128
    experts = make_experts(E, H, I, seed=T + E)
    ids, wts = route(T, E, k, seed=T + E)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(14)).bfloat16()
    y = run_gpu(x, ids, wts, experts)
    ref = O.woq_moe(x, ids, wts, *experts[:4])
    torch.testing.assert_close(y.float(), ref.float(), **TOL)


def test_moe_decode_single_token():
    T, H, I, E, k = 1, 1024, 512, 8, 2
    experts = make_experts(E, H, I, seed=5)
    ids, wts = route(T, E, k, seed=5)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(10)).bfloat16()
    y = run_gpu(x, ids, wts, experts)
    ref = O.woq_moe(x, ids, wts, *experts[:4])
    torch.testing.assert_close(y.float(), ref.float(), **TOL)


def test_mixtral_layer_subset_and_permutation():
    # 8 experts, hidden 4096, intermediate 14336, top-2
    # over 256 tokens.  Rows are independent, so the oracle checks a subset
    # of tokens; permuting the tokens permutes the output bit for bit.
    T, H, I, E, k = 256, 4096, 14336, 8, 2
    experts = make_experts(E, H, I, seed=6)
    ids, wts = route(T, E, k, seed=6)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(11)).bfloat16()
    y = run_gpu(x, ids, wts, experts)
    sub = torch.tensor([0, 1, 77, 128, 200, 255])
    ref = O.woq_moe(x[sub], ids[sub], wts[sub], *experts[:4])
    torch.testing.assert_close(y[sub].float(), ref.float(), **TOL)
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(12))
    yp = run_gpu(x[perm], ids[perm], wts[perm], experts)
    assert torch.equal(yp, y[perm])


def test_torch_op_writes_output():
    import zentorch  # noqa: F401
    T, H, I, E, k = 16, 512, 256, 4, 2
    w13, s13, w2, s2, _, _ = dev(*make_experts(E, H, I, seed=7))
    ids, wts = route(T, E, k, seed=7)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(13)).bfloat16().to(DEV)
    out = torch.zeros_like(x)
    ret = torch.ops.zentorch.zentorch_fused_moe(out, x, w13, w2, None, None, wts.to(DEV),
                                                ids.to(DEV), False, "silu", s13, s2)
    assert ret is None
    ref = C.woq_moe(x, ids.to(DEV), wts.to(DEV), w13, s13, w2, s2)
    assert torch.equal(out, ref)
    with pytest.raises(RuntimeError, match="w2 must be int8"):
        torch.ops.zentorch.zentorch_fused_moe(out, x, w13.to(torch.int8), w2, None, None,
                                              wts.to(DEV), ids.to(DEV), False, "silu", s13, s2)
    with pytest.raises(RuntimeError, match="swigluoai"):
        torch.ops.zentorch.zentorch_fused_moe(out, x, w13, w2, None, None, wts.to(DEV),
                                              ids.to(DEV), False, "swigluoai", s13, s2)


def test_moe_replays_from_a_hip_graph():
    # no host synchronisation inside the op: it can be captured, and every
    # replay with new inputs matches the eager result
    import zentorch  # noqa: F401
    T, H, I, E, k = 32, 512, 256, 4, 2
    w13, s13, w2, s2, _, _ = dev(*make_experts(E, H, I, seed=8))
    x = torch.zeros(T, H, dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros(T, k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(T, k, device=DEV)
    out = torch.zeros(T, H, dtype=torch.bfloat16, device=DEV)
    op = torch.ops.zentorch.zentorch_fused_moe

    def step():
        op(out, x, w13, w2, None, None, wts, ids, False, "silu", s13, s2)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for r in range(3):
        i_r, w_r = route(T, E, k, seed=20 + r)
        x.copy_(torch.randn(T, H, generator=torch.Generator().manual_seed(30 + r)).bfloat16())
        ids.copy_(i_r)
        wts.copy_(w_r)
        graph.replay()
        torch.cuda.synchronize()
        eager = C.woq_moe(x, ids, wts, w13, s13, w2, s2)
        assert torch.equal(out, eager), f"replay {r}"



# The reference's own expert formats (docs/zentorch_fused_moe.md:80-101):
# float experts in the input's dtype, and int8 experts with per-channel
# scales and per-token dynamic activation quantisation.  The references are
# the reference's per-expert fallback loop (vllm/_int8_moe_patch.py:149-206)
# restated on the CPU: the oracle's dynamic_qlinear for int8 experts, fp32
# F.linear on the same weights for float experts.
def _act(name):
    import torch.nn.functional as F
    return {"silu": F.silu, "gelu": F.gelu,
            "gelu_tanh": lambda t: F.gelu(t, approximate="tanh")}[name]


def moe_reference(x, ids, wts, w13, w2, b13, b2, act, skip, per_expert):
    """sum_k w[t, k] * expert(ids[t, k])(x[t]) with per_expert(xe, e) ->
    [n, H]; ids outside [0, E) contribute nothing."""
    T, k = ids.shape
    E = w13.shape[0]
    out = torch.zeros(T, x.shape[1], dtype=torch.float32)
    for e in range(E):
        rows = (ids == e).nonzero()
        if rows.numel() == 0:
            continue
        t, kk = rows[:, 0], rows[:, 1]
        y = per_expert(x[t], e).float()
        w = torch.ones(len(t)) if skip else wts[t, kk].float()
        out.index_add_(0, t, y * w[:, None])
    return out


def float_experts(E, H, I, dtype, seed, bias):
    g = torch.Generator().manual_seed(seed)
    w13 = (torch.randn(E, 2 * I, H, generator=g) / H ** 0.5).to(dtype)
    w2 = (torch.randn(E, H, I, generator=g) / I ** 0.5).to(dtype)
    b13 = (torch.randn(E, 2 * I, generator=g) * 0.1).to(dtype) if bias else None
    b2 = (torch.randn(E, H, generator=g) * 0.1).to(dtype) if bias else None
    return w13, w2, b13, b2


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-3)])
@pytest.mark.parametrize("act", ["silu", "gelu", "gelu_tanh"])
@pytest.mark.parametrize("bias", [False, True])
def test_fused_moe_float_experts(dtype, tol, act, bias):
    # bf16 experts round the gate_up GEMM output and the intermediate to
    # bf16, as the reference's bf16 GEMMs do; the fp32 reference does not:
    # 2e-2 for bf16, 1e-3 for fp32
    import torch.nn.functional as F
    import zentorch  # noqa: F401
    T, H, I, E, k = 24, 256, 128, 5, 2
    w13, w2, b13, b2 = float_experts(E, H, I, dtype, seed=21, bias=bias)
    ids, wts = route(T, E, k, seed=21)
    ids[3, 1] = -1  # dropped
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(22)).to(dtype)
    out = torch.empty(T, H, dtype=dtype, device=DEV)
    torch.ops.zentorch.zentorch_fused_moe(out, *dev(x, w13, w2, b13, b2, wts, ids), False, act)

    def expert(xe, e):
        gu = F.linear(xe.float(), w13[e].float(), None if b13 is None else b13[e].float())
        h = _act(act)(gu[:, :I]) * gu[:, I:]
        return F.linear(h, w2[e].float(), None if b2 is None else b2[e].float())

    ref = moe_reference(x, ids, wts, w13, w2, b13, b2, act, False, expert)
    torch.testing.assert_close(out.cpu().float(), ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("act", ["silu", "gelu", "gelu_tanh"])
@pytest.mark.parametrize("bias,scale_shape", [(False, "flat"), (True, "col")])
def test_fused_moe_int8_experts(act, bias, scale_shape):
    import zentorch  # noqa: F401
    T, H, I, E, k = 20, 256, 192, 4, 2
    g = torch.Generator().manual_seed(31)
    w13 = torch.randint(-127, 128, (E, 2 * I, H), generator=g, dtype=torch.int8)
    w2 = torch.randint(-127, 128, (E, H, I), generator=g, dtype=torch.int8)
    s13 = torch.rand(E, 2 * I, generator=g) * 0.004 / H ** 0.5 * 16
    s2 = torch.rand(E, H, generator=g) * 0.004 / I ** 0.5 * 16
    b13 = (torch.randn(E, 2 * I, generator=g) * 0.1).bfloat16() if bias else None
    b2 = (torch.randn(E, H, generator=g) * 0.1).bfloat16() if bias else None
    ids, wts = route(T, E, k, seed=31)
    ids[2, 0] = E + 1  # dropped
    x = torch.randn(T, H, generator=g).bfloat16()
    s13d = s13.unsqueeze(-1) if scale_shape == "col" else s13  # [E, N, 1] as torchao
    out = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    torch.ops.zentorch.zentorch_fused_moe(out, *dev(x, w13, w2, b13, b2, wts, ids), False, act,
                                          s13d.to(DEV), s2.to(DEV))

    def expert(xe, e):
        bg = None if b13 is None else b13[e, :I]
        bu = None if b13 is None else b13[e, I:]
        # h = act(gate accumulator) * rounded up half, one rounding (the
        # fused epilogue; the int4 path's convention)
        up = O.dynamic_qlinear(xe, w13[e, I:], s13[e, I:], bu)
        name = {"silu": "silu", "gelu": "gelu_erf", "gelu_tanh": "gelu_tanh"}[act]
        h = O.dynamic_qlinear(xe, w13[e, :I], s13[e, :I], bg, post_ops=(name, "mul"),
                              post_bufs=[up])
        return O.dynamic_qlinear(h, w2[e], s2[e], None if b2 is None else b2[e])

    ref = moe_reference(x, ids, wts, w13, w2, b13, b2, act, False, expert)
    torch.testing.assert_close(out.cpu().float(), ref, **TOL)


def test_fused_moe_dense_errors_and_skip_weighted():
    import zentorch  # noqa: F401
    T, H, I, E = 6, 128, 128, 3
    w13, w2, _, _ = float_experts(E, H, I, torch.bfloat16, seed=41, bias=False)
    ids = torch.tensor([[0], [2], [1], [2], [0], [1]], dtype=torch.int32)
    wts = torch.ones(T, 1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(42)).bfloat16()
    out = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    op = torch.ops.zentorch.zentorch_fused_moe
    op(out, *dev(x, w13, w2), None, None, *dev(wts * 3, ids), True, "silu")
    out2 = torch.empty_like(out)
    op(out2, *dev(x, w13, w2), None, None, *dev(wts, ids), False, "silu")
    assert torch.equal(out, out2)  # skip_weighted ignores the weights
    with pytest.raises(RuntimeError, match="input's dtype"):
        op(out, *dev(x, w13.float(), w2), None, None, *dev(wts, ids), False, "silu")
    with pytest.raises(RuntimeError, match="need w13_scales"):
        op(out, *dev(x, w13.to(torch.int8), w2.to(torch.int8)), None, None, *dev(wts, ids),
           False, "silu")
    with pytest.raises(RuntimeError, match="per-group"):
        op(out, *dev(x, w13.to(torch.int8), w2.to(torch.int8)), None, None, *dev(wts, ids),
           False, "silu", torch.ones(E, 2, 2 * I, device=DEV), torch.ones(E, H, device=DEV))
    with pytest.raises(RuntimeError, match="swigluoai"):
        op(out, *dev(x, w13, w2), None, None, *dev(wts, ids), False, "swigluoai")
