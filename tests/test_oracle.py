"""Pins the CPU oracle (oracle/zt_oracle.c) before it is trusted as the checker.

Each check compares the oracle with something that does not share its code:
hand-computed known answers, stock-torch routines (F.linear on torch-dequantised
weights, aten's int4pack/tinygemm kernels, torch._int_mm), the reference tests'
own closed forms, and the committed golden fixtures.  Tolerances are the
reference tests' where they exist.
"""
import os

import pytest
import torch
from safetensors.torch import load_file

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    return load_file(os.path.join(GOLDEN, name + ".safetensors"))


def _ulp(y):
    return torch.finfo(torch.bfloat16).eps * y.float().abs().clamp(min=2.0 ** -126)


# ----------------------------------------------------------------- repack
def test_repack_known_answers():
    # WOQ_Linear.cpp:345-350: nibble i of word c is element 8c+i, LSB first.
    w = torch.tensor([[1, 2, 3, 4, 5, 6, 7, -8],
                      [-1, 0, 0, 0, 0, 0, 0, 0],
                      [0, 0, 0, 0, 0, 0, 0, -1],
                      [7, -8, 7, -8, 7, -8, 7, -8]], dtype=torch.int8)
    out = O.woq_repack_weight(w)
    expect = [0x87654321, 0x0000000F, 0xF0000000, 0x87878787]
    assert [v & 0xFFFFFFFF for v in out.view(-1).tolist()] == expect


def test_repack_round_trip_all_values():
    # every value in every nibble position; unpack by shifting back
    vals = torch.arange(-8, 8, dtype=torch.int8)
    w = torch.stack([vals.roll(i) for i in range(16)])  # [16, 16]
    out = O.woq_repack_weight(w).view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    K = w.shape[1]
    back = torch.empty_like(w)
    for k in range(K):
        nib = (out[:, k // 8] >> (4 * (k % 8))) & 0xF
        back[:, k] = torch.where(nib >= 8, nib - 16, nib).to(torch.int8)
    assert torch.equal(back, w)


def test_repack_rejects_bad_k():
    with pytest.raises(ValueError):
        O.woq_repack_weight(torch.zeros(4, 12, dtype=torch.int8))


def test_unpack_int4pack_matches_torch_packing():
    g = torch.Generator().manual_seed(3)
    for N, K in [(64, 64), (128, 256), (192, 32)]:
        u = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
        packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(u, 1)
        assert torch.equal(O.unpack_int4pack(packed, K), u.to(torch.int8))


# ------------------------------------------------------------------- WOQ
def _dq_torch(q, s, gs):
    return (q.float() * s.float().repeat_interleave(gs, 0).t()).bfloat16().float()


@pytest.mark.parametrize("M,K,N,gs", [(1, 128, 32, 128), (4, 256, 64, 128),
                                      (16, 512, 48, 256), (5, 64, 40, 64)])
def test_woq_symmetric_vs_torch_linear(M, K, N, gs):
    g = torch.Generator().manual_seed(M * 1000 + K + N)
    x = torch.randn(M, K, generator=g).bfloat16()
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(K // gs, N, generator=g) * 0.015 + 0.005).bfloat16()
    b = torch.randn(N, generator=g).bfloat16()
    y = O.woq_linear(x, O.woq_repack_weight(q), s, bias=b)
    ref = torch.nn.functional.linear(x.float(), _dq_torch(q, s, gs), b.float()).bfloat16()
    assert ((y.float() - ref.float()).abs() <= _ulp(ref)).all()


def test_woq_per_channel_reference_test_formula():
    # test_woq_linear.py:107-136 at its own tolerance (1e-3)
    g = torch.Generator().manual_seed(11)
    for M, K, N in [(1, 32, 32), (4, 64, 48), (16, 128, 64), (32, 128, 32)]:
        x = torch.randn(M, K, generator=g).bfloat16()
        w = torch.randn(N, K, generator=g).bfloat16()
        b = torch.randn(N, generator=g).bfloat16()
        scale = torch.clamp(w.abs().max(dim=1, keepdim=True)[0] / 8, min=1e-8).float()
        q = torch.clamp(torch.round(w / scale), -8, 7).to(torch.int8)
        y = O.woq_linear(x, O.woq_repack_weight(q), scale.t().contiguous(), bias=b)
        ref = torch.nn.functional.linear(x, (q.to(torch.bfloat16) * scale).to(torch.bfloat16), b)
        assert torch.allclose(y, ref, rtol=1e-3, atol=1e-3)


def test_woq_fp32_activations_keep_fp32_weights():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(3, 64, generator=g)
    q = torch.randint(-8, 8, (16, 64), generator=g, dtype=torch.int8)
    s = torch.rand(1, 16, generator=g) * 0.02
    y = O.woq_linear(x, O.woq_repack_weight(q), s)
    ref = x.double() @ (q.double() * s.double().t()).t()
    assert y.dtype == torch.float32
    assert torch.allclose(y.double(), ref, rtol=1e-5, atol=1e-5)


def test_woq_asymmetric_vs_tinygemm():
    # test_woq_linear_asymmetric.py:100-141 compares against aten's tinygemm
    g = torch.Generator().manual_seed(5)
    for M, K, N, gs in [(1, 256, 64, 128), (8, 512, 128, 256), (4, 1024, 64, 128)]:
        x = torch.randn(M, K, generator=g).bfloat16()
        u = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
        s = (torch.rand(K // gs, N, generator=g) * 0.015 + 0.005).bfloat16()
        z = (torch.randn(K // gs, N, generator=g) * 0.01).bfloat16()
        packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(u, 1)
        wp = O.woq_repack_weight(O.unpack_int4pack(packed, K))
        y = O.woq_linear(x, wp, s, zero_points=z)
        tg = torch.ops.aten._weight_int4pack_mm_for_cpu(x, packed, gs,
                                                        torch.stack([s, z], -1).contiguous())
        assert torch.allclose(y.float(), tg.float(), atol=1e-2, rtol=1e-2)


def test_woq_integer_zero_point():
    g = torch.Generator().manual_seed(6)
    M, K, N, gs = 2, 128, 16, 64
    x = torch.randn(M, K, generator=g).bfloat16()
    u = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand(K // gs, N, generator=g) * 0.02
    zp = torch.randint(0, 16, (K // gs, N), generator=g, dtype=torch.int32)
    y = O.woq_linear(x, O.woq_repack_weight(u), s, zero_points=zp)
    w = ((u.float() - zp.float().repeat_interleave(gs, 0).t()) *
         s.repeat_interleave(gs, 0).t()).bfloat16().float()
    ref = (x.float() @ w.t()).bfloat16()
    assert ((y.float() - ref.float()).abs() <= _ulp(ref)).all()


@pytest.mark.parametrize("post", ["relu", "sigmoid", "gelu_tanh", "gelu_erf", "silu", "tanh"])
def test_woq_unary_post_ops(post):
    g = torch.Generator().manual_seed(21)
    M, K, N = 4, 128, 32
    x = torch.randn(M, K, generator=g).bfloat16()
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(1, N, generator=g) * 0.1).bfloat16()
    b = torch.randn(N, generator=g).bfloat16()
    y = O.woq_linear(x, O.woq_repack_weight(q), s, bias=b, post_ops=[post])
    pre = torch.nn.functional.linear(x.float(), _dq_torch(q, s, K), b.float())
    F = torch.nn.functional
    ref = {"relu": F.relu, "sigmoid": torch.sigmoid, "silu": F.silu, "tanh": torch.tanh,
           "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"),
           "gelu_erf": lambda t: F.gelu(t, approximate="none")}[post](pre).bfloat16()
    assert torch.allclose(y.float(), ref.float(), rtol=1e-2, atol=1e-2)
    # a wrong activation would not pass: relu and gelu differ on this data
    if post == "gelu_erf":
        assert not torch.allclose(y.float(), F.relu(pre).bfloat16().float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("ops", [("mul", "add"), ("add", "add"), ("add",), ("silu", "mul")])
def test_woq_binary_post_ops_in_list_order(ops):
    g = torch.Generator().manual_seed(22)
    M, K, N = 3, 64, 48
    x = torch.randn(M, K, generator=g).bfloat16()
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(1, N, generator=g) * 0.1).bfloat16()
    bufs = [torch.randn(M, N, generator=g).bfloat16() for o in ops if o in ("add", "mul")]
    y = O.woq_linear(x, O.woq_repack_weight(q), s, post_ops=list(ops), post_bufs=bufs)
    v = torch.nn.functional.linear(x.float(), _dq_torch(q, s, K))
    bi = 0
    for o in ops:
        if o == "add":
            v = v + bufs[bi].float(); bi += 1
        elif o == "mul":
            v = v * bufs[bi].float(); bi += 1
        else:
            v = torch.nn.functional.silu(v)
    assert ((y.float() - v.bfloat16().float()).abs() <= _ulp(v) + 1e-6).all()


# ------------------------------------------------------------ dynamic int8
def _qdq_ref(src):
    # test_dynamic_qlinear.py:32-36
    abs_max = src.abs().amax(dim=1, keepdim=True).clamp(min=1e-12)
    scale = abs_max / 127.0
    return torch.clamp(torch.round(src / scale), -128, 127), scale


@pytest.mark.parametrize("M,K", [(1, 4), (7, 12), (16, 16), (33, 4096), (4, 11008)])
def test_dynamic_quantize_matches_reference_closed_form(M, K):
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g) * 3
    qx, sx = O.dynamic_quantize(x)
    q, s = _qdq_ref(x)
    assert torch.equal(qx, q.to(torch.int8))
    assert torch.equal(sx, s.squeeze(1))


def test_dynamic_quantize_edge_rows():
    x = torch.zeros(4, 32)
    x[1, 3] = 1.0                     # single element -> q = 127
    x[2] = torch.linspace(-1, 1, 32)  # exact halves at the ends
    x[3, :] = -5.0                    # constant row
    qx, sx = O.dynamic_quantize(x)
    q, s = _qdq_ref(x)
    assert torch.equal(qx, q.to(torch.int8)) and torch.equal(sx, s.squeeze(1))
    assert qx[0].abs().sum() == 0 and sx[0].item() == pytest.approx(1e-12 / 127)


def test_dynamic_quantize_bf16_widens_exactly():
    g = torch.Generator().manual_seed(4)
    xb = torch.randn(6, 256, generator=g).bfloat16()
    qx, sx = O.dynamic_quantize(xb)
    q, s = _qdq_ref(xb.float())
    assert torch.equal(qx, q.to(torch.int8)) and torch.equal(sx, s.squeeze(1))


def test_s8_gemm_matches_int_mm():
    g = torch.Generator().manual_seed(8)
    for M, N, K in [(17, 33, 64), (64, 128, 256), (3, 5, 4)]:
        a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
        w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
        ref = a.int() @ w.int().t()
        assert torch.equal(O.s8s8s32_gemm(a, w), ref)


def test_dynamic_qlinear_reference_test_formula():
    # test_dynamic_qlinear.py:53-103: fp32 input, atol=rtol=1e-2
    g = torch.Generator().manual_seed(9)
    for M, K, N in [(1, 4, 8), (5, 16, 32), (64, 128, 48)]:
        x = torch.randn(M, K, generator=g)
        w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
        sw = 1 + torch.randn(N, generator=g).abs()
        b = torch.randn(N, generator=g)
        y = O.dynamic_qlinear(x, w, sw, b)
        q, s = _qdq_ref(x)
        ref = torch.matmul(q * s, (w.float() * sw.unsqueeze(1)).t()) + b
        assert y.dtype == torch.float32
        torch.testing.assert_close(y, ref, atol=1e-2, rtol=1e-2)


# ------------------------------------------------------------ golden files
def test_oracle_reproduces_golden_fixtures():
    c = _golden("woq_symmetric_group128")
    assert torch.equal(O.woq_repack_weight(c["q"]), c["w_packed"])
    assert torch.equal(O.woq_linear(c["x"], c["w_packed"], c["scales"]), c["y"])
    assert torch.equal(O.woq_linear(c["x"], c["w_packed"], c["scales"], bias=c["bias"]), c["y_bias"])
    c = _golden("woq_per_channel_fp32_scale")
    assert torch.equal(O.woq_linear(c["x"], c["w_packed"], c["scales"], bias=c["bias"]), c["y"])
    c = _golden("woq_asymmetric_tinygemm")
    K = c["x"].shape[1]
    assert torch.equal(O.woq_repack_weight(O.unpack_int4pack(c["int4pack"], K)), c["w_packed"])
    assert torch.equal(O.woq_linear(c["x"], c["w_packed"], c["scales"], zero_points=c["zero_points"]), c["y"])
    c = _golden("dynamic_qlinear")
    y, qx, sx, acc = O.dynamic_qlinear(c["x"], c["w"], c["w_scales"], c["bias"], return_intermediates=True)
    assert torch.equal(qx, c["qx"]) and torch.equal(sx, c["sx"]) and torch.equal(acc, c["acc"])
    assert torch.equal(y, c["y"])
    qb, sb = O.dynamic_quantize(c["x_bf16"])
    assert torch.equal(qb, c["qx_bf16"]) and torch.equal(sb, c["sx_bf16"])



# ------------------------------------------------------------------ MoE
def _dequant_rows(q, s):
    """q int [N, K] (signed int4 values), s [G, N] -> bf16-rounded q*s in fp32
    (the dequantised weight of the reference test, test_woq_linear.py:118-128)."""
    N, K = q.shape
    G = s.shape[0]
    return (q.float().view(N, G, K // G) * s.float().t().unsqueeze(-1)).view(N, K).bfloat16().float()


@pytest.mark.parametrize("act", ["silu", "gelu", "gelu_tanh"])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_oracle_vs_torch_composition(act, bias):
    # independent restatement with torch ops: per pair, gated activation of
    # the w13 product, bf16 h, bf16 w2 product, weighted sum over k
    g = torch.Generator().manual_seed(11)
    T, H, I, E, k = 12, 256, 128, 4, 2
    x = torch.randn(T, H, generator=g).bfloat16()
    q13 = torch.randint(-8, 8, (E, 2 * I, H), generator=g, dtype=torch.int8)
    q2 = torch.randint(-8, 8, (E, H, I), generator=g, dtype=torch.int8)
    s13 = (torch.rand(E, H // 128, 2 * I, generator=g) * 0.01 + 0.005).bfloat16()
    s2 = (torch.rand(E, I // 128, H, generator=g) * 0.01 + 0.005).bfloat16()
    b13 = (torch.randn(E, 2 * I, generator=g) * 0.1).bfloat16() if bias else None
    b2 = (torch.randn(E, H, generator=g) * 0.1).bfloat16() if bias else None
    wts, ids = torch.topk(torch.softmax(torch.randn(T, E, generator=g), -1), k)
    ids[3, 1] = -1  # dropped pair (expert-parallel remote id)
    w13 = torch.stack([O.woq_repack_weight(q13[e]) for e in range(E)])
    w2 = torch.stack([O.woq_repack_weight(q2[e]) for e in range(E)])
    y = O.woq_moe(x, ids.int(), wts, w13, s13, w2, s2, b13, b2, act=act)
    f = {"silu": torch.nn.functional.silu,
         "gelu": torch.nn.functional.gelu,
         "gelu_tanh": lambda v: torch.nn.functional.gelu(v, approximate="tanh")}[act]
    ref = torch.zeros(T, H)
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if e < 0:
                continue
            gu = x[t].float() @ _dequant_rows(q13[e], s13[e]).t()
            if bias:
                gu = gu + b13[e].float()
            h = (f(gu[:I]) * gu[I:]).bfloat16().float()
            yy = h @ _dequant_rows(q2[e], s2[e]).t()
            if bias:
                yy = yy + b2[e].float()
            ref[t] += wts[t, j] * yy.bfloat16().float()
    torch.testing.assert_close(y.float(), ref, rtol=1e-2, atol=1e-2)


def test_moe_oracle_single_expert_is_the_woq_pipeline():
    # k = 1, skip_weighted: out = w2(act(w13 x)) exactly as two woq_linear
    # calls and the gated activation (a closed special case)
    g = torch.Generator().manual_seed(5)
    T, H, I, E = 6, 256, 128, 3
    x = torch.randn(T, H, generator=g).bfloat16()
    q13 = torch.randint(-8, 8, (E, 2 * I, H), generator=g, dtype=torch.int8)
    q2 = torch.randint(-8, 8, (E, H, I), generator=g, dtype=torch.int8)
    s13 = (torch.rand(E, 1, 2 * I, generator=g) * 0.01 + 0.005).bfloat16()
    s2 = (torch.rand(E, 1, H, generator=g) * 0.01 + 0.005).bfloat16()
    w13 = torch.stack([O.woq_repack_weight(q13[e]) for e in range(E)])
    w2 = torch.stack([O.woq_repack_weight(q2[e]) for e in range(E)])
    ids = torch.tensor([[1], [0], [2], [1], [1], [0]], dtype=torch.int32)
    y = O.woq_moe(x, ids, torch.ones(T, 1), w13, s13, w2, s2, skip_weighted=True)
    for t in range(T):
        e = int(ids[t, 0])
        gu = O.woq_linear(x[t:t + 1], w13[e], s13[e]).float()  # bf16-rounded gate/up
        gu32 = x[t:t + 1].float() @ _dequant_rows(q13[e], s13[e]).t()
        h = (torch.nn.functional.silu(gu32[:, :I]) * gu32[:, I:]).bfloat16()
        yy = O.woq_linear(h, w2[e], s2[e])
        assert torch.equal(y[t:t + 1], yy)
        del gu
