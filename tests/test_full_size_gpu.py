"""Parity at the exact shapes bench.py times, against the CPU oracle.

Output columns of a linear are independent (column n depends only on weight
row n, its scales and the bias entry n), and so are output rows.  Each test
runs the whole call on the GPU at its full size and compares a column subset
of the result with the oracle evaluated on just those weight rows, so the
oracle finishes in seconds.  Tolerance rtol = atol = 1e-2 as in the other
parity tests.
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


def full_weights(N, K, G, seed):
    """int4 values [N, K] and bf16 group scales [G, N] (CPU), plus the packed
    [N, K/8] weight repacked on the GPU (bit-exact against the oracle's
    repack in test_woq_gpu)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(G, N, generator=g) * 0.015 + 0.005).bfloat16()
    wp = C.woq_repack_weight(q.to(DEV))
    return q, s, wp


def column_subset(n, count, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randperm(n, generator=g)[:count]
    # always include both ends (first and last row tiles, ragged edges)
    return torch.unique(torch.cat([idx, torch.tensor([0, n - 1])]))


def oracle_cols(x, q, s, cols, bias=None, post=(), bufs=()):
    """The oracle on weight rows `cols` only: y[:, cols].  `bufs` are the
    binary post-op operands already restricted to those columns."""
    qs = q[cols].contiguous()
    return O.woq_linear(x, O.woq_repack_weight(qs), s[:, cols].contiguous(),
                        bias=None if bias is None else bias[cols].contiguous(),
                        post_ops=post, post_bufs=[b.contiguous() for b in bufs])


@pytest.mark.parametrize("M", [1, 4, 8, 16, 64])
@pytest.mark.parametrize("name,N,K", [("qkv", 6144, 4096), ("o", 4096, 4096)])
def test_llama_projection_full_size(M, name, N, K):
    G = K // 128
    q, s, wp = full_weights(N, K, G, seed=N + M)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).bfloat16()
    y = C.woq_linear(x.to(DEV), wp, s.to(DEV)).cpu()
    cols = column_subset(N, 192, seed=M)
    torch.testing.assert_close(y[:, cols].float(), oracle_cols(x, q, s, cols).float(), **TOL)


@pytest.mark.parametrize("M", [1, 8, 16, 64])
def test_down_projection_residual_add_full_size(M):
    # 4096 x 14336 with the residual add of the decode layer, full N
    N, K = 4096, 14336
    G = K // 128
    q, s, wp = full_weights(N, K, G, seed=M + 1)
    g = torch.Generator().manual_seed(M + 2)
    x = torch.randn(M, K, generator=g).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    y = C.woq_linear(x.to(DEV), wp, s.to(DEV), post_ops=("add",), post_bufs=[res.to(DEV)]).cpu()
    cols = column_subset(N, 160, seed=M + 3)
    ref = oracle_cols(x, q, s, cols, post=("add",), bufs=[res[:, cols]])
    torch.testing.assert_close(y[:, cols].float(), ref.float(), **TOL)


@pytest.mark.parametrize("M", [1, 8, 16, 17, 64])
def test_merged_gate_up_full_size(M):
    # the merged 28672 x 4096 gate_up with silu(gate) * up, against the
    # two-op composition on the oracle for a subset of output columns j
    # (gate row j, up row I + j)
    I, K = 14336, 4096
    G = K // 128
    q, s, wp = full_weights(2 * I, K, G, seed=M + 7)
    g = torch.Generator().manual_seed(M + 8)
    x = torch.randn(M, K, generator=g).bfloat16()
    b = torch.randn(2 * I, generator=g).bfloat16()
    y = C.woq_linear_gate_up(x.to(DEV), wp, s.to(DEV), bias=b.to(DEV)).cpu()
    j = column_subset(I, 128, seed=M + 9)
    up = oracle_cols(x, q, s, j + I, bias=b)
    ref = oracle_cols(x, q, s, j, bias=b, post=("silu", "mul"), bufs=[up])
    torch.testing.assert_close(y[:, j].float(), ref.float(), **TOL)


@pytest.mark.parametrize("name,N,K", [("qkv", 6144, 4096), ("o", 4096, 4096),
                                      ("gate_up", 28672, 4096), ("down", 4096, 14336)])
def test_prefill_int4_full_size(name, N, K):
    # config 3, int4 path: M = 2048 on the bf16-MFMA GEMM kernel
    M, G = 2048, K // 128
    q, s, wp = full_weights(N, K, G, seed=N + K)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, K, generator=g).bfloat16()
    y = C.woq_linear(x.to(DEV), wp, s.to(DEV)).cpu()
    cols = column_subset(N, 48, seed=N)
    rows = column_subset(M, 256, seed=K)  # a row subset keeps the oracle fast
    ref = oracle_cols(x[rows].contiguous(), q, s, cols)
    torch.testing.assert_close(y[rows][:, cols].float(), ref.float(), **TOL)


def dyn_case(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.009 + 0.001
    b = (torch.randn(N, generator=g) * 0.1).bfloat16()
    return x, w, sw, b


@pytest.mark.parametrize("name,N,K", [("qkv", 6144, 4096), ("o", 4096, 4096),
                                      ("gate_up", 28672, 4096), ("down", 4096, 14336)])
def test_prefill_int8_full_op_full_size(name, N, K):
    # config 3, int8 path: the whole op (quantise + GEMM + epilogue) at
    # M = 2048; quantised rows and int32 accumulators are exact, so a row and
    # column subset of the oracle pins every stage
    M = 2048
    x, w, sw, b = dyn_case(M, N, K, seed=N + 1)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)).cpu()
    cols = column_subset(N, 64, seed=N + 2)
    rows = column_subset(M, 192, seed=N + 3)
    ref = O.dynamic_qlinear(x[rows].contiguous(), w[cols].contiguous(), sw[cols].contiguous(),
                            b[cols].contiguous())
    torch.testing.assert_close(y[rows][:, cols].float(), ref.float(), **TOL)
