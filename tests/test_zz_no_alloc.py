"""zt_dynamic_qlinear_scratch, the allocation-free variant of
zt_dynamic_qlinear (its scratch is a device array the library holds per
GPU), against zt_dynamic_qlinear with a caller workspace, through the C-ABI.

Both run the same kernels, so the outputs must be identical bit for bit
(the integer stages are exact and the epilogue is the same code).  Two calls
in a row, the second smaller, check that the scratch keeps no state a call
depends on; a call that needs more scratch than the array holds is refused
before anything is launched.
"""
import ctypes

import pytest
import torch

import zt_capi as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
_vp, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[case] {request.node.name}", flush=True)


def _bind():
    L = C.lib()
    L.zt_dynamic_qlinear_scratch.argtypes = [_vp, _i32, _i64, _i64, _vp, _i64, _vp, _i32, _vp,
                                             _i32, ctypes.POINTER(C.PostOps), _vp, _i32, _vp]
    L.zt_dynamic_qlinear_scratch.restype = ctypes.c_int
    L.zt_dynamic_qlinear_scratch_max.restype = ctypes.c_size_t
    return L


def scratch_call(x, w, sw, bias=None, post_ops=(), post_bufs=()):
    L = _bind()
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty(M, N, dtype=x.dtype, device=x.device)
    po, keep = C.make_post(post_ops, post_bufs, N)
    rc = L.zt_dynamic_qlinear_scratch(
        C._p(x), C.DT[x.dtype], M, K, C._p(w), N, C._p(sw), C.DT[sw.dtype], C._p(bias),
        C.DT[bias.dtype] if bias is not None else -1,
        ctypes.byref(po) if post_ops else None, C._p(y), C.DT[y.dtype], C._stream())
    C._check(rc)
    torch.cuda.synchronize()
    del keep
    return y


def case(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.009 + 0.001
    b = (torch.randn(N, generator=g) * 0.1).bfloat16()
    return x, w, sw, b


@pytest.mark.parametrize("first,second", [((128, 11008, 4096), (16, 512, 1024)),
                                          ((2048, 1024, 4096), (33, 4096, 4096)),
                                          ((300, 136, 1024), (1, 96, 256))])
def test_scratch_matches_workspace_two_calls(first, second):
    for i, (M, N, K) in enumerate((first, second)):
        x, w, sw, b = case(M, N, K, seed=M + N + i)
        xd, wd, sd, bd = x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)
        y_ws = C.dynamic_qlinear(xd, wd, sd, bd)
        y_sc = scratch_call(xd, wd, sd, bd)
        assert torch.equal(y_sc, y_ws), (M, N, K)
        rows = slice(0, min(M, 64))
        torch.testing.assert_close(
            y_sc[rows].cpu().float(),
            O.dynamic_qlinear(x[rows].contiguous(), w, sw, b).float(), rtol=1e-2, atol=1e-2)


def test_scratch_post_ops():
    M, N, K = 48, 136, 512
    x, w, sw, b = case(M, N, K, seed=3)
    g = torch.Generator().manual_seed(4)
    add = torch.randn(M, N, generator=g).bfloat16().to(DEV)
    xd, wd, sd, bd = x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)
    y_ws = C.dynamic_qlinear(xd, wd, sd, bd, post_ops=("relu", "add"), post_bufs=[add])
    y_sc = scratch_call(xd, wd, sd, bd, post_ops=("relu", "add"), post_bufs=[add])
    assert torch.equal(y_sc, y_ws)


def test_scratch_refuses_oversized_call():
    L = _bind()
    cap = L.zt_dynamic_qlinear_scratch_max()
    assert cap == 32 << 20
    K = 8192
    M = cap // K + 64  # needs more than the array holds
    rc = L.zt_dynamic_qlinear_scratch(None, C.DT[torch.bfloat16], M, K, None, 16, None,
                                      C.DT[torch.float32], None, -1, None, None,
                                      C.DT[torch.bfloat16], C._stream())
    assert rc == 1
    assert b"scratch" in L.zt_last_error_string()


def test_scratch_on_a_side_stream():
    # a stream other than the null stream: the call takes the array of the
    # stream's device and leaves the caller's current device as it was
    M, N, K = 64, 1000, 2048
    x, w, sw, b = case(M, N, K, seed=5)
    xd, wd, sd, bd = x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)
    y_ws = C.dynamic_qlinear(xd, wd, sd, bd)
    dev_before = torch.cuda.current_device()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y_sc = scratch_call(xd, wd, sd, bd)
    assert torch.cuda.current_device() == dev_before
    assert torch.equal(y_sc, y_ws)
