"""GPU parity of the int4 WOQ kernels against the CPU oracle, through the
C-ABI (libzentorch_hip.so), at sizes the oracle finishes in seconds.

Tolerance: rtol = atol = 1e-2 on bf16/fp32 outputs (the bar of the path's
specification and of the reference's fused-op tests,
test/unittests/op_tests/test_woq_linear.py:165).  The repack ops are integer
work and must be bit-exact.
"""
import os

import pytest
import torch
from safetensors.torch import load_file

import zt_capi as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = dict(rtol=1e-2, atol=1e-2)


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[case] {request.node.name}", flush=True)


def make_case(M, K, N, G, seed, zp=None, bias=False, s_dtype=torch.bfloat16,
              x_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(x_dtype)
    if zp is None:
        q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    else:
        q = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(G, N, generator=g) * 0.015 + 0.005).to(s_dtype)
    z = None
    if zp == "float":
        z = (torch.randn(G, N, generator=g) * 0.01).bfloat16()
    elif zp == "int":
        z = torch.randint(0, 16, (G, N), generator=g, dtype=torch.int32)
    b = torch.randn(N, generator=g).bfloat16() if bias else None
    return x, q, O.woq_repack_weight(q), s, z, b


def gpu(*ts):
    return [t.to(DEV) if t is not None else None for t in ts]


def check_close(y_gpu, y_ref, **tol):
    tol = tol or TOL
    torch.testing.assert_close(y_gpu.cpu().float(), y_ref.float(), **tol)


def run_case(M, K, N, G, kernel=None, seed=0, post=(), nbuf=0, **kw):
    """kernel: force one kernel for this call only (None: the library's choice)."""
    x, q, wp, s, z, b = make_case(M, K, N, G, seed, **kw)
    g = torch.Generator().manual_seed(seed + 1)
    bufs = [torch.randn(M, N, generator=g).to(x.dtype) for _ in range(nbuf)]
    y_ref = O.woq_linear(x, wp, s, zero_points=z, bias=b, post_ops=post, post_bufs=bufs)
    xd, wd, sd, zd, bd = gpu(x, wp, s, z, b)
    with C.tuning(ZT_WOQ_FORCE_KERNEL=kernel):
        y = C.woq_linear(xd, wd, sd, zd, bd, post_ops=post, post_bufs=gpu(*bufs))
    check_close(y, y_ref)
    return y, y_ref


# decode kernel: M <= 32, K % 128 == 0
@pytest.mark.parametrize("M", [1, 4, 8, 16, 17, 32])
@pytest.mark.parametrize("K,N,G", [(128, 64, 1), (256, 48, 2), (1024, 112, 8),
                                   (4096, 256, 32), (512, 100, 2), (2048, 64, 1)])
def test_decode_kernel_vs_oracle(M, K, N, G):
    run_case(M, K, N, G, kernel="decode", seed=M * 7 + K + N, bias=(M % 2 == 0))


@pytest.mark.parametrize("zp", ["float", "int"])
@pytest.mark.parametrize("kernel", ["decode", "gemm", "generic"])
def test_zero_points_all_kernels(zp, kernel):
    run_case(8 if kernel != "gemm" else 40, 512, 64, 4, kernel=kernel, zp=zp, seed=3)


@pytest.mark.parametrize("post,nbuf", [(("relu",), 0), (("sigmoid",), 0),
                                       (("gelu_tanh",), 0), (("gelu_erf",), 0),
                                       (("add",), 1), (("mul", "add"), 2),
                                       (("add", "add"), 2), (("silu", "mul"), 1)])
@pytest.mark.parametrize("kernel,M", [("decode", 4), ("decode", 24), ("gemm", 96),
                                      ("generic", 3)])
def test_post_ops_all_kernels(post, nbuf, kernel, M):
    run_case(M, 256, 80, 2, kernel=kernel, post=post, nbuf=nbuf, seed=11, bias=True)


@pytest.mark.parametrize("M,K,N,G", [(33, 128, 64, 1), (64, 256, 96, 2), (130, 512, 200, 4),
                                     (256, 1024, 256, 8), (2048, 256, 128, 2)])
def test_gemm_kernel_vs_oracle(M, K, N, G):
    run_case(M, K, N, G, kernel="gemm", seed=M + K, bias=True)


# the wide decode kernel (17..64 rows, bf16 scales, no zero points,
# K % 256 == 0, N % 4 == 0): one or two 32-token tiles, K split over several
# workgroups (partials + reduce) or not (epilogue in the kernel), ragged N,
# group 128 / 256 / per-channel; K = 768 and 1280 give splits of 3 and 5
# phases (the padded kernel form)
@pytest.mark.parametrize("M", [17, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("K,N,G", [(4096, 1000, 32), (2048, 200, 8), (1024, 2052, 1),
                                   (14336, 384, 112), (768, 260, 6), (1280, 132, 5)])
def test_wide_kernel_vs_oracle(M, K, N, G):
    run_case(M, K, N, G, kernel="wide", seed=M + K + N, bias=(M % 2 == 1))


@pytest.mark.parametrize("splits", ["1", "2", "4", "8"])
@pytest.mark.parametrize("post,nbuf", [(("gelu_tanh",), 0), (("mul", "add"), 2),
                                       (("silu", "mul"), 1)])
def test_wide_kernel_post_ops_and_splits(splits, post, nbuf, knobs):
    knobs.set("ZT_WOQ_WIDE", splits)
    run_case(40, 2048, 264, 16, kernel="wide", post=post, nbuf=nbuf, seed=21, bias=True)


# split counts of the reduce kernel's remaining unrolled form (6) and of its
# general form past eight splits (12 = eight, then four one by one); K =
# 3072 is 12 phases of 256
@pytest.mark.parametrize("splits", ["6", "12"])
def test_wide_kernel_reduce_split_counts(splits, knobs):
    knobs.set("ZT_WOQ_WIDE", splits)
    run_case(33, 3072, 136, 24, kernel="wide", post=("add",), nbuf=1, seed=int(splits), bias=True)


# uneven K splits, where no divisor of the phase count (K / 256) gives whole
# rounds of four phases: splits of whole rounds with a shorter last split
# (43 phases at K = 11008, 74 at 18944, 14 at 3584), chosen by the planner
# or forced (ZT_WOQ_WIDE: 5 splits of 43 phases -> 12, 12, 12, 7; 3 of 14
# -> 8, 6)
@pytest.mark.parametrize("M,K,N,splits,post,nbuf", [(17, 11008, 136, None, (), 0),
                                                     (40, 18944, 200, None, ("add",), 1),
                                                     (64, 11008, 264, "5", ("mul", "add"), 2),
                                                     (33, 3584, 96, "3", (), 0)])
def test_wide_kernel_uneven_splits(M, K, N, splits, post, nbuf, knobs):
    if splits:
        knobs.set("ZT_WOQ_WIDE", splits)
    run_case(M, K, N, K // 128, kernel="wide", post=post, nbuf=nbuf, seed=M + K, bias=True)


# 4608 x 3584 at 17..64 rows (Qwen2's QKV): more than one round of 16-row
# tiles, so the library's own choice is the wide kernel (14 phases in 4
# uneven splits), with post-ops
@pytest.mark.parametrize("M", [17, 40, 64])
def test_wide_kernel_default_past_one_round(M, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    run_case(M, 3584, 4608, 28, post=("add",), nbuf=1, seed=M, bias=True)
    assert "woq wide" in capfd.readouterr().err


# Up to 16 rows the wide kernel takes the calls for which the stream kernel
# has no x layout (K = 11008 at 15-16 rows: two phases do not fit the LDS and
# 86 chunks do not split in four; K = 28672 at 11-16 rows: four phases do not
# fit, eight have no compiled case) or whose phased grid of one workgroup per
# CU makes more than one round (5120 rows at K = 13824 from 12 rows, 4160 at
# K = 28672 from 4 rows)
@pytest.mark.parametrize("M,K,N", [(15, 11008, 2048), (16, 11008, 1544), (8, 28672, 4160),
                                   (16, 28672, 1032), (12, 13824, 5120), (6, 28672, 4160)])
def test_wide_kernel_below_17_rows_without_stream_layout(M, K, N, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    run_case(M, K, N, K // 128, post=("add",), nbuf=1, seed=M + K, bias=True)
    assert "woq wide" in capfd.readouterr().err


# past a round of workgroups the stream kernel takes K phases that fit two
# workgroups per CU: two phases instead of x whole (6 rows, 520 tiles two
# per workgroup), four instead of two (10 rows, 260 tiles)
@pytest.mark.parametrize("M,N,P", [(6, 8320, 2), (10, 4160, 4)])
def test_stream_kernel_phase_preference(M, N, P, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    run_case(M, 8192, N, 64, post=("add",), nbuf=1, seed=M + N, bias=True)
    assert f"P={P} " in capfd.readouterr().err


# K = 28672 (224 chunks, 28 per wave): the lean kernel at 1-2 rows, the
# stream kernel with x whole at 1-2 rows (lean kernel off) and in two K
# phases at 3 rows
@pytest.mark.parametrize("M,N,lean", [(1, 256, None), (2, 264, None), (1, 264, "0"),
                                      (2, 256, "0"), (3, 136, None)])
def test_28_chunks_per_wave(M, N, lean, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    if lean:
        knobs.set("ZT_WOQ_LEAN", lean)
    capfd.readouterr()
    run_case(M, 28672, N, 224, post=("add",), nbuf=1, seed=M + N, bias=True)
    assert ("woq lean" if M <= 2 and not lean else "woq stream") in capfd.readouterr().err


# prefill GEMM with a K split: when its 128 x 128 tiles make less than one
# round (65..~500 rows on small matrices) the workgroups write fp32 partials
# of whole 64-k step ranges into the workspace and the reduce kernel adds
# them in split order and applies bias and post-ops
@pytest.mark.parametrize("M,K,N,post,nbuf", [(65, 4096, 264, (), 0), (128, 11008, 256, ("add",), 1),
                                             (300, 2048, 512, ("gelu_tanh",), 0),
                                             (512, 8192, 136, ("mul", "add"), 2),
                                             (256, 2048, 16384, (), 0)])
def test_gemm32_kernel_k_split(M, K, N, post, nbuf, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    run_case(M, K, N, K // 128, post=post, nbuf=nbuf, seed=M + N, bias=True)
    assert "K splits" in capfd.readouterr().err


def test_wide_kernel_strided_x():
    M, K, N, G = 48, 4096, 512, 32
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=77)
    xs = torch.randn(M, K + 64).bfloat16()
    xs[:, :K] = x
    y_ref = O.woq_linear(x, wp, s)
    xd = xs.to(DEV)[:, :K]
    assert xd.stride(0) == K + 64
    y = C.woq_linear(xd, wp.to(DEV), s.to(DEV))
    check_close(y, y_ref)


# the 32x32 prefill kernel (bf16 scales, no zero points, N % 8 == 0):
# 128 x 128 and 256 x 128 tiles, ragged M and N, group sizes 128 / 256 /
# per-channel, more tiles than CUs
@pytest.mark.parametrize("M,K,N,G", [(300, 1024, 200, 8), (520, 512, 264, 2),
                                     (1100, 2048, 1032, 1), (2100, 768, 4104, 6)])
def test_gemm32_kernel_vs_oracle(M, K, N, G):
    run_case(M, K, N, G, kernel="gemm", seed=M + N, bias=True)


@pytest.mark.parametrize("M,K,N,G", [(1, 32, 32, 1), (4, 64, 48, 1), (24, 128, 64, 2),
                                     (3, 72, 16, 9), (5, 256, 40, 2)])
def test_generic_kernel_vs_oracle(M, K, N, G):
    run_case(M, K, N, G, kernel="generic", seed=M + N, bias=True)


def test_fp32_activations():
    run_case(6, 256, 64, 2, x_dtype=torch.float32, s_dtype=torch.float32, seed=5)


def test_fp32_scales_decode():
    run_case(4, 512, 64, 4, kernel="decode", s_dtype=torch.float32, seed=6)


def test_split_k_counters_reset_between_calls():
    # down-proj shape: K split across workgroups; run twice with the same
    # workspace semantics the torch op uses and compare both calls
    M, K, N, G = 16, 14336, 512, 112
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=42)
    y_ref = O.woq_linear(x, wp, s)
    xd, wd, sd = gpu(x, wp, s)
    y1 = C.woq_linear(xd, wd, sd)
    y2 = C.woq_linear(xd, wd, sd)
    check_close(y1, y_ref)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_config0_full_size(M):
    # BASELINE config 0 shape (M=4, N=K=4096, group 128, bf16 scales)
    run_case(M, 4096, 4096, 32, seed=100 + M)


@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (4096, 14336)])
def test_llama_decode_shapes_m16(N, K):
    run_case(16, K, N, K // 128, seed=N + K)


@pytest.mark.parametrize("M", [1, 3, 4])
@pytest.mark.parametrize("N,K", [(8192, 1024), (3072, 4096), (8192, 8192), (97, 1024)])
def test_stream_kernel_small_m_shapes(M, N, K):
    # M <= 4: one row tile per wave below and above 512 tiles, K of 8 to
    # 64 chunks; odd N takes the general bf16-scale mode
    run_case(M, K, N, K // 128, seed=M + N + K, bias=True)


# the general modes on the stream kernel (zero points, fp32 scales), with
# their weight, scale and zero-point loads pipelined like the fast mode's
@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("zp,s_dtype", [("int", torch.bfloat16), ("float", torch.bfloat16),
                                        (None, torch.float32)])
def test_stream_kernel_general_modes(M, zp, s_dtype):
    run_case(M, 4096, 272, 32, zp=zp, s_dtype=s_dtype, seed=M + 31, bias=True)


@pytest.mark.parametrize("M,N", [(10, 12816), (16, 12800)])
def test_stream_kernel_four_tiles(M, N):
    # x [M, 4096] past 76 KB with at least 800 row tiles: four tiles per
    # wave; N = 12816 leaves a last workgroup with one real tile
    run_case(M, 4096, N, 32, post=("add",), nbuf=1, seed=M + N, bias=True)


def run_gate_up(M, K, I, G, seed, zp=None, x_dtype=torch.bfloat16, bias=True):
    """Merged gate_up against the two-op composition on the oracle: the up
    half through woq_linear, the gate half with the post-ops silu, mul."""
    x, q, wp, s, z, b = make_case(M, K, 2 * I, G, seed, zp=zp, bias=bias, x_dtype=x_dtype)
    half = lambda t, lo: None if t is None else (t[lo:lo + I] if t.dim() == 1 else
                                                 t[:, lo:lo + I].contiguous())
    up = O.woq_linear(x, wp[I:].contiguous(), half(s, I), zero_points=half(z, I),
                      bias=half(b, I))
    y_ref = O.woq_linear(x, wp[:I].contiguous(), half(s, 0), zero_points=half(z, 0),
                         bias=half(b, 0), post_ops=("silu", "mul"), post_bufs=[up])
    xd, wd, sd, zd, bd = gpu(x, wp, s, z, b)
    y = C.woq_linear_gate_up(xd, wd, sd, zd, bd)
    check_close(y, y_ref)
    return y, y_ref


# one launch: bf16, up to 16 rows, I % 16 == 0 (one gate/up tile pair per
# wave, or two once x fills a CU's LDS and there are 800 tiles)
@pytest.mark.parametrize("M", [1, 4, 9, 16])
@pytest.mark.parametrize("K,I,G", [(1024, 64, 8), (4096, 256, 32), (2048, 1040, 1)])
def test_gate_up_one_launch(M, K, I, G):
    run_gate_up(M, K, I, G, seed=M + K + I)


def test_gate_up_two_tile_pairs():
    run_gate_up(16, 4096, 6400, 32, seed=5)


# two steps (fp32 linear into the workspace, then silu * up): more rows,
# fp32 activations, zero points, I % 16 != 0
@pytest.mark.parametrize("M,K,I,G,zp,x_dtype", [
    (20, 1024, 64, 8, None, torch.bfloat16),
    (300, 512, 96, 4, None, torch.bfloat16),
    (4, 1024, 64, 8, None, torch.float32),
    (8, 512, 64, 4, "int", torch.bfloat16),
    (3, 256, 40, 2, None, torch.bfloat16)])
def test_gate_up_two_steps(M, K, I, G, zp, x_dtype):
    run_gate_up(M, K, I, G, seed=M + I, zp=zp, x_dtype=x_dtype)


# one launch on the wide kernel (17-64 rows, no K split, N % 128 == 0):
# forced with one K split at small shapes, and the Llama-3 8B gate_up shape
# that takes it by default.  The 12-row case has x [12, 8192] (196 KB),
# more than the stream kernel's LDS holds, so the stream gate_up refuses it
# and the wide kernel runs it below 17 rows.
@pytest.mark.parametrize("M,K,I,G,bias", [
    (17, 1024, 64, 8, True), (40, 2048, 192, 16, True), (64, 4096, 256, 32, False),
    (33, 512, 128, 1, True), (12, 8192, 64, 64, True)])
def test_gate_up_wide(M, K, I, G, bias, knobs):
    knobs.set("ZT_WOQ_WIDE", "1")
    run_gate_up(M, K, I, G, seed=M + K + I, bias=bias)


@pytest.mark.parametrize("M", [9, 12, 16])
def test_wide_kernel_below_17_rows(M, knobs):
    # the plain linear on the wide kernel at 9-16 rows (one K split)
    knobs.set("ZT_WOQ_WIDE", "1")
    run_case(M, 8192, 384, 64, kernel="wide", seed=M + 3, bias=True)


@pytest.mark.parametrize("M", [17, 64])
def test_gate_up_wide_llama(M):
    run_gate_up(M, 4096, 14336, 32, seed=M)


# 8-16 rows whose x leaves the stream kernel one workgroup per CU over more
# than a round of workgroups (K = 5120, where the persistent kernel has no
# case; 258 workgroups of two gate/up tile pairs): the wide kernel's merged
# form when it takes the call in one launch.  With one round (I = 8192) the
# stream kernel keeps it.
@pytest.mark.parametrize("M,I,kernel", [(8, 8256, "woq wide gate_up"), (14, 8256, "woq wide gate_up"),
                                        (14, 8192, "woq gate_up stream")])
def test_gate_up_wide_below_17_rows(M, I, kernel, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    run_gate_up(M, 5120, I, 40, seed=M)
    assert kernel in capfd.readouterr().err


def test_gate_up_torch_op():
    import zentorch  # noqa: F401
    M, K, I, G = 4, 1024, 128, 8
    x, q, wp, s, z, b = make_case(M, K, 2 * I, G, seed=9, bias=True)
    y = torch.ops.zentorch.zentorch_woq_linear_gate_up_silu_mul(
        x.to(DEV), wp.to(DEV).t(), s.to(DEV), None, b.to(DEV))
    y2 = C.woq_linear_gate_up(*gpu(x, wp, s), None, b.to(DEV))
    assert y.shape == (M, I) and torch.equal(y, y2)


@pytest.mark.parametrize("M,K", [(4, 3328), (16, 3328), (8, 3584)])
def test_stream_kernel_x_copy_paths(M, K):
    # 26 or 28 chunks of K: the stream kernel, x copied by loads when its
    # rows are not whole 1 KB pieces (K % 512 != 0), by DMA otherwise
    run_case(M, K, 96, K // 128, seed=M + K)


@pytest.mark.parametrize("M", [9, 16])
def test_stream_kernel_phases_k8192(M):
    # K = 8192 with M > 9: two K phases of 32 chunks, 4 per wave
    run_case(M, 8192, 208, 64, seed=M + 8192, bias=True)


@pytest.mark.parametrize("M", [5, 8, 9, 16])
@pytest.mark.parametrize("post,nbuf", [((), 0), (("add",), 1)])
def test_stream_kernel_phases_down_shape(M, post, nbuf):
    # K = 14336 with M > 4: x does not fit LDS whole, so it is staged in 2
    # (M <= 8) or 4 K-phases; 256 of the 4096 output rows keep the oracle fast
    run_case(M, 14336, 256, 112, post=post, nbuf=nbuf, seed=M + 3 * nbuf, bias=True)


# K phases whose rows are not whole 1 KB pieces (K / P % 512 != 0): the
# last DMA piece of each row is partial and lands in the row's padding.
# 4096 x 11008 at M = 8 (Llama-2's down projection) runs in 2 phases of
# 5504; before, it fell to the wide kernel on 32 workgroups.  ZT_WOQ_DEBUG
# names the stream kernel and its phase count.
@pytest.mark.parametrize("M,K,N,post,nbuf", [(8, 11008, 136, (), 0), (7, 10496, 64, ("add",), 1),
                                             (8, 18944, 72, (), 0), (6, 18944, 40, ("add",), 1)])
def test_stream_kernel_phases_partial_pieces(M, K, N, post, nbuf, knobs, capfd):
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    run_case(M, K, N, K // 128, post=post, nbuf=nbuf, seed=M + K, bias=True)
    err = capfd.readouterr().err
    assert "woq stream" in err and " P=1 " not in err, err


# 17..64 rows on the stream kernel: 2 or 4 token tiles per weight fragment,
# x staged in 1, 2, 4 or 8 K-phases (M = 17: whole; 20..32: 2; 33..48: 4;
# 49..64: 8 at K = 4096)
@pytest.mark.parametrize("M", [17, 20, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("post,nbuf", [((), 0), (("mul", "add"), 2)])
def test_stream_kernel_token_tiles(M, post, nbuf):
    run_case(M, 4096, 160, 32, post=post, nbuf=nbuf, seed=M + 7 * nbuf, bias=True)


def test_stream_kernel_token_tiles_strided_x():
    M, K, N = 64, 4096, 96
    x, q, wp, s, _, _ = make_case(M, K, N, K // 128, seed=640)
    wide = torch.zeros(M, K + 256, dtype=x.dtype)
    wide[:, 128:128 + K] = x
    y_ref = O.woq_linear(x, wp, s)
    wd = wide.to(DEV)
    y = C.woq_linear(wd[:, 128:128 + K], *gpu(wp, s))
    check_close(y, y_ref)


# M = 33..64 runs as blocks of 16 rows on the decode kernels, with x, y and
# the binary post-op buffers offset to each block's first row
@pytest.mark.parametrize("M", [33, 40, 64])
@pytest.mark.parametrize("post,nbuf", [((), 0), (("mul", "add"), 2), (("silu", "mul"), 1)])
def test_row_blocks_vs_oracle(M, post, nbuf):
    run_case(M, 1024, 112, 8, post=post, nbuf=nbuf, seed=M + 5 * nbuf, bias=True)


def test_row_blocks_strided_x_down_shape():
    # M = 64 rows of a down-projection-shaped call (K = 14336, 512 of its
    # output rows), x a column slice of a wider buffer (ldx > K), residual add
    M, K, N = 64, 14336, 512
    x, q, wp, s, _, b = make_case(M, K, N, K // 128, seed=64, bias=True)
    wide = torch.zeros(M, K + 64, dtype=x.dtype)
    wide[:, 32:32 + K] = x
    res = torch.randn(M, N, generator=torch.Generator().manual_seed(65)).bfloat16()
    y_ref = O.woq_linear(x, wp, s, bias=b, post_ops=("add",), post_bufs=[res])
    wd = wide.to(DEV)
    y = C.woq_linear(wd[:, 32:32 + K], *gpu(wp, s), None, b.to(DEV), post_ops=("add",),
                     post_bufs=[res.to(DEV)])
    check_close(y, y_ref)


def test_llama_gate_up_silu_mul_m8():
    # gate half with the up half as the multiplier, N = 14336 per half
    run_case(8, 4096, 14336, 32, post=("silu", "mul"), nbuf=1, seed=77)


def test_golden_fixtures_on_gpu():
    c = load_file(os.path.join(GOLDEN, "woq_symmetric_group128.safetensors"))
    y = C.woq_linear(*gpu(c["x"], c["w_packed"], c["scales"]), None, c["bias"].to(DEV))
    check_close(y, c["y_bias"])
    c = load_file(os.path.join(GOLDEN, "woq_per_channel_fp32_scale.safetensors"))
    y = C.woq_linear(*gpu(c["x"], c["w_packed"], c["scales"]), None, c["bias"].to(DEV))
    check_close(y, c["y"])
    c = load_file(os.path.join(GOLDEN, "woq_asymmetric_tinygemm.safetensors"))
    y = C.woq_linear(*gpu(c["x"], c["w_packed"], c["scales"], c["zero_points"]))
    check_close(y, c["y"])
    check_close(y, c["y_tinygemm"])


def test_repack_bit_exact():
    g = torch.Generator().manual_seed(1)
    for N, K in [(1, 8), (64, 4096), (37, 264)]:
        q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
        assert torch.equal(C.woq_repack_weight(q.to(DEV)).cpu(), O.woq_repack_weight(q))
    c = load_file(os.path.join(GOLDEN, "woq_asymmetric_tinygemm.safetensors"))
    out = C.woq_repack_from_int4pack(c["int4pack"].to(DEV)).cpu()
    assert torch.equal(out, c["w_packed"])
    u = torch.randint(0, 16, (128, 512), generator=g, dtype=torch.int32)
    packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(u, 1)
    assert torch.equal(C.woq_repack_from_int4pack(packed.to(DEV)).cpu(),
                       O.woq_repack_weight(u.to(torch.int8)))


def test_empty_and_error_paths():
    x, q, wp, s, z, b = make_case(4, 256, 32, 2, seed=0)
    xd, wd, sd = gpu(x, wp, s)
    y = C.woq_linear(xd[:0], wd, sd)  # M = 0
    assert y.shape == (0, 32)
    with pytest.raises(RuntimeError, match="divide K"):
        C.woq_linear(xd, wd, torch.ones(3, 32, dtype=torch.bfloat16, device=DEV))


# the wave-independent decode kernel (fast mode, M <= 16, even N, K = 16
# waves x 1 / 2 / 4 chunks; forced, as the library keeps it for more than
# 4096 rows): group sizes 128 / 256 / 1024 and per channel, every M up to
# the LDS limit, bias and post-ops, strided x, and the same result as the
# stream kernel on these shapes
@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 8, 13, 16])
@pytest.mark.parametrize("K,N,G", [(2048, 16, 16), (4096, 4096, 32), (4096, 496, 16),
                                   (8192, 256, 8), (8192, 112, 1)])
def test_wave_kernel_vs_oracle(M, K, N, G, knobs):
    knobs.set("ZT_WOQ_DEBUG", None)
    knobs.set("ZT_WOQ_WAVE", "1")  # also on 4096 rows or fewer
    y, y_ref = run_case(M, K, N, G, seed=M * 3 + G)
    knobs.set("ZT_WOQ_WAVE", "0")
    y_stream, _ = run_case(M, K, N, G, seed=M * 3 + G)
    check_close(y, y_stream.cpu())


@pytest.mark.parametrize("post,nbuf", [(("relu",), 0), (("gelu_erf",), 0), (("add",), 1),
                                       (("mul", "add"), 2)])
def test_wave_kernel_post_ops(post, nbuf, knobs):
    knobs.set("ZT_WOQ_WAVE", "1")
    run_case(4, 4096, 512, 32, post=post, nbuf=nbuf, seed=5, bias=True)


def test_wave_kernel_strided_x(knobs):
    knobs.set("ZT_WOQ_WAVE", "1")
    M, K, N, G = 4, 4096, 256, 32
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=78)
    xs = torch.randn(M, K + 64).bfloat16()
    xs[:, :K] = x
    y_ref = O.woq_linear(x, wp, s)
    xd = xs.to(DEV)[:, :K]
    y = C.woq_linear(xd, wp.to(DEV), s.to(DEV))
    check_close(y, y_ref)


@pytest.mark.parametrize("M,K,N,G", [(1, 8192, 4100, 64), (2, 8192, 514, 8),
                                     (1, 4096, 1000, 32), (3, 2048, 50, 16)])
def test_wave_kernel_ragged_n(M, K, N, G, knobs):
    knobs.set("ZT_WOQ_WAVE", "1")
    y, _ = run_case(M, K, N, G, seed=M + N)
    knobs.set("ZT_WOQ_WAVE", "0")
    y_stream, _ = run_case(M, K, N, G, seed=M + N)
    check_close(y, y_stream.cpu())


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("K,I,G", [(4096, 256, 32), (2048, 1040, 1), (8192, 64, 64)])
def test_wave_kernel_gate_up(M, K, I, G, knobs):
    knobs.set("ZT_WOQ_PERSIST", "0")
    knobs.set("ZT_WOQ_WAVE", "1")  # also below 3 rows
    y, y_ref = run_gate_up(M, K, I, G, seed=M + I)
    knobs.set("ZT_WOQ_WAVE", "0")
    y_stream, _ = run_gate_up(M, K, I, G, seed=M + I)
    check_close(y, y_stream.cpu())


# the persistent decode kernel (fast mode, M <= 16, K = 8 or 16 waves x
# CPW chunks; forced by ZT_WOQ_PERSIST: "1" 8 waves, "2" 16 waves): every
# workgroup loops over row units with the next units' weights in flight;
# units past N (ragged last unit), more units than workgroups, group sizes
# and per channel, bias and post-ops, and the merged gate_up
# None: the library's choice, the persistent kernel from 12288 rows
@pytest.mark.parametrize("variant", ["1", "2", None])
@pytest.mark.parametrize("M", [1, 4, 9, 16])
@pytest.mark.parametrize("K,N,G", [(2048, 16, 16), (4096, 4096, 32), (4096, 12304, 32),
                                   (2048, 9000, 1), (4096, 496, 16), (4096, 14336, 32)])
def test_persist_kernel_vs_oracle(variant, M, K, N, G, knobs):
    if variant:
        knobs.set("ZT_WOQ_PERSIST", variant)
    y, y_ref = run_case(M, K, N, G, seed=M * 5 + N + G)


@pytest.mark.parametrize("post,nbuf", [(("relu",), 0), (("add",), 1), (("mul", "add"), 2)])
def test_persist_kernel_post_ops(post, nbuf, knobs):
    knobs.set("ZT_WOQ_PERSIST", "1")
    run_case(8, 4096, 8200, 32, post=post, nbuf=nbuf, seed=6, bias=True)


# None: the library's choice, the persistent kernel from 3 rows; "1" / "2"
# 8 / 16 waves over units of 8 gate rows and their 8 up rows, "1p" / "2p"
# over gate/up tile pairs
@pytest.mark.parametrize("variant", ["1", "2", "1p", "2p", None])
@pytest.mark.parametrize("M", [1, 5, 12, 16])
@pytest.mark.parametrize("K,I,G", [(4096, 256, 32), (2048, 4112, 1), (4096, 14336, 32)])
def test_persist_kernel_gate_up(variant, M, K, I, G, knobs):
    if variant:
        knobs.set("ZT_WOQ_PERSIST", variant)
    run_gate_up(M, K, I, G, seed=M + I + 1)


def test_persist_kernel_gate_up_strided_x():
    M, K, I, G = 12, 4096, 1040, 32
    x, q, wp, s, z, b = make_case(M, K, 2 * I, G, seed=3, bias=True)
    xs = torch.randn(M, K + 64).bfloat16()
    xs[:, :K] = x
    xd, wd, sd, bd = gpu(x, wp, s, b)
    y0 = C.woq_linear_gate_up(xd, wd, sd, None, bd).cpu()
    y = C.woq_linear_gate_up(xs.to(DEV)[:, :K], wd, sd, None, bd).cpu()
    assert torch.equal(y, y0)


# every prefill GEMM variant by name (ZT_WOQ_GEMM): "1" the 32x32 kernel with
# 128 x 128 tiles (256 x 128 is the default at this size), "w" / "v" its
# load-wave form with 4 / 3 stages, "x" with 256 x 192 tiles (ragged in N
# here), "d" the 16x16 DMA kernel, "2" its
# 256 x 128 tiles, "o" the 16x16 kernel without DMA; ragged M and N, two
# scale dtypes
@pytest.mark.parametrize("variant", ["1", "w", "v", "x", "d", "2", "o"])
@pytest.mark.parametrize("M,K,N,G,s_dtype", [(300, 1024, 264, 8, torch.bfloat16),
                                             (520, 2048, 520, 16, torch.bfloat16),
                                             (97, 512, 136, 4, torch.float32)])
def test_prefill_gemm_variants(variant, M, K, N, G, s_dtype):
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=M + N, bias=True, s_dtype=s_dtype)
    y_ref = O.woq_linear(x, wp, s, bias=b)
    xd, wd, sd, bd = gpu(x, wp, s, b)
    with C.tuning(ZT_WOQ_FORCE_KERNEL="gemm", ZT_WOQ_GEMM=variant):
        y = C.woq_linear(xd, wd, sd, None, bd)
    check_close(y, y_ref)


# post-ops in the prefill variants' epilogues: the 32x32 kernel ("1"), its
# load-wave form with 256 x 128 and 256 x 192 tiles ("w", "x") and the
# 16x16 DMA kernel ("2"), with bias, elementwise and binary post-ops
@pytest.mark.parametrize("variant", ["1", "w", "x", "2"])
@pytest.mark.parametrize("post,nbuf", [(("gelu_erf",), 0), (("mul", "add"), 2),
                                       (("silu", "mul"), 1)])
def test_prefill_variants_post_ops(variant, post, nbuf):
    M, K, N, G = 300, 1024, 264, 8
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=23, bias=True)
    g = torch.Generator().manual_seed(24)
    bufs = [torch.randn(M, N, generator=g).to(x.dtype) for _ in range(nbuf)]
    y_ref = O.woq_linear(x, wp, s, bias=b, post_ops=post, post_bufs=bufs)
    xd, wd, sd, bd = gpu(x, wp, s, b)
    with C.tuning(ZT_WOQ_FORCE_KERNEL="gemm", ZT_WOQ_GEMM=variant):
        y = C.woq_linear(xd, wd, sd, None, bd, post_ops=post, post_bufs=gpu(*bufs))
    check_close(y, y_ref)


# the default prefill dispatch at one round of 256 x 128 tiles (128 tiles
# here) takes the load-wave kernel
def test_prefill_one_round_default_kernel():
    M, K, N, G = 2048, 256, 2048, 2
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=11, bias=True)
    y_ref = O.woq_linear(x, wp, s, bias=b)
    xd, wd, sd, bd = gpu(x, wp, s, b)
    y = C.woq_linear(xd, wd, sd, None, bd)
    check_close(y, y_ref)


# 256 x 192 tiles by default where they make one round and 256 x 128 do not:
# 9 x 24 = 216 tiles of 256 x 192 against 9 x 36 = 324 of 256 x 128 (ragged M)
def test_prefill_one_round_192_default_kernel():
    M, K, N, G = 2100, 256, 4608, 2
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=12, bias=True)
    y_ref = O.woq_linear(x, wp, s, bias=b)
    xd, wd, sd, bd = gpu(x, wp, s, b)
    y = C.woq_linear(xd, wd, sd, None, bd)
    check_close(y, y_ref)


# the lean decode kernel (fast mode, M <= 16, K = 8 waves x 2 / 4 / 8 / 14
# chunks, x whole in LDS; forced by ZT_WOQ_LEAN=1, as the library takes it
# only for the shapes where it measured faster): group sizes 128 / 256 /
# 1024 and per channel, ragged N, every M up to 16, and the same result as
# the other decode kernels on these shapes
# (only the cases whose x [M, K] fits the lean kernel's LDS; the other
# kernels take the rest)
_LEAN_CASES = [(M, K, N, G) for M in (1, 2, 3, 4, 7, 8, 13, 16)
               for K, N, G in ((2048, 16, 16), (4096, 4096, 32), (4096, 1000, 16),
                               (8192, 256, 8), (8192, 112, 1), (14336, 4096, 112))
               if M * (K + 8) * 2 <= 160 * 1024]


@pytest.mark.parametrize("M,K,N,G", _LEAN_CASES)
def test_lean_kernel_vs_oracle(M, K, N, G, knobs):
    knobs.set("ZT_WOQ_LEAN", "1")
    y, y_ref = run_case(M, K, N, G, seed=M * 7 + G)
    knobs.set("ZT_WOQ_LEAN", "0")
    y_other, _ = run_case(M, K, N, G, seed=M * 7 + G)
    check_close(y, y_other.cpu())


@pytest.mark.parametrize("post,nbuf", [(("relu",), 0), (("gelu_tanh",), 0), (("add",), 1),
                                       (("mul", "add"), 2)])
def test_lean_kernel_post_ops(post, nbuf, knobs):
    knobs.set("ZT_WOQ_LEAN", "1")
    run_case(3, 4096, 520, 32, post=post, nbuf=nbuf, seed=9, bias=True)


def test_lean_kernel_strided_x(knobs):
    knobs.set("ZT_WOQ_LEAN", "1")
    M, K, N, G = 2, 14336, 256, 112
    x, q, wp, s, z, b = make_case(M, K, N, G, seed=79)
    xs = torch.randn(M, K + 64).bfloat16()
    xs[:, :K] = x
    y_ref = O.woq_linear(x, wp, s)
    y = C.woq_linear(xs.to(DEV)[:, :K], wp.to(DEV), s.to(DEV))
    check_close(y, y_ref)


# form "1": one 16-row tile per workgroup, its rows 0-7 gate and 8-15 up;
# "p": a gate tile and its up tile per workgroup
@pytest.mark.parametrize("form", ["1", "p"])
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("K,I,G", [(4096, 256, 32), (2048, 1040, 1), (8192, 64, 64)])
def test_lean_kernel_gate_up(M, K, I, G, form, knobs):
    knobs.set("ZT_WOQ_LEAN", form)
    y, y_ref = run_gate_up(M, K, I, G, seed=M + I + 2)
    knobs.set("ZT_WOQ_LEAN", "0")
    y_other, _ = run_gate_up(M, K, I, G, seed=M + I + 2)
    check_close(y, y_other.cpu())
