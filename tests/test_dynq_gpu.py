"""GPU parity of the dynamic int8 path against the CPU oracle, through the
C-ABI.  Quantised activations (qx, sx) and int32 accumulators are integer /
exact-closed-form results and must be bit-exact; bf16/fp32 outputs are held
to rtol = atol = 1e-2 (test/unittests/op_tests/test_dynamic_qlinear.py:103).
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


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[case] {request.node.name}", flush=True)


def make(M, K, N, seed, x_dtype=torch.bfloat16, sw_dtype=torch.float32, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(x_dtype)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = (torch.rand(N, generator=g) * 0.009 + 0.001).to(sw_dtype)
    b = (torch.randn(N, generator=g) * 0.1).bfloat16() if bias else None
    return x, w, sw, b


# long rows (7, 14 and 16 vectors per thread, and past 16 the element-wise
# kernel), a partial last 16-byte vector per thread, odd row counts
@pytest.mark.parametrize("M,K", [(1, 4), (3, 12), (16, 16), (128, 4096), (7, 11008),
                                 (2048, 4096), (5, 1), (1025, 14336), (3001, 2056), (1024, 8),
                                 (5, 28672), (3, 32768), (2, 32776), (9, 24584)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_quantize_bit_exact(M, K, x_dtype):
    g = torch.Generator().manual_seed(M * 31 + K)
    x = (torch.randn(M, K, generator=g) * 2).to(x_dtype)
    if M > 2:
        x[1] = 0  # all-zero row -> scale 1e-12/127
    qx, sx = C.dynamic_quantize(x.to(DEV))
    qr, sr = O.dynamic_quantize(x)
    assert torch.equal(sx.cpu(), sr)
    assert torch.equal(qx.cpu(), qr)


# quotients x / s that are exactly half-integers (ties, rounded to even) or
# within an ulp of one: rows whose amax is 127 * 2^e make s = 2^e exact
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_quantize_ties_bit_exact(x_dtype):
    rows = []
    for e in (0, -3, 5):
        h = (torch.arange(-127, 127, dtype=torch.float32) + 0.5) * 2.0 ** e
        row = torch.cat([torch.tensor([127.0 * 2.0 ** e]), h, -h[:1]])
        rows.append(row)
        # one ulp either side of every half-integer (fp32 rows only keep it)
        rows.append(torch.cat([torch.tensor([127.0 * 2.0 ** e]), torch.nextafter(h, h + 1),
                               torch.nextafter(h, h - 1)])[:256])
    K = 256
    x = torch.stack([torch.nn.functional.pad(r, (0, K - r.numel()))[:K] for r in rows]).to(x_dtype)
    qx, sx = C.dynamic_quantize(x.to(DEV))
    qr, sr = O.dynamic_quantize(x)
    assert torch.equal(sx.cpu(), sr)
    assert torch.equal(qx.cpu(), qr)


@pytest.mark.parametrize("M,N,K", [(1, 8, 16), (5, 33, 48), (64, 96, 256), (128, 11008, 4096),
                                   (300, 130, 512), (2048, 256, 1024), (4, 17, 12),
                                   # large-M tiled kernel: ragged M, N and K % 128 != 0
                                   (257, 200, 144), (520, 4160, 272), (1024, 1000, 2064),
                                   # skinny weight-streaming kernel: ragged N, K % 64 != 0
                                   (33, 100, 4112), (100, 4100, 272), (17, 50, 80),
                                   # more tiles than CUs (workgroups loop over tiles),
                                   # ragged M and N, K % 64 != 0
                                   (2100, 4100, 144), (4096, 2080, 208),
                                   # 129..255 rows on the tiled kernels, and at most
                                   # half a round of 256 x 128 tiles (128 x 128)
                                   (129, 300, 1024), (200, 4096, 2048), (255, 136, 4112),
                                   (512, 4096, 1024)])
def test_s8_gemm_accumulators_bit_exact(M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    acc = C.s8s8s32_gemm(a.to(DEV), w.to(DEV)).cpu()
    ref = O.s8s8s32_gemm(a, w) if M * N * K <= 2 ** 28 else torch._int_mm(a, w.t().contiguous())
    assert torch.equal(acc, ref)


@pytest.mark.parametrize("M,K,N", [(1, 4, 8), (4, 12, 16), (16, 16, 32), (24, 128, 48),
                                   (128, 4096, 11008), (33, 4096, 4096), (256, 1024, 640),
                                   (160, 2048, 4096), (512, 1024, 3584)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_dynamic_qlinear_vs_oracle(M, K, N, x_dtype):
    x, w, sw, b = make(M, K, N, seed=M + K + N, x_dtype=x_dtype)
    y_ref = O.dynamic_qlinear(x, w, sw, b)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)).cpu()
    assert y.dtype == x_dtype
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


def test_dynamic_qlinear_bf16_scales_no_bias():
    x, w, sw, _ = make(8, 256, 64, seed=9, sw_dtype=torch.bfloat16, bias=False)
    y_ref = O.dynamic_qlinear(x, w, sw, None)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), None).cpu()
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


def test_golden_dynamic_fixture():
    c = load_file(os.path.join(GOLDEN, "dynamic_qlinear.safetensors"))
    qx, sx = C.dynamic_quantize(c["x"].to(DEV))
    assert torch.equal(qx.cpu(), c["qx"]) and torch.equal(sx.cpu(), c["sx"])
    acc = C.s8s8s32_gemm(c["qx"].to(DEV), c["w"].to(DEV)).cpu()
    assert torch.equal(acc, c["acc"])
    y = C.dynamic_qlinear(c["x"].to(DEV), c["w"].to(DEV), c["w_scales"].to(DEV),
                          c["bias"].to(DEV)).cpu()
    torch.testing.assert_close(y, c["y"], rtol=1e-2, atol=1e-2)
    qb, sb = C.dynamic_quantize(c["x_bf16"].to(DEV))
    assert torch.equal(qb.cpu(), c["qx_bf16"]) and torch.equal(sb.cpu(), c["sx_bf16"])


def test_prefill_shape_accumulator_checksum():
    # M = 2048 prefill (int8 path, one linear): exact
    # accumulators against torch._int_mm on the CPU
    g = torch.Generator().manual_seed(2048)
    M, K, N = 2048, 4096, 6144
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    acc = C.s8s8s32_gemm(a.to(DEV), w.to(DEV)).cpu()
    assert torch.equal(acc, torch._int_mm(a, w.t().contiguous()))


# 17..128 tokens run on the 32x32x32 skinny kernel over qx in fragment
# order: ragged M inside the last 32-token tile, N not a multiple of the
# 16-row weight tiles (an odd last tile pairs with zeros), K of one chunk
# (waves with no chunks) up to 64, and K of 8192 and of 25 64-k chunks.
@pytest.mark.parametrize("M,K,N", [(17, 64, 50), (31, 320, 100), (32, 4096, 96),
                                   (33, 1024, 4100), (64, 448, 48), (100, 4096, 1000),
                                   (128, 192, 47), (20, 8192, 64), (45, 1600, 96)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_dynamic_qlinear_fragment_kernel(M, K, N, x_dtype):
    x, w, sw, b = make(M, K, N, seed=7 * M + K + N, x_dtype=x_dtype)
    y_ref = O.dynamic_qlinear(x, w, sw, b)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)).cpu()
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


# every compiled (TPW, PF, NW) shape of the 32x32 kernel, forced; M = 1..16
# forced onto it too
@pytest.mark.parametrize("M,shape", [(20, "4,4,8"), (40, "4,2,8"), (64, "3,2,8"), (90, "2,2,8"),
                                     (128, "4,2,8"), (128, "3,4,4"), (97, "4,4,4"),
                                     (20, "2,4,8"), (31, "1,4,8"), (40, "2,2,8"), (64, "2,4,8"),
                                     (50, "1,4,8"), (1, None), (9, None), (16, None)])
def test_dynamic_qlinear_fragment_kernel_shapes(M, shape, knobs):
    K, N = 1344, 232
    if shape:
        knobs.set("ZT_S8_SKINNY32", shape)
    knobs.set("ZT_S8_FRAG", "1")
    x, w, sw, b = make(M, K, N, seed=M + 5)
    y_ref = O.dynamic_qlinear(x, w, sw, b)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV)).cpu()
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


# 17..64 tokens on the 32-token kernel: the default tile shape (16- or
# 32-row tiles up to 8192 rows) bit-identical to 64-row tiles
@pytest.mark.parametrize("M,N,K", [(17, 4096, 4096), (64, 4096, 14336), (33, 6144, 4096),
                                   (24, 11008, 1024)])
def test_dynamic_qlinear_fragment_kernel_default_tiles(M, N, K, knobs):
    x, w, sw, b = make(M, K, N, seed=M + N)
    args = (x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV))
    y = C.dynamic_qlinear(*args).cpu()
    knobs.set("ZT_S8_SKINNY32", "4,4,8" if M <= 32 else "4,2,8")
    assert torch.equal(C.dynamic_qlinear(*args).cpu(), y)
    torch.testing.assert_close(y.float(), O.dynamic_qlinear(x, w, sw, b).float(),
                               rtol=1e-2, atol=1e-2)


# The skinny GEMM with the per-token quantisation in its prologue (one
# launch for at most 16 tokens of bf16 x): bit-identical to the quantise
# launch + skinny GEMM (the same qx, sx and int32 sums) for every register
# layout it has (1, 2, 4 and 8 vectors per thread and row, 2 to 16 rows), ragged N and K,
# with and without bias.  ZT_WOQ_DEBUG names the kernel that ran.
@pytest.mark.parametrize("M,K,N", [(1, 64, 8), (2, 4096, 11008), (3, 192, 70), (5, 4096, 6144),
                                   (8, 4096, 4096), (9, 4096, 200), (16, 4096, 136),
                                   (4, 8192, 300), (3, 5120, 77), (2, 14336, 4096),
                                   (1, 16384, 64), (4, 4096, 28672), (1, 28672, 8192),
                                   (2, 24640, 130), (2, 32768, 72), (3, 14336, 4096),
                                   (3, 11008, 136)])
@pytest.mark.parametrize("bias", [True, False])
def test_dynamic_qlinear_fused_quantise(M, K, N, bias, knobs, capfd):
    x, w, sw, b = make(M, K, N, seed=M * 31 + K + N, bias=bias)
    args = (x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV) if bias else None)
    knobs.set("ZT_S8_FUSED", "0")
    y0 = C.dynamic_qlinear(*args).cpu()
    knobs.set("ZT_S8_FUSED", "1")
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    y1 = C.dynamic_qlinear(*args).cpu()
    assert "s8 fused quantise" in capfd.readouterr().err
    assert torch.equal(y1, y0)
    y_ref = O.dynamic_qlinear(x, w, sw, b if bias else None)
    torch.testing.assert_close(y1.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


# every tile shape of both one-token-tile paths (ZT_S8_SKINNY "TPW,PF,NW":
# 64-, 32- and 16-row weight tiles, 4 or 8 chunks in flight), with the
# quantisation in the GEMM's prologue and as its own launch: all
# bit-identical to one another and within tolerance of the oracle
@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (7, 1024, 300), (16, 2048, 11008),
                                   (2, 14336, 520), (8, 192, 36), (4, 28672, 264),
                                   (9, 24576, 72)])
def test_dynamic_qlinear_skinny_tile_shapes(M, K, N, knobs):
    x, w, sw, b = make(M, K, N, seed=M * 13 + K + N)
    args = (x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV))
    ys = []
    for fused in ("0", "1"):
        for shape in ("4,4,8", "2,4,8", "1,4,8", "1,8,8"):
            knobs.set("ZT_S8_FUSED", fused)
            knobs.set("ZT_S8_SKINNY", shape)
            ys.append(C.dynamic_qlinear(*args).cpu())
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    torch.testing.assert_close(ys[0].float(), O.dynamic_qlinear(x, w, sw, b).float(),
                               rtol=1e-2, atol=1e-2)


# post-ops in the fused kernel's epilogue (row scales read from LDS), with
# N a multiple of 4 and not
@pytest.mark.parametrize("N", [136, 130])
@pytest.mark.parametrize("post", [("relu",), ("add",), ("mul", "add"), ("silu",)])
def test_dynamic_qlinear_fused_quantise_post_ops(post, N, knobs):
    M, K = 6, 1024
    x, w, sw, b = make(M, K, N, seed=N + len(post))
    g = torch.Generator().manual_seed(17)
    bufs = [torch.randn(M, N, generator=g).bfloat16() for p in post if p in ("add", "mul")]
    args = (x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV))
    kw = dict(post_ops=post, post_bufs=[t.to(DEV) for t in bufs])
    knobs.set("ZT_S8_FUSED", "0")
    y0 = C.dynamic_qlinear(*args, **kw).cpu()
    knobs.set("ZT_S8_FUSED", "1")
    y1 = C.dynamic_qlinear(*args, **kw).cpu()
    assert torch.equal(y1, y0)
    y_ref = O.dynamic_qlinear(x, w, sw, b, post_ops=post, post_bufs=bufs)
    torch.testing.assert_close(y1.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


# 64 < M <= 128 with K % 256 == 0 runs the split-K kernel when the workspace
# holds its exchange (two K halves per 96-column tile, the second to finish
# adds the other's int32 partial): bit-identical to the unsplit kernel (the
# least workspace), on ragged M, N past a tile, N % 4 != 0, one or an odd
# number of 128-k chunks per half, every load depth.  Calls alternate two
# inputs, so a partial left from the previous call cannot pass for the
# current one; each call reuses the freed workspace, whose tile counters the
# quantise kernel clears.
@pytest.mark.parametrize("M,K,N,depth", [(65, 256, 1, None), (70, 512, 95, None),
                                         (96, 768, 96, "3"), (97, 1024, 97, "4"),
                                         (128, 2816, 203, None), (128, 4096, 11008, None),
                                         (128, 4096, 11008, "3"), (100, 1536, 4100, "4")])
def test_dynamic_qlinear_split_k(M, K, N, depth, knobs):
    if depth:
        knobs.set("ZT_S8_SPLIT", depth)
    x, w, sw, b = make(M, K, N, seed=M * 7 + K + N)
    x2 = torch.randn(M, K, generator=torch.Generator().manual_seed(K)).to(x.dtype)
    wd, swd, bd = w.to(DEV), sw.to(DEV), b.to(DEV)
    xs = [x.to(DEV), x2.to(DEV)]
    y0 = [C.dynamic_qlinear(xi, wd, swd, bd, split=False).cpu() for xi in xs]
    for i in (0, 1, 0, 1):
        assert torch.equal(C.dynamic_qlinear(xs[i], wd, swd, bd).cpu(), y0[i])
    torch.testing.assert_close(y0[0].float(), O.dynamic_qlinear(x, w, sw, b).float(),
                               rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("post", [("relu",), ("add",), ("mul", "add"), ("silu",)])
def test_dynamic_qlinear_split_k_post_ops(post):
    M, K, N = 112, 1280, 300
    x, w, sw, b = make(M, K, N, seed=5)
    g = torch.Generator().manual_seed(13)
    bufs = [torch.randn(M, N, generator=g).bfloat16() for p in post if p in ("add", "mul")]
    args = (x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV))
    kw = dict(post_ops=post, post_bufs=[t.to(DEV) for t in bufs])
    y = C.dynamic_qlinear(*args, **kw).cpu()
    assert torch.equal(y, C.dynamic_qlinear(*args, split=False, **kw).cpu())
    y_ref = O.dynamic_qlinear(x, w, sw, b, post_ops=post, post_bufs=bufs)
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("post", [("relu",), ("add",), ("mul", "add"), ("gelu_tanh",)])
def test_dynamic_qlinear_fragment_kernel_post_ops(post):
    M, K, N = 48, 512, 136
    x, w, sw, b = make(M, K, N, seed=3)
    g = torch.Generator().manual_seed(11)
    bufs = [torch.randn(M, N, generator=g).bfloat16() for p in post if p in ("add", "mul")]
    y_ref = O.dynamic_qlinear(x, w, sw, b, post_ops=post, post_bufs=bufs)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV), post_ops=post,
                          post_bufs=[t.to(DEV) for t in bufs]).cpu()
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


# past 128 tokens with at most half a round of 256 x 128 tiles, the tiled
# kernel's K split (128 x 128 tiles, int32 partials in the workspace, then
# the sum kernel's epilogue): bit-identical to the unsplit kernel (the least
# workspace), including a last step past K and post-ops; the asymmetric op
# takes it too
@pytest.mark.parametrize("M,K,N,post", [(129, 4096, 4096, ()), (300, 5008, 520, ("add",)),
                                        (512, 14336, 1024, ("mul", "add")),
                                        (200, 2048, 136, ("gelu_tanh",))])
def test_dynamic_qlinear_tiled_k_split(M, K, N, post, knobs, capfd):
    x, w, sw, b = make(M, K, N, seed=M + K)
    g = torch.Generator().manual_seed(3)
    bufs = [torch.randn(M, N, generator=g).bfloat16() for p in post if p in ("add", "mul")]
    args = (x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV))
    kw = dict(post_ops=post, post_bufs=[t.to(DEV) for t in bufs])
    knobs.set("ZT_WOQ_DEBUG", "1")
    capfd.readouterr()
    y = C.dynamic_qlinear(*args, **kw).cpu()
    assert "K splits" in capfd.readouterr().err
    assert torch.equal(y, C.dynamic_qlinear(*args, split=False, **kw).cpu())
    torch.testing.assert_close(y.float(), O.dynamic_qlinear(x, w, sw, b, post_ops=post,
                                                            post_bufs=bufs).float(),
                               rtol=1e-2, atol=1e-2)
    if not post:
        import zentorch  # noqa: F401  (registers the column-sum op)
        cs = torch.ops.zentorch.zentorch_s8_weight_colsum(w.to(DEV))
        ya = C.dynamic_qlinear_asym(x.to(DEV), w.to(DEV), sw.to(DEV), cs, b.to(DEV)).cpu()
        yb = C.dynamic_qlinear_asym(x.to(DEV), w.to(DEV), sw.to(DEV), cs, b.to(DEV),
                                    split=False).cpu()
        assert torch.equal(ya, yb)


# post-ops in the large-M load-wave kernel's epilogue (the general path of
# its tile epilogue), with 256 x 128 and 256 x 192 tiles
@pytest.mark.parametrize("tile", ["2", "9"])
@pytest.mark.parametrize("post", [("gelu_erf",), ("mul", "add"), ("silu", "mul")])
def test_dynamic_qlinear_large_m_post_ops(tile, post, knobs):
    M, K, N = 300, 272, 400
    knobs.set("ZT_S8_TILE", tile)
    x, w, sw, b = make(M, K, N, seed=17)
    g = torch.Generator().manual_seed(19)
    bufs = [torch.randn(M, N, generator=g).bfloat16() for p in post if p in ("add", "mul")]
    y_ref = O.dynamic_qlinear(x, w, sw, b, post_ops=post, post_bufs=bufs)
    y = C.dynamic_qlinear(x.to(DEV), w.to(DEV), sw.to(DEV), b.to(DEV), post_ops=post,
                          post_bufs=[t.to(DEV) for t in bufs]).cpu()
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1e-2, atol=1e-2)


# the large-M kernels by name: the load-wave kernel (default, also with its
# 128 x 128 tiles: ZT_S8_TILE 1 / 0, and 256 x 192: 9) and the kernels it replaced (n: 32x32
# DMA, r: register-staged, 2 / 3: 16x16 DMA with 2 / 3 stages), on ragged
# shapes (M, N past a tile, K not a multiple of the 128-byte step)
@pytest.mark.parametrize("kind", ["w", "w1", "w0", "w9", "n", "r", "2", "3"])
@pytest.mark.parametrize("M,N,K", [(257, 200, 144), (520, 4160, 272), (2100, 130, 2064),
                                   (512, 384, 4096),
                                   # 216 tiles of 256 x 192, 324 of 256 x 128: the
                                   # default takes 256 x 192
                                   (2100, 4608, 272)])
def test_s8_large_m_kernels_bit_exact(kind, M, N, K, knobs):
    knobs.set("ZT_S8_KIND", kind[0])
    if len(kind) > 1:
        knobs.set("ZT_S8_TILE", kind[1])
    g = torch.Generator().manual_seed(M * 3 + N + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    acc = C.s8s8s32_gemm(a.to(DEV), w.to(DEV)).cpu()
    assert torch.equal(acc, torch._int_mm(a, w.t().contiguous()))
    x, w2, sw, b = make(M, K, N, seed=M + K)
    y = C.dynamic_qlinear(x.to(DEV), w2.to(DEV), sw.to(DEV), b.to(DEV)).cpu()
    torch.testing.assert_close(y.float(), O.dynamic_qlinear(x, w2, sw, b).float(), rtol=1e-2,
                               atol=1e-2)
