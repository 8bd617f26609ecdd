"""GPU parity of the static int8 linear (zentorch_qlinear, _relu, _sigmoid,
_mul_add and the .out forms; src/cpu/cpp/QLinear.cpp:367-573) against the
CPU oracle.  Argument forms follow the reference's op tests
(test/unittests/op_tests/test_qlinear.py): per-tensor input scale with an
int32 zero point (u8) or none (s8), per-tensor or per-channel weight scales,
float / bf16 / u8 / s8 inputs, bias or none, float outputs and u8 / s8
requantised ones, 2-D to 4-D inputs.  The integer part (quantised input,
int32 accumulators) is exact; float outputs are held to rtol = atol = 1e-4
(fp32) / 1e-2 (bf16) and int8 outputs to one step.
"""
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ops = torch.ops.zentorch


@pytest.fixture(autouse=True)
def _announce(request):
    import zentorch  # noqa: F401
    print(f"\n[case] {request.node.name}", flush=True)


def make(seed, shape=(7, 96), N=40, in_dtype=torch.float32, zp=True, per_channel=True,
         bias_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    K = shape[-1]
    if in_dtype in (torch.float32, torch.bfloat16):
        x = torch.randn(*shape, generator=g).to(in_dtype)
    elif in_dtype == torch.uint8:
        x = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
    else:
        x = torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    xs = torch.rand(1, generator=g) * 0.02 + 0.01
    xz = torch.randint(0, 256, (1,), generator=g, dtype=torch.int32) if zp else None
    ws = torch.rand(N if per_channel else 1, generator=g) * 0.01 + 0.001
    b = torch.randn(N, generator=g).to(bias_dtype) if bias_dtype is not None else None
    return x, w, xs, xz, ws, b


def dev(*ts):
    return [t.to(DEV) if t is not None else None for t in ts]


def check(y, ref):
    assert y.dtype == ref.dtype and y.shape == ref.shape
    y, ref = y.cpu(), ref
    if y.dtype in (torch.uint8, torch.int8):
        assert (y.int() - ref.int()).abs().max() <= 1
    elif y.dtype == torch.bfloat16:
        torch.testing.assert_close(y.float(), ref.float(), rtol=1e-2, atol=1e-2)
    else:
        torch.testing.assert_close(y, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.uint8, torch.int8])
@pytest.mark.parametrize("zp", [True, False])
@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("shape", [(7, 96), (2, 3, 64), (2, 2, 3, 32)])
def test_qlinear_float_out(in_dtype, zp, per_channel, shape):
    x, w, xs, xz, ws, b = make(len(shape) * 10 + int(zp), shape=shape, in_dtype=in_dtype, zp=zp,
                               per_channel=per_channel)
    y = ops.zentorch_qlinear(*dev(x, w, xs, xz, ws, None, b, None, None),
                             output_dtype=torch.float32)
    check(y, O.qlinear(x, w, xs, xz, ws, b, out_dtype=torch.float32))


@pytest.mark.parametrize("name,post", [("zentorch_qlinear", []),
                                       ("zentorch_qlinear_relu", ["relu"]),
                                       ("zentorch_qlinear_sigmoid", ["sigmoid"])])
@pytest.mark.parametrize("out", ["u8", "s8", "bf16", "f32"])
def test_qlinear_unary_outputs(name, post, out):
    x, w, xs, xz, ws, b = make(3, shape=(9, 64), N=24,
                               bias_dtype=torch.bfloat16 if out == "bf16" else torch.float32)
    dt = {"u8": torch.uint8, "s8": torch.int8, "bf16": torch.bfloat16, "f32": torch.float32}[out]
    ys = torch.tensor([0.05]) if out in ("u8", "s8") else None
    yz = torch.tensor([17], dtype=torch.int32) if out == "u8" else None
    y = getattr(ops, name)(*dev(x, w, xs, xz, ws, None, b, ys, yz), output_dtype=dt)
    check(y, O.qlinear(x, w, xs, xz, ws, b, post_ops=post, out_dtype=dt, y_scale=ys, y_zp=yz))


def test_qlinear_default_output_dtype_is_float32():
    x, w, xs, xz, ws, b = make(4, in_dtype=torch.bfloat16)
    y = ops.zentorch_qlinear(*dev(x, w, xs, xz, ws, None, b, None, None))
    assert y.dtype == torch.float32


@pytest.mark.parametrize("shape", [(5, 32), (2, 4, 48)])
def test_qlinear_mul_add(shape):
    x, w, xs, xz, ws, b = make(5, shape=shape, N=16)
    g = torch.Generator().manual_seed(6)
    osz = (*shape[:-1], 16)
    mul, add = torch.randn(*osz, generator=g), torch.randn(*osz, generator=g)
    y = ops.zentorch_qlinear_mul_add(*dev(x, w, xs, xz, ws, None, mul, add, b, None, None),
                                     output_dtype=torch.float32)
    check(y, O.qlinear(x, w, xs, xz, ws, b, post_ops=["mul", "add"], post_bufs=[mul, add]))


@pytest.mark.parametrize("variant", ["zentorch_qlinear", "zentorch_qlinear_relu"])
def test_qlinear_out_forms(variant):
    x, w, xs, xz, ws, b = make(7, shape=(6, 64), N=32)
    out = torch.empty(6, 32, dtype=torch.uint8, device=DEV)
    ys, yz = torch.tensor([0.04]), torch.tensor([100], dtype=torch.int32)
    getattr(ops, variant).out(out, *dev(x, w, xs, xz, ws, None, b, ys, yz),
                              output_dtype=torch.uint8)
    post = ["relu"] if variant.endswith("relu") else []
    check(out, O.qlinear(x, w, xs, xz, ws, b, post_ops=post, out_dtype=torch.uint8, y_scale=ys,
                         y_zp=yz))
    with pytest.raises(RuntimeError, match="does not match the dtype"):
        getattr(ops, variant).out(out, *dev(x, w, xs, xz, ws, None, b, ys, yz),
                                  output_dtype=torch.int8)


# (M, N, K): each row reaches another int8 GEMM kernel (skinny 16-token,
# split-K 32-token (twice: a ragged last tile), 32-token, 16x16, load-wave,
# generic)
@pytest.mark.parametrize("M,N,K", [(1, 264, 512), (100, 520, 1024), (128, 1000, 2048),
                                   (40, 130, 256), (200, 264, 512), (2048, 512, 1024),
                                   (5, 33, 12),
                                   # 216 tiles of 256 x 192: requantised outputs
                                   # through the half-tile epilogue
                                   (2100, 4608, 272),
                                   # 16 tiles of 128 x 128: K split in four over
                                   # int32 partials, outputs from the sum kernel
                                   (200, 1024, 4096)])
@pytest.mark.parametrize("kind", ["u8_in_u8_out", "f32_zp_s8_out", "bf16_sym_bf16_out"])
def test_qlinear_kernels(M, N, K, kind):
    in_dtype = {"u8_in_u8_out": torch.uint8, "f32_zp_s8_out": torch.float32,
                "bf16_sym_bf16_out": torch.bfloat16}[kind]
    x, w, xs, xz, ws, b = make(M + N, shape=(M, K), N=N, in_dtype=in_dtype,
                               zp=kind != "bf16_sym_bf16_out",
                               bias_dtype=torch.bfloat16 if in_dtype == torch.bfloat16
                               else torch.float32)
    if kind == "u8_in_u8_out":
        dt, ys, yz = torch.uint8, torch.tensor([2.0]), torch.tensor([128], dtype=torch.int32)
    elif kind == "f32_zp_s8_out":
        dt, ys, yz = torch.int8, torch.tensor([0.1]), None
    else:
        dt, ys, yz = torch.bfloat16, None, None
    y = ops.zentorch_qlinear(*dev(x, w, xs, xz, ws, None, b, ys, yz), output_dtype=dt)
    check(y, O.qlinear(x, w, xs, xz, ws, b, out_dtype=dt, y_scale=ys, y_zp=yz))


def test_qlinear_errors():
    x, w, xs, xz, ws, b = dev(*make(8))
    with pytest.raises(RuntimeError, match="only int8 is supported"):
        ops.zentorch_qlinear(x, w.int(), xs, xz, ws, None, b, None, None)
    with pytest.raises(RuntimeError, match="input_zero_points, only int32"):
        ops.zentorch_qlinear(x, w, xs, xz.to(torch.uint8), ws, None, b, None, None)
    with pytest.raises(RuntimeError, match="uint8 are supported dtype"):
        ops.zentorch_qlinear(x, w, xs, xz, ws, None, b, xs, xz, output_dtype=torch.int8)
    with pytest.raises(RuntimeError, match="int8 are supported dtype"):
        ops.zentorch_qlinear(x, w, xs, xz, ws, None, b, xs, None, output_dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="weight_scales with respect"):
        ops.zentorch_qlinear(x, w, xs, xz, torch.ones(3, device=DEV), None, b, None, None)
    with pytest.raises(RuntimeError, match="per-tensor quantization for input"):
        ops.zentorch_qlinear(x, w, xs, torch.zeros(2, dtype=torch.int32, device=DEV), ws, None,
                             b, None, None)


def test_qlinear_weight_column_sums_cached_and_updated():
    # the column sums an input offset needs are computed once per weight and
    # recomputed after an in-place update; a new weight in a reused block
    # (same address) gets its own
    x, w, xs, xz, ws, b = make(11, shape=(5, 64), N=24)
    xd, wd, xsd, xzd, wsd, bd = dev(x, w, xs, xz, ws, b)
    call = lambda wt: ops.zentorch_qlinear(xd, wt, xsd, xzd, wsd, None, bd, None, None,
                                           output_dtype=torch.float32)
    y1 = call(wd)
    assert torch.equal(call(wd), y1)
    check(y1, O.qlinear(x, w, xs, xz, ws, b, out_dtype=torch.float32))
    w2 = torch.randint(-128, 128, w.shape, generator=torch.Generator().manual_seed(12),
                       dtype=torch.int8)
    wd.copy_(w2.to(DEV))
    check(call(wd), O.qlinear(x, w2, xs, xz, ws, b, out_dtype=torch.float32))
    ptr = wd.data_ptr()
    del wd
    w3 = torch.randint(-128, 128, w.shape, generator=torch.Generator().manual_seed(13),
                       dtype=torch.int8)
    wd3 = w3.to(DEV)
    check(call(wd3), O.qlinear(x, w3, xs, xz, ws, b, out_dtype=torch.float32))
    assert wd3.data_ptr() == ptr or True  # the caching allocator usually reuses the block
