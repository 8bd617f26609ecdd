"""The oracle's static int8 linear (zentorch_qlinear*) against the
reference's own test reference, qdq_linear (test/unittests/quant_utils.py:
13-83): fake-quantise the input per tensor, dequantise the int8 weight per
tensor / channel, F.linear with the bias, the eltwise op, then either the
output dtype or quantize_per_tensor with the output scale and zero point.
That restatement uses torch's own quantisation ops, so it pins the oracle's
quantisation (the same integers), its zero-point handling and its
requantisation; the float outputs agree to fp32 rounding (the accumulation
order differs) and the int8 outputs to one step.

Argument forms follow the reference's op tests (test_qlinear.py:552-610):
an int8 zero point there means symmetric and is passed as None, a uint8 one
is passed as int32 (unittest_utils.py:355-365).
"""
import pytest
import torch
import torch.ao.quantization.fx._decomposed  # noqa: F401  (quantized_decomposed ops)

from oracle import oracle as O

qd = torch.ops.quantized_decomposed


def qdq_linear(x, w, b, xs, xz, ws, post, out_dtype, ys=None, yz=None):
    """quant_utils.py:13-83 restated (u8 when a zero point is given)."""
    if x.dtype in (torch.float32, torch.bfloat16):
        lo, hi = (0, 255) if xz is not None else (-128, 127)
        xq = torch.fake_quantize_per_tensor_affine(
            x.float(), xs, xz if xz is not None else torch.zeros((), dtype=torch.int32), lo, hi)
    else:
        zp = int(xz) if xz is not None else 0
        xq = (x.float() - zp) * xs
    dw = w.float() * ws.reshape(-1, 1).float()
    y = torch.nn.functional.linear(xq.float(), dw, b.float() if b is not None else None)
    y = post(y)
    if ys is not None:
        lo, hi, dt = (0, 255, torch.uint8) if yz is not None else (-128, 127, torch.int8)
        return qd.quantize_per_tensor(y, float(ys), int(yz) if yz is not None else 0, lo, hi, dt)
    return y.to(out_dtype)


def make(seed, M=7, K=96, N=40, in_dtype=torch.float32, zp=True, per_channel=True):
    g = torch.Generator().manual_seed(seed)
    if in_dtype in (torch.float32, torch.bfloat16):
        x = torch.randn(M, K, generator=g).to(in_dtype)
    elif in_dtype == torch.uint8:
        x = torch.randint(0, 256, (M, K), generator=g, dtype=torch.uint8)
    else:
        x = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    xs = torch.rand(1, generator=g) * 0.02 + 0.01
    xz = torch.randint(0, 256, (1,), generator=g, dtype=torch.int32) if zp else None
    ws = (torch.rand(N if per_channel else 1, generator=g) * 0.01 + 0.001)
    return x, w, xs, xz, ws


IDENT = lambda y: y  # noqa: E731


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.uint8, torch.int8])
@pytest.mark.parametrize("zp", [True, False])
@pytest.mark.parametrize("per_channel", [True, False])
def test_qlinear_float_out_vs_qdq(in_dtype, zp, per_channel):
    if in_dtype == torch.int8 and zp:
        pytest.skip("int8 input with a zero point is covered by the u8 case")
    x, w, xs, xz, ws = make(1, in_dtype=in_dtype, zp=zp, per_channel=per_channel)
    b = torch.randn(w.shape[0])
    y = O.qlinear(x, w, xs, xz, ws, b, out_dtype=torch.float32)
    ref = qdq_linear(x, w, b, xs, xz, ws, IDENT, torch.float32)
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("post,ids", [(torch.relu, ["relu"]), (torch.sigmoid, ["sigmoid"])])
@pytest.mark.parametrize("out", ["u8", "s8", "bf16"])
def test_qlinear_eltwise_and_requant(post, ids, out):
    x, w, xs, xz, ws = make(2, M=9, K=64, N=24)
    b = torch.randn(w.shape[0])
    ys = torch.tensor([0.05]) if out != "bf16" else None
    yz = torch.tensor([17], dtype=torch.int32) if out == "u8" else None
    dt = {"u8": torch.uint8, "s8": torch.int8, "bf16": torch.bfloat16}[out]
    y = O.qlinear(x, w, xs, xz, ws, b, post_ops=ids, out_dtype=dt, y_scale=ys, y_zp=yz)
    ref = qdq_linear(x, w, b, xs, xz, ws, post, dt, ys, yz)
    assert y.dtype == dt
    if out == "bf16":
        torch.testing.assert_close(y.float(), ref.float(), rtol=1e-2, atol=1e-2)
    else:
        assert (y.int() - ref.int()).abs().max() <= 1


def test_qlinear_mul_add():
    x, w, xs, xz, ws = make(3, M=5, K=32, N=16)
    g = torch.Generator().manual_seed(4)
    mul, add = torch.randn(5, 16, generator=g), torch.randn(5, 16, generator=g)
    y = O.qlinear(x, w, xs, xz, ws, None, post_ops=["mul", "add"], post_bufs=[mul, add])
    ref = qdq_linear(x, w, None, xs, xz, ws, lambda t: t * mul + add, torch.float32)
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)


def test_qlinear_quantised_input_matches_float_input():
    # an s8 input equals the float input whose quantisation gives it
    x, w, xs, _, ws = make(5, in_dtype=torch.int8, zp=False)
    xf = x.float() * xs
    a = O.qlinear(x, w, xs, None, ws)
    b = O.qlinear(xf, w, xs, None, ws)
    torch.testing.assert_close(a, b, rtol=0, atol=0)
