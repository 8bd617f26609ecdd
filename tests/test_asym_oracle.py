"""The oracle's per-token asymmetric uint8 quantisation (an opt-in beside
the reference's symmetric s8; the reference holds no golden data for it),
pinned by what the definition fixes:

* range: sx = fp32((hi - lo) / 255) with lo = min(0, min x), hi = max(0, max
  x); zp and q are integers in [0, 255];
* zero is exact: x = 0 quantises to q = zp;
* one-signed rows: a row >= 0 has zp = 0 and its maximum at q = 255; a row
  <= 0 has zp = 255 and its minimum at q = 0;
* round trip: |(q - zp) * sx - x| <= sx / 2 where q is not clamped, <= sx
  everywhere;
* the GEMM: sum_k (q - zp) * w equals q . w - zp * colsum(w) and, scaled,
  approximates the fp64 product within the quantisation error.

A sign error in zp, a 256-level scale, a range that leaves out zero or a
dropped zero-point term fails one of these.
"""
import pytest
import torch

from oracle import oracle as O


def _rows(seed, M=6, K=200, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * 3
    x[1] = x[1].abs() + 0.5          # positive row (no zero inside)
    x[2] = -x[2].abs() - 0.25        # negative row
    x[3] = 0                         # all zero
    x[4, :] = 1.75                   # constant
    x[5] = torch.nn.functional.silu(x[5])  # SiLU output: mostly >= -0.28
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_asym_quant_identities(dtype):
    x = _rows(1, dtype=dtype)
    q, sx, zp = O.dynamic_quantize_asym(x)
    xf = x.float()
    lo = torch.minimum(xf.min(1).values, torch.zeros(()))
    hi = torch.maximum(xf.max(1).values, torch.zeros(()))
    rng = torch.clamp(hi - lo, min=1e-12)
    assert torch.equal(sx, rng / 255.0)
    assert int(zp.min()) >= 0 and int(zp.max()) <= 255
    # one-signed rows
    assert zp[1] == 0 and int(q[1].max()) == 255
    assert zp[2] == 255 and int(q[2].min()) == 0
    # zero and the constant row
    assert torch.all(q[3] == zp[3])
    assert torch.all(q[4] == 255) and zp[4] == 0
    # round trip
    deq = (q.double() - zp[:, None].double()) * sx[:, None].double()
    err = (deq - xf.double()).abs()
    s = sx[:, None].double()
    assert torch.all(err <= s * (1 + 1e-6))
    inner = (q > 0) & (q < 255)
    assert torch.all(err[inner] <= (s * 0.5 * (1 + 1e-6)).expand_as(err)[inner])


def test_asym_zero_exact_in_mixed_rows():
    x = torch.tensor([[-1.0, 0.0, 2.0, 0.0, 0.5]]).bfloat16()
    q, sx, zp = O.dynamic_quantize_asym(x)
    assert q[0, 1] == zp[0] and q[0, 3] == zp[0]
    assert q[0, 0] == 0 and q[0, 2] == 255


def test_asym_qlinear_accumulator_identity_and_error():
    g = torch.Generator().manual_seed(7)
    x = torch.nn.functional.silu(torch.randn(9, 256, generator=g) * 2).bfloat16()
    w = torch.randint(-127, 128, (40, 256), generator=g, dtype=torch.int8)
    sw = torch.rand(40, generator=g) * 0.01 + 0.001
    q, sx, zp = O.dynamic_quantize_asym(x)
    acc = O.dynamic_qlinear_asym(x, w, sw, out_dtype=torch.int32)
    colsum = w.long().sum(1)
    ref = q.long() @ w.long().t() - zp[:, None].long() * colsum[None, :]
    assert torch.equal(acc.long(), ref)
    y = O.dynamic_qlinear_asym(x, w, sw, out_dtype=torch.float32)
    exact = x.double() @ (w.double() * sw.double()[:, None]).t()
    # per element: sum_k |dx_k * w_k| * sw <= K * sx / 2 * 127 * sw (loose)
    bound = sx.double()[:, None] * 0.5 * w.abs().double().sum(1)[None, :] * sw.double()[None, :]
    assert torch.all((y.double() - exact).abs() <= bound * 1.01 + 1e-6)
    # the asymmetric grid is finer than the symmetric one on one-signed data
    y_asym = O.dynamic_qlinear_asym(x, w, sw).double()   # bf16 output, as the symmetric op
    y_sym = O.dynamic_qlinear(x, w, sw, None).double()
    assert (y_asym - exact).abs().mean() < (y_sym - exact).abs().mean()
