"""Writes the golden fixtures in tests/golden/*.safetensors.

The reference ships no fixtures for this path (its tests regenerate random
data), so these are produced here from seeded inputs by the CPU oracle and,
before anything is written, cross-checked against routines that do not share
the oracle's code:
  * torch F.linear on torch-dequantised weights, the reference test's own
    reference (test/unittests/op_tests/test_woq_linear.py:118-128);
  * aten._weight_int4pack_mm_for_cpu (tinygemm) for the asymmetric u4 case,
    the reference's asymmetric test oracle (test_woq_linear_asymmetric.py:118-125);
  * the reference test's per-token qdq closed form and torch._int_mm for the
    dynamic int8 case (test_dynamic_qlinear.py:32-36, 83-92).
Run: python tests/golden/make_golden.py   (deterministic; rewrites the files)
"""
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402


def bf16_ulp(y):
    return torch.finfo(torch.bfloat16).eps * y.float().abs().clamp(min=2.0 ** -126)


def woq_symmetric_group():
    g = torch.Generator().manual_seed(1234)
    M, K, N, gs = 4, 256, 64, 128
    x = torch.randn(M, K, generator=g).bfloat16()
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(K // gs, N, generator=g) * 0.015 + 0.005).bfloat16()
    b = torch.randn(N, generator=g).bfloat16()
    wp = O.woq_repack_weight(q)
    y = O.woq_linear(x, wp, s)
    yb = O.woq_linear(x, wp, s, bias=b)
    # cross-check: torch dequant (bf16 rounding of q*s) then fp32 linear
    dq = (q.float() * s.float().repeat_interleave(gs, 0).t()).bfloat16().float()
    ref = torch.nn.functional.linear(x.float(), dq).bfloat16()
    refb = torch.nn.functional.linear(x.float(), dq, b.float()).bfloat16()
    assert ((y.float() - ref.float()).abs() <= bf16_ulp(ref)).all()
    assert ((yb.float() - refb.float()).abs() <= bf16_ulp(refb)).all()
    return {"x": x, "q": q, "w_packed": wp, "scales": s, "bias": b, "y": y, "y_bias": yb}


def woq_per_channel_fp32_scale():
    # The reference op test's data: randn weight quantised per channel with
    # scale = absmax/8 in fp32 (test_woq_linear.py:71-96), bf16 activations.
    g = torch.Generator().manual_seed(99)
    M, K, N = 16, 64, 48
    x = torch.randn(M, K, generator=g).bfloat16()
    w = torch.randn(N, K, generator=g).bfloat16()
    b = torch.randn(N, generator=g).bfloat16()
    absmax = w.abs().max(dim=1, keepdim=True)[0]
    scale = torch.clamp(absmax / 8, min=1e-8).to(torch.float32)
    q = torch.clamp(torch.round(w / scale), -8, 7).to(torch.int8)
    wp = O.woq_repack_weight(q)
    y = O.woq_linear(x, wp, scale.t().contiguous(), bias=b)
    ref = torch.nn.functional.linear(x, (q.to(torch.bfloat16) * scale).to(torch.bfloat16), b)
    assert torch.allclose(y, ref, rtol=1e-3, atol=1e-3)  # the reference test's bar
    return {"x": x, "q": q, "w_packed": wp, "scales": scale.t().contiguous(), "bias": b, "y": y}


def woq_asymmetric_tinygemm():
    g = torch.Generator().manual_seed(7)
    M, K, N, gs = 3, 256, 64, 128
    x = torch.randn(M, K, generator=g).bfloat16()
    u = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
    s = (torch.rand(K // gs, N, generator=g) * 0.015 + 0.005).bfloat16()
    z = (torch.randn(K // gs, N, generator=g) * 0.01).bfloat16()
    packed = torch.ops.aten._convert_weight_to_int4pack_for_cpu(u, 1)
    wp = O.woq_repack_weight(O.unpack_int4pack(packed, K))
    assert torch.equal(wp, O.woq_repack_weight(u.to(torch.int8)))
    y = O.woq_linear(x, wp, s, zero_points=z)
    tg = torch.ops.aten._weight_int4pack_mm_for_cpu(x, packed, gs, torch.stack([s, z], -1).contiguous())
    assert torch.allclose(y.float(), tg.float(), atol=1e-2, rtol=1e-2)
    return {"x": x, "u": u.to(torch.int8), "int4pack": packed, "w_packed": wp, "scales": s,
            "zero_points": z, "y": y, "y_tinygemm": tg}


def dynamic_qlinear_case():
    g = torch.Generator().manual_seed(2024)
    M, K, N = 8, 64, 32
    x = torch.randn(M, K, generator=g)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    sw = 1 + torch.randn(N, generator=g).abs()
    b = torch.randn(N, generator=g)
    y, qx, sx, acc = O.dynamic_qlinear(x, w, sw, b, return_intermediates=True)
    amax = x.abs().amax(dim=1, keepdim=True).clamp(min=1e-12)
    scale = amax / 127.0
    qref = torch.clamp(torch.round(x / scale), -128, 127)
    assert torch.equal(qx, qref.to(torch.int8)) and torch.equal(sx, scale.squeeze(1))
    assert torch.equal(acc, torch._int_mm(qx, w.t().contiguous()))
    ref = torch.matmul(qref * scale, (w.float() * sw.unsqueeze(1)).t()) + b
    assert torch.allclose(y, ref, atol=1e-2, rtol=1e-2)
    xb = torch.randn(5, 4096, generator=g).bfloat16()
    qxb, sxb = O.dynamic_quantize(xb)
    xf = xb.float()
    sb = xf.abs().amax(1, keepdim=True).clamp(min=1e-12) / 127.0
    assert torch.equal(qxb, torch.clamp(torch.round(xf / sb), -128, 127).to(torch.int8))
    return {"x": x, "w": w, "w_scales": sw, "bias": b, "qx": qx, "sx": sx, "acc": acc, "y": y,
            "x_bf16": xb, "qx_bf16": qxb, "sx_bf16": sxb}


def main():
    cases = {
        "woq_symmetric_group128": woq_symmetric_group(),
        "woq_per_channel_fp32_scale": woq_per_channel_fp32_scale(),
        "woq_asymmetric_tinygemm": woq_asymmetric_tinygemm(),
        "dynamic_qlinear": dynamic_qlinear_case(),
    }
    for name, tensors in cases.items():
        path = os.path.join(HERE, name + ".safetensors")
        save_file({k: v.contiguous() for k, v in tensors.items()}, path)
        print("wrote", path)


if __name__ == "__main__":
    main()
