"""GPU parity of the per-token asymmetric uint8 dynamic qlinear (the opt-in
extension beside the reference's symmetric s8) against the CPU oracle,
through the C-ABI and the torch op.  q, sx, zp and the corrected int32
accumulators sum_k (q - zp) * w are integer / closed-form results and must
be bit-exact, on every int8 GEMM kernel (skinny 16- and 32-token, tiled,
load-wave and 16x16 kernels, chosen by M, N, K and the selection knobs);
bf16/fp32 outputs are held to rtol = atol = 1e-2 as the symmetric op.
"""
import pytest
import torch

import zt_capi as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _announce(request):
    import zentorch  # noqa: F401  (the torch ops)
    print(f"\n[case] {request.node.name}", flush=True)


def _x(M, K, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * 2
    if M > 3:
        x[1] = torch.nn.functional.silu(x[1])  # mostly positive
        x[2] = x[2].abs()                      # positive
        x[3] = 0                               # zero row
    return x.to(dtype)


@pytest.mark.parametrize("M,K", [(1, 8), (5, 12), (16, 4096), (7, 11008), (130, 1024),
                                 (3, 33), (64, 20000), (1500, 4096), (1025, 14336)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_asym_quantize_bit_exact(M, K, dtype):
    x = _x(M, K, seed=M * 7 + K, dtype=dtype)
    qx, sx, azp = C.dynamic_quantize_asym(x.to(DEV))
    q, sr, zr = O.dynamic_quantize_asym(x)
    assert torch.equal(sx.cpu(), sr)
    assert torch.equal(azp.cpu() + 128, zr)
    assert torch.equal(qx.cpu().int() + 128, q.int())


def test_colsum_exact():
    g = torch.Generator().manual_seed(3)
    for N, K in [(1, 1), (7, 33), (300, 4096), (64, 4100)]:
        w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
        assert torch.equal(C.s8_weight_colsum(w.to(DEV)).cpu(), w.int().sum(1).int())
    # a row start that is not 16-byte aligned (K odd): the scalar path
    w = torch.randint(-128, 128, (9, 1001), generator=g, dtype=torch.int8)
    assert torch.equal(torch.ops.zentorch.zentorch_s8_weight_colsum(w.to(DEV)).cpu(),
                       w.int().sum(1).int())


# (M, N, K, knobs): each row reaches one GEMM kernel
KERNEL_CASES = [
    (1, 264, 512, {}), (8, 258, 512, {}), (16, 512, 1024, {}),          # skinny 16-token
    (17, 264, 512, {}), (100, 520, 1024, {"ZT_S8_SPLIT": "0"}),         # skinny 32-token
    (20, 64, 8192, {}), (45, 96, 1600, {}),
    (100, 520, 1024, {}), (128, 1032, 4096, {}), (65, 97, 256, {}),     # split-K
    (96, 1000, 768, {"ZT_S8_SPLIT": "3"}), (128, 11008, 4096, {"ZT_S8_SPLIT": "4"}),
    (200, 264, 512, {}),                                                # 16x16 kernel
    (300, 130, 144, {}), (2048, 512, 1024, {}), (1500, 600, 272, {}),   # load-wave kernel
    (1500, 600, 272, {"ZT_S8_TILE": "9"}),                              # 256 x 192 tiles
    (2048, 512, 1024, {"ZT_S8_KIND": "n"}),                             # 32x32 DMA kernel
    (64, 100, 48, {"ZT_S8_FORCE": "o"}),                                # 16x16 kernel
    (5, 33, 12, {}),                                                     # generic (K % 16)
]


@pytest.mark.parametrize("M,N,K,kn", KERNEL_CASES)
def test_asym_accumulators_bit_exact(M, N, K, kn, knobs):
    x = _x(M, K, seed=M + N + K)
    g = torch.Generator().manual_seed(N)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 0.009 + 0.001
    wd = w.to(DEV)
    cs = C.s8_weight_colsum(wd)
    for k, v in kn.items():
        knobs.set(k, v)
    acc = C.dynamic_qlinear_asym(x.to(DEV), wd, sw.to(DEV), cs, out_dtype=torch.int32).cpu()
    ref = O.dynamic_qlinear_asym(x, w, sw, out_dtype=torch.int32)
    assert torch.equal(acc, ref)
    y = C.dynamic_qlinear_asym(x.to(DEV), wd, sw.to(DEV), cs).cpu()
    torch.testing.assert_close(y.float(), O.dynamic_qlinear_asym(x, w, sw).float(),
                               rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,K,N", [(1, 256, 64), (33, 4096, 4096), (128, 4096, 11008)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_asym_op_vs_oracle(M, K, N, x_dtype):
    g = torch.Generator().manual_seed(M + K)
    x = torch.nn.functional.silu(torch.randn(2, M, K, generator=g) * 2).to(x_dtype)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = (torch.rand(N, 1, generator=g) * 0.009 + 0.001).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16()
    ops = torch.ops.zentorch
    wd = w.to(DEV)
    cs = ops.zentorch_s8_weight_colsum(wd)
    y = ops.zentorch_dynamic_qlinear_asym(x.to(DEV), wd, sw.to(DEV), cs, b.to(DEV)).cpu()
    assert y.shape == (2, M, N) and y.dtype == x_dtype
    ref = O.dynamic_qlinear_asym(x, w, sw.reshape(-1), b)
    torch.testing.assert_close(y.float(), ref.float(), rtol=1e-2, atol=1e-2)


def test_asym_op_errors():
    ops = torch.ops.zentorch
    x = torch.randn(4, 64, device=DEV).bfloat16()
    w = torch.randint(-127, 128, (16, 64), dtype=torch.int8, device=DEV)
    sw = torch.rand(16, device=DEV)
    with pytest.raises(RuntimeError, match="weight_colsum"):
        ops.zentorch_dynamic_qlinear_asym(x, w, sw, torch.zeros(15, dtype=torch.int32,
                                                                device=DEV))
    with pytest.raises(RuntimeError, match="weight_colsum"):
        ops.zentorch_dynamic_qlinear_asym(x, w, sw, torch.zeros(16, device=DEV))
