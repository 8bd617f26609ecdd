"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every symbol include/*.h declares, the torch ops carry the reference's exact
schemas, Meta kernels give the reference's output shapes, and a CPU tensor
is an error (no CPU fallback).  No GPU compute is called here."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
PKG = os.path.join(ROOT, "zendnn-pytorch-plugin_amd", "zentorch")


def declared(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:zt|aoti_torch_cuda_zentorch)_\w+)\s*\(", text)))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True,
                         check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


def test_c_abi_exports_every_declared_symbol():
    names = declared("zentorch_hip.h")
    assert "zt_woq_linear" in names and "zt_dynamic_qlinear" in names
    lib = os.path.join(PKG, "libzentorch_hip.so")
    syms = exported(lib)
    missing = [n for n in names if n not in syms]
    assert not missing, missing
    L = ctypes.CDLL(lib)
    for n in names:
        getattr(L, n)
    L.zt_version.restype = ctypes.c_int32
    assert L.zt_version() >= 100


def test_c_abi_needs_no_torch():
    out = subprocess.run(["readelf", "-d", os.path.join(PKG, "libzentorch_hip.so")],
                         capture_output=True, text=True, check=True).stdout
    needed = [ln.split("[", 1)[1].rstrip("]") for ln in out.splitlines() if "(NEEDED)" in ln]
    assert needed, out
    assert not any("torch" in n or "c10" in n for n in needed), needed


def test_aoti_shims_exported():
    names = declared("shim_cuda_zentorch.h")
    # the reference's 9 WOQ/dynamic + 6 static qlinear shims, and 4 extensions
    assert len(names) == 19
    syms = exported(os.path.join(PKG, "_C.so"))
    assert not [n for n in names if n not in syms]


def test_c_abi_validates_without_gpu():
    import zt_capi as C
    L = C.lib()
    # K not a multiple of 8 is rejected before any device work
    rc = L.zt_woq_linear(None, 1, 4, 12, 12, None, 16, None, 1, 1, None, -1, None, -1,
                         None, None, 1, 16, None, 0, None)
    assert rc == 1 and b"K" in L.zt_last_error_string()
    rc = L.zt_woq_repack_from_int4pack(None, 10, 64, None, None)
    assert rc == 1 and b"multiple of 64" in L.zt_last_error_string()
    assert L.zt_dynamic_qlinear_workspace_size(128, 4096, 0) >= 128 * 4096 + 128 * 4
    # the split-K exchange (64 < M <= 128, K % 256 == 0): int32 partials of
    # both K halves of every 96-column tile, then the tile counters
    base = L.zt_dynamic_qlinear_workspace_size(128, 4096, 0)
    tiles = (11008 + 95) // 96
    assert L.zt_dynamic_qlinear_workspace_size(128, 4096, 11008) >= base + tiles * 2 * 128 * 96 * 4
    assert L.zt_dynamic_qlinear_workspace_size(64, 4096, 11008) == \
        L.zt_dynamic_qlinear_workspace_size(64, 4096, 0)
    # MoE: H, I multiples of 128; E <= 1024; activations the kernels have
    rc = L.zt_woq_moe(None, 4, 100, None, None, 0, 2, 0, 4, None, None, 1, None, None, None,
                      1, None, 8, 256, None, None, 0, None)
    assert rc == 1 and b"multiples of 128" in L.zt_last_error_string()
    rc = L.zt_woq_moe(None, 4, 256, None, None, 0, 2, 0, 1, None, None, 1, None, None, None,
                      1, None, 8, 256, None, None, 0, None)
    assert rc == 2 and b"act" in L.zt_last_error_string()
    rc = L.zt_woq_moe(None, 4, 256, None, None, 0, 2, 0, 4, None, None, 1, None, None, None,
                      1, None, 2048, 256, None, None, 0, None)
    assert rc == 2 and b"1024 experts" in L.zt_last_error_string()
    assert L.zt_woq_moe_workspace_size(256, 4096, 2, 8, 14336) >= 512 * (14336 + 4096) * 2
    # merged gate_up: an odd N is refused before any device work; the
    # two-step path's workspace holds the fp32 [M, N] result
    rc = L.zt_woq_linear_gate_up(None, 1, 4, 128, 128, None, 17, None, 1, 1, None, -1, None,
                                 -1, None, 1, 8, None, 0, None)
    assert rc == 1 and b"even" in L.zt_last_error_string()
    assert L.zt_woq_linear_gate_up_workspace_size(20, 4096, 1024, 32) >= 20 * 1024 * 4
    # the WOQ kernels reduce K inside a workgroup: no device workspace
    assert L.zt_woq_linear_workspace_size(16, 14336, 4096, 112) == 0
    assert L.zt_woq_linear_workspace_size(2048, 4096, 4096, 32) == 0
    # up to 16 rows a shape without a stream-kernel x layout takes the wide
    # kernel, whose K splits keep fp32 partials [splits][M][N] (4096 x 11008
    # at M = 16: 43 phases in 6 splits of 8); with a layout it needs none
    assert L.zt_woq_linear_workspace_size(16, 11008, 4096, 86) == 6 * 16 * 4096 * 4
    assert L.zt_woq_linear_workspace_size(14, 11008, 4096, 86) == 0
    # prefill GEMMs whose tiles make less than one round split K: fp32 (int4)
    # or int32 (int8) partials [splits][M][N] follow the base workspace
    assert L.zt_woq_linear_workspace_size(512, 4096, 4096, 32) == 4 * 512 * 4096 * 4
    assert L.zt_woq_linear_workspace_size(128, 11008, 4096, 86) == 8 * 128 * 4096 * 4
    # exactly half a round of 256 x 128 tiles (128) splits too: 2 ways
    assert L.zt_woq_linear_workspace_size(512, 8192, 8192, 64) == 2 * 512 * 8192 * 4
    assert L.zt_dynamic_qlinear_workspace_size(512, 4096, 4096) >= \
        L.zt_dynamic_qlinear_workspace_size(512, 4096, 0) + 2 * 512 * 4096 * 4
    # empty sizes (N = 0 asks for the least workspace) plan no split
    assert L.zt_dynamic_qlinear_workspace_size(512, 4096, 0) >= 512 * 4096 + 512 * 4
    assert L.zt_dynamic_qlinear_asym_workspace_size(512, 4096, 0) >= 512 * 4096 + 512 * 8
    assert L.zt_woq_linear_workspace_size(512, 4096, 0, 32) == 0
    assert L.zt_dynamic_qlinear_workspace_size(0, 4096, 4096) == 0


# Schemas as the reference registers them (src/cpu/cpp/WOQ_Linear.cpp:435-480,
# DynamicQLinear.cpp:184-189), in torch's canonical printing.
REFERENCE_SCHEMAS = {
    "zentorch_woq_linear": "zentorch::zentorch_woq_linear(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear\") -> Tensor",
    "zentorch_woq_linear_relu": "zentorch::zentorch_woq_linear_relu(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_relu\") -> Tensor",
    "zentorch_woq_linear_sigmoid": "zentorch::zentorch_woq_linear_sigmoid(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_sigmoid\") -> Tensor",
    "zentorch_woq_linear_gelu_tanh": "zentorch::zentorch_woq_linear_gelu_tanh(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_gelu_tanh\") -> Tensor",
    "zentorch_woq_linear_gelu_erf": "zentorch::zentorch_woq_linear_gelu_erf(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_gelu_erf\") -> Tensor",
    "zentorch_woq_linear_add": "zentorch::zentorch_woq_linear_add(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor add_input, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_add\") -> Tensor",
    "zentorch_woq_linear_mul_add": "zentorch::zentorch_woq_linear_mul_add(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor mul_input, Tensor add_input, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_mul_add\") -> Tensor",
    "zentorch_woq_linear_add_add": "zentorch::zentorch_woq_linear_add_add(Tensor input, Tensor weight, Tensor weight_scales, Tensor? weight_zero_points, Tensor add_input, Tensor add_input_2, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_woq_linear_add_add\") -> Tensor",
    "zentorch_woq_repack_weight": "zentorch::zentorch_woq_repack_weight(Tensor unpacked_weight) -> Tensor",
    "zentorch_woq_repack_from_int4pack": "zentorch::zentorch_woq_repack_from_int4pack(Tensor packed_weight) -> Tensor",
    "zentorch_dynamic_qlinear": "zentorch::zentorch_dynamic_qlinear(Tensor input, Tensor weight, Tensor weight_scales, Tensor? bias=None, *, str zentorch_op_name=\"zentorch::zentorch_dynamic_qlinear\") -> Tensor",
    # src/cpu/cpp/FusedMoE.cpp:729-741
    "zentorch_fused_moe": "zentorch::zentorch_fused_moe(Tensor(a!) output, Tensor input, Tensor w13, Tensor w2, Tensor? w13_bias, Tensor? w2_bias, Tensor topk_weights, Tensor topk_id, bool skip_weighted, str act, Tensor? w13_scales=None, Tensor? w2_scales=None, *, str zentorch_op_name=\"zentorch::zentorch_fused_moe\") -> ()",
    "zentorch_flush_moe_weight_cache": "zentorch::zentorch_flush_moe_weight_cache() -> ()",
}


@pytest.mark.parametrize("op", sorted(REFERENCE_SCHEMAS))
def test_op_schema_matches_reference(op):
    import zentorch  # noqa: F401
    assert str(getattr(torch.ops.zentorch, op).default._schema) == REFERENCE_SCHEMAS[op]


def test_reference_tags_kept():
    import zentorch  # noqa: F401
    ops = torch.ops.zentorch
    assert torch.Tag.needs_contiguous_strides in ops.zentorch_woq_linear_add.default.tags
    assert torch.Tag.needs_fixed_stride_order in ops.zentorch_woq_linear_mul_add.default.tags
    assert torch.Tag.needs_fixed_stride_order in ops.zentorch_woq_linear_add_add.default.tags


def test_meta_shapes():
    import zentorch  # noqa: F401
    ops = torch.ops.zentorch
    m = dict(device="meta")
    x = torch.empty(2, 3, 4096, dtype=torch.bfloat16, **m)
    w = torch.empty(512, 6144, dtype=torch.int32, **m)
    s = torch.empty(32, 6144, dtype=torch.bfloat16, **m)
    y = ops.zentorch_woq_linear(x, w, s, None)
    assert y.shape == (2, 3, 6144) and y.dtype == torch.bfloat16
    buf = torch.empty(2, 3, 6144, dtype=torch.bfloat16, **m)
    assert ops.zentorch_woq_linear_mul_add(x, w, s, None, buf, buf).shape == (2, 3, 6144)
    assert ops.zentorch_woq_linear_silu_mul(x, w, s, None, buf).shape == (2, 3, 6144)
    # merged gate_up [K/8, 2I] -> [*, I]
    assert ops.zentorch_woq_linear_gate_up_silu_mul(x, w, s, None).shape == (2, 3, 3072)
    xw = torch.empty(128, 4096, dtype=torch.float32, **m)
    wq = torch.empty(11008, 4096, dtype=torch.int8, **m)
    y = ops.zentorch_dynamic_qlinear(xw, wq, torch.empty(11008, **m))
    assert y.shape == (128, 11008) and y.dtype == torch.float32
    r = ops.zentorch_woq_repack_weight(torch.empty(64, 256, dtype=torch.int8, **m))
    assert r.shape == (64, 32) and r.dtype == torch.int32
    r = ops.zentorch_woq_repack_from_int4pack(torch.empty(64, 128, dtype=torch.uint8, **m))
    assert r.shape == (64, 32) and r.dtype == torch.int32
    xm = torch.empty(8, 256, dtype=torch.bfloat16, **m)
    assert ops.zentorch_fused_moe(
        torch.empty_like(xm), xm, torch.empty(4, 256, 32, dtype=torch.int32, **m),
        torch.empty(4, 256, 16, dtype=torch.int32, **m), None, None,
        torch.empty(8, 2, **m), torch.empty(8, 2, dtype=torch.int32, **m), False, "silu",
        torch.empty(4, 1, 256, dtype=torch.bfloat16, **m),
        torch.empty(4, 1, 256, dtype=torch.bfloat16, **m)) is None


def test_cpu_tensors_are_rejected_not_computed():
    import zentorch  # noqa: F401
    x = torch.randn(4, 64).bfloat16()
    with pytest.raises(NotImplementedError):
        torch.ops.zentorch.zentorch_woq_linear(x, torch.zeros(8, 16, dtype=torch.int32),
                                               torch.ones(1, 16).bfloat16(), None)
    with pytest.raises(NotImplementedError):
        torch.ops.zentorch.zentorch_dynamic_qlinear(x, torch.zeros(16, 64, dtype=torch.int8),
                                                    torch.ones(16))
