"""ctypes binding of libzentorch_hip.so's C-ABI (include/zentorch_hip.h) for
the tests: GPU tensors go in as raw device pointers with sizes and the
current torch stream, exactly as a non-torch caller would pass them."""
import contextlib
import ctypes
import os

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "zendnn-pytorch-plugin_amd", "zentorch", "libzentorch_hip.so")

DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int8: 3,
      torch.uint8: 4, torch.int32: 5}
PO = {"none": 0, "relu": 1, "gelu_tanh": 2, "gelu_erf": 3, "silu": 4,
      "sigmoid": 5, "tanh": 6, "mul": 7, "add": 8}
MAX_POST_OPS = 4

_vp, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t


class PostOps(ctypes.Structure):
    _fields_ = [("count", ctypes.c_int32),
                ("ids", ctypes.c_int32 * MAX_POST_OPS),
                ("bufs", ctypes.c_void_p * MAX_POST_OPS),
                ("buf_dtypes", ctypes.c_int32 * MAX_POST_OPS),
                ("buf_ld", ctypes.c_int64 * MAX_POST_OPS)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH, mode=os.RTLD_GLOBAL | os.RTLD_NOW)
        L.zt_woq_linear.argtypes = [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i32,
                                    _i64, _vp, _i32, _vp, _i32, ctypes.POINTER(PostOps),
                                    _vp, _i32, _i64, _vp, _sz, _vp]
        L.zt_woq_linear.restype = ctypes.c_int
        L.zt_woq_linear_workspace_size.argtypes = [_i64, _i64, _i64, _i64]
        L.zt_woq_linear_workspace_size.restype = _sz
        L.zt_woq_linear_gate_up.argtypes = [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i32,
                                            _i64, _vp, _i32, _vp, _i32, _vp, _i32, _i64,
                                            _vp, _sz, _vp]
        L.zt_woq_linear_gate_up.restype = ctypes.c_int
        L.zt_woq_linear_gate_up_workspace_size.argtypes = [_i64, _i64, _i64, _i64]
        L.zt_woq_linear_gate_up_workspace_size.restype = _sz
        L.zt_dynamic_qlinear.argtypes = [_vp, _i32, _i64, _i64, _vp, _i64, _vp, _i32, _vp,
                                         _i32, ctypes.POINTER(PostOps), _vp, _i32, _vp,
                                         _sz, _vp]
        L.zt_dynamic_qlinear_workspace_size.argtypes = [_i64, _i64, _i64]
        L.zt_dynamic_qlinear_workspace_size.restype = _sz
        L.zt_dynamic_quantize.argtypes = [_vp, _i32, _i64, _i64, _vp, _vp, _vp]
        L.zt_s8s8s32_gemm.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp, _vp]
        L.zt_dynamic_qlinear_asym.argtypes = [_vp, _i32, _i64, _i64, _vp, _i64, _vp, _i32,
                                              _vp, _vp, _i32, ctypes.POINTER(PostOps), _vp,
                                              _i32, _vp, _sz, _vp]
        L.zt_dynamic_qlinear_asym_workspace_size.argtypes = [_i64, _i64, _i64]
        L.zt_dynamic_qlinear_asym_workspace_size.restype = _sz
        L.zt_dynamic_quantize_asym.argtypes = [_vp, _i32, _i64, _i64, _vp, _vp, _vp, _vp]
        L.zt_s8_weight_colsum.argtypes = [_vp, _i64, _i64, _vp, _vp]
        L.zt_woq_repack_weight.argtypes = [_vp, _i64, _i64, _vp, _vp]
        L.zt_woq_repack_from_int4pack.argtypes = [_vp, _i64, _i64, _vp, _vp]
        L.zt_woq_moe.argtypes = [_vp, _i64, _i64, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp,
                                 _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp, _sz, _vp]
        L.zt_woq_moe_workspace_size.argtypes = [_i64, _i64, _i64, _i64, _i64]
        L.zt_woq_moe_workspace_size.restype = _sz
        L.zt_last_error_string.restype = ctypes.c_char_p
        L.zt_set_tuning.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        L.zt_set_tuning.restype = ctypes.c_int
        L.zt_get_tuning.argtypes = [ctypes.c_char_p]
        L.zt_get_tuning.restype = ctypes.c_char_p
        L.zt_version.restype = ctypes.c_int32
        _lib = L
    return _lib


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(rc):
    if rc != 0:
        raise RuntimeError(f"C-ABI error {rc}: {lib().zt_last_error_string().decode()}")


def set_tuning(name, value):
    """Set a kernel-selection knob of the library (None unsets it)."""
    v = None if value is None else str(value).encode()
    _check(lib().zt_set_tuning(name.encode(), v))


def get_tuning(name):
    v = lib().zt_get_tuning(name.encode())
    return None if v is None else v.decode()


@contextlib.contextmanager
def tuning(**knobs):
    """Set knobs for the duration of a with-block, then restore them."""
    saved = {k: get_tuning(k) for k in knobs}
    try:
        for k, v in knobs.items():
            set_tuning(k, v)
        yield
    finally:
        for k, v in saved.items():
            set_tuning(k, v)


def make_post(post_ops, bufs, N):
    po = PostOps()
    po.count = len(post_ops)
    bi = 0
    keep = []
    for i, name in enumerate(post_ops):
        po.ids[i] = PO[name]
        if name in ("add", "mul"):
            b = bufs[bi].reshape(-1, N).contiguous()
            keep.append(b)
            po.bufs[bi] = b.data_ptr()
            po.buf_dtypes[bi] = DT[b.dtype]
            po.buf_ld[bi] = N
            bi += 1
    return po, keep


def woq_linear(x, w_nk, scales, zp=None, bias=None, post_ops=(), post_bufs=(),
               out_dtype=None, sync=True):
    """x [M,K] (GPU), w_nk int32 [N,K/8], scales/zp [G,N], bias [N]."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    N = w_nk.shape[0]
    G = scales.shape[0]
    y = torch.empty(M, N, dtype=out_dtype or x.dtype, device=x.device)
    po, keep = make_post(post_ops, post_bufs, N)
    ws_bytes = lib().zt_woq_linear_workspace_size(M, K, N, G)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    rc = lib().zt_woq_linear(
        _p(x2), DT[x2.dtype], M, K, x2.stride(0), _p(w_nk), N, _p(scales), DT[scales.dtype], G,
        _p(zp), DT[zp.dtype] if zp is not None else -1, _p(bias),
        DT[bias.dtype] if bias is not None else -1, ctypes.byref(po), _p(y), DT[y.dtype], N,
        _p(ws), ws_bytes, _stream())
    _check(rc)
    if sync:
        torch.cuda.synchronize()
    del keep
    return y


def woq_linear_gate_up(x, w_nk, scales, zp=None, bias=None, sync=True):
    """Merged gate_up: w_nk int32 [2I,K/8] (gate rows, then up rows); y [M, I]."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    N = w_nk.shape[0]
    G = scales.shape[0]
    y = torch.empty(M, N // 2, dtype=x.dtype, device=x.device)
    ws_bytes = lib().zt_woq_linear_gate_up_workspace_size(M, K, N, G)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    rc = lib().zt_woq_linear_gate_up(
        _p(x2), DT[x2.dtype], M, K, x2.stride(0), _p(w_nk), N, _p(scales), DT[scales.dtype], G,
        _p(zp), DT[zp.dtype] if zp is not None else -1, _p(bias),
        DT[bias.dtype] if bias is not None else -1, _p(y), DT[y.dtype], N // 2,
        _p(ws), ws_bytes, _stream())
    _check(rc)
    if sync:
        torch.cuda.synchronize()
    return y


def dynamic_qlinear(x, w, sw, bias=None, post_ops=(), post_bufs=(), sync=True, split=True):
    """split=False passes the least workspace (no room for the split-K
    exchange), which runs the unsplit kernel."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    N = w.shape[0]
    y = torch.empty(M, N, dtype=x.dtype, device=x.device)
    po, keep = make_post(post_ops, post_bufs, N)
    ws_bytes = lib().zt_dynamic_qlinear_workspace_size(M, K, N if split else 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    rc = lib().zt_dynamic_qlinear(
        _p(x2), DT[x2.dtype], M, K, _p(w), N, _p(sw), DT[sw.dtype], _p(bias),
        DT[bias.dtype] if bias is not None else -1,
        ctypes.byref(po) if post_ops else None, _p(y), DT[y.dtype], _p(ws), ws_bytes,
        _stream())
    _check(rc)
    if sync:
        torch.cuda.synchronize()
    del keep
    return y


def dynamic_quantize(x):
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    qx = torch.empty(M, K, dtype=torch.int8, device=x.device)
    sx = torch.empty(M, dtype=torch.float32, device=x.device)
    _check(lib().zt_dynamic_quantize(_p(x2), DT[x2.dtype], M, K, _p(qx), _p(sx), _stream()))
    torch.cuda.synchronize()
    return qx, sx


def s8_weight_colsum(w):
    N, K = w.shape
    out = torch.empty(N, dtype=torch.int32, device=w.device)
    _check(lib().zt_s8_weight_colsum(_p(w), N, K, _p(out), _stream()))
    torch.cuda.synchronize()
    return out


def dynamic_quantize_asym(x):
    """(qx int8 = q - 128, sx fp32, azp int32 = zp - 128)."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    qx = torch.empty(M, K, dtype=torch.int8, device=x.device)
    sx = torch.empty(M, dtype=torch.float32, device=x.device)
    azp = torch.empty(M, dtype=torch.int32, device=x.device)
    _check(lib().zt_dynamic_quantize_asym(_p(x2), DT[x2.dtype], M, K, _p(qx), _p(sx), _p(azp),
                                          _stream()))
    torch.cuda.synchronize()
    return qx, sx, azp


def dynamic_qlinear_asym(x, w, sw, colsum, bias=None, out_dtype=None, post_ops=(),
                         post_bufs=(), split=True):
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    N = w.shape[0]
    y = torch.empty(M, N, dtype=out_dtype or x.dtype, device=x.device)
    po, keep = make_post(post_ops, post_bufs, N)
    ws_bytes = lib().zt_dynamic_qlinear_asym_workspace_size(M, K, N if split else 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    rc = lib().zt_dynamic_qlinear_asym(
        _p(x2), DT[x2.dtype], M, K, _p(w), N, _p(sw), DT[sw.dtype], _p(colsum), _p(bias),
        DT[bias.dtype] if bias is not None else -1,
        ctypes.byref(po) if post_ops else None, _p(y), DT[y.dtype], _p(ws), ws_bytes,
        _stream())
    _check(rc)
    torch.cuda.synchronize()
    del keep
    return y


def s8s8s32_gemm(qa, w):
    M, K = qa.shape
    N = w.shape[0]
    acc = torch.empty(M, N, dtype=torch.int32, device=qa.device)
    _check(lib().zt_s8s8s32_gemm(_p(qa), _p(w), M, N, K, _p(acc), _stream()))
    torch.cuda.synchronize()
    return acc


def woq_repack_weight(w):
    N, K = w.shape
    out = torch.empty(N, K // 8, dtype=torch.int32, device=w.device)
    _check(lib().zt_woq_repack_weight(_p(w), N, K, _p(out), _stream()))
    torch.cuda.synchronize()
    return out


def woq_repack_from_int4pack(packed):
    N = packed.shape[0]
    K = packed.shape[1] * 2
    out = torch.empty(N, K // 8, dtype=torch.int32, device=packed.device)
    _check(lib().zt_woq_repack_from_int4pack(_p(packed), N, K, _p(out), _stream()))
    torch.cuda.synchronize()
    return out


MOE_ACT = {"silu": PO["silu"], "gelu": PO["gelu_erf"], "gelu_tanh": PO["gelu_tanh"]}


def woq_moe(x, topk_ids, topk_weights, w13, w13_scales, w2, w2_scales, w13_bias=None,
            w2_bias=None, act="silu", skip_weighted=False, sync=True):
    """zt_woq_moe on device tensors; returns bf16 [T, H]."""
    T, H = x.shape
    topk = topk_ids.shape[1]
    E, N13, _ = w13.shape
    I = N13 // 2
    out = torch.empty(T, H, dtype=torch.bfloat16, device=x.device)
    ws_bytes = lib().zt_woq_moe_workspace_size(T, H, topk, E, I)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    ids = topk_ids.to(torch.int32).contiguous()
    _check(lib().zt_woq_moe(
        _p(x), T, H, _p(ids), _p(topk_weights), DT[topk_weights.dtype], topk,
        int(skip_weighted), MOE_ACT[act], _p(w13), _p(w13_scales), w13_scales.shape[1],
        _p(w13_bias), _p(w2), _p(w2_scales), w2_scales.shape[1], _p(w2_bias), E, I, _p(out),
        _p(ws), ws_bytes, _stream()))
    if sync:
        torch.cuda.synchronize()
    return out
