"""ctypes front end of the CPU oracle (oracle/zt_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing
measured or shipped.  The product path (torch.ops.zentorch.*) has no CPU
kernel and never reaches this module.

Every function takes and returns CPU torch tensors.  Semantics and the
reference lines they restate are documented in zt_oracle.c.
"""
import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libzt_oracle.so")
_lib = None

DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int8: 3,
      torch.uint8: 4, torch.int32: 5}
# Post-op ids, numbered as the reference's UNARY_POST_OP / BINARY_POST_OP
# (src/cpu/cpp/Utils.hpp:56-71).
PO = {"none": 0, "relu": 1, "gelu_tanh": 2, "gelu_erf": 3, "silu": 4,
      "sigmoid": 5, "tanh": 6, "mul": 7, "add": 8}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build():
    """Compile libzt_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.zto_woq_repack_weight.argtypes = [_vp, _i64, _i64, _vp]
        L.zto_unpack_int4pack.argtypes = [_vp, _i64, _i64, _vp]
        L.zto_woq_linear.argtypes = [
            _vp, _int, _i64, _i64, _i64, _vp, _i64, _vp, _int, _i64, _vp, _int,
            _vp, _int, _int, _vp, _vp, _vp, _vp, _vp, _int, _i64, _int]
        L.zto_dynamic_quantize.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _int]
        L.zto_s8s8s32_gemm.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp, _int]
        L.zto_dynamic_qlinear.argtypes = [
            _vp, _int, _i64, _i64, _vp, _i64, _vp, _int, _vp, _int, _int, _vp,
            _vp, _vp, _vp, _vp, _int, _vp, _vp, _vp, _int]
        L.zto_dynamic_quantize_asym.argtypes = [_vp, _int, _i64, _i64, _vp, _vp, _vp, _int]
        L.zto_dynamic_qlinear_asym.argtypes = [
            _vp, _int, _i64, _i64, _vp, _i64, _vp, _int, _vp, _int, _vp, _int, _vp, _vp, _vp,
            _int]
        L.zto_qlinear.argtypes = [
            _vp, _int, _i64, _i64, ctypes.c_float, _int, ctypes.c_int32, _vp, _i64, _vp, _i64,
            _vp, _int, _int, _vp, _vp, _vp, _vp, _vp, _int, _int, ctypes.c_float, _int,
            ctypes.c_int32, _int]
        L.zto_woq_moe.argtypes = [
            _vp, _i64, _i64, _vp, _vp, _int, _i64, _int, _int, _vp, _vp, _i64, _vp, _vp,
            _vp, _i64, _vp, _i64, _i64, _vp, _int]
        L.zto_max_threads.restype = _int
        _lib = L
    return _lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (rc={rc})")


def _post_arrays(post_ops, post_bufs):
    post_ops = list(post_ops or [])
    bufs = [b.contiguous() for b in (post_bufs or [])]
    n = len(post_ops)
    ids = (ctypes.c_int * max(n, 1))(*[PO[p] for p in post_ops])
    nb = max(len(bufs), 1)
    bp = (ctypes.c_void_p * nb)(*[b.data_ptr() for b in bufs])
    bd = (ctypes.c_int * nb)(*[DT[b.dtype] for b in bufs])
    bl = (ctypes.c_int64 * nb)(*[b.reshape(-1, b.shape[-1]).stride(0) for b in bufs])
    return n, ids, bp, bd, bl, bufs


def max_threads():
    return lib().zto_max_threads()


def woq_repack_weight(w_int8):
    """int8 [N, K] -> int32 [N, K/8] (WOQ_Linear.cpp:294-357)."""
    w = w_int8.contiguous()
    N, K = w.shape
    out = torch.empty(N, K // 8, dtype=torch.int32)
    _check(lib().zto_woq_repack_weight(_ptr(w), N, K, _ptr(out)), "repack")
    return out


def unpack_int4pack(packed_u8, K):
    """torch CPU int4pack uint8 [N, K/2] -> int8 [N, K] nibbles (0..15)."""
    p = packed_u8.contiguous()
    N = p.shape[0]
    out = torch.empty(N, K, dtype=torch.int8)
    _check(lib().zto_unpack_int4pack(_ptr(p), N, K, _ptr(out)), "unpack_int4pack")
    return out


def woq_linear(x, w_packed_nk, scales, zero_points=None, bias=None,
               post_ops=(), post_bufs=(), nthreads=0):
    """Reference semantics of zentorch_woq_linear[_*].

    x: [..., K] bf16/fp32; w_packed_nk: int32 [N, K/8] (storage of the op's
    [K/8, N] weight view); scales / zero_points: [G, N]; bias: [N].
    post_ops: names in list order; binary ops consume post_bufs in order.
    """
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    w = w_packed_nk.contiguous()
    N = w.shape[0]
    s = scales.contiguous()
    G = s.shape[0]
    zp = zero_points.contiguous() if zero_points is not None else None
    b = bias.contiguous() if bias is not None else None
    y = torch.empty(M, N, dtype=x.dtype)
    n, ids, bp, bd, bl, keep = _post_arrays(post_ops, [pb.reshape(-1, N) for pb in post_bufs])
    rc = lib().zto_woq_linear(
        _ptr(x2), DT[x2.dtype], M, K, K, _ptr(w), N, _ptr(s), DT[s.dtype], G,
        _ptr(zp), DT[zp.dtype] if zp is not None else -1,
        _ptr(b), DT[b.dtype] if b is not None else -1,
        n, ids, bp, bd, bl, _ptr(y), DT[y.dtype], N, nthreads)
    _check(rc, "woq_linear")
    del keep
    return y.reshape(*x.shape[:-1], N)


def dynamic_quantize(x, nthreads=0):
    """Per-token symmetric s8: returns (qx int8 [M,K], sx fp32 [M])."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    qx = torch.empty(M, K, dtype=torch.int8)
    sx = torch.empty(M, dtype=torch.float32)
    lib().zto_dynamic_quantize(_ptr(x2), DT[x2.dtype], M, K, _ptr(qx), _ptr(sx), nthreads)
    return qx, sx


def s8s8s32_gemm(qa, w, nthreads=0):
    qa = qa.contiguous()
    w = w.contiguous()
    M, K = qa.shape
    N = w.shape[0]
    acc = torch.empty(M, N, dtype=torch.int32)
    lib().zto_s8s8s32_gemm(_ptr(qa), _ptr(w), M, N, K, _ptr(acc), nthreads)
    return acc


def dynamic_qlinear(x, w, w_scales, bias=None, post_ops=(), post_bufs=(),
                    nthreads=0, return_intermediates=False):
    """Reference semantics of zentorch_dynamic_qlinear (DynamicQLinear.cpp:74-181)."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    wc = w.contiguous()
    N = wc.shape[0]
    sw = w_scales.reshape(-1).contiguous()
    b = bias.contiguous() if bias is not None else None
    y = torch.empty(M, N, dtype=x.dtype)
    qx = torch.empty(M, K, dtype=torch.int8)
    sx = torch.empty(M, dtype=torch.float32)
    acc = torch.empty(M, N, dtype=torch.int32)
    n, ids, bp, bd, bl, keep = _post_arrays(post_ops, [pb.reshape(-1, N) for pb in post_bufs])
    lib().zto_dynamic_qlinear(
        _ptr(x2), DT[x2.dtype], M, K, _ptr(wc), N, _ptr(sw), DT[sw.dtype],
        _ptr(b), DT[b.dtype] if b is not None else -1, n, ids, bp, bd, bl,
        _ptr(y), DT[y.dtype], _ptr(qx), _ptr(sx), _ptr(acc), nthreads)
    del keep
    y = y.reshape(*x.shape[:-1], N)
    if return_intermediates:
        return y, qx, sx, acc
    return y


def dynamic_quantize_asym(x, nthreads=0):
    """Per-token asymmetric uint8 (extension, zt_oracle.c): returns
    (q uint8 [M,K], sx fp32 [M], zp int32 [M])."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    q = torch.empty(M, K, dtype=torch.uint8)
    sx = torch.empty(M, dtype=torch.float32)
    zp = torch.empty(M, dtype=torch.int32)
    lib().zto_dynamic_quantize_asym(_ptr(x2), DT[x2.dtype], M, K, _ptr(q), _ptr(sx), _ptr(zp),
                                    nthreads)
    return q, sx, zp


def dynamic_qlinear_asym(x, w, w_scales, bias=None, out_dtype=None, nthreads=0):
    """zentorch_dynamic_qlinear_asym semantics (extension, zt_oracle.c);
    out_dtype torch.int32 returns sum_k (q - zp) * w."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    wc = w.contiguous()
    N = wc.shape[0]
    sw = w_scales.reshape(-1).contiguous()
    b = bias.contiguous() if bias is not None else None
    y = torch.empty(M, N, dtype=out_dtype or x.dtype)
    lib().zto_dynamic_qlinear_asym(
        _ptr(x2), DT[x2.dtype], M, K, _ptr(wc), N, _ptr(sw), DT[sw.dtype],
        _ptr(b), DT[b.dtype] if b is not None else -1, _ptr(y), DT[y.dtype],
        None, None, None, nthreads)
    return y.reshape(*x.shape[:-1], N)


def qlinear(x, w, x_scale, x_zp, w_scales, bias=None, post_ops=(), post_bufs=(),
            out_dtype=torch.float32, y_scale=None, y_zp=None, nthreads=0):
    """zentorch_qlinear* semantics (QLinear.cpp:66-347; zt_oracle.c).  Scales
    and zero points are one-element tensors (or None for the zero points and
    the output scale); w is [N, K] int8."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    wc = w.contiguous()
    N = wc.shape[0]
    sw = w_scales.reshape(-1).float().contiguous()
    b = bias.contiguous() if bias is not None else None
    y = torch.empty(M, N, dtype=out_dtype)
    n, ids, bp, bd, bl, keep = _post_arrays(post_ops, [pb.reshape(-1, N) for pb in post_bufs])
    lib().zto_qlinear(
        _ptr(x2), DT[x2.dtype], M, K, float(x_scale.reshape(-1)[0]), int(x_zp is not None),
        int(x_zp.reshape(-1)[0]) if x_zp is not None else 0, _ptr(wc), N, _ptr(sw), sw.numel(),
        _ptr(b), DT[b.dtype] if b is not None else -1, n, ids, bp, bd, bl, _ptr(y), DT[y.dtype],
        int(y_scale is not None), float(y_scale.reshape(-1)[0]) if y_scale is not None else 1.0,
        int(y_zp is not None), int(y_zp.reshape(-1)[0]) if y_zp is not None else 0, nthreads)
    del keep
    return y.reshape(*x.shape[:-1], N)


MOE_ACT = {"silu": PO["silu"], "gelu": PO["gelu_erf"], "gelu_tanh": PO["gelu_tanh"]}


def woq_moe(x, topk_ids, topk_weights, w13, w13_scales, w2, w2_scales,
            w13_bias=None, w2_bias=None, act="silu", skip_weighted=False, nthreads=0):
    """Grouped int4 MoE (FusedMoE.cpp:443-700 with int4 experts).

    x [T, H] bf16; topk_ids [T, k] int32; topk_weights [T, k]; w13 int32
    [E, 2I, H/8]; w13_scales bf16 [E, G13, 2I]; w2 int32 [E, H, I/8];
    w2_scales bf16 [E, G2, H]; biases bf16 [E, 2I] / [E, H].  Returns bf16 [T, H].
    """
    x = x.contiguous()
    T, H = x.shape
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.contiguous()
    topk = ids.shape[1]
    E, N13, _ = w13.shape
    I = N13 // 2
    out = torch.empty(T, H, dtype=torch.bfloat16)
    args = [w13.contiguous(), w13_scales.contiguous(), w2.contiguous(), w2_scales.contiguous(),
            None if w13_bias is None else w13_bias.contiguous(),
            None if w2_bias is None else w2_bias.contiguous()]
    w13c, s13, w2c, s2, b13, b2 = args
    rc = lib().zto_woq_moe(
        _ptr(x), T, H, _ptr(ids), _ptr(wts), DT[wts.dtype], topk, int(skip_weighted),
        MOE_ACT[act], _ptr(w13c), _ptr(s13), s13.shape[1], _ptr(b13), _ptr(w2c), _ptr(s2),
        s2.shape[1], _ptr(b2), E, I, _ptr(out), nthreads)
    _check(rc, "woq_moe")
    return out
