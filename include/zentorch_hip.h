/*
 * zentorch_hip.h -- C-ABI of libzentorch_hip.so, the gfx950 kernels behind
 * zentorch's quantized-linear ops.
 *
 * Plain pointers, sizes and a HIP stream; no torch types.  Every pointer is a
 * device pointer unless stated otherwise.  All entry points are asynchronous
 * on `stream`, allocate nothing, are thread-safe, and return 0 on success or
 * a ZT_E* code; zt_last_error_string() gives the message of the calling
 * thread's last failure.
 *
 * The reference calls ZenDNNL's C++ matmul_direct from its ATen ops; each
 * entry point below names the reference code it stands in for (paths are
 * relative to the amd/ZenDNN-pytorch-plugin checkout).
 */
#ifndef ZENTORCH_HIP_H
#define ZENTORCH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t (0 = the null stream). */
typedef struct ihipStream_t *zt_stream_t;

/* Element types (src/cpu/cpp/Memory.hpp:20-44 maps the same torch dtypes). */
enum zt_dtype {
  ZT_DT_NONE = -1,
  ZT_DT_F32 = 0,
  ZT_DT_BF16 = 1,
  ZT_DT_F16 = 2,
  ZT_DT_S8 = 3,
  ZT_DT_U8 = 4,
  ZT_DT_S32 = 5
};

/* Post-op ids with the reference's numbering (src/cpu/cpp/Utils.hpp:56-71):
 * unary ops act on the running value, MUL/ADD combine it with the next
 * buffer, applied in list order (src/cpu/cpp/MatmulUtils.hpp:36-77). */
enum zt_post_op {
  ZT_PO_NONE = 0,
  ZT_PO_RELU = 1,
  ZT_PO_GELU_TANH = 2,
  ZT_PO_GELU_ERF = 3,
  ZT_PO_SILU = 4,
  ZT_PO_SIGMOID = 5,
  ZT_PO_TANH = 6,
  ZT_PO_MUL = 7,
  ZT_PO_ADD = 8
};

enum zt_status {
  ZT_OK = 0,
  ZT_EINVAL = 1,     /* bad argument (shape, dtype, null pointer) */
  ZT_EUNSUPPORTED = 2, /* valid request this build does not implement */
  ZT_EHIP = 3        /* a HIP runtime call failed */
};

#define ZT_MAX_POST_OPS 4

/* Fused epilogue: up to ZT_MAX_POST_OPS ops.  Binary buffers are [M, ld]
 * (row m at buf + m*ld elements) in bf16 or fp32. */
typedef struct zt_post_ops {
  int32_t count;
  int32_t ids[ZT_MAX_POST_OPS];
  const void *bufs[ZT_MAX_POST_OPS]; /* i-th binary op uses bufs[i-th binary] */
  int32_t buf_dtypes[ZT_MAX_POST_OPS];
  int64_t buf_ld[ZT_MAX_POST_OPS];
} zt_post_ops;

/*
 * int4 weight-only linear: y = post(x . dequant(W)^T + bias).
 *
 * Replaces zentorch_woq_linear_impl's matmul_direct call
 * (src/cpu/cpp/WOQ_Linear.cpp:14-112, call at :103-108) and, through the
 * post-op list, the _relu/_sigmoid/_gelu_tanh/_gelu_erf/_add/_mul_add/_add_add
 * wrappers (:178-292, registered :435-512).
 *
 *  x        [M, ldx] bf16 or fp32 activations (K used columns)
 *  w_packed [N, K/8] int32, row-major: the storage of the op's [K/8, N]
 *           transposed weight view; nibble i of word (n, c) is element
 *           (n, 8c+i), LSB first (WOQ_Linear.cpp:345-350)
 *  scales   [G, N] bf16 or fp32 (G = 1: per channel; K % G == 0)
 *  zp       [G, N] or NULL.  NULL: signed int4 (s4).  Otherwise unsigned
 *           int4 (u4, WOQ_Linear.cpp:47-49): a bf16/fp32 zp is the tinygemm
 *           float zero point, w = (u-8)*s + z; an s8/s32 zp gives w = (u-zp)*s
 *  bias     [N] bf16/fp32 or NULL
 *  y        [M, ldy] in y_dtype (bf16 or fp32)
 */
int zt_woq_linear(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                  int64_t ldx, const int32_t *w_packed, int64_t N,
                  const void *scales, int32_t scales_dtype, int64_t G,
                  const void *zp, int32_t zp_dtype, const void *bias,
                  int32_t bias_dtype, const zt_post_ops *post, void *y,
                  int32_t y_dtype, int64_t ldy, void *workspace,
                  size_t workspace_bytes, zt_stream_t stream);

/* Bytes of device workspace zt_woq_linear needs for these sizes.  Calls that
 * split K over several workgroups keep fp32 partials [splits][M][N] there
 * (no initial contents needed): 17..64 rows on large matrices (and from 4
 * rows where the decode kernels have no good layout for x, e.g. K = 11008
 * at 15-16 rows; a smaller workspace is refused for these), and prefill
 * calls whose row tiles make at most one round of the GPU (a smaller
 * workspace runs those unsplit); other sizes need none (0).  Calls that
 * overlap in time must not share a workspace. */
size_t zt_woq_linear_workspace_size(int64_t M, int64_t K, int64_t N,
                                    int64_t G);

/*
 * Merged gate_up int4 linear with the SiLU-and-mul epilogue.  No counterpart
 * in the reference: it is the merged-weight form of the extension
 * zentorch_woq_linear_silu_mul, for callers that hold the gate and up
 * projections as one [2I, K] weight (vLLM's merged gate_up + SiluAndMul).
 *   g = x . dequant(W[0:I])^T + bias[0:I]
 *   u = x . dequant(W[I:2I])^T + bias[I:2I]
 *   y[m][j] = silu(g[m][j]) * round_y(u[m][j]),   I = N/2
 * round_y rounds u to y_dtype first, so y equals the two-op composition
 * u = zt_woq_linear(x, W[I:2I]) then zt_woq_linear(x, W[0:I]) with the
 * post-ops {SILU, MUL u}.  Arguments as zt_woq_linear without post-ops;
 * N even, y [M, ldy] with N/2 columns.  Pass a workspace of
 * zt_woq_linear_gate_up_workspace_size(M, K, N, G) bytes on every call:
 * calls the fused kernels take (bf16 x and scales, no zero points, up to 64
 * rows, I % 16 == 0, x within the kernel's LDS, no K split) run as one
 * launch and leave it untouched; the others run the full linear into fp32
 * there, then the epilogue.
 */
int zt_woq_linear_gate_up(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                          int64_t ldx, const int32_t *w_packed, int64_t N,
                          const void *scales, int32_t scales_dtype, int64_t G,
                          const void *zp, int32_t zp_dtype, const void *bias,
                          int32_t bias_dtype, void *y, int32_t y_dtype, int64_t ldy,
                          void *workspace, size_t workspace_bytes, zt_stream_t stream);

size_t zt_woq_linear_gate_up_workspace_size(int64_t M, int64_t K, int64_t N,
                                            int64_t G);

/*
 * Dynamic int8 linear: per-token symmetric s8 quantisation of x inside the
 * op, int8 x int8 -> int32 GEMM, y = acc * sx[m] * sw[n] + bias[n].
 *
 * Replaces zentorch_dynamic_qlinear_impl's matmul_direct(dynamic_quant)
 * (src/cpu/cpp/DynamicQLinear.cpp:74-135, call at :124-129).
 *
 *  x        [M, K] bf16 or fp32, contiguous (DynamicQLinear.cpp:160-162)
 *  w        [N, K] int8 row-major (transB=true, ldb=K, :124-126)
 *  w_scales [N] fp32 or bf16 per output channel
 *  bias     [N] fp32/bf16 or NULL
 *  post     NULL for the reference op (it has no post-ops,
 *           docs/zentorch_dynamic_qlinear.md:99); non-NULL is an extension
 *  y        [M, N] in y_dtype
 *  workspace: zt_dynamic_qlinear_workspace_size(M, K, N) bytes.  Its first
 *           part holds the quantised activations and row scales; the rest
 *           holds the exchange of the split-K GEMM (64 < M <= 128,
 *           K % 256 == 0) or, past 128 rows when the tiled GEMM's tiles make
 *           less than one round, its int32 K-split partials.  A workspace
 *           holding only the first part (zt_dynamic_qlinear_workspace_size(M,
 *           K, 0)) is accepted and runs the unsplit kernels, with the same
 *           results.
 */
int zt_dynamic_qlinear(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                       const int8_t *w, int64_t N, const void *w_scales,
                       int32_t w_scales_dtype, const void *bias,
                       int32_t bias_dtype, const zt_post_ops *post, void *y,
                       int32_t y_dtype, void *workspace, size_t workspace_bytes,
                       zt_stream_t stream);

size_t zt_dynamic_qlinear_workspace_size(int64_t M, int64_t K, int64_t N);

/*
 * zt_dynamic_qlinear without a workspace argument: allocates nothing.  No
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP-graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The quantised activations and row
 * scales go to a scratch array of ZT_DYN_SCRATCH_BYTES that each GPU holds
 * from the first call on it until the process ends, so a call is limited to
 * zt_dynamic_qlinear_workspace_size(M, K, 0) <= ZT_DYN_SCRATCH_BYTES (about
 * M * K <= 32 Mi; larger calls return ZT_EINVAL and launch nothing); the
 * split-K exchange uses the rest of the array when it fits.  Every
 * call on one GPU shares that GPU's array: calls that overlap in time on one
 * GPU (different streams, or threads without ordering) race and must not be
 * issued.  Nothing in the scratch needs to start at zero; it keeps the last
 * call's contents.  Results equal zt_dynamic_qlinear's bit for bit (the same
 * kernels).  The call uses the array of the stream's device (the null stream:
 * the current device), making that device current for the call and
 * restoring the caller's current device afterwards.
 */
#define ZT_DYN_SCRATCH_BYTES (32u << 20)

int zt_dynamic_qlinear_scratch(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                               const int8_t *w, int64_t N, const void *w_scales,
                               int32_t w_scales_dtype, const void *bias, int32_t bias_dtype,
                               const zt_post_ops *post, void *y, int32_t y_dtype,
                               zt_stream_t stream);

/* ZT_DYN_SCRATCH_BYTES, for callers that bind the library at run time. */
size_t zt_dynamic_qlinear_scratch_max(void);

/*
 * The quantisation stage of zt_dynamic_qlinear on its own (same kernel):
 * qx[M, K] int8 and sx[M] fp32, sx = max(amax_k|x|, 1e-12)/127,
 * qx = clamp(round_half_even(x/sx), -128, 127).  Exposes what ZenDNNL
 * computes inside matmul_direct (DynamicQLinear.cpp:100-110) so it can be
 * checked bit for bit.
 */
int zt_dynamic_quantize(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                        int8_t *qx, float *sx, zt_stream_t stream);

/*
 * The GEMM stage of zt_dynamic_qlinear on its own (same kernels, int32
 * epilogue): acc[M, N] = qa[M, K] . w[N, K]^T exactly in int32.
 */
int zt_s8s8s32_gemm(const int8_t *qa, const int8_t *w, int64_t M, int64_t N,
                    int64_t K, int32_t *acc, zt_stream_t stream);

/*
 * Dynamic int8 linear with per-token ASYMMETRIC uint8 activations.  No
 * counterpart in the reference, whose dynamic qlinear is symmetric s8
 * (DynamicQLinear.cpp:94-110); this is an opt-in for callers whose
 * activations are one-signed (after SiLU / GELU / ReLU), where a zero point
 * spends all 256 levels on the row's range.  Per row m:
 *   lo = min(0, min_k x), hi = max(0, max_k x),
 *   sx = max(hi - lo, 1e-12) / 255, zp = clamp(rint(-lo / sx), 0, 255),
 *   q  = clamp(rint(x / sx) + zp, 0, 255)       (fp32, rint half-to-even)
 *   y  = (float)(sum_k (q - zp) * w[n][k]) * sx * sw[n] + bias[n]
 * The GEMM runs on q - 128 stored as s8 (the symmetric kernels unchanged)
 * and the epilogue subtracts (zp - 128) * w_colsum[n] from each int32
 * accumulator, which is exact.
 *
 *  w_colsum  [N] int32, sum_k w[n][k] (zt_s8_weight_colsum), 16-byte aligned;
 *            computed once per weight and kept beside it
 *  y_dtype   bf16 / fp32, or ZT_DT_S32 for the corrected accumulators
 *            sum_k (q - zp) * w exactly (no scales, bias or post-ops)
 *  workspace zt_dynamic_qlinear_asym_workspace_size(M, K, N) bytes (as for
 *            zt_dynamic_qlinear: N = 0 gives the least that is accepted)
 * Other arguments as zt_dynamic_qlinear.
 */
int zt_dynamic_qlinear_asym(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                            const int8_t *w, int64_t N, const void *w_scales,
                            int32_t w_scales_dtype, const int32_t *w_colsum,
                            const void *bias, int32_t bias_dtype, const zt_post_ops *post,
                            void *y, int32_t y_dtype, void *workspace,
                            size_t workspace_bytes, zt_stream_t stream);

size_t zt_dynamic_qlinear_asym_workspace_size(int64_t M, int64_t K, int64_t N);

/* The asymmetric quantisation stage on its own (same kernel): qx[M, K] =
 * q - 128 as int8, sx[M] fp32, azp[M] = zp - 128 int32.  No reference
 * counterpart (extension above). */
int zt_dynamic_quantize_asym(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                             int8_t *qx, float *sx, int32_t *azp, zt_stream_t stream);

/*
 * Static int8 linear: per-tensor quantisation of x with a given scale (and
 * zero point), int8 x int8 -> int32 GEMM, y = acc * x_scale * w_scale[n] +
 * bias[n], post-ops, then a float output or one requantised to u8 / s8.
 *
 * Replaces zendnnl_quantized_matmul_impl (src/cpu/cpp/QLinear.cpp:66-347)
 * behind zentorch_qlinear / _relu / _sigmoid / _mul_add and the .out forms
 * (QLinear.cpp:367-521, schemas :525-573).
 *
 *  x             [M, K]: fp32 / bf16 (quantised here, QLinear.cpp:118-157),
 *                or already quantised s8 / u8 (:113-116)
 *  x_scale       device fp32 scalar; q = clamp(rint(x * (1 / x_scale)) + zp)
 *  x_zero_point  device int32 scalar or NULL.  Given: u8 activations over
 *                [0, 255] (QLinear.cpp:16-22).  NULL: symmetric s8 over
 *                [-128, 127].  acc = sum_k (q - zp) * w.
 *  w             [N, K] int8 row-major (the op's weight, used as weight.t())
 *  w_scales      fp32, 1 (per tensor) or N (per channel) entries
 *  w_colsum      [N] int32 sum_k w[n][k], 16-byte aligned; required when x is
 *                u8 or x_zero_point is given, ignored otherwise
 *  post          relu / sigmoid / mul + add (QLinear.cpp:367-521), or NULL
 *  y             y_dtype fp32 / bf16 without y_scale; with y_scale (device
 *                fp32 scalar) u8 when y_zero_point (device int32) is given
 *                and s8 when not, y = clamp(rint(v * (1 / y_scale)) + zp)
 *                (the reference scales by 1 / output_scales, QLinear.cpp:163-166).
 *  workspace     zt_qlinear_workspace_size(M, K, N) bytes (N = 0: the least
 *                that is accepted, without the split-K exchange)
 * Weight zero points are not an argument: the reference's matmul path leaves
 * them unused (QLinear.cpp:248-262), so weights are symmetric.
 */
int zt_qlinear(const void *x, int32_t x_dtype, int64_t M, int64_t K, const float *x_scale,
               const int32_t *x_zero_point, const int8_t *w, int64_t N, const float *w_scales,
               int64_t n_w_scales, const int32_t *w_colsum, const void *bias,
               int32_t bias_dtype, const zt_post_ops *post, void *y, int32_t y_dtype,
               const float *y_scale, const int32_t *y_zero_point, void *workspace,
               size_t workspace_bytes, zt_stream_t stream);

size_t zt_qlinear_workspace_size(int64_t M, int64_t K, int64_t N);

/* colsum[n] = sum_k w[n][k] of an int8 [N, K] row-major weight, exactly in
 * int32.  No reference counterpart (extension above). */
int zt_s8_weight_colsum(const int8_t *w, int64_t N, int64_t K, int32_t *colsum,
                        zt_stream_t stream);

/* Repack int8 [N, K] int4 values into int32 [N, K/8] on the GPU.
 * Replaces zentorch_woq_repack_weight (src/cpu/cpp/WOQ_Linear.cpp:294-357). */
int zt_woq_repack_weight(const int8_t *w, int64_t N, int64_t K, int32_t *out,
                         zt_stream_t stream);

/* torch CPU int4pack uint8 [N, K/2] -> int32 [N, K/8] on the GPU.
 * Replaces zentorch_woq_repack_from_int4pack (WOQ_Linear.cpp:361-433). */
int zt_woq_repack_from_int4pack(const uint8_t *packed, int64_t N, int64_t K,
                                int32_t *out, zt_stream_t stream);

/*
 * Grouped int4 weight-only mixture of experts: for every token t and each
 * of its topk experts e = topk_ids[t, k],
 *   h = act(x[t] . dq(w13[e, :I])^T + b13[e, :I]) * (x[t] . dq(w13[e, I:])^T + b13[e, I:])
 *   y = h . dq(w2[e])^T + b2[e]                      (h and y rounded to bf16)
 *   out[t] = sum_k topk_weights[t, k] * y            (fp32, k in order; all
 *                                                     weights 1 if skip_weighted)
 * Replaces zentorch_fused_moe (src/cpu/cpp/FusedMoE.cpp:443-700, schema
 * :728-736) for int4-packed expert weights (the reference takes bf16 or int8
 * experts); pairs whose id is outside [0, E) are dropped, as the reference's
 * expert-parallel path drops remote ids (vllm/_int8_moe_patch.py:170-180).
 *
 *  x            [T, H] bf16;  out [T, H] bf16 (overwritten)
 *  topk_ids     [T, topk] int32;  topk_weights [T, topk] fp32 or bf16
 *  act          ZT_PO_SILU, ZT_PO_GELU_ERF or ZT_PO_GELU_TANH
 *  w13          [E, 2I, H/8] int32 packed int4 (zt_woq_repack_weight per
 *               expert), w13_scales [E, G13, 2I] bf16, w13_bias [E, 2I] bf16
 *               or NULL
 *  w2           [E, H, I/8], w2_scales [E, G2, H] bf16, w2_bias [E, H] or NULL
 *  H, I multiples of 128; group sizes H/G13, I/G2 multiples of 128 (or one
 *  group), powers of two times 128.  E <= 1024.
 *  workspace    zt_woq_moe_workspace_size(T, H, topk, E, I) bytes; no host
 *               synchronisation (the routing runs on the GPU).
 */
int zt_woq_moe(const void *x, int64_t T, int64_t H, const int32_t *topk_ids,
               const void *topk_weights, int32_t weights_dtype, int64_t topk,
               int32_t skip_weighted, int32_t act, const int32_t *w13,
               const void *w13_scales, int64_t G13, const void *w13_bias,
               const int32_t *w2, const void *w2_scales, int64_t G2,
               const void *w2_bias, int64_t E, int64_t I, void *out,
               void *workspace, size_t workspace_bytes, zt_stream_t stream);

size_t zt_woq_moe_workspace_size(int64_t T, int64_t H, int64_t topk, int64_t E,
                                 int64_t I);

/* Message of the calling thread's last failed call ("" if none). */
const char *zt_last_error_string(void);

/*
 * Kernel-selection overrides, for tests and tuning.  No counterpart in the
 * reference (its EnvReader, src/cpu/cpp/EnvReader.hpp, reads ZenDNN's own
 * variables on every call).  Each knob is named after the environment
 * variable that sets it when the library is loaded (ZT_WOQ_FORCE_KERNEL,
 * ZT_WOQ_DECODE_PLAN, ZT_WOQ_STREAM, ZT_WOQ_WIDE, ZT_WOQ_GEMM, ZT_WOQ_DEBUG,
 * ZT_WOQ_WAVE, ZT_WOQ_PERSIST, ZT_S8_SKINNY32, ZT_S8_SKINNY, ZT_S8_FRAG, ZT_S8_FORCE,
 * ZT_S8_TILE, ZT_S8_KIND, ZT_S8_SPLIT, ZT_MOE_BN, ZT_WOQ_LEAN, ZT_S8_FUSED); the environment is not
 * read again.  value NULL or
 * "" unsets the knob.  Returns ZT_EINVAL for an unknown name.  Launches
 * already enqueued are not affected.
 */
int zt_set_tuning(const char *name, const char *value);

/* Current value of a knob (NULL if unset or unknown). */
const char *zt_get_tuning(const char *name);

/* Library ABI version (major*10000 + minor*100 + patch). */
int32_t zt_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ZENTORCH_HIP_H */
