/*
 * zt_oracle.c -- CPU restatement of zentorch's quantized-linear semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels in
 * zendnn-pytorch-plugin_amd/csrc.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never calls it
 * (the torch ops have no CPU kernel and fail loudly without the HIP library).
 *
 * What each function restates (paths relative to the reference checkout):
 *   zto_woq_repack_weight   src/cpu/cpp/WOQ_Linear.cpp:294-357 (LSB-first, 8
 *                           nibbles per int32, order_map is the identity :326)
 *   zto_unpack_int4pack     src/cpu/cpp/WOQ_Linear.cpp:361-428 (torch CPU
 *                           int4pack, BLOCK_N=64, 16x4 interleave)
 *   zto_woq_linear          src/cpu/cpp/WOQ_Linear.cpp:14-176 (matmul_direct
 *                           with s4/u4 weights, [G,N] scales, optional zp),
 *                           post-ops in list order MatmulUtils.hpp:36-77,
 *                           post-op ids Utils.hpp:56-71.  Numerics follow the
 *                           reference's own test reference
 *                           test/unittests/op_tests/test_woq_linear.py:118-128:
 *                           dequantised weight rounded to the input dtype,
 *                           fp32 accumulation, one rounding of the output.
 *   zto_dynamic_quantize    test/unittests/op_tests/test_dynamic_qlinear.py:32-36
 *                           and DynamicQLinear.cpp:94-110: per-token symmetric
 *                           s8, scale = max(amax,1e-12)/127 (fp32 IEEE divide),
 *                           q = clamp(round_half_even(x/scale), -128, 127).
 *   zto_s8s8s32_gemm        exact int32 accumulation of DynamicQLinear.cpp:124-129
 *                           (compute=s8, transB=true, ldb=K).
 *   zto_dynamic_qlinear     DynamicQLinear.cpp:74-181: y = acc*sx[m]*sw[n] + b[n]
 *                           in fp32, rounded once to the output dtype.
 *   zto_dynamic_quantize_asym, zto_dynamic_qlinear_asym
 *                           no reference counterpart: the per-token
 *                           asymmetric-uint8 opt-in beside the reference's
 *                           symmetric s8 (DynamicQLinear.cpp:94-110); the
 *                           epilogue is zto_dynamic_qlinear's with
 *                           acc = sum_k (q - zp) * w.  Parity unpinned by the
 *                           reference (no golden data exists); pinned by the
 *                           round-trip, zero-point and range identities the
 *                           CPU tests check.
 *   zto_qlinear             QLinear.cpp:66-347 (zentorch_qlinear*): per-tensor
 *                           input quantisation q = clamp(rint(x * (1/s)) + zp)
 *                           over u8 with a zero point (QLinear.cpp:16-22,
 *                           :139-149) or s8 without; s8/u8 inputs as given;
 *                           acc = sum_k (q - zp) * w exactly; y = acc * s_x *
 *                           s_w[n] + b[n]; post-ops; output float, or
 *                           clamp(rint(y * (1/s_out)) + zp_out) in u8 (zero
 *                           point given) / s8 (:163-166, validators
 *                           MatmulUtils.hpp:325-433).
 *   zto_woq_moe             FusedMoE.cpp:443-700 and the per-expert loop of
 *                           vllm/_int8_moe_patch.py:149-206 with int4 expert
 *                           weights: per (token, k) pair of expert e,
 *                           gate/up = zto_woq_linear (fp32), h = bf16(act(gate)
 *                           * up), y = bf16(zto_woq_linear(h) + b2), out[t] =
 *                           bf16(sum_k w[t,k] * y) in fp32, k ascending; ids
 *                           outside [0, E) are dropped.
 *
 * Where the reference leaves numerics to ZenDNNL (accumulation order, the
 * rounding of the dequantised weight, the u4 zero-point convention) the
 * choice made here is stated at the function.  Compiled with
 * -ffp-contract=off so a*b+c is always two roundings.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* dtype codes shared with include/zentorch_hip.h */
enum { ZT_DT_NONE = -1, ZT_DT_F32 = 0, ZT_DT_BF16 = 1, ZT_DT_F16 = 2,
       ZT_DT_S8 = 3, ZT_DT_U8 = 4, ZT_DT_S32 = 5 };
/* post-op ids: same numbering as the reference's UNARY_POST_OP/BINARY_POST_OP
 * (src/cpu/cpp/Utils.hpp:56-71) */
enum { PO_NONE = 0, PO_RELU = 1, PO_GELU_TANH = 2, PO_GELU_ERF = 3,
       PO_SILU = 4, PO_SIGMOID = 5, PO_TANH = 6, PO_MUL = 7, PO_ADD = 8 };

#define ZTO_OK 0
#define ZTO_EINVAL 1

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE round-to-nearest-even fp32 -> bf16; NaN stays NaN (quiet). */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float round_to_dtype(float v, int dt) {
  if (dt == ZT_DT_BF16) return bf16_to_f32(f32_to_bf16(v));
  return v;
}

static inline float load_f(const void *p, int dt, int64_t i) {
  switch (dt) {
  case ZT_DT_F32: return ((const float *)p)[i];
  case ZT_DT_BF16: return bf16_to_f32(((const uint16_t *)p)[i]);
  case ZT_DT_S8: return (float)((const int8_t *)p)[i];
  case ZT_DT_U8: return (float)((const uint8_t *)p)[i];
  case ZT_DT_S32: return (float)((const int32_t *)p)[i];
  default: return 0.f;
  }
}

static inline void store_f(void *p, int dt, int64_t i, float v) {
  if (dt == ZT_DT_F32) ((float *)p)[i] = v;
  else ((uint16_t *)p)[i] = f32_to_bf16(v);
}

static inline float unary(int id, float v) {
  switch (id) {
  case PO_RELU: return v > 0.f ? v : 0.f;
  case PO_GELU_TANH: {
    const float k0 = 0.7978845608028654f; /* sqrt(2/pi) */
    return 0.5f * v * (1.f + tanhf(k0 * (v + 0.044715f * v * v * v)));
  }
  case PO_GELU_ERF: return 0.5f * v * (1.f + erff(v * 0.7071067811865476f));
  case PO_SILU: return v / (1.f + expf(-v));
  case PO_SIGMOID: return 1.f / (1.f + expf(-v));
  case PO_TANH: return tanhf(v);
  default: return v;
  }
}

/* Post-ops are applied in list order; a binary op consumes the next buffer
 * (MatmulUtils.hpp:62-76).  Buffers are [M, ld] in their own dtype. */
static inline float apply_post_ops(float v, int n_post, const int *ids,
                                   const void *const *bufs, const int *dts,
                                   const int64_t *lds, int64_t m, int64_t n) {
  int b = 0;
  for (int i = 0; i < n_post; ++i) {
    int id = ids[i];
    if (id == PO_ADD || id == PO_MUL) {
      float o = load_f(bufs[b], dts[b], m * lds[b] + n);
      ++b;
      v = (id == PO_ADD) ? v + o : v * o;
    } else {
      v = unary(id, v);
    }
  }
  return v;
}

static void set_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
}

int zto_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ A1 */
/* WOQ_Linear.cpp:294-357: word[n][c] = sum_i (w[n][8c+i] & 0xF) << 4i. */
int zto_woq_repack_weight(const int8_t *w, int64_t N, int64_t K, int32_t *out) {
  if (K < 8 || K % 8 != 0 || N < 0) return ZTO_EINVAL;
  const int64_t KW = K / 8;
  for (int64_t n = 0; n < N; ++n) {
    const int8_t *src = w + n * K;
    for (int64_t c = 0; c < KW; ++c) {
      uint32_t word = 0;
      for (int i = 0; i < 8; ++i)
        word |= ((uint32_t)(uint8_t)src[8 * c + i] & 0xFu) << (4 * i);
      out[n * KW + c] = (int32_t)word;
    }
  }
  return ZTO_OK;
}

/* ------------------------------------------------------------------ A2 */
/* WOQ_Linear.cpp:361-428.  packed: uint8 [N, K/2] in torch's CPU int4pack
 * layout; out: int8 [N, K] holding the unsigned nibble (0..15). */
int zto_unpack_int4pack(const uint8_t *packed, int64_t N, int64_t K,
                        int8_t *out) {
  const int BLOCK_N = 64;
  if (N % BLOCK_N != 0 || K % 2 != 0) return ZTO_EINVAL;
  for (int64_t nb = 0; nb < N / BLOCK_N; ++nb) {
    const uint8_t *src = packed + nb * K * BLOCK_N / 2;
    int8_t *dst = out + nb * BLOCK_N * K;
    for (int64_t k = 0; k < K; ++k) {
      for (int d = 0; d < 16; ++d) {
        uint8_t p02 = src[k * 32 + d];
        uint8_t p13 = src[k * 32 + 16 + d];
        dst[(d + 0) * K + k] = (int8_t)(p02 & 0xF);
        dst[(d + 16) * K + k] = (int8_t)(p13 & 0xF);
        dst[(d + 32) * K + k] = (int8_t)((p02 >> 4) & 0xF);
        dst[(d + 48) * K + k] = (int8_t)((p13 >> 4) & 0xF);
      }
    }
  }
  return ZTO_OK;
}

/* ------------------------------------------------------------- A3-A5 */
/* Dequantised weight element (n, k):
 *   no zero points (s4, WOQ_Linear.cpp:47-49): q = signed nibble, w = q*s
 *   floating zero points (u4): tinygemm convention w = (u-8)*s + z, the
 *     convention of aten._weight_int4pack_mm_for_cpu that the reference's
 *     asymmetric test compares against (test_woq_linear_asymmetric.py:28-42)
 *   integer zero points (u4): w = (u - zp)*s
 * then rounded to the compute (= input) dtype, as the reference test does
 * with dq_weight.to(bfloat16) (test_woq_linear.py:121,127). */
static inline float woq_dequant(uint32_t nib, float s, const void *zp,
                                int zp_dt, int64_t zidx, int compute_dt) {
  float w;
  if (!zp) {
    int q = (int)(nib ^ 8u) - 8; /* sign-extend 4 bits */
    w = (float)q * s;
  } else if (zp_dt == ZT_DT_F32 || zp_dt == ZT_DT_BF16) {
    float z = load_f(zp, zp_dt, zidx);
    w = (float)((int)nib - 8) * s;
    w = w + z;
  } else {
    float z = load_f(zp, zp_dt, zidx);
    w = ((float)nib - z) * s;
  }
  return round_to_dtype(w, compute_dt);
}

/* x: [M, ldx] in x_dt (bf16/fp32); wpk: [N, K/8] int32 (the storage of the
 * [K/8, N] transposed view the op receives); scales/zp: [G, N]; bias: [N];
 * y: [M, ldy] in y_dt.  Accumulates each output in fp32, k ascending. */
int zto_woq_linear(const void *x, int x_dt, int64_t M, int64_t K, int64_t ldx,
                   const int32_t *wpk, int64_t N, const void *scales, int s_dt,
                   int64_t G, const void *zp, int zp_dt, const void *bias,
                   int b_dt, int n_post, const int *post_ids,
                   const void *const *post_bufs, const int *post_dts,
                   const int64_t *post_lds, void *y, int y_dt, int64_t ldy,
                   int nthreads) {
  if (K % 8 != 0 || G <= 0 || K % G != 0) return ZTO_EINVAL;
  const int64_t KW = K / 8, gs = K / G;
  set_threads(nthreads);
  int err = 0;
#pragma omp parallel
  {
    const int NB = 16;
    float *wdq = (float *)malloc(sizeof(float) * (size_t)K * NB);
    float *xr = (float *)malloc(sizeof(float) * (size_t)K);
    if (!wdq || !xr) {
#pragma omp atomic write
      err = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t n0 = 0; n0 < N; n0 += NB) {
        const int nb = (int)((N - n0) < NB ? (N - n0) : NB);
        /* dequantise a [K, nb] block, k-major so the inner loop runs over n */
        for (int j = 0; j < nb; ++j) {
          const int64_t n = n0 + j;
          for (int64_t c = 0; c < KW; ++c) {
            uint32_t word = (uint32_t)wpk[n * KW + c];
            for (int i = 0; i < 8; ++i) {
              int64_t k = 8 * c + i;
              int64_t sidx = (k / gs) * N + n;
              float s = load_f(scales, s_dt, sidx);
              wdq[k * NB + j] = woq_dequant((word >> (4 * i)) & 0xFu, s, zp,
                                            zp_dt, sidx, x_dt);
            }
          }
        }
        for (int64_t m = 0; m < M; ++m) {
          float acc[16];
          for (int j = 0; j < NB; ++j) acc[j] = 0.f;
          for (int64_t k = 0; k < K; ++k) xr[k] = load_f(x, x_dt, m * ldx + k);
          for (int64_t k = 0; k < K; ++k) {
            const float xv = xr[k];
            const float *wr = wdq + k * NB;
            for (int j = 0; j < NB; ++j) acc[j] += xv * wr[j];
          }
          for (int j = 0; j < nb; ++j) {
            const int64_t n = n0 + j;
            float v = acc[j];
            if (bias) v = v + load_f(bias, b_dt, n);
            v = apply_post_ops(v, n_post, post_ids, post_bufs, post_dts,
                               post_lds, m, n);
            store_f(y, y_dt, m * ldy + n, v);
          }
        }
      }
    }
    free(wdq);
    free(xr);
  }
  return err ? ZTO_EINVAL : ZTO_OK;
}

/* ------------------------------------------------------------------ A6 */
/* Per-token symmetric s8 quantisation.  All arithmetic in fp32 after the
 * exact bf16->fp32 widening:
 *   amax = max_k |x[m,k]|; sx = max(amax, 1e-12f) / 127.0f  (IEEE divide)
 *   q = clamp(rint(x / sx), -128, 127)   (rint: round half to even) */
int zto_dynamic_quantize(const void *x, int x_dt, int64_t M, int64_t K,
                         int8_t *qx, float *sx, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      float v = fabsf(load_f(x, x_dt, m * K + k));
      amax = v > amax ? v : amax;
    }
    if (!(amax >= 1e-12f)) amax = 1e-12f;
    const float s = amax / 127.0f;
    sx[m] = s;
    for (int64_t k = 0; k < K; ++k) {
      float r = rintf(load_f(x, x_dt, m * K + k) / s);
      r = r < -128.f ? -128.f : (r > 127.f ? 127.f : r);
      qx[m * K + k] = (int8_t)r;
    }
  }
  return ZTO_OK;
}

/* acc[m,n] = sum_k qa[m,k] * w[n,k], exact in int32 (w is [N,K] row-major,
 * the transB=true / ldb=K layout of DynamicQLinear.cpp:124-126). */
int zto_s8s8s32_gemm(const int8_t *qa, const int8_t *w, int64_t M, int64_t N,
                     int64_t K, int32_t *acc, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const int8_t *wr = w + n * K;
    for (int64_t m = 0; m < M; ++m) {
      const int8_t *ar = qa + m * K;
      int32_t s = 0;
      for (int64_t k = 0; k < K; ++k) s += (int32_t)ar[k] * (int32_t)wr[k];
      acc[m * N + n] = s;
    }
  }
  return ZTO_OK;
}

/* Full op: quantise, exact int32 GEMM, then y = ((float)acc*sx[m])*sw[n] + b[n]
 * with the post-ops (an extension; the reference op has none) and one
 * rounding to y_dt.  Returns qx/sx/acc through the optional out pointers. */
int zto_dynamic_qlinear(const void *x, int x_dt, int64_t M, int64_t K,
                        const int8_t *w, int64_t N, const void *sw, int sw_dt,
                        const void *bias, int b_dt, int n_post,
                        const int *post_ids, const void *const *post_bufs,
                        const int *post_dts, const int64_t *post_lds, void *y,
                        int y_dt, int8_t *qx_out, float *sx_out,
                        int32_t *acc_out, int nthreads) {
  int8_t *qx = qx_out ? qx_out : (int8_t *)malloc((size_t)(M * K > 0 ? M * K : 1));
  float *sx = sx_out ? sx_out : (float *)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1));
  int32_t *acc = acc_out ? acc_out
                         : (int32_t *)malloc(sizeof(int32_t) * (size_t)(M * N > 0 ? M * N : 1));
  if (!qx || !sx || !acc) return ZTO_EINVAL;
  zto_dynamic_quantize(x, x_dt, M, K, qx, sx, nthreads);
  zto_s8s8s32_gemm(qx, w, M, N, K, acc, nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float v = (float)acc[m * N + n] * sx[m];
      v = v * load_f(sw, sw_dt, n);
      if (bias) v = v + load_f(bias, b_dt, n);
      v = apply_post_ops(v, n_post, post_ids, post_bufs, post_dts, post_lds, m, n);
      store_f(y, y_dt, m * N + n, v);
    }
  }
  if (!qx_out) free(qx);
  if (!sx_out) free(sx);
  if (!acc_out) free(acc);
  return ZTO_OK;
}

/* Per-token asymmetric uint8 (extension).  fp32 after the exact widening:
 *   lo = min(0, min_k x), hi = max(0, max_k x)
 *   sx = max(hi - lo, 1e-12f) / 255.0f              (IEEE divide)
 *   zp = clamp(rint(-lo / sx), 0, 255)
 *   q  = clamp(rint(x / sx) + zp, 0, 255)           (rint: half to even) */
int zto_dynamic_quantize_asym(const void *x, int x_dt, int64_t M, int64_t K,
                              uint8_t *q, float *sx, int32_t *zp, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float lo = 0.f, hi = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      const float v = load_f(x, x_dt, m * K + k);
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
    }
    float range = hi - lo;
    if (!(range >= 1e-12f)) range = 1e-12f;
    const float s = range / 255.0f;
    float z = rintf(-lo / s);
    z = z < 0.f ? 0.f : (z > 255.f ? 255.f : z);
    sx[m] = s;
    zp[m] = (int32_t)z;
    for (int64_t k = 0; k < K; ++k) {
      float r = rintf(load_f(x, x_dt, m * K + k) / s) + z;
      r = r < 0.f ? 0.f : (r > 255.f ? 255.f : r);
      q[m * K + k] = (uint8_t)r;
    }
  }
  return ZTO_OK;
}

/* y = ((float)acc * sx[m]) * sw[n] + b[n] with acc = sum_k (q - zp[m]) *
 * w[n,k] exactly (int64, then int32: |acc| < 2^31 for K < 2^16); y_dt
 * ZT_DT_S32 stores acc itself.  q/sx/zp go to the optional out pointers. */
int zto_dynamic_qlinear_asym(const void *x, int x_dt, int64_t M, int64_t K,
                             const int8_t *w, int64_t N, const void *sw, int sw_dt,
                             const void *bias, int b_dt, void *y, int y_dt,
                             uint8_t *q_out, float *sx_out, int32_t *zp_out, int nthreads) {
  uint8_t *q = q_out ? q_out : (uint8_t *)malloc((size_t)(M * K > 0 ? M * K : 1));
  float *sx = sx_out ? sx_out : (float *)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1));
  int32_t *zp = zp_out ? zp_out : (int32_t *)malloc(sizeof(int32_t) * (size_t)(M > 0 ? M : 1));
  if (!q || !sx || !zp) return ZTO_EINVAL;
  zto_dynamic_quantize_asym(x, x_dt, M, K, q, sx, zp, nthreads);
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      int64_t a = 0;
      for (int64_t k = 0; k < K; ++k)
        a += ((int64_t)q[m * K + k] - zp[m]) * (int64_t)w[n * K + k];
      const int32_t acc = (int32_t)a;
      if (y_dt == ZT_DT_S32) {
        ((int32_t *)y)[m * N + n] = acc;
        continue;
      }
      float v = (float)acc * sx[m];
      v = v * load_f(sw, sw_dt, n);
      if (bias) v = v + load_f(bias, b_dt, n);
      store_f(y, y_dt, m * N + n, v);
    }
  }
  if (!q_out) free(q);
  if (!sx_out) free(sx);
  if (!zp_out) free(zp);
  return ZTO_OK;
}

/* ------------------------------------------------------------ (f)4 */
/* Static int8 linear.  x_dt f32/bf16/s8/u8; w_scales 1 or N fp32; y_dt
 * f32/bf16 (has_y_scale = 0) or u8/s8 (requantised). */
int zto_qlinear(const void *x, int x_dt, int64_t M, int64_t K, float x_scale, int has_x_zp,
                int32_t x_zp, const int8_t *w, int64_t N, const float *w_scales,
                int64_t n_w_scales, const void *bias, int b_dt, int n_post,
                const int *post_ids, const void *const *post_bufs, const int *post_dts,
                const int64_t *post_lds, void *y, int y_dt, int has_y_scale, float y_scale,
                int has_y_zp, int32_t y_zp, int nthreads) {
  int32_t *q = (int32_t *)malloc(sizeof(int32_t) * (size_t)(M * K > 0 ? M * K : 1));
  if (!q) return ZTO_EINVAL;
  const int32_t off = has_x_zp ? x_zp : 0;
  const float inv = 1.0f / x_scale;
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * K; ++i) {
    if (x_dt == ZT_DT_S8) {
      q[i] = ((const int8_t *)x)[i];
    } else if (x_dt == ZT_DT_U8) {
      q[i] = ((const uint8_t *)x)[i];
    } else {
      float r = rintf(load_f(x, x_dt, i) * inv);
      if (has_x_zp) {
        r += (float)x_zp;
        r = r < 0.f ? 0.f : (r > 255.f ? 255.f : r);
      } else {
        r = r < -128.f ? -128.f : (r > 127.f ? 127.f : r);
      }
      q[i] = (int32_t)r;
    }
  }
  const float inv_y = has_y_scale ? 1.0f / y_scale : 0.f;
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      int64_t a = 0;
      for (int64_t k = 0; k < K; ++k)
        a += (int64_t)(q[m * K + k] - off) * (int64_t)w[n * K + k];
      float v = (float)(int32_t)a * x_scale;
      v = v * w_scales[n_w_scales == 1 ? 0 : n];
      if (bias) v = v + load_f(bias, b_dt, n);
      v = apply_post_ops(v, n_post, post_ids, post_bufs, post_dts, post_lds, m, n);
      if (has_y_scale) {
        float r = rintf(v * inv_y) + (has_y_zp ? (float)y_zp : 0.f);
        if (y_dt == ZT_DT_U8)
          ((uint8_t *)y)[m * N + n] = (uint8_t)(r < 0.f ? 0.f : (r > 255.f ? 255.f : r));
        else
          ((int8_t *)y)[m * N + n] = (int8_t)(r < -128.f ? -128.f : (r > 127.f ? 127.f : r));
      } else {
        store_f(y, y_dt, m * N + n, v);
      }
    }
  }
  free(q);
  return ZTO_OK;
}

/* ------------------------------------------------------------------ MoE */
/* x [T, H] bf16; ids [T, topk] int32; wts [T, topk] (wts_dt); w13 [E, 2I,
 * H/8] packed; s13 [E, G13, 2I] bf16; b13 [E, 2I] bf16 or NULL; w2 [E, H,
 * I/8]; s2 [E, G2, H]; b2 [E, H] or NULL; out [T, H] bf16. */
int zto_woq_moe(const uint16_t *x, int64_t T, int64_t H, const int32_t *ids,
                const void *wts, int wts_dt, int64_t topk, int skip_weighted,
                int act, const int32_t *w13, const uint16_t *s13, int64_t G13,
                const uint16_t *b13, const int32_t *w2, const uint16_t *s2,
                int64_t G2, const uint16_t *b2, int64_t E, int64_t I,
                uint16_t *out, int nthreads) {
  const int64_t P = T * topk;
  float *acc = (float *)calloc((size_t)T * H, sizeof(float));
  uint16_t *xe = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(P > 0 ? P : 1) * H);
  int64_t *pe = (int64_t *)malloc(sizeof(int64_t) * (size_t)(P > 0 ? P : 1));
  float *gu = (float *)malloc(sizeof(float) * (size_t)(P > 0 ? P : 1) * 2 * I);
  uint16_t *h = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(P > 0 ? P : 1) * I);
  uint16_t *y = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(P > 0 ? P : 1) * H);
  int rc = ZTO_OK;
  if (!acc || !xe || !pe || !gu || !h || !y) rc = ZTO_EINVAL;
  float *yfull = rc == ZTO_OK ? (float *)malloc(sizeof(float) * (size_t)(P > 0 ? P : 1) * H) : NULL;
  if (rc == ZTO_OK && !yfull) rc = ZTO_EINVAL;
  for (int64_t e = 0; e < E && rc == ZTO_OK; ++e) {
    /* the pairs of expert e, in pair order */
    int64_t me = 0;
    for (int64_t p = 0; p < P; ++p)
      if (ids[p] == e) {
        pe[me] = p;
        memcpy(xe + me * H, x + (p / topk) * H, sizeof(uint16_t) * (size_t)H);
        ++me;
      }
    if (me == 0) continue;
    const int32_t *we13 = w13 + e * 2 * I * (H / 8);
    const uint16_t *se13 = s13 + e * G13 * 2 * I;
    rc = zto_woq_linear(xe, ZT_DT_BF16, me, H, H, we13, 2 * I, se13, ZT_DT_BF16, G13,
                        NULL, ZT_DT_NONE, b13 ? (const void *)(b13 + e * 2 * I) : NULL,
                        ZT_DT_BF16, 0, NULL, NULL, NULL, NULL, gu, ZT_DT_F32, 2 * I, nthreads);
    if (rc != ZTO_OK) break;
    for (int64_t m = 0; m < me; ++m)
      for (int64_t j = 0; j < I; ++j)
        h[m * I + j] = f32_to_bf16(unary(act, gu[m * 2 * I + j]) * gu[m * 2 * I + I + j]);
    rc = zto_woq_linear(h, ZT_DT_BF16, me, I, I, w2 + e * H * (I / 8), H, s2 + e * G2 * H,
                        ZT_DT_BF16, G2, NULL, ZT_DT_NONE,
                        b2 ? (const void *)(b2 + e * H) : NULL, ZT_DT_BF16, 0, NULL, NULL,
                        NULL, NULL, y, ZT_DT_BF16, H, nthreads);
    if (rc != ZTO_OK) break;
    for (int64_t m = 0; m < me; ++m)
      for (int64_t j = 0; j < H; ++j) yfull[pe[m] * H + j] = bf16_to_f32(y[m * H + j]);
  }
  if (rc == ZTO_OK) {
    for (int64_t t = 0; t < T; ++t)
      for (int64_t k = 0; k < topk; ++k) {
        const int64_t p = t * topk + k;
        if (ids[p] < 0 || ids[p] >= E) continue;
        const float wk = skip_weighted ? 1.f : load_f(wts, wts_dt, p);
        for (int64_t j = 0; j < H; ++j) acc[t * H + j] += wk * yfull[p * H + j];
      }
    for (int64_t i = 0; i < T * H; ++i) out[i] = f32_to_bf16(acc[i]);
  }
  free(acc); free(xe); free(pe); free(gu); free(h); free(y); free(yfull);
  return rc;
}
