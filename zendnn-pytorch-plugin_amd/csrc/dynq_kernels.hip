// Dynamic int8 linear kernels for gfx950 (zentorch_dynamic_qlinear).
//
//  * dyn_quantize_kernel  one workgroup per token row: fp32 amax of |x|,
//    sx = max(amax, 1e-12) / 127 (correctly rounded divide), then
//    q = clamp(rint(x / sx), -128, 127).  This is the closed form of the
//    reference's test reference (test_dynamic_qlinear.py:32-36) evaluated in
//    fp32, bit for bit.
//  * s8_gemm_kernel       int8 x int8 -> int32 MFMA (16x16x64) GEMM over
//    LDS tiles of qx [M, K] and W [N, K] (both K-contiguous, the transB=true
//    layout of DynamicQLinear.cpp:124-126), epilogue
//    y = ((float)acc * sx[m]) * sw[n] + bias[n] (+ post-ops), or the raw
//    int32 accumulators.
//  * s8_generic_kernel    K not a multiple of 16: one wave per output.
//
// Per-token asymmetric uint8 (an opt-in beside the reference's symmetric
// s8): lo = min(0, min_k x), hi = max(0, max_k x), sx = max(hi - lo, 1e-12)
// / 255, zp = clamp(rint(-lo / sx), 0, 255), q = clamp(rint(x / sx) + zp,
// 0, 255).  qx stores q - 128 as s8 so the s8 x s8 GEMMs run unchanged, and
// the epilogue subtracts (zp - 128) * colsum[n] from the int32 accumulator,
// which leaves sum_k (q - zp) * w exactly.
#include <cstdio>
#include <cstdlib>

#include "zt_launch.hpp"
#include "zt_tuning.hpp"

namespace zt {

namespace {

// Byte offset of qx[m][k] in the fragment order read by s8_skinny32_kernel
// (K % 64 == 0): 32-token tiles, each a run of 64-k chunks, each chunk two
// 1 KB B-operand fragments of v_mfma_i32_32x32x32_i8.  Fragment f holds the
// 16-byte k blocks f (lanes 0-31) and f + 2 (lanes 32-63) of the chunk; lane
// 32*h + (m % 32) holds block f + 2h of token m.
__device__ __forceinline__ int64_t qx_frag_offset(int64_t m, int64_t k, int64_t K) {
  return (((m >> 5) * (K >> 6) + (k >> 6)) * 2 + ((k >> 4) & 1)) * 1024 +
         ((((k >> 5) & 1) * 32 + (m & 31)) * 16) + (k & 15);
}

// Row scale (and zero point) from the row's extremes: symmetric s8 from
// lo = -amax, hi = amax; asymmetric u8 from lo <= 0 <= hi.  Sets s and the
// value added to rint(x / s) before the clamp to [qlo, qlo + 255].
template <bool ASYM>
__device__ __forceinline__ void row_qparams(float lo, float hi, float &s, float &zp) {
  if (ASYM) {
    float range = hi - lo;
    if (!(range >= 1e-12f)) range = 1e-12f;
    s = __fdiv_rn(range, 255.0f);
    zp = fminf(fmaxf(rintf(__fdiv_rn(-lo, s)), 0.f), 255.f);
  } else {
    float amax = hi;
    if (!(amax >= 1e-12f)) amax = 1e-12f;
    s = __fdiv_rn(amax, 127.0f);
    zp = 0.f;
  }
}

// rint(x / s) with x / s the correctly rounded quotient, |x / s| < 256,
// given inv = 1 / s correctly rounded.  y = x * inv is within 2 ulp of the
// exact quotient (two roundings of relative size 2^-24) and the rounded
// quotient within 0.5 ulp of it: 2.5 ulp <= 2.5 * 2^-16 < 2^-14 below 256.
// So unless y lies within 2^-14 of a half-integer, both have the same
// nearest integer and neither is a tie; only those rare elements take the
// IEEE division.  (A product that underflows leaves |x / s| far below 0.5:
// 0 either way; NaN and infinite inputs give NaN or 0 in both forms.)
__device__ __forceinline__ float rint_div(float x, float s, float inv) {
  const float y = x * inv;
  const float r = rintf(y);
  if (fabsf(y - r) > 0.5f - 0x1p-14f) return rintf(__fdiv_rn(x, s));
  return r;
}

// q as stored in qx: clamp(rint(x / s) + zp) in [-128, 127] (symmetric) or
// [0, 255] (asymmetric, stored minus 128); inv = 1 / s correctly rounded
template <bool ASYM>
__device__ __forceinline__ int quant_one(float x, float s, float inv, float zp) {
  float r = rint_div(x, s, inv);
  if (ASYM) return (int)fminf(fmaxf(r + zp, 0.f), 255.f) - 128;
  return (int)fminf(fmaxf(r, -128.f), 127.f);
}

// Reduce (lo, hi) over the 256 threads; returns the workgroup's values.
__device__ __forceinline__ void block_minmax(float &lo, float &hi, float *red, int tid) {
  const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off, kWave));
    hi = fmaxf(hi, __shfl_xor(hi, off, kWave));
  }
  if (lane == 0) red[wv] = lo, red[4 + wv] = hi;
  __syncthreads();
  lo = fminf(fminf(red[0], red[1]), fminf(red[2], red[3]));
  hi = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
}

// The quantise kernels also clear the tile counters of the split-K GEMM that
// follows them on the stream (workgroup 0, 256 threads).
__device__ __forceinline__ void zero_counters(int32_t *zero, int nzero, int tid) {
  if (blockIdx.x == 0)
    for (int i = tid; i < nzero; i += 256) zero[i] = 0;
}

template <bool ASYM>
__global__ __launch_bounds__(256) void dyn_quantize_kernel(
    const void *x, int x_dt, int64_t K, int8_t *qx, float *sx, int frag, int32_t *azp,
    int32_t *zero, int nzero) {
  __shared__ float red[8];
  const int tid = threadIdx.x;
  const int64_t m = blockIdx.x;
  zero_counters(zero, nzero, tid);
  const int64_t base = m * K;
  float lo = 0.f, hi = 0.f;
  for (int64_t k = tid; k < K; k += 256) {
    const float v = load_elem(x, x_dt, base + k);
    if (ASYM) {
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    } else {
      hi = fmaxf(hi, fabsf(v));
    }
  }
  block_minmax(lo, hi, red, tid);
  float s, zp;
  row_qparams<ASYM>(lo, hi, s, zp);
  if (tid == 0) {
    sx[m] = s;
    if (ASYM) azp[m] = (int32_t)zp - 128;
  }
  const float inv = __fdiv_rn(1.0f, s);
  for (int64_t k = tid; k < K; k += 256)
    qx[frag ? qx_frag_offset(m, k, K) : base + k] =
        (int8_t)quant_one<ASYM>(load_elem(x, x_dt, base + k), s, inv, zp);
}

// The same per-row quantisation for bf16 rows with K % 8 == 0, 16-byte
// aligned: each thread holds up to VPT 8-element vectors of its row in
// registers between the amax and the quantise pass and writes 8 bytes of qx
// at a time (row-major, or in fragment order when FRAG).  Bit-identical to
// dyn_quantize_kernel.
template <int VPT, bool FRAG, bool ASYM>
__global__ __launch_bounds__(256) void dyn_quantize_bf16_kernel(const uint16_t *x, int64_t K,
                                                                 int8_t *qx, float *sx,
                                                                 int32_t *azp, int32_t *zero,
                                                                 int nzero) {
  __shared__ float red[8];
  const int tid = threadIdx.x;
  const int64_t m = blockIdx.x;
  zero_counters(zero, nzero, tid);
  const u32x4_t *row = reinterpret_cast<const u32x4_t *>(x + m * K);
  const int nv = (int)(K / 8);
  u32x4_t v[VPT];
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int j = tid + 256 * i;
    v[i] = j < nv ? row[j] : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float e0 = __uint_as_float(v[i][w] << 16);
      const float e1 = __uint_as_float(v[i][w] & 0xffff0000u);
      if (ASYM) {
        lo = fminf(lo, fminf(e0, e1));
        hi = fmaxf(hi, fmaxf(e0, e1));
      } else {
        hi = fmaxf(hi, fmaxf(fabsf(e0), fabsf(e1)));
      }
    }
  }
  block_minmax(lo, hi, red, tid);
  float s, zp;
  row_qparams<ASYM>(lo, hi, s, zp);
  if (tid == 0) {
    sx[m] = s;
    if (ASYM) azp[m] = (int32_t)zp - 128;
  }
  const float inv = __fdiv_rn(1.0f, s);
  auto q1 = [&](float f) { return (uint32_t)(uint8_t)(int8_t)quant_one<ASYM>(f, s, inv, zp); };
  u32x2_t *out = reinterpret_cast<u32x2_t *>(qx + m * K);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int j = tid + 256 * i;
    if (j >= nv) break;
    u32x2_t o;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t a0 = v[i][2 * h], a1 = v[i][2 * h + 1];
      o[h] = q1(__uint_as_float(a0 << 16)) | (q1(__uint_as_float(a0 & 0xffff0000u)) << 8) |
             (q1(__uint_as_float(a1 << 16)) << 16) | (q1(__uint_as_float(a1 & 0xffff0000u)) << 24);
    }
    if (FRAG)
      *reinterpret_cast<u32x2_t *>(qx + qx_frag_offset(m, 8 * (int64_t)j, K)) = o;
    else
      out[j] = o;
  }
}

// Static per-tensor quantisation of zentorch_qlinear's activations, one
// workgroup per row.  fp32 / bf16 x: q = clamp(rint(x * inv) + zp) with
// inv = 1 / scale in fp32, over [0, 255] when a zero point is given (stored
// q - 128, offset zp - 128) and over [-128, 127] when not (offset 0).  s8 x
// is taken as is (offset zp, or 0); u8 x is stored x - 128 (offset zp - 128,
// zp = 0 when absent).  sx[m] = scale; azp[m] = the offset, when azp is set.
__global__ __launch_bounds__(256) void static_quantize_kernel(
    const void *x, int x_dt, int64_t K, int8_t *qx, int frag, const float *scale,
    const int32_t *zp, float *sx, int32_t *azp, int32_t *zero, int nzero) {
  const int tid = threadIdx.x;
  const int64_t m = blockIdx.x, base = m * K;
  zero_counters(zero, nzero, tid);
  const float s = *scale;
  const int32_t z = zp ? *zp : 0;
  const bool u8 = x_dt == ZT_DT_U8 || ((x_dt == ZT_DT_F32 || x_dt == ZT_DT_BF16) && zp);
  if (tid == 0) {
    sx[m] = s;
    if (azp) azp[m] = u8 ? z - 128 : z;
  }
  const float inv = __fdiv_rn(1.0f, s);
  for (int64_t k = tid; k < K; k += 256) {
    int q;
    if (x_dt == ZT_DT_S8) {
      q = reinterpret_cast<const int8_t *>(x)[base + k];
    } else if (x_dt == ZT_DT_U8) {
      q = (int)reinterpret_cast<const uint8_t *>(x)[base + k] - 128;
    } else {
      const float r = rintf(load_elem(x, x_dt, base + k) * inv);
      q = u8 ? (int)fminf(fmaxf(r + (float)z, 0.f), 255.f) - 128
             : (int)fminf(fmaxf(r, -128.f), 127.f);
    }
    qx[frag ? qx_frag_offset(m, k, K) : base + k] = (int8_t)q;
  }
}

// Requantised int8 output (zentorch_qlinear with output scales):
// clamp(rint(v * inv) + zp) with inv = 1 / scale in fp32.
__device__ __forceinline__ void store_q8(const DynArgs &a, int64_t i, float v) {
  const float inv = __fdiv_rn(1.0f, *a.out_scale);
  float r = rintf(v * inv) + (a.out_zp ? (float)*a.out_zp : 0.f);
  if (a.y_dt == ZT_DT_U8)
    reinterpret_cast<uint8_t *>(a.y)[i] = (uint8_t)(int)fminf(fmaxf(r, 0.f), 255.f);
  else
    reinterpret_cast<int8_t *>(a.y)[i] = (int8_t)(int)fminf(fmaxf(r, -128.f), 127.f);
}

// The weight scale of column n (one shared scale when sw_bcast).
__device__ __forceinline__ float wscale(const DynArgs &a, int64_t n) {
  return load_elem(a.sw, a.sw_dt, a.sw_bcast ? 0 : n);
}

// sxp, when set, replaces a.sx (the fused kernel keeps the row scales in LDS).
__device__ __forceinline__ void dyn_epilogue(const DynArgs &a, int64_t m,
                                             int64_t n, int32_t acc,
                                             const float *sxp = nullptr) {
  if (a.azp) acc -= a.azp[m] * a.colsum[n];
  if (a.y_dt == ZT_DT_S32) {
    reinterpret_cast<int32_t *>(a.y)[m * a.N + n] = acc;
    return;
  }
  float v = (float)acc * (sxp ? sxp[m] : a.sx[m]);
  v = v * wscale(a, n);
  if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
  v = apply_post_ops(v, a.post, m, n);
  if (a.y_dt == ZT_DT_U8 || a.y_dt == ZT_DT_S8)
    store_q8(a, m * a.N + n, v);
  else
    store_elem(a.y, a.y_dt, m * a.N + n, v);
}

__global__ __launch_bounds__(256) void s8_generic_kernel(DynArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= a.M * a.N) return;
  const int64_t m = wid / a.N, n = wid % a.N;
  int32_t acc = 0;
  for (int64_t k = lane; k < a.K; k += kWave)
    acc += (int32_t)a.qx[m * a.K + k] * (int32_t)a.w[n * a.K + k];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  if (lane == 0) dyn_epilogue(a, m, n, acc);
}

constexpr int kS8BK = 128;

template <int BM, int BN>
__global__ __launch_bounds__(256) void s8_gemm_kernel(DynArgs a) {
  constexpr int LD = kS8BK + 16;  // bytes per LDS row, padded
  constexpr int WTM = BM / 32, WTN = BN / 32;
  __shared__ __attribute__((aligned(16))) int8_t As[BM * LD];
  __shared__ __attribute__((aligned(16))) int8_t Bs[BN * LD];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 15, lg = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t M = a.M, N = a.N, K = a.K;

  i32x4_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) acc[i][j] = i32x4_t{0, 0, 0, 0};

  for (int64_t k0 = 0; k0 < K; k0 += kS8BK) {
    for (int i = tid; i < BM * 8; i += 256) {
      const int r = i >> 3, cc = i & 7;
      const int64_t m = m0 + r, k = k0 + cc * 16;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (m < M && k < K)
        v = *reinterpret_cast<const u32x4_t *>(a.qx + m * K + k);
      *reinterpret_cast<u32x4_t *>(As + r * LD + cc * 16) = v;
    }
    for (int i = tid; i < BN * 8; i += 256) {
      const int r = i >> 3, cc = i & 7;
      const int64_t n = n0 + r, k = k0 + cc * 16;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (n < N && k < K)
        v = *reinterpret_cast<const u32x4_t *>(a.w + n * K + k);
      *reinterpret_cast<u32x4_t *>(Bs + r * LD + cc * 16) = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kS8BK / 64; ++kk) {
      i32x4_t Af[WTM], Bf[WTN];
#pragma unroll
      for (int i = 0; i < WTM; ++i)
        Af[i] = *reinterpret_cast<const i32x4_t *>(
            As + (wm * (BM / 2) + i * 16 + lr) * LD + kk * 64 + 16 * lg);
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        Bf[j] = *reinterpret_cast<const i32x4_t *>(
            Bs + (wn * (BN / 2) + j * 16 + lr) * LD + kk * 64 + 16 * lg);
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] =
              __builtin_amdgcn_mfma_i32_16x16x64_i8(Af[i], Bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * (BM / 2) + i * 16 + 4 * lg + r;
        const int64_t n = n0 + wn * (BN / 2) + j * 16 + lr;
        if (m < M && n < N) dyn_epilogue(a, m, n, acc[i][j][r]);
      }
}

// Large-M int8 GEMM.  A BM x BN output tile walks K in steps of BK = 128
// with 4 waves (2 x 2), each owning a (BM/2) x (BN/2) sub-tile of
// WTM x WTN 16x16x64 MFMAs.  LDS holds two stages of the qx [BM, BK] and
// W [BN, BK] slabs (rows padded to 144 B); while a step computes from one
// stage, every thread's 16-byte chunks of the next step are already in
// flight into registers (raw buffer loads: rows past M/N and columns past
// K read as zero), and are written to the other stage before the step's
// single barrier.  Tiles are ordered in groups of GM m-tiles (so a group
// reuses the same W tiles) and each XCD takes one contiguous range of that
// order, so the tiles sharing W and qx rows share an L2.
constexpr int kTBK = 128;
constexpr int kTLDR = kTBK + 16;

// int32 row pitch of the accumulator tile staged in LDS for the epilogue
template <int BN>
constexpr int acc_pitch() { return BN + 4; }

template <int BM, int BN>
constexpr size_t s8_tiled_lds() {
  const size_t stages = 2 * (size_t)(BM + BN) * kTLDR;
  const size_t acc = (size_t)BM * acc_pitch<BN>() * 4 + (size_t)BM * 4;
  return stages > acc ? stages : acc;
}

// Epilogue of four consecutive columns n..n+3 of row m: one 8/16-byte store
// when the row has them all, element by element otherwise.
// The asymmetric-activation correction of four accumulators of row m from
// column n (the row's four columns are n..n+3 < N).
__device__ __forceinline__ i32x4_t asym_fix4(const DynArgs &a, int m, int n, i32x4_t v) {
  const int32_t z = a.azp[m];
  const i32x4_t c = *reinterpret_cast<const i32x4_t *>(a.colsum + n);
  return v - c * z;
}

__device__ __forceinline__ void dyn_epilogue4(const DynArgs &a, int m, int n, i32x4_t v,
                                              const float *sxp = nullptr) {
  const int N = (int)a.N;
  const bool vec_out = a.y_dt == ZT_DT_S32 || a.y_dt == ZT_DT_BF16 || a.y_dt == ZT_DT_F32;
  if (n + 3 < N && (N & 3) == 0 && vec_out) {
    if (a.azp) v = asym_fix4(a, m, n, v);
    if (a.y_dt == ZT_DT_S32) {
      *reinterpret_cast<i32x4_t *>(reinterpret_cast<int32_t *>(a.y) + (int64_t)m * N + n) = v;
      return;
    }
    float f[4];
    const float sxm = sxp ? sxp[m] : a.sx[m];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float t = (float)v[r] * sxm;
      t = t * wscale(a, n + r);
      if (a.bias) t = t + load_elem(a.bias, a.b_dt, n + r);
      f[r] = apply_post_ops(t, a.post, m, n + r);
    }
    if (a.y_dt == ZT_DT_BF16) {
      u32x2_t p;
      p[0] = pack_bf16x2(f[0], f[1]);
      p[1] = pack_bf16x2(f[2], f[3]);
      *reinterpret_cast<u32x2_t *>(reinterpret_cast<uint16_t *>(a.y) + (int64_t)m * N + n) = p;
      return;
    }
    if (a.y_dt == ZT_DT_F32) {
      *reinterpret_cast<f32x4_t *>(reinterpret_cast<float *>(a.y) + (int64_t)m * N + n) =
          f32x4_t{f[0], f[1], f[2], f[3]};
      return;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (n + r < N) dyn_epilogue(a, m, n + r, v[r], sxp);
}

// Epilogue of a BM x BN int32 tile staged in LDS (row pitch acc_pitch),
// 256 threads.  BN/4 divides 256, so each thread keeps the same four columns
// for all its rows: their weight scales and bias are loaded once, and the
// row scales come from LDS (sx_l).  Same arithmetic as dyn_epilogue:
// ((float)acc * sx[m]) * sw[n] + bias[n].  Post-ops, int32 output and a row
// length that is not a multiple of 4 take the general path.
template <int BM, int BN, int NT = 256>
__device__ __forceinline__ void s8_tile_epilogue(const DynArgs &a, const int32_t *tile,
                                                 const float *sx_l, int m0, int n0, int tid) {
  constexpr int AP = acc_pitch<BN>();
  constexpr int G4 = BN / 4;
  // the first NTE threads keep the same four columns for all their rows
  // (NT / G4 rows at a time); the rest of the threads sit this loop out
  constexpr int NTE = NT / G4 * G4;
  static_assert(NTE > 0, "four-column groups must fit the threads");
  const int M = (int)a.M, N = (int)a.N;
  const int c4 = (tid % G4) * 4, n = n0 + c4;
  if ((a.y_dt == ZT_DT_BF16 || a.y_dt == ZT_DT_F32) && a.post.count == 0 && (N & 3) == 0) {
    if (n >= N || tid >= NTE) return;
    float sw[4], b[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sw[r] = wscale(a, n + r);
      b[r] = a.bias ? load_elem(a.bias, a.b_dt, n + r) : 0.f;
    }
    for (int row = tid / G4; row < BM && m0 + row < M; row += NTE / G4) {
      const int m = m0 + row;
      i32x4_t v = *reinterpret_cast<const i32x4_t *>(tile + row * AP + c4);
      if (a.azp) v = asym_fix4(a, m, n, v);
      const float sxm = sx_l[row];
      float f[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = (float)v[r] * sxm;
        t = t * sw[r];
        f[r] = a.bias ? t + b[r] : t;
      }
      if (a.y_dt == ZT_DT_BF16) {
        u32x2_t pk;
        pk[0] = pack_bf16x2(f[0], f[1]);
        pk[1] = pack_bf16x2(f[2], f[3]);
        *reinterpret_cast<u32x2_t *>(reinterpret_cast<uint16_t *>(a.y) + (int64_t)m * N + n) = pk;
      } else {
        *reinterpret_cast<f32x4_t *>(reinterpret_cast<float *>(a.y) + (int64_t)m * N + n) =
            f32x4_t{f[0], f[1], f[2], f[3]};
      }
    }
    return;
  }
  for (int idx = tid; idx < BM * G4; idx += NT) {
    const int row = idx / G4, cc = (idx % G4) * 4;
    const int m = m0 + row, nn = n0 + cc;
    if (m < M && nn < N)
      dyn_epilogue4(a, m, nn, *reinterpret_cast<const i32x4_t *>(tile + row * AP + cc));
  }
}

// Stage the row scales of rows m0..m0+BM of the tile for s8_tile_epilogue.
template <int BM, int NT = 256>
__device__ __forceinline__ void s8_stage_row_scales(const DynArgs &a, float *sx_l, int m0, int tid) {
  if (a.y_dt == ZT_DT_S32) return;
  for (int r = tid; r < BM; r += NT) sx_l[r] = m0 + r < (int)a.M ? a.sx[m0 + r] : 0.f;
}

template <int BM, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void s8_gemm_tiled_kernel(DynArgs a, int tiles_m, int tiles_n, int group_m) {
  constexpr int WTM = BM / 32, WTN = BN / 32;
  constexpr int ACH = BM * (kTBK / 16) / 256, BCH = BN * (kTBK / 16) / 256;
  constexpr int STAGE = (BM + BN) * kTLDR;
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 15, lg = lane >> 4;

  // grouped tile order, contiguous per XCD
  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int m0 = tm * BM, n0 = tn * BN;

  const auto a_rs = make_rsrc(a.qx, (uint32_t)((int64_t)M * K));
  const auto b_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));

  // this thread's 16-byte chunks: row = idx / 8, column chunk = idx % 8
  uint32_t a_off[ACH], b_off[BCH];
  int a_col[ACH], b_col[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const int idx = tid + 256 * c, row = idx >> 3;
    a_col[c] = (idx & 7) * 16;
    a_off[c] = m0 + row < M ? (uint32_t)((m0 + row) * K + a_col[c]) : kOobOffset;
  }
#pragma unroll
  for (int c = 0; c < BCH; ++c) {
    const int idx = tid + 256 * c, row = idx >> 3;
    b_col[c] = (idx & 7) * 16;
    b_off[c] = n0 + row < N ? (uint32_t)((n0 + row) * K + b_col[c]) : kOobOffset;
  }

  u32x4_t ra[ACH], rb[BCH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const uint32_t off = (a_off[c] == kOobOffset || k0 + a_col[c] >= K) ? kOobOffset
                                                                         : a_off[c] + k0;
      ra[c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(a_rs, off, 0, 0));
    }
#pragma unroll
    for (int c = 0; c < BCH; ++c) {
      const uint32_t off = (b_off[c] == kOobOffset || k0 + b_col[c] >= K) ? kOobOffset
                                                                         : b_off[c] + k0;
      rb[c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rs, off, 0, 0));
    }
  };
  auto swrite = [&](int stage) {
    int8_t *base = s8_smem + stage * STAGE;
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const int idx = tid + 256 * c;
      *reinterpret_cast<u32x4_t *>(base + (idx >> 3) * kTLDR + (idx & 7) * 16) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < BCH; ++c) {
      const int idx = tid + 256 * c;
      *reinterpret_cast<u32x4_t *>(base + (BM + (idx >> 3)) * kTLDR + (idx & 7) * 16) = rb[c];
    }
  };

  i32x4_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) acc[i][j] = i32x4_t{0, 0, 0, 0};

  const int nk = (K + kTBK - 1) / kTBK;
  gload(0);
  swrite(0);
  __syncthreads();
  for (int ks = 0; ks < nk; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nk) gload((ks + 1) * kTBK);
    const int8_t *As = s8_smem + cur * STAGE + (wm * (BM / 2) + lr) * kTLDR + 16 * lg;
    const int8_t *Bs = s8_smem + cur * STAGE + (BM + wn * (BN / 2) + lr) * kTLDR + 16 * lg;
    // both 64-wide halves of the step's fragments are read up front, so the
    // second half's LDS reads overlap the first half's MFMAs
    i32x4_t Af[2][WTM], Bf[2][WTN];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        Bf[kk][j] = *reinterpret_cast<const i32x4_t *>(Bs + j * 16 * kTLDR + kk * 64);
#pragma unroll
      for (int i = 0; i < WTM; ++i)
        Af[kk][i] = *reinterpret_cast<const i32x4_t *>(As + i * 16 * kTLDR + kk * 64);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Af[kk][i], Bf[kk][j], acc[i][j],
                                                             0, 0, 0);
    if (ks + 1 < nk) swrite(cur ^ 1);
    __syncthreads();
  }

  // Stage the accumulator tile in LDS (static register indices only, so
  // acc stays in registers), then write rows of four columns per thread.
  constexpr int AP = acc_pitch<BN>();
  int32_t *tile = reinterpret_cast<int32_t *>(s8_smem);
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        tile[(wm * (BM / 2) + i * 16 + 4 * lg + r) * AP + wn * (BN / 2) + j * 16 + lr] =
            acc[i][j][r];
  float *sx_l = reinterpret_cast<float *>(tile + BM * AP);
  s8_stage_row_scales<BM>(a, sx_l, m0, tid);
  __syncthreads();
  s8_tile_epilogue<BM, BN>(a, tile, sx_l, m0, n0, tid);
}

// The same tiling with the K slabs moved by the buffer unit straight into
// LDS (buffer_load_dwordx4 ... lds, range-checked like the register loads),
// S stages deep.  LDS rows are 128 B with no padding; the 16-byte chunk c
// of row r sits at position c ^ (r & 7), so one wave's 1 KB load fills 8
// whole rows and a fragment read (16 rows, one chunk) touches every bank
// once per 8 rows.  Each step first reads all its fragments into registers,
// then starts the loads of step ks + S - 1 into the stage read one step
// earlier, then runs its MFMAs; only the loads of step ks + 1 are waited for
// before the barrier.
template <int BM, int BN, int S>
constexpr size_t s8_dma_lds() {
  const size_t stages = (size_t)S * (BM + BN) * kTBK;
  const size_t acc = (size_t)BM * acc_pitch<BN>() * 4 + (size_t)BM * 4;
  return stages > acc ? stages : acc;
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

template <int BM, int BN, int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void s8_gemm_dma_kernel(DynArgs a, int tiles_m, int tiles_n, int group_m) {
  constexpr int WTM = BM / 32, WTN = BN / 32;
  constexpr int STAGE = (BM + BN) * kTBK;
  constexpr int GROUPS = (BM + BN) / 8;      // 8-row groups per stage
  constexpr int GPW = GROUPS / 4;            // per wave
  static_assert(GROUPS % 4 == 0, "row groups must split over 4 waves");
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  // wave index as a scalar, so the row groups (and A/B choice) are uniform
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 15, lg = lane >> 4;

  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int m0 = tm * BM, n0 = tn * BN;

  const auto a_rs = make_rsrc(a.qx, (uint32_t)((int64_t)M * K));
  const auto b_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));

  // lane's source for each of the wave's row groups: row (group*8 + lane/8),
  // logical chunk (lane%8) ^ (lane/8)
  const int lrow = lane >> 3, lchunk = ((lane & 7) ^ lrow) * 16;
  uint32_t src[GPW];
  bool is_a[GPW];
#pragma unroll
  for (int q = 0; q < GPW; ++q) {
    const int grp = wv * GPW + q;
    const int row = grp * 8 + lrow;
    is_a[q] = grp * 8 < BM;  // whole groups lie in A or in B
    if (is_a[q])
      src[q] = m0 + row < M ? (uint32_t)((m0 + row) * K + lchunk) : kOobOffset;
    else
      src[q] = n0 + row - BM < N ? (uint32_t)((n0 + row - BM) * K + lchunk) : kOobOffset;
  }
  auto dma = [&](int step) {
    const int k0 = step * kTBK;
    int8_t *stage = s8_smem + (step % S) * STAGE;
#pragma unroll
    for (int q = 0; q < GPW; ++q) {
      const uint32_t off = (src[q] == kOobOffset || k0 + lchunk >= K) ? kOobOffset : src[q] + k0;
      lds_ptr_t dst = (lds_ptr_t)(stage + (wv * GPW + q) * 1024);
      if (is_a[q])
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, dst, 16, off, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rs, dst, 16, off, 0, 0, 0);
    }
  };

  i32x4_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) acc[i][j] = i32x4_t{0, 0, 0, 0};

  const int nk = (K + kTBK - 1) / kTBK;
#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p < nk) dma(p);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // fragment rows of this lane: A rows wm*BM/2 + i*16 + lr, B rows likewise;
  // row & 7 == lr & 7 for every i, j
  const int sw = lr & 7;
  for (int ks = 0; ks < nk; ++ks) {
    const int8_t *stage = s8_smem + (ks % S) * STAGE;
    const int8_t *As = stage + (wm * (BM / 2) + lr) * kTBK;
    const int8_t *Bs = stage + (BM + wn * (BN / 2) + lr) * kTBK;
    i32x4_t Af[2][WTM], Bf[2][WTN];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int pos = (((kk * 4 + lg) ^ sw) * 16);
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        Bf[kk][j] = *reinterpret_cast<const i32x4_t *>(Bs + j * 16 * kTBK + pos);
#pragma unroll
      for (int i = 0; i < WTM; ++i)
        Af[kk][i] = *reinterpret_cast<const i32x4_t *>(As + i * 16 * kTBK + pos);
    }
    if (ks + S - 1 < nk) dma(ks + S - 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Af[kk][i], Bf[kk][j], acc[i][j],
                                                             0, 0, 0);
    // keep the MFMAs ahead of the wait (the scheduler would otherwise hoist
    // the wait and barrier above them and expose the load latency)
    __builtin_amdgcn_sched_barrier(0);
    // the loads of step ks + 1 have landed once at most the GPW loads issued
    // this step are outstanding
    if (S > 2 && ks + S - 1 < nk)
      __builtin_amdgcn_s_waitcnt((GPW & 15) | ((GPW >> 4) << 14) | (7 << 4) | (15 << 8));
    else
      __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  constexpr int AP = acc_pitch<BN>();
  int32_t *tile = reinterpret_cast<int32_t *>(s8_smem);
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        tile[(wm * (BM / 2) + i * 16 + 4 * lg + r) * AP + wn * (BN / 2) + j * 16 + lr] =
            acc[i][j][r];
  float *sx_l = reinterpret_cast<float *>(tile + BM * AP);
  s8_stage_row_scales<BM>(a, sx_l, m0, tid);
  __syncthreads();
  s8_tile_epilogue<BM, BN>(a, tile, sx_l, m0, n0, tid);
}

// Prefill int8 GEMM on v_mfma_i32_32x32x32_i8: BM x BN tiles, 4 waves of
// (BM/2) x (BN/2), K in steps of 64 bytes moved straight into LDS by the
// buffer unit, S stages deep, two workgroups per CU (at most 256 registers
// and 80 KB of LDS each), so one workgroup's epilogue and barriers overlap
// the other's MFMAs.
//
// LDS rows are 64 B; the 16-byte chunk c of row r sits at position
// c ^ f(r), f(r) = ((r >> 2) ^ (r >> 1)) & 3, and one wave's 1 KB load fills
// 16 whole rows.  f gives the 16 rows a fragment read touches 16 distinct
// 16-byte bank groups over 256 bytes, and any 8 of them (rows of equal
// parity) distinct groups over 128 bytes.
// Step ks: wait for this wave's loads of step ks (those of the S - 2 later
// steps stay in flight), barrier (a bare s_barrier: __syncthreads' release
// fence would wait for every load in flight), start the loads of step
// ks + S - 1 into the buffer step ks - 1 used, read the step's fragments
// and run its MFMAs.  Loads past the last step read zeros into a buffer no
// step reads, so the loop has no branches (a branch join makes the compiler
// wait for LDS reads still in flight).
//
// The MFMA takes W as A and qx as B, so D is [n][m]: register r of lane l
// holds n = 8*(r/4) + 4*(l/32) + r%4 and m = l%32, four runs of four
// consecutive n per lane.  The epilogue stages one half of the tile (the
// rows of the waves with wm == h) as fp32 [m][n] in LDS at a time.
constexpr int kS32BK = 64;

__host__ __device__ constexpr int s32_swz(int r) { return ((r >> 2) ^ (r >> 1)) & 3; }

__host__ __device__ constexpr int vmcnt_wait_imm(int n) {
  return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

template <int BM, int BN, int S>
constexpr size_t s8_gemm32_lds() {
  const size_t stages = (size_t)S * (BM + BN) * kS32BK;
  const size_t half = (size_t)(BM / 2) * acc_pitch<BN>() * 4 + (size_t)(BM / 2) * 4;
  return stages > half ? stages : half;
}

template <int BM, int BN, int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void s8_gemm32_kernel(DynArgs a, int tiles_m, int tiles_n, int group_m) {
  constexpr int WTM = BM / 64, WTN = BN / 64;  // 32 x 32 tiles per wave
  constexpr int STAGE = (BM + BN) * kS32BK;
  constexpr int GROUPS = (BM + BN) / 16;        // 1 KB loads (16 rows) per stage
  constexpr int LPW = GROUPS / 4;               // per wave
  static_assert(GROUPS % 4 == 0 && S >= 2 && S <= 5 && (S - 2) * LPW <= 63, "tile shape");
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv >> 1, wn = wv & 1;

  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int m0 = tm * BM, n0 = tn * BN;

  const auto a_rs = make_rsrc(a.qx, (uint32_t)((int64_t)M * K));
  const auto b_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));

  // this lane's source in each of the wave's loads: row grp*16 + lane/4 of
  // the [A | B] slab, logical chunk (lane % 4) ^ f(row)
  const int lrow = lane >> 2;
  const int lchunk = ((lane & 3) ^ s32_swz(lrow)) * 16;
  uint32_t src[LPW];
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int row = (wv * LPW + q) * 16 + lrow;
    if (row < BM)
      src[q] = m0 + row < M ? (uint32_t)((m0 + row) * K + lchunk) : kOobOffset;
    else
      src[q] = n0 + row - BM < N ? (uint32_t)((n0 + row - BM) * K + lchunk) : kOobOffset;
  }
  auto dma = [&](int step) {
    const int k0 = step * kS32BK;
    int8_t *stage = s8_smem + (step % S) * STAGE;
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      // K % 16 == 0: a chunk lies wholly inside or past K
      const uint32_t off = (src[q] == kOobOffset || k0 + lchunk >= K) ? kOobOffset : src[q] + k0;
      lds_ptr_t dst = (lds_ptr_t)(stage + (wv * LPW + q) * 1024);
      if ((wv * LPW + q) * 16 < BM)  // whole loads lie in A or in B
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, dst, 16, off, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rs, dst, 16, off, 0, 0, 0);
    }
  };

  // fragments: row R (R % 32 == lane % 32), k block kb = 2*sub + lane/32
  const int fsw = s32_swz(lane & 31);
  const int a_base = (wm * (BM / 2) + (lane & 31)) * kS32BK;
  const int b_base = (BM + wn * (BN / 2) + (lane & 31)) * kS32BK;
  i32x16_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = (K + kS32BK - 1) / kS32BK;
#pragma unroll
  for (int p = 0; p < S - 1; ++p) dma(p);
  for (int ks = 0; ks < nk; ++ks) {
    __builtin_amdgcn_s_waitcnt(vmcnt_wait_imm((S - 2) * LPW));
    asm volatile("s_barrier" ::: "memory");
    dma(ks + S - 1);
    const int8_t *stage = s8_smem + (ks % S) * STAGE;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int pos = ((2 * sub + (lane >> 5)) ^ fsw) * 16;
      i32x4_t Af[WTM], Bf[WTN];
#pragma unroll
      for (int i = 0; i < WTM; ++i)
        Af[i] = *reinterpret_cast<const i32x4_t *>(stage + a_base + i * 32 * kS32BK + pos);
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        Bf[j] = *reinterpret_cast<const i32x4_t *>(stage + b_base + j * 32 * kS32BK + pos);
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Bf[j], Af[i], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue in two halves of BM/2 rows: the waves with wm == h stage
  // their accumulators as [m][n], then all threads finish those rows
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_barrier" ::: "memory");
  constexpr int AP = acc_pitch<BN>();
  int32_t *tile = reinterpret_cast<int32_t *>(s8_smem);
  float *sx_l = reinterpret_cast<float *>(tile + (BM / 2) * AP);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (wm == h) {
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<i32x4_t *>(
                tile + (i * 32 + (lane & 31)) * AP + wn * (BN / 2) + j * 32 + 8 * q + 4 * (lane >> 5)) =
                i32x4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]};
    }
    s8_stage_row_scales<BM / 2>(a, sx_l, m0 + h * (BM / 2), tid);
    __syncthreads();
    s8_tile_epilogue<BM / 2, BN>(a, tile, sx_l, m0 + h * (BM / 2), n0, tid);
    __syncthreads();
  }
}

template <int BM, int BN, int S>
hipError_t launch_s8_gemm32(const DynArgs &a, hipStream_t s) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  s8_gemm32_kernel<BM, BN, S><<<dim3((unsigned)(tiles_m * tiles_n)), dim3(256),
                                s8_gemm32_lds<BM, BN, S>(), s>>>(a, tiles_m, tiles_n, group_m);
  return hipGetLastError();
}

template <int BM, int BN, int S>
hipError_t launch_s8_dma(const DynArgs &a, hipStream_t s) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  s8_gemm_dma_kernel<BM, BN, S><<<dim3((unsigned)(tiles_m * tiles_n)), dim3(256),
                                  s8_dma_lds<BM, BN, S>(), s>>>(a, tiles_m, tiles_n, group_m);
  return hipGetLastError();
}

// Large-M int8 GEMM with warp-specialised loads: BM x BN tiles, K in steps
// of 128 bytes (each row's slab is one whole 128-byte line), S stages in LDS.
//  * NC = WM x WN compute waves only read fragments from LDS and run
//    v_mfma_i32_32x32x32_i8 (each wave (BM/WM) x (BN/WN), fragments of the
//    next 32-k sub-step read while the current sub-step's MFMAs run);
//  * ND load waves only move the stages into LDS with the buffer unit
//    (buffer_load_dwordx4 ... lds, 8 rows x 128 B per instruction).
// When the same waves issued both, every load instruction the buffer unit
// could not yet accept held up the MFMAs queued behind it, and the loop ran
// at the sum of its load and MFMA times.  One s_barrier per step: a load
// wave first waits for its own loads of the step (in-order vmcnt), so after
// the barrier the stage is whole, and every compute wave has finished the
// previous step's reads, so its stage can be refilled.
// LDS rows are 128 B; the 16-byte chunk c of tile row R sits at
// c ^ ((R >> 1) & 7), so the 16 rows one read pass touches hit 16 distinct
// bank groups.  The epilogue stages the int32 tile in LDS (whole, or one
// half of the rows at a time for tiles wider than 128 columns) and all
// threads finish it (s8_tile_epilogue).
constexpr int kWsBK = 128;

// tiles wider than 128 columns stage their int32 epilogue tile in two halves
// of BM/2 rows
template <int BN>
constexpr bool s8_ws_half() { return BN > 128; }

template <int BM, int BN, int S>
constexpr size_t s8_ws_lds() {
  const size_t stages = (size_t)S * (BM + BN) * kWsBK;
  constexpr int R = s8_ws_half<BN>() ? BM / 2 : BM;
  const size_t tile = (size_t)R * acc_pitch<BN>() * 4 + (size_t)R * 4;
  return stages > tile ? stages : tile;
}

// With a K split (partial set, grid.y splits of sps steps) a workgroup
// walks its split's steps only and writes its int32 tile to
// partial[split][M][N] (N % 4 == 0); s8_splitk_sum_kernel adds the splits
// and applies the epilogue.
template <int BM, int BN, int WM, int WN, int ND, int S>
__global__ __launch_bounds__(64 * (WM * WN + ND)) __attribute__((amdgpu_waves_per_eu(2, 2)))
void s8_gemm_ws_kernel(DynArgs a, int tiles_m, int tiles_n, int group_m, int32_t *partial,
                       int sps) {
  constexpr int NC = WM * WN, NT = 64 * (NC + ND);
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // 32 x 32 tiles per compute wave
  constexpr int STAGE = (BM + BN) * kWsBK;
  constexpr int GROUPS = (BM + BN) / 8;  // 1 KB loads (8 rows) per stage
  constexpr int LPW = GROUPS / ND;       // per load wave
  static_assert(GROUPS % ND == 0 && (S - 2) * LPW <= 63 && S >= 2, "tile shape");
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = (K + kWsBK - 1) / kWsBK;
  const int kb = partial ? (int)blockIdx.y * sps : 0;  // this workgroup's steps [kb, ke)
  const int ke = partial ? min(kb + sps, nk) : nk;
  // the accumulators are set (zeroed) only on the compute waves' path, so
  // the load waves' loop does not hold their registers
  i32x16_t acc[TM][TN];
  const int wm = wv / WN, wn = wv % WN;
  if (wv >= NC) {
    // load wave: rows (dw * LPW + q) * 8 + lane / 8 of the [A | B] slab
    const int dw = wv - NC;
    const auto a_rs = make_rsrc(a.qx, (uint32_t)((int64_t)M * K));
    const auto b_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));
    // the 16-byte chunk of row (dw * LPW + q) * 8 + lane / 8 this lane moves
    auto chunk = [&](int q) {
      const int row = (dw * LPW + q) * 8 + (lane >> 3);
      return ((lane & 7) ^ ((row >> 1) & 7)) * 16;
    };
    uint32_t src[LPW];
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      const int row = (dw * LPW + q) * 8 + (lane >> 3);
      if (row < BM) src[q] = m0 + row < M ? (uint32_t)((m0 + row) * K + chunk(q)) : kOobOffset;
      else src[q] = n0 + row - BM < N ? (uint32_t)((n0 + row - BM) * K + chunk(q)) : kOobOffset;
    }
    auto dma = [&](int step) {
      const int k0 = step * kWsBK;
      int8_t *stage = s8_smem + (step % S) * STAGE;
#pragma unroll
      for (int q = 0; q < LPW; ++q) {
        // K % 16 == 0: a 16-byte chunk lies wholly inside or past its row
        const uint32_t off = (src[q] == kOobOffset || step >= ke || k0 + chunk(q) >= K)
                                 ? kOobOffset : src[q] + (uint32_t)k0;
        lds_ptr_t dst = (lds_ptr_t)(stage + (dw * LPW + q) * 1024);
        if ((dw * LPW + q) * 8 < BM)  // whole loads lie in A or in B
          __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, dst, 16, off, 0, 0, 0);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rs, dst, 16, off, 0, 0, 0);
      }
    };
#pragma unroll
    for (int p = 0; p < S - 1; ++p) dma(kb + p);
    for (int ks = kb; ks < ke; ++ks) {
      __builtin_amdgcn_s_waitcnt(vmcnt_wait_imm((S - 2) * LPW));
      asm volatile("s_barrier" ::: "memory");
      dma(ks + S - 1);
    }
    __builtin_amdgcn_s_waitcnt(0);
  } else {
    // compute wave: fragments of row R = lane % 32 (+ tile offsets), k
    // block 2 * sub + lane / 32 of the 128-byte step
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    const int fsw = (lane >> 1) & 7;
    const int a_base = (wm * (BM / WM) + (lane & 31)) * kWsBK;
    const int b_base = (BM + wn * (BN / WN) + (lane & 31)) * kWsBK;
    i32x4_t Fa[2][TM], Fb[2][TN];
    auto read = [&](int ks, int sub, int buf) {
      const int8_t *stage = s8_smem + (ks % S) * STAGE;
      const int pos = ((2 * sub + (lane >> 5)) ^ fsw) * 16;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        Fa[buf][i] = *reinterpret_cast<const i32x4_t *>(stage + a_base + i * 32 * kWsBK + pos);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        Fb[buf][j] = *reinterpret_cast<const i32x4_t *>(stage + b_base + j * 32 * kWsBK + pos);
    };
    for (int ks = kb; ks < ke; ++ks) {
      asm volatile("s_barrier" ::: "memory");
      read(ks, 0, 0);
#pragma unroll
      for (int sub = 0; sub < kWsBK / 32; ++sub) {
        if (sub + 1 < kWsBK / 32) read(ks, sub + 1, (sub + 1) & 1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Fb[sub & 1][j], Fa[sub & 1][i],
                                                              acc[i][j], 0, 0, 0);
      }
    }
  }
  // epilogue: the whole int32 tile [m][n] in LDS (D is [n][m]: register r of
  // lane l holds n = 8*(r/4) + 4*(l/32) + r%4, m = l%32 of its 32 x 32
  // tile), then every thread finishes four columns of its rows
  __syncthreads();
  constexpr int AP = acc_pitch<BN>();
  constexpr bool HALF = s8_ws_half<BN>();
  static_assert(!HALF || WM == 2, "half-tile epilogue: one row half per wm");
  constexpr int R = HALF ? BM / 2 : BM;  // rows staged at a time
  int32_t *tile = reinterpret_cast<int32_t *>(s8_smem);
  float *sx_l = reinterpret_cast<float *>(tile + R * AP);
#pragma unroll
  for (int h = 0; h < (HALF ? 2 : 1); ++h) {
    if (h) __syncthreads();  // the first half's reads are done
    if (wv < NC && (!HALF || wm == h)) {
      const int rb = HALF ? 0 : wm * (BM / WM);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<i32x4_t *>(tile + (rb + i * 32 + (lane & 31)) * AP +
                                         wn * (BN / WN) + j * 32 + 8 * q + 4 * (lane >> 5)) =
                i32x4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]};
    }
    if (partial) {
      // the split's int32 tile, four columns at a time (N % 4 == 0)
      __syncthreads();
      int32_t *pp = partial + (size_t)blockIdx.y * M * N;
      for (int idx = tid; idx < R * (BN / 4); idx += NT) {
        const int r = idx / (BN / 4), c = (idx - r * (BN / 4)) * 4;
        const int m = m0 + h * R + r, n = n0 + c;
        if (m < M && n < N)
          *reinterpret_cast<i32x4_t *>(pp + (size_t)m * N + n) =
              *reinterpret_cast<const i32x4_t *>(tile + r * AP + c);
      }
      continue;
    }
    s8_stage_row_scales<R, NT>(a, sx_l, m0 + h * R, tid);
    __syncthreads();
    s8_tile_epilogue<R, BN, NT>(a, tile, sx_l, m0 + h * R, n0, tid);
  }
}

// y = epilogue(the sum of the K splits' int32 partials [splits][M][N]),
// four columns per thread (N % 4 == 0); the sums are exact, so the result
// is the unsplit kernel's bit for bit
__global__ __launch_bounds__(256) void s8_splitk_sum_kernel(DynArgs a, const int32_t *partial,
                                                            int splits) {
  const int M = (int)a.M, N = (int)a.N;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * (N / 4)) return;
  const int m = (int)(idx / (N / 4)), n = (int)(idx % (N / 4)) * 4;
  const size_t stride = (size_t)M * N;
  const int32_t *p = partial + (size_t)m * N + n;
  i32x4_t q[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    q[s] = s < splits ? *reinterpret_cast<const i32x4_t *>(p + s * stride) : i32x4_t{0, 0, 0, 0};
  i32x4_t v = q[0];
#pragma unroll
  for (int s = 1; s < 8; ++s) v += q[s];
  dyn_epilogue4(a, m, n, v);
}

// splits > 1: K split over a.split_part (int32 partials), then the sum
template <int BM, int BN, int WM, int WN, int ND, int S>
hipError_t launch_s8_ws(const DynArgs &a, hipStream_t s, int splits = 1) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  const int nk = (int)((a.K + kWsBK - 1) / kWsBK);
  const bool split = splits > 1 && a.split_part;
  const int sps = split ? (nk + splits - 1) / splits : nk;
  const int gy = split ? (nk + sps - 1) / sps : 1;
  s8_gemm_ws_kernel<BM, BN, WM, WN, ND, S>
      <<<dim3((unsigned)(tiles_m * tiles_n), (unsigned)gy), dim3(64 * (WM * WN + ND)),
         s8_ws_lds<BM, BN, S>(), s>>>(a, tiles_m, tiles_n, group_m,
                                      split ? a.split_part : nullptr, sps);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !split) return err;
  const int64_t n4 = a.M * (a.N / 4);
  s8_splitk_sum_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s>>>(a, a.split_part, gy);
  return hipGetLastError();
}

// Skinny int8 GEMM (M <= 16*MT tokens, weight-streaming: the whole of qx
// is reused by every workgroup from L2, W is read once).  One workgroup per
// block of TPW 16-row weight tiles over all of K; its NW waves split K into
// 64-wide chunks.  Per chunk a lane loads one 16-byte fragment of each of
// its TPW weight rows (A operand) and of each of the MT token tiles
// (B operand) into a ring of PF register slots; a slot is refilled right
// after its MFMAs, PF chunks ahead (a scheduling barrier keeps the compiler
// from sinking the refills).  D[n][m] leaves each lane four consecutive n of
// one token; the K partials meet in LDS in a fixed order (4 slabs; with 8
// waves the upper four first add onto the lower four) and the epilogue
// writes rows of 4 columns.
constexpr int kSkPitchPad = 4;

template <int MT, int TPW>
constexpr size_t s8_skinny_lds() {
  return (size_t)4 * (16 * MT) * (16 * TPW + kSkPitchPad) * 4;
}

// Sum of the four K-partial slabs [4][ROWS][16*TPW + pad] int32 and the
// dequantising epilogue, for the skinny kernels (ROWS tokens, TPW 16-row
// weight tiles from n0, 64*NW threads).
// Epilogue of a ROWS x COLS int32 tile (rows 0.., columns n0..) over NT
// threads.  Thread t < T = RP * Q (Q = COLS / 4 column quads, RP = NT / Q
// rows per pass) keeps quad t % Q for rows t / Q + k RP, so its weight
// scales, bias and column sums and its rows' scales and offsets are loaded
// once, by prefetch(), which the kernels call before their final reductions
// so that those loads are in flight meanwhile.  Same arithmetic as
// dyn_epilogue4; post-ops, requantised or int32 outputs and a row length
// that is not a multiple of 4 take dyn_epilogue4 itself.
template <int ROWS, int COLS, int NT>
struct QuadEpi {
  static constexpr int Q = COLS / 4, RP = NT / Q, T = RP * Q, KR = (ROWS + RP - 1) / RP;
  bool fast;
  int c4, r0;
  float sw[4], b[4], sx[KR];
  int32_t cs[4], az[KR];

  // sxp, when set, replaces a.sx
  const float *sxp;

  __device__ __forceinline__ void prefetch(const DynArgs &a, int n0, int tid,
                                           const float *sx_override = nullptr) {
    sxp = sx_override;
    const int M = (int)a.M, N = (int)a.N;
    fast = (a.y_dt == ZT_DT_BF16 || a.y_dt == ZT_DT_F32) && a.post.count == 0 && (N & 3) == 0;
    c4 = (tid % Q) * 4;
    r0 = tid / Q;
    if (!fast || tid >= T || n0 + c4 >= N) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sw[r] = wscale(a, n0 + c4 + r);
      b[r] = a.bias ? load_elem(a.bias, a.b_dt, n0 + c4 + r) : 0.f;
      cs[r] = a.azp ? a.colsum[n0 + c4 + r] : 0;
    }
#pragma unroll
    for (int k = 0; k < KR; ++k) {
      const int m = r0 + k * RP;
      sx[k] = m < M && m < ROWS ? (sxp ? sxp[m] : a.sx[m]) : 0.f;
      az[k] = a.azp && m < M && m < ROWS ? a.azp[m] : 0;
    }
  }

  // v(m, c) returns the int32 sums of row m, columns c .. c + 3
  template <typename V>
  __device__ __forceinline__ void finish(const DynArgs &a, int n0, int tid, V v) {
    const int M = (int)a.M, N = (int)a.N;
    if (!fast) {
      for (int idx = tid; idx < ROWS * Q; idx += NT) {
        const int m = idx / Q, c = (idx % Q) * 4;
        if (m < M && n0 + c < N) dyn_epilogue4(a, m, n0 + c, v(m, c), sxp);
      }
      return;
    }
    const int n = n0 + c4;
    if (tid >= T || n >= N) return;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
      const int m = r0 + k * RP;
      if (m >= M || m >= ROWS) break;
      i32x4_t s = v(m, c4);
      if (a.azp) s -= i32x4_t{cs[0], cs[1], cs[2], cs[3]} * az[k];
      float f[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = (float)s[r] * sx[k];
        t = t * sw[r];
        f[r] = a.bias ? t + b[r] : t;
      }
      if (a.y_dt == ZT_DT_BF16) {
        u32x2_t pk;
        pk[0] = pack_bf16x2(f[0], f[1]);
        pk[1] = pack_bf16x2(f[2], f[3]);
        *reinterpret_cast<u32x2_t *>(reinterpret_cast<uint16_t *>(a.y) + (int64_t)m * N + n) = pk;
      } else {
        *reinterpret_cast<f32x4_t *>(reinterpret_cast<float *>(a.y) + (int64_t)m * N + n) =
            f32x4_t{f[0], f[1], f[2], f[3]};
      }
    }
  }
};

// Epilogue of the skinny kernels: the four K-partial slabs [4][ROWS][P] are
// added and finished by ep (prefetched by the kernel).
template <int ROWS, int TPW, int NW>
__device__ __forceinline__ void skinny_epilogue(const DynArgs &a, const int32_t *slab, int n0,
                                                int tid, QuadEpi<ROWS, 16 * TPW, 64 * NW> &ep) {
  constexpr int P = 16 * TPW + kSkPitchPad;
  ep.finish(a, n0, tid, [&](int m, int c) {
    i32x4_t v = *reinterpret_cast<const i32x4_t *>(slab + m * P + c);
#pragma unroll
    for (int w = 1; w < 4; ++w) v += *reinterpret_cast<const i32x4_t *>(slab + (w * ROWS + m) * P + c);
    return v;
  });
}

template <int MT, int TPW, int PF, int NW>
__global__ __launch_bounds__(64 * NW) void s8_skinny_kernel(DynArgs a, int chunks_per_wave) {
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int n0 = blockIdx.x * (16 * TPW);
  const auto q_rs = make_rsrc(a.qx, (uint32_t)((int64_t)M * K));
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));

  uint32_t w_row[TPW], q_row[MT];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int n = n0 + t * 16 + lr;
    w_row[t] = n < N ? (uint32_t)(n * K) : kOobOffset;
  }
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int m = j * 16 + lr;
    q_row[j] = m < M ? (uint32_t)(m * K) : kOobOffset;
  }
  const int c_begin = wv * chunks_per_wave;
  const int total = K / 64;
  const int nch = max(0, min(chunks_per_wave, total - c_begin));

  // K % 64 == 0 (host-checked): every lane's k of a chunk inside the wave's
  // range is < K.  A row past M/N starts at kOobOffset and stays out of
  // range after adding k; a chunk past the wave's range (c >= nch, the
  // same for the whole wave) is read at kOobOffset too.  (A row past M/N in
  // a chunk past the range wraps to a small in-range offset: the read is in
  // bounds and only feeds an output row or column that is never stored.)
  i32x4_t wf[PF][TPW], qf[PF][MT];
  auto load = [&](int slot, int c) {
    const uint32_t kc = c < nch ? (uint32_t)((c_begin + c) * 64) : kOobOffset;
    const uint32_t k = kc + 16u * lg;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
      wf[slot][t] = __builtin_bit_cast(
          i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rs, w_row[t] + k, 0, 0));
#pragma unroll
    for (int j = 0; j < MT; ++j)
      qf[slot][j] = __builtin_bit_cast(
          i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(q_rs, q_row[j] + k, 0, 0));
  };

  i32x4_t acc[TPW][MT];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[t][j] = i32x4_t{0, 0, 0, 0};

  // the epilogue's per-column and per-row values, in flight with the chunks
  QuadEpi<16 * MT, 16 * TPW, 64 * NW> ep;
  ep.prefetch(a, n0, tid);
#pragma unroll
  for (int p = 0; p < PF; ++p) load(p, p);
  for (int c = 0; c < nch; c += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[p][t], qf[p][j], acc[t][j], 0, 0, 0);
      load(p, c + p + PF);  // chunks past nch read as zero and are never used
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // K partials: slab[w][m][n_local], n_local = t*16 + 4*lg + r
  constexpr int P = 16 * TPW + kSkPitchPad;
  int32_t *slab = reinterpret_cast<int32_t *>(s8_smem);
  auto slab_at = [&](int w, int t, int j) {
    return reinterpret_cast<i32x4_t *>(slab + ((w * 16 * MT) + j * 16 + lr) * P + t * 16 + 4 * lg);
  };
  if (NW == 8 && wv >= 4) {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < MT; ++j) *slab_at(wv - 4, t, j) = acc[t][j];
  }
  if (NW == 8) __syncthreads();
  if (wv < 4) {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        i32x4_t v = acc[t][j];
        if (NW == 8) v += *slab_at(wv, t, j);
        *slab_at(wv, t, j) = v;
      }
  }
  __syncthreads();
  skinny_epilogue<16 * MT, TPW, NW>(a, slab, n0, tid, ep);
}

// The 16-token skinny GEMM with the per-token quantisation in its
// prologue (symmetric s8; bf16 x [M, K] in 16-byte rows, M <= RM, and each
// row at most VR vectors of 8 elements per thread).  Every workgroup
// quantises all of x itself into an LDS copy of qx [M][K + 16] and of sx,
// with the quantise kernel's arithmetic (the row's amax over the whole
// workgroup, sx = max(amax, 1e-12) / 127, q = clamp(rint(x / sx), -128,
// 127)), so qx and sx are bit-identical to that pass.  Its first PF chunks
// of weights are requested in the prologue, so the quantisation runs while
// they are in flight (the compiler issues them once x has landed; pinning
// them before x, right after it or before the amax shuffles measured 1-4 %
// slower); the chunk loop then reads its B operands from LDS (token
// columns past M read row M - 1; their sums are never stored).  The call
// loses the quantise launch and the trip of qx through memory; in exchange
// every workgroup reads x (2 M K bytes, from its XCD's L2) and repeats the
// quantisation, so it serves few tokens only.
template <int TPW, int PF, int NW, int RM, int VR>
__global__ __launch_bounds__(64 * NW) void s8_skinny_fused_kernel(DynArgs a, int chunks_per_wave) {
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int n0 = blockIdx.x * (16 * TPW);
  const int QP = K + 16;  // qx row pitch (K % 64 == 0: rows stay 16-byte aligned)
  // LDS: the K-partial slabs, qx [M][QP], sx [16], the amax partials [NW][RM]
  int32_t *slab = reinterpret_cast<int32_t *>(s8_smem);
  int8_t *ql = s8_smem + s8_skinny_lds<1, TPW>();
  float *sxl = reinterpret_cast<float *>(ql + (size_t)M * QP);
  float *red = sxl + 16;
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));
  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)M * K * 2));

  uint32_t w_row[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int n = n0 + t * 16 + lr;
    w_row[t] = n < N ? (uint32_t)(n * K) : kOobOffset;
  }
  const int c_begin = wv * chunks_per_wave;
  const int total = K / 64;
  const int nch = max(0, min(chunks_per_wave, total - c_begin));
  // weight chunks past the wave's slice read zeros (as in s8_skinny_kernel);
  // the qx reads of those chunks are clamped into the row and never used
  i32x4_t wf[PF][TPW], qf[PF];
  auto load_w = [&](int slot, int c) {
    const uint32_t kc = c < nch ? (uint32_t)((c_begin + c) * 64) : kOobOffset;
    const uint32_t k = kc + 16u * lg;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
      wf[slot][t] = __builtin_bit_cast(
          i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rs, w_row[t] + k, 0, 0));
  };
  const int qrow = min(lr, M - 1) * QP + 16 * lg;
  auto load_q = [&](int slot, int c) {
    const int kc = min(c_begin + c, total - 1) * 64;
    qf[slot] = *reinterpret_cast<const i32x4_t *>(ql + qrow + kc);
  };

  // 1. the first PF chunks of weights and x: thread tid holds the vectors
  //    j = tid + NT * i (i < VR) of each row m < RM (rows past M and vectors
  //    past the row read zeros)
#pragma unroll
  for (int p = 0; p < PF; ++p) load_w(p, p);
  const int nv = K >> 3;
  u32x4_t xv[RM][VR];
#pragma unroll
  for (int m = 0; m < RM; ++m)
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int j = tid + NT * i;
      const uint32_t off = m < M && j < nv ? (uint32_t)(m * K + j * 8) * 2u : kOobOffset;
      xv[m][i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rs, off, 0, 0));
    }
  // 2. each row's amax: per thread, per wave, then over the NW waves
  float hi[RM];
#pragma unroll
  for (int m = 0; m < RM; ++m) {
    hi[m] = 0.f;
#pragma unroll
    for (int i = 0; i < VR; ++i)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float e0 = __uint_as_float(xv[m][i][w] << 16);
        const float e1 = __uint_as_float(xv[m][i][w] & 0xffff0000u);
        hi[m] = fmaxf(hi[m], fmaxf(fabsf(e0), fabsf(e1)));
      }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) hi[m] = fmaxf(hi[m], __shfl_xor(hi[m], off, kWave));
  }
  if (lane == 0)
#pragma unroll
    for (int m = 0; m < RM; ++m) red[wv * RM + m] = hi[m];
  __syncthreads();
  // 3. lane m < RM of every wave forms row m's scale and its reciprocal;
  //    the wave shares them by shuffles
  float s_l, inv_l;
  {
    const int m = lane < RM ? lane : 0;
    float amax = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) amax = fmaxf(amax, red[w * RM + m]);
    float zp;
    row_qparams<false>(-amax, amax, s_l, zp);
    inv_l = __fdiv_rn(1.0f, s_l);
  }
  if (wv == 0 && lane < RM && lane < M) sxl[lane] = s_l;
  // 4. qx into LDS, eight bytes per vector
#pragma unroll
  for (int m = 0; m < RM; ++m) {
    const float sm = __shfl(s_l, m, kWave), im = __shfl(inv_l, m, kWave);
    if (m >= M) break;
    auto q1 = [&](float f) { return (uint32_t)(uint8_t)(int8_t)quant_one<false>(f, sm, im, 0.f); };
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int j = tid + NT * i;
      if (j >= nv) break;
      u32x2_t o;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t a0 = xv[m][i][2 * h], a1 = xv[m][i][2 * h + 1];
        o[h] = q1(__uint_as_float(a0 << 16)) | (q1(__uint_as_float(a0 & 0xffff0000u)) << 8) |
               (q1(__uint_as_float(a1 << 16)) << 16) | (q1(__uint_as_float(a1 & 0xffff0000u)) << 24);
      }
      *reinterpret_cast<u32x2_t *>(ql + m * QP + j * 8) = o;
    }
  }
  __syncthreads();

  // 5. the chunks, as in s8_skinny_kernel; the epilogue reads sx from LDS
  QuadEpi<16, 16 * TPW, NT> ep;
  ep.prefetch(a, n0, tid, sxl);
  i32x4_t acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = i32x4_t{0, 0, 0, 0};
#pragma unroll
  for (int p = 0; p < PF; ++p) load_q(p, p);
  for (int c = 0; c < nch; c += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
#pragma unroll
      for (int t = 0; t < TPW; ++t)
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[p][t], qf[p], acc[t], 0, 0, 0);
      load_w(p, c + p + PF);
      load_q(p, c + p + PF);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // 6. K partials: slab[w][m][n_local], n_local = t*16 + 4*lg + r
  constexpr int P = 16 * TPW + kSkPitchPad;
  auto slab_at = [&](int w, int t) {
    return reinterpret_cast<i32x4_t *>(slab + (w * 16 + lr) * P + t * 16 + 4 * lg);
  };
  if (NW == 8 && wv >= 4) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) *slab_at(wv - 4, t) = acc[t];
  }
  if (NW == 8) __syncthreads();
  if (wv < 4) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      i32x4_t v = acc[t];
      if (NW == 8) v += *slab_at(wv, t);
      *slab_at(wv, t) = v;
    }
  }
  __syncthreads();
  skinny_epilogue<16, TPW, NW>(a, slab, n0, tid, ep);
}

// The skinny GEMM on v_mfma_i32_32x32x32_i8 (twice the int8 rate of the
// 16x16x64 shape on gfx950), for qx in fragment order (qx_frag_offset,
// written by the quantise kernels of zt_dynamic_qlinear).  MT 32-token tiles,
// TPW 16-row weight tiles per workgroup, NW waves splitting K into 64-wide
// chunks, PF chunks of loads in flight per wave, as in s8_skinny_kernel.
// Weights load as two 16-row x 64 B tiles; one v_permlane16_swap per dword
// turns a pair into the two 32-row A operands of a chunk (k blocks {0, 2}
// and {1, 3} of each row), which pair with qx fragments 0 and 1.  An odd
// last tile pairs with zeros.  D[n][m] leaves each lane four runs of four
// consecutive n of one token; the K partials meet in LDS as in the 16-token
// kernel.
template <int MT, int TPW, int PF, int NW>
__global__ __launch_bounds__(64 * NW) void s8_skinny32_kernel(DynArgs a, int chunks_per_wave) {
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];
  constexpr int NG = (TPW + 1) / 2;  // 32-row groups
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4, lh = lane >> 5;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int n0 = blockIdx.x * (16 * TPW);
  const int tiles_m = (M + 31) >> 5;
  const auto q_rs = make_rsrc(a.qx, (uint32_t)(tiles_m * 32 * K));
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));

  uint32_t w_row[TPW], q_tile[MT];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int n = n0 + t * 16 + lr;
    w_row[t] = n < N ? (uint32_t)(n * K + 16 * lg) : kOobOffset;
  }
#pragma unroll
  for (int j = 0; j < MT; ++j) q_tile[j] = j < tiles_m ? (uint32_t)(j * 32 * K) : kOobOffset;
  const int c_begin = wv * chunks_per_wave;
  const int nch = max(0, min(chunks_per_wave, K / 64 - c_begin));

  // K % 64 == 0 (host-checked).  A weight row past N, a token tile past M
  // and a chunk past the wave's range start at kOobOffset and read zeros;
  // two of them together wrap to a small in-range offset, whose data only
  // reaches an output row or column that is never stored.  Tokens of the
  // last tile past M read whatever the workspace holds, with the same
  // effect.
  i32x4_t wf[PF][TPW], qf[PF][MT][2];
  auto load = [&](int slot, int c) {
    const bool in = c < nch;
    const uint32_t kw = in ? (uint32_t)((c_begin + c) * 64) : kOobOffset;
    const uint32_t kq = in ? (uint32_t)((c_begin + c) * 2048) + 16u * lane : kOobOffset;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
      wf[slot][t] = __builtin_bit_cast(
          i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rs, w_row[t] + kw, 0, 0));
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int f = 0; f < 2; ++f)
        qf[slot][j][f] = __builtin_bit_cast(
            i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(q_rs, q_tile[j] + kq + 1024u * f, 0, 0));
  };

  i32x16_t acc[NG][MT];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][j][r] = 0;

  // the epilogue's per-column and per-row values, in flight with the chunks
  QuadEpi<32 * MT, 16 * TPW, 64 * NW> ep;
  ep.prefetch(a, n0, tid);
#pragma unroll
  for (int p = 0; p < PF; ++p) load(p, p);
  for (int c = 0; c < nch; c += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        i32x4_t a0 = wf[p][2 * g], a1 = 2 * g + 1 < TPW ? wf[p][2 * g + 1] : i32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const auto sw = __builtin_amdgcn_permlane16_swap((uint32_t)a0[e], (uint32_t)a1[e],
                                                          false, false);
          a0[e] = (int32_t)sw[0];
          a1[e] = (int32_t)sw[1];
        }
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          acc[g][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qf[p][j][0], acc[g][j], 0, 0, 0);
          acc[g][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qf[p][j][1], acc[g][j], 0, 0, 0);
        }
      }
      load(p, c + p + PF);  // chunks past nch read as zero and are never used
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // K partials: slab[w][m][n_local]; D register r of lane l holds
  // n_local = 32*g + 8*(r/4) + 4*(l/32) + r%4 of token 32*j + l%32
  constexpr int ROWS = 32 * MT, P = 16 * TPW + kSkPitchPad;
  int32_t *slab = reinterpret_cast<int32_t *>(s8_smem);
  auto put = [&](int w, bool add) {
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (2 * g + 1 >= TPW && q >= 2) continue;  // rows of the zero half
          i32x4_t *d = reinterpret_cast<i32x4_t *>(
              slab + (w * ROWS + 32 * j + (lane & 31)) * P + 32 * g + 8 * q + 4 * lh);
          i32x4_t v = {acc[g][j][4 * q], acc[g][j][4 * q + 1], acc[g][j][4 * q + 2],
                       acc[g][j][4 * q + 3]};
          if (add) v += *d;
          *d = v;
        }
  };
  if (NW == 8 && wv >= 4) put(wv - 4, false);
  if (NW == 8) __syncthreads();
  if (wv < 4) put(wv, NW == 8);
  __syncthreads();
  skinny_epilogue<ROWS, TPW, NW>(a, slab, n0, tid, ep);
}

template <int MT, int TPW, int PF, int NW>
hipError_t launch_s8_skinny32_t(const DynArgs &a, hipStream_t s) {
  const int total = (int)(a.K / 64);
  int cpw = (total + NW - 1) / NW;
  cpw = (cpw + PF - 1) / PF * PF;
  const int blocks = (int)((a.N + 16 * TPW - 1) / (16 * TPW));
  const size_t lds = (size_t)4 * (32 * MT) * (16 * TPW + kSkPitchPad) * 4;
  s8_skinny32_kernel<MT, TPW, PF, NW><<<dim3((unsigned)blocks), dim3(64 * NW), lds, s>>>(a, cpw);
  return hipGetLastError();
}

hipError_t launch_s8_skinny32(const DynArgs &a, hipStream_t s) {
  const int mt = (int)((a.M + 31) / 32);
  const char *e = knob(kKnobS8Skinny32);  // "TPW,PF,NW"
  int tpw = 0, pf = 0, nw = 0;
  if (e) {
    std::sscanf(e, "%d,%d,%d", &tpw, &pf, &nw);
  } else if (mt <= 2 && a.N <= 8192) {
    // up to 64 tokens: 16-row weight tiles up to 4096 rows, 32-row tiles up
    // to 8192, so that those matrices give at least 128 workgroups (graph
    // replays over rotating weights, one box, against 64-row tiles: at M =
    // 17 / 64 O 4096 x 4096 20.3 -> 12.5 / 22.1 -> 15.3 us, down 4096 x
    // 14336 51.9 -> 27.0 / 58.8 -> 34.4, QKV 6144 x 4096 20.7 -> 16.1 /
    // 22.8 -> 18.7; 11008 and 28672 rows keep 64-row tiles, 4-30 % faster)
    tpw = a.N <= 4096 ? 1 : 2, pf = 4, nw = 8;
  }
#define ZT_SK(MT_, TPW_, PF_, NW_)                                            \
  if (mt <= MT_ && (!tpw || (tpw == TPW_ && pf == PF_ && nw == NW_)))          \
    return launch_s8_skinny32_t<MT_, TPW_, PF_, NW_>(a, s);
  ZT_SK(1, 4, 4, 8) ZT_SK(2, 4, 2, 8) ZT_SK(4, 3, 2, 8) ZT_SK(4, 2, 2, 8) ZT_SK(4, 4, 2, 8)
  ZT_SK(4, 3, 4, 4) ZT_SK(4, 4, 4, 4) ZT_SK(1, 2, 4, 8) ZT_SK(1, 1, 4, 8) ZT_SK(2, 2, 2, 8)
  ZT_SK(2, 2, 4, 8) ZT_SK(2, 1, 4, 8)
#undef ZT_SK
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------- split-K skinny
// Skinny int8 GEMM for 64 < M <= 128 tokens with K split in two halves
// across workgroups (qx in fragment order, K % 256 == 0).  The
// weight-streaming kernels above give each workgroup all of K, so every CU
// pulls the whole of qx through its vector memory path (at M = 128, 2.7 x
// the weight bytes it streams); here a CU pulls half of it.
//
// Workgroup (tile, half) takes 96 weight rows (three 32-row groups) over K
// half `half`; its eight waves are (token tile j = w % 4, chunk parity
// h = w / 4).  A step covers two 128-k chunks, one per parity:
//  * the weight slab [2][96][128 B] moves into LDS by DMA, three 1 KB
//    instructions per wave, each eight whole 128-byte rows (the 16-byte
//    blocks of row r are XOR-swizzled by (r >> 1) & 7, so the 32-row
//    fragment reads hit each bank once);
//  * a wave loads the qx fragments of its token tile and chunk straight to
//    registers;
//  * a wave runs 12 v_mfma_i32_32x32x32_i8 (3 row groups x 4 32-k steps):
//    W is A (row 32g + l%32, k block f + 2 (l/32) of each 64-k half, the
//    blocks qx fragment f pairs with), qx is B.
// PD steps of loads are in flight (PD + 1 LDS stages, one barrier a step;
// steps past the half read zeros).  The two parities meet in LDS.  Both
// halves of a tile write their int32 partial tile to the workspace; the
// second workgroup of the tile to finish (a per-tile counter) adds the
// other half's partial and runs the epilogue.  The partials are written and
// read with device-scope (sc1) accesses, the memory instructions of relaxed
// device-scope atomic stores and loads, and the writer waits for its stores
// to complete before the counter's atomic add: the exchange needs neither an
// L2 writeback nor an invalidate (a release / acquire fence pair makes every
// workgroup write back its XCD's whole dirty L2).  The sums are integers, so the result does not depend on which
// half finishes last.  Workgroups b and b + 8 of every 16 are the two
// halves of one tile (the same XCD under round-robin dispatch).
constexpr int kSpBN = 96;                 // weight rows per workgroup
constexpr int kSpChunk = kSpBN * 128;     // LDS bytes of one 128-k weight chunk
constexpr int kSpStep = 2 * kSpChunk;     // one chunk per parity
constexpr int kSpPart = 128 * kSpBN;      // int32 partials of a workgroup
constexpr int kSpTileP = kSpBN + 4;       // row pitch of the staged output tile
constexpr int kSpSlabB = 4 * 48 * 64 * 4;  // the parity-1 waves' accumulators
constexpr int kSpFlagOff = kSpSlabB + 128 * kSpTileP * 4;
constexpr int kSc1 = 16;  // cache-policy bit of device-scope accesses (sc1)

template <int PD>
constexpr size_t s8_splitk_lds() {
  const size_t stages = (size_t)(PD + 1) * kSpStep;
  const size_t tail = (size_t)kSpFlagOff + 16;
  return stages > tail ? stages : tail;
}

template <int PD>
__global__ __launch_bounds__(512) void s8_splitk_kernel(DynArgs a, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) int8_t s8_smem[];
  constexpr int NS = PD + 1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  const int tile = (b >> 4) * 8 + (b & 7), half = (b >> 3) & 1;
  if (tile >= tiles_n) return;  // the grid is a whole number of 16-blocks
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int n0 = tile * kSpBN;
  const int tiles_m = (M + 31) >> 5;
  const int nch = K >> 8;  // 128-k chunks per half
  const int kc0 = half * nch;
  const int nsteps = (((nch + 1) >> 1) + PD - 1) / PD * PD;
  const int j = wv & 3, h = wv >> 2;
  const auto q_rs = make_rsrc(a.qx, (uint32_t)(tiles_m * 32 * K));
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * K));

  // DMA instruction 3 wv + u of a step: rows 8 (q % 12) .. + 7 of chunk
  // parity q / 12 (= h); lane l takes 16-byte block (l % 8) ^ swz of row
  // 8 (q % 12) + l / 8 (N * K < 2^31, host-checked)
  uint32_t w_src[3];
  int w_dst[3];
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int rb = (3 * wv + u) % 12;
    const int lr = 8 * rb + (lane >> 3), n = n0 + lr;
    const int blk = (lane & 7) ^ ((lr >> 1) & 7);
    w_src[u] = n < N ? (uint32_t)(n * K + blk * 16) : kOobOffset;
    w_dst[u] = h * kSpChunk + rb * 1024;
  }
  auto dma = [&](int st) {
    int8_t *stage = s8_smem + (st % NS) * kSpStep;
    const int c = 2 * st + h;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const uint32_t off = (w_src[u] == kOobOffset || c >= nch)
                               ? kOobOffset : w_src[u] + (uint32_t)((kc0 + c) * 128);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (lds_ptr_t)(stage + w_dst[u]), 16, off, 0, 0,
                                               0);
    }
  };
  // qx fragment (tile j, 64-k chunk c64, f) at ((j (K/64) + c64) 2 + f) KB
  const uint32_t q_base = j < tiles_m ? (uint32_t)(j * (K >> 6) * 2048) + 16u * lane : kOobOffset;
  i32x4_t qf[PD][2][2];
  auto ldq = [&](int st, int slot) {
    const int c = 2 * st + h;
    const bool in = q_base != kOobOffset && c < nch;
    const uint32_t base = in ? q_base + (uint32_t)((kc0 + c) * 4096) : 0u;
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int f = 0; f < 2; ++f)
        qf[slot][e][f] = __builtin_bit_cast(
            i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         q_rs, in ? base + (uint32_t)(e * 2048 + f * 1024) : kOobOffset, 0, 0));
  };

  i32x16_t acc[3];
#pragma unroll
  for (int g = 0; g < 3; ++g)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[g][r] = 0;
  const int swz = ((lane & 31) >> 1) & 7;
  const int a_row = (lane & 31) * 128;
  auto compute = [&](int st, int slot) {
    const int8_t *stage = s8_smem + (st % NS) * kSpStep + h * kSpChunk + a_row;
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int pos = ((4 * e + f + 2 * (lane >> 5)) ^ swz) << 4;
        i32x4_t wa[3];
#pragma unroll
        for (int g = 0; g < 3; ++g)
          wa[g] = *reinterpret_cast<const i32x4_t *>(stage + g * 32 * 128 + pos);
#pragma unroll
        for (int g = 0; g < 3; ++g)
          acc[g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa[g], qf[slot][e][f], acc[g], 0, 0, 0);
      }
  };

  // the epilogue's per-column and per-row values, loaded first: a step's
  // wait below then counts only the loads issued after its own
  QuadEpi<128, kSpBN, 512> ep;
  ep.prefetch(a, n0, tid);
#pragma unroll
  for (int p = 0; p < PD; ++p) {
    dma(p);
    ldq(p, p);
  }
  for (int st0 = 0; st0 < nsteps; st0 += PD) {
#pragma unroll
    for (int p = 0; p < PD; ++p) {
      const int st = st0 + p;
      // this step's 3 DMA + 4 qx loads are the oldest of the PD steps in flight
      __builtin_amdgcn_s_waitcnt(vmcnt_wait_imm(7 * (PD - 1)));
      asm volatile("s_barrier" ::: "memory");
      dma(st + PD);  // into the stage of step st - 1, which every wave has finished
      compute(st, p);
      ldq(st + PD, p);
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_wait_imm(0));  // the zero-filling DMA past the end
  __syncthreads();

  // the parities meet: slab[j][g][r][lane]
  int32_t *slab = reinterpret_cast<int32_t *>(s8_smem);
  if (h == 1) {
#pragma unroll
    for (int g = 0; g < 3; ++g)
#pragma unroll
      for (int r = 0; r < 16; ++r) slab[((j * 3 + g) * 16 + r) * 64 + lane] = acc[g][r];
  }
  __syncthreads();
  if (h == 0) {
#pragma unroll
    for (int g = 0; g < 3; ++g)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][r] += slab[((j * 3 + g) * 16 + r) * 64 + lane];
    const auto mine = make_rsrc(a.split_part + ((size_t)tile * 2 + half) * kSpPart, kSpPart * 4);
#pragma unroll
    for (int g = 0; g < 3; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4_t{(uint32_t)acc[g][4 * q], (uint32_t)acc[g][4 * q + 1],
                    (uint32_t)acc[g][4 * q + 2], (uint32_t)acc[g][4 * q + 3]},
            mine, (uint32_t)((((j * 3 + g) * 4 + q) * 64 + lane) * 16), 0, kSc1);
    __builtin_amdgcn_s_waitcnt(vmcnt_wait_imm(0));  // the partial is at device scope
  }
  // count the halves done; the first to finish leaves
  __syncthreads();
  int32_t *flag = reinterpret_cast<int32_t *>(s8_smem + kSpFlagOff);
  if (tid == 0) *flag = atomicAdd(a.split_cnt + tile, 1);
  __syncthreads();
  if (*flag == 0) return;
  int32_t *tl = reinterpret_cast<int32_t *>(s8_smem + kSpSlabB);
  if (h == 0) {
    const auto other =
        make_rsrc(a.split_part + ((size_t)tile * 2 + (half ^ 1)) * kSpPart, kSpPart * 4);
    // D[n][m]: register r of lane l holds row 32g + 8 (r/4) + 4 (l/32) + r%4
    // of the tile and token 32 j + l%32
#pragma unroll
    for (int g = 0; g < 3; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const i32x4_t o = __builtin_bit_cast(
            i32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         other, (uint32_t)((((j * 3 + g) * 4 + q) * 64 + lane) * 16), 0, kSc1));
        *reinterpret_cast<i32x4_t *>(tl + (32 * j + (lane & 31)) * kSpTileP + 32 * g + 8 * q +
                                     4 * (lane >> 5)) =
            i32x4_t{acc[g][4 * q] + o[0], acc[g][4 * q + 1] + o[1], acc[g][4 * q + 2] + o[2],
                    acc[g][4 * q + 3] + o[3]};
      }
  }
  __syncthreads();
  ep.finish(a, n0, tid, [&](int m, int c) {
    return *reinterpret_cast<const i32x4_t *>(tl + m * kSpTileP + c);
  });
}

template <int PD>
hipError_t launch_s8_splitk_t(const DynArgs &a, hipStream_t s) {
  const int tiles_n = s8_split_counters(a.N);
  const unsigned blocks = (unsigned)((tiles_n + 7) / 8 * 16);
  s8_splitk_kernel<PD><<<dim3(blocks), dim3(512), s8_splitk_lds<PD>(), s>>>(a, tiles_n);
  return hipGetLastError();
}

bool s8_split_shape(int64_t M, int64_t K, int64_t N) {
  const int64_t rows = (M + 31) / 32 * 32;
  return M > 64 && M <= 128 && K % 256 == 0 && N > 0 && N * K < (int64_t)kOobOffset &&
         rows * K < (int64_t)kOobOffset;
}

bool s8_split_ok(const DynArgs &a) {
  const char *e = knob(kKnobS8Split);
  if (e && e[0] == '0') return false;
  return a.qx_frag && a.split_part && a.split_cnt && s8_split_shape(a.M, a.K, a.N) &&
         ((reinterpret_cast<uintptr_t>(a.split_part) | reinterpret_cast<uintptr_t>(a.w) |
           reinterpret_cast<uintptr_t>(a.qx)) & 15u) == 0;
}

hipError_t launch_s8_splitk(const DynArgs &a, hipStream_t s) {
  // "2" .. "4": steps of loads in flight (2 measured fastest at M = 128,
  // N = 11008, K = 4096: 19.6 us against 20.8 for 3)
  const char *e = knob(kKnobS8Split);
  const int pd = e && e[0] >= '2' && e[0] <= '4' ? e[0] - '0' : 2;
  if (pd == 3) return launch_s8_splitk_t<3>(a, s);
  if (pd == 4) return launch_s8_splitk_t<4>(a, s);
  return launch_s8_splitk_t<2>(a, s);
}

template <int MT, int TPW, int PF, int NW>
hipError_t launch_s8_skinny_t(const DynArgs &a, hipStream_t s) {
  const int total = (int)(a.K / 64);
  int cpw = (total + NW - 1) / NW;
  cpw = (cpw + PF - 1) / PF * PF;
  const int blocks = (int)((a.N + 16 * TPW - 1) / (16 * TPW));
  s8_skinny_kernel<MT, TPW, PF, NW><<<dim3((unsigned)blocks), dim3(64 * NW),
                                      s8_skinny_lds<MT, TPW>(), s>>>(a, cpw);
  return hipGetLastError();
}

hipError_t launch_s8_skinny(const DynArgs &a, hipStream_t s) {
  const int mt = (int)((a.M + 15) / 16);
  const char *e = knob(kKnobS8Skinny);  // "TPW,PF,NW"
  int tpw = 0, pf = 0, nw = 0;
  if (e) {
    std::sscanf(e, "%d,%d,%d", &tpw, &pf, &nw);
  } else if (mt == 1) {
    // one token tile: 16-row weight tiles, as many workgroups as CUs or
    // more, except 32-row tiles from 4097 to 8192 rows and 64-row tiles
    // past 12288 (graph replays over rotating weights, M = 1..16, one box:
    // at M = 1 O 4096 x 4096 18.1 -> 11.0 us, down 4096 x 14336 44.9 ->
    // 20.3, QKV 6144 x 4096 18.7 -> 13.8, 11008 x 4096 20.4 -> 17.8, all
    // against 64-row tiles; gate_up 28672 x 4096 keeps them, 37.4 against
    // 40.2 with 16-row tiles at M = 8; at M = 9 / 16 14336 x 4096 22.3 /
    // 23.2 against 23.5 / 26.3 with 16-row tiles, 16384 x 3072 19.2 / 19.8
    // against 20.2 / 22.5)
    tpw = a.N > 12288 ? 4 : (a.N > 4096 && a.N <= 8192) ? 2 : 1;
    pf = 4, nw = 8;
  }
#define ZT_SK(MT_, TPW_, PF_, NW_)                                            \
  if (mt <= MT_ && (!tpw || (tpw == TPW_ && pf == PF_ && nw == NW_)))          \
    return launch_s8_skinny_t<MT_, TPW_, PF_, NW_>(a, s);
  ZT_SK(1, 4, 4, 8) ZT_SK(1, 1, 4, 8) ZT_SK(1, 1, 8, 8) ZT_SK(1, 2, 4, 8)
  ZT_SK(2, 4, 4, 8) ZT_SK(4, 2, 4, 8)
  ZT_SK(8, 3, 2, 8) ZT_SK(8, 2, 3, 8) ZT_SK(8, 2, 4, 4) ZT_SK(8, 1, 4, 8) ZT_SK(8, 4, 2, 8)
  ZT_SK(8, 3, 4, 4)
#undef ZT_SK
  return hipErrorInvalidValue;
}

template <int TPW, int PF, int RM, int VR>
hipError_t launch_s8_skinny_fused_t(const DynArgs &a, hipStream_t s) {
  constexpr int NW = 8;
  const int total = (int)(a.K / 64);
  int cpw = (total + NW - 1) / NW;
  cpw = (cpw + PF - 1) / PF * PF;
  const int blocks = (int)((a.N + 16 * TPW - 1) / (16 * TPW));
  s8_skinny_fused_kernel<TPW, PF, NW, RM, VR><<<dim3((unsigned)blocks), dim3(64 * NW),
                                                 s8_fused_lds(a.M, a.K, TPW), s>>>(a, cpw);
  return hipGetLastError();
}

template <int BM, int BN>
hipError_t launch_s8_tiled(const DynArgs &a, hipStream_t s) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  s8_gemm_tiled_kernel<BM, BN><<<dim3((unsigned)(tiles_m * tiles_n)), dim3(256),
                                  s8_tiled_lds<BM, BN>(), s>>>(a, tiles_m, tiles_n, group_m);
  return hipGetLastError();
}

}  // namespace

// Tokens up to which the fused kernel takes a call by default.
constexpr int64_t kS8FusedRows = 8;

// Vectors of 8 elements per thread and row of the fused kernel (512
// threads), and the fused kernel's LDS.
static int s8_fused_vr(int64_t K) { return (int)((K / 8 + 511) / 512); }
size_t s8_fused_lds(int64_t M, int64_t K, int tpw) {
  // the K-partial slabs (s8_skinny_lds<1, tpw>), qx, sx, the amax partials
  return (size_t)4 * 16 * (16 * tpw + kSkPitchPad) * 4 + (size_t)M * (size_t)(K + 16) + 16 * 4 +
         8 * 16 * 4;
}

bool s8_fused_ok(const DynArgs &a) {
  // "0": never; "1": wherever it applies; unset: up to kS8FusedRows tokens
  const char *e = knob(kKnobS8Fused);
  if (e && e[0] == '0') return false;
  if (a.x_dt != ZT_DT_BF16 || a.azp || a.qx_frag || a.out_scale || a.y_dt == ZT_DT_S32 ||
      a.M < 1 || a.M > 16 || a.K % 64 != 0 || a.N < 1)
    return false;
  if (((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.w)) & 15u) != 0)
    return false;
  if (a.N * a.K >= (int64_t)kOobOffset || a.M * a.K * 2 >= (int64_t)kOobOffset) return false;
  const int vr = s8_fused_vr(a.K);
  // rows the fused form takes per register layout; at 3-4 vectors per row
  // three (four rows held as 4 x 4 vectors measured 1-4 % slower than two
  // launches at M = 4 on 8192 x 16384, 6-10 % faster at M = 3)
  const int64_t rm = vr <= 1 ? 16 : vr <= 2 ? 4 : vr <= 4 ? 3 : vr <= 8 ? 2 : 0;
  if (a.M > rm || s8_fused_lds(a.M, a.K, 4) > 160 * 1024) return false;
  return (e && e[0] == '1') || a.M <= kS8FusedRows;
}

template <int TPW, int PF>
hipError_t launch_s8_skinny_fused_tp(const DynArgs &a, hipStream_t s) {
  const int vr = s8_fused_vr(a.K);
  if (vr == 1) return a.M <= 8 ? launch_s8_skinny_fused_t<TPW, PF, 8, 1>(a, s)
                               : launch_s8_skinny_fused_t<TPW, PF, 16, 1>(a, s);
  if (vr == 2) return launch_s8_skinny_fused_t<TPW, PF, 4, 2>(a, s);
  if (vr <= 4) return a.M <= 2 ? launch_s8_skinny_fused_t<TPW, PF, 2, 4>(a, s)
                               : launch_s8_skinny_fused_t<TPW, PF, 4, 4>(a, s);
  return launch_s8_skinny_fused_t<TPW, PF, 2, 8>(a, s);
}

hipError_t launch_s8_skinny_fused(const DynArgs &a, hipStream_t s) {
  if (!s8_fused_ok(a)) return hipErrorInvalidValue;
  // ZT_S8_SKINNY "TPW,PF,8" picks the tile shape as for the 16-token
  // kernel.  By default 16-row tiles with 8 chunks in flight up to 4096
  // rows (one workgroup per CU), else 32-row tiles (graph replays over
  // rotating weights, M = 1..8, one box: at M = 1 O 4096 x 4096 8.6 us
  // against 9.3 / 10.5 / 15.4 with 16-row tiles and 4 chunks / 32 / 64-row
  // tiles; QKV 6144 x 4096 11.2 against 11.6 / 16.1 with 16 / 64-row tiles;
  // gate_up 28672 x 4096 33.0 against 36.1 with 64-row tiles)
  const char *e = knob(kKnobS8Skinny);
  int tpw = a.N <= 4096 ? 1 : 2, pf = a.N <= 4096 ? 8 : 4, nw = 8;
  if (e) std::sscanf(e, "%d,%d,%d", &tpw, &pf, &nw);
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr, "[zt] s8 fused quantise + skinny GEMM M=%lld N=%lld K=%lld TPW=%d PF=%d\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, tpw, pf);
  if (tpw == 1 && pf == 8) return launch_s8_skinny_fused_tp<1, 8>(a, s);
  if (tpw == 1) return launch_s8_skinny_fused_tp<1, 4>(a, s);
  if (tpw == 2) return launch_s8_skinny_fused_tp<2, 4>(a, s);
  return launch_s8_skinny_fused_tp<4, 4>(a, s);
}

hipError_t launch_dyn_quantize(const void *x, int x_dt, int64_t M, int64_t K,
                               int8_t *qx, float *sx, bool frag, hipStream_t s,
                               int32_t *azp, int32_t *zero, int nzero) {
  if (M == 0) return hipSuccess;
  if (frag && K % 64 != 0) return hipErrorInvalidValue;
  const bool vec = x_dt == ZT_DT_BF16 && K % 8 == 0 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(qx)) & 15u) == 0;
  const int64_t per = (K / 8 + 255) / 256;  // 8-element vectors per thread
  const dim3 grid((unsigned)M), block(256);
  // up to 16 vectors per thread (K <= 32768); longer rows take the
  // element-wise kernel (measured: at K = 28672 the element-wise kernel made
  // the op at M = 3..5, N = 8192 take 113-114 us)
  if (vec && per <= 16) {
    const uint16_t *xb = static_cast<const uint16_t *>(x);
#define ZT_QB(V_)                                                                          \
  if (per <= V_) {                                                                         \
    if (azp)                                                                               \
      frag ? dyn_quantize_bf16_kernel<V_, true, true><<<grid, block, 0, s>>>(xb, K, qx, sx, azp, zero, nzero) \
           : dyn_quantize_bf16_kernel<V_, false, true><<<grid, block, 0, s>>>(xb, K, qx, sx, azp, zero, nzero); \
    else                                                                                   \
      frag ? dyn_quantize_bf16_kernel<V_, true, false><<<grid, block, 0, s>>>(xb, K, qx, sx, azp, zero, nzero) \
           : dyn_quantize_bf16_kernel<V_, false, false><<<grid, block, 0, s>>>(xb, K, qx, sx, azp, zero, nzero); \
    return hipGetLastError();                                                              \
  }
    ZT_QB(2) ZT_QB(4) ZT_QB(8) ZT_QB(16)
#undef ZT_QB
  }
  if (azp)
    dyn_quantize_kernel<true><<<grid, block, 0, s>>>(x, x_dt, K, qx, sx, (int)frag, azp,
                                                    zero, nzero);
  else
    dyn_quantize_kernel<false><<<grid, block, 0, s>>>(x, x_dt, K, qx, sx, (int)frag, azp,
                                                     zero, nzero);
  return hipGetLastError();
}

hipError_t launch_static_quantize(const void *x, int x_dt, int64_t M, int64_t K, int8_t *qx,
                                  bool frag, const float *scale, const int32_t *zp, float *sx,
                                  int32_t *azp, hipStream_t s, int32_t *zero, int nzero) {
  if (M == 0) return hipSuccess;
  if (frag && K % 64 != 0) return hipErrorInvalidValue;
  static_quantize_kernel<<<dim3((unsigned)M), dim3(256), 0, s>>>(x, x_dt, K, qx, (int)frag, scale,
                                                                 zp, sx, azp, zero, nzero);
  return hipGetLastError();
}

// colsum[n] = sum_k w[n][k]: one wave per weight row, 16 bytes per lane per
// step where the row is 16-byte aligned.
__global__ __launch_bounds__(256) void s8_colsum_kernel(const int8_t *w, int64_t N, int64_t K,
                                                       int32_t *colsum) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int8_t *row = w + n * K;
  int32_t acc = 0;
  int64_t k0 = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15u) == 0) {
    const int64_t nv = K / 16;
    for (int64_t j = lane; j < nv; j += kWave) {
      const i32x4_t v = *reinterpret_cast<const i32x4_t *>(row + 16 * j);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc += (int32_t)(int8_t)(v[r] >> (8 * b));
    }
    k0 = nv * 16;
  }
  for (int64_t k = k0 + lane; k < K; k += kWave) acc += row[k];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  if (lane == 0) colsum[n] = acc;
}

hipError_t launch_s8_colsum(const int8_t *w, int64_t N, int64_t K, int32_t *colsum,
                            hipStream_t s) {
  if (N == 0) return hipSuccess;
  s8_colsum_kernel<<<dim3((unsigned)((N + 3) / 4)), dim3(256), 0, s>>>(w, N, K, colsum);
  return hipGetLastError();
}

int s8_split_counters(int64_t N) { return (int)((N + kSpBN - 1) / kSpBN); }

int s8_ws_splits(int64_t M, int64_t N, int64_t K) {
  if (M <= 128 || N < 4 || K < 1 || N % 4 || knob(kKnobS8Tile) || knob(kKnobS8Kind) ||
      knob(kKnobS8Force))
    return 1;
  if (M * K >= (int64_t)kOobOffset || N * K >= (int64_t)kOobOffset) return 1;
  const int64_t t256 = ((M + 255) / 256) * ((N + 127) / 128);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (t256 > 128 || t128 >= 256) return 1;
  const int64_t nk = (K + kWsBK - 1) / kWsBK;
  const int64_t sp = std::min<int64_t>(std::min<int64_t>(8, 256 / t128), nk / 8);
  return sp >= 2 ? (int)sp : 1;
}

size_t s8_split_bytes(int64_t M, int64_t K, int64_t N) {
  if (M > 128) {
    const int sp = s8_ws_splits(M, N, K);
    return sp > 1 ? ((size_t)sp * (size_t)M * (size_t)N * 4 + 255) & ~(size_t)255 : 0;
  }
  if (!s8_split_shape(M, K, N)) return 0;
  const size_t tiles = (size_t)s8_split_counters(N);
  return tiles * 2 * kSpPart * 4 + ((tiles * 4 + 255) & ~(size_t)255);
}

bool s8_frag_ok(const DynArgs &a) {
  // 17..128 tokens: the 32x32 kernel's tiles are at least half full there
  // (one 16-token tile is cheaper on the 16x16 kernel)
  const char *e = knob(kKnobS8Frag);  // "0": never, "1": from M = 1
  const int64_t lo = e && e[0] == '1' ? 1 : 17;
  if ((e && e[0] == '0') || a.M < lo || a.M > 128 || a.K % 64 != 0) return false;
  const int64_t rows = (a.M + 31) / 32 * 32;
  return rows * a.K < (int64_t)kOobOffset && a.N * a.K < (int64_t)kOobOffset &&
         ((reinterpret_cast<uintptr_t>(a.qx) | reinterpret_cast<uintptr_t>(a.w)) & 15u) == 0;
}

hipError_t launch_s8_gemm(const DynArgs &a, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  if (a.qx_frag) {
    if (!s8_frag_ok(a)) return hipErrorInvalidValue;
    return s8_split_ok(a) ? launch_s8_splitk(a, s) : launch_s8_skinny32(a, s);
  }
  const bool aligned = ((reinterpret_cast<uintptr_t>(a.qx) |
                         reinterpret_cast<uintptr_t>(a.w)) & 15u) == 0;
  if (a.K % 16 != 0 || !aligned) {
    const int64_t blocks = (a.M * a.N + 3) / 4;
    hipLaunchKernelGGL(s8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  // the fast kernels address qx and W with 32-bit byte offsets
  const bool fits32 = a.M * a.K < (int64_t)kOobOffset && a.N * a.K < (int64_t)kOobOffset;
  const char *force = knob(kKnobS8Force);  // t: tiled, s: skinny, o: old
  // past the skinny kernels' 128 tokens the tiled kernels (129..255 had
  // fallen to the 16x16 kernel below: O 4096 x 4096 at M = 192 took 176 us
  // against 40 at M = 256)
  const bool tiled = force ? force[0] == 't' : a.M > 128;
  const bool skinny = force ? force[0] == 's' : a.M <= 128;
  if (skinny && fits32 && a.K % 64 == 0) return launch_s8_skinny(a, s);
  if (tiled && fits32) {
    // 256x128 tiles once there are half a round of them (measured on the
    // Llama prefill shapes: 2-stage DMA 256x128 is fastest from M = 2048 up)
    const int64_t t256 = ((a.M + 255) / 256) * ((a.N + 127) / 128);
    const char *tile = knob(kKnobS8Tile);
    const bool big = tile ? tile[0] == '2' : t256 >= 128;
    const char *kind = knob(kKnobS8Kind);  // w: load-wave kernel, n: 32x32x32 kernel, r, 2, 3
    if (!kind || kind[0] == 'w') {
      // ZT_S8_TILE: "2" 256 x 128 tiles, "1" 128 x 128 with 3 stages, "0" 128 x 128 with 2
      // stages (two workgroups per CU)
      if (tile && tile[0] == '1') return launch_s8_ws<128, 128, 2, 2, 4, 3>(a, s);
      if (tile && tile[0] == '0') return launch_s8_ws<128, 128, 2, 2, 4, 2>(a, s);
      // at most half a round of 256 x 128 tiles: 128 x 128 tiles, twice as
      // many workgroups (graph replays, one box: 4096 x 14336 at M = 256 /
      // 512 / 1024 90.1 / 92.4 / 96.9 -> 57.8 / 59.7 / 77.5 us, 4096 x 4096
      // 40.3 / 38.1 / 39.9 -> 38.6 / 27.0 / 32.7, 6144 x 4096 at M = 256 /
      // 512 36.9 / 38.0 -> 26.0 / 28.4; more tiles keep 256 x 128: 11008 x
      // 4096 at M = 512 39.0 against 47.1)
      if (!tile && t256 <= 128) {
        // and, when the workspace holds the partials, a K split
        if (a.gemm_splits > 1 && a.split_part && !a.split_cnt && knob(kKnobWoqDebug))
          std::fprintf(stderr, "[zt] s8 ws M=%lld N=%lld K=%lld: 128x128 tiles, %d K splits\n",
                       (long long)a.M, (long long)a.N, (long long)a.K, a.gemm_splits);
        return a.gemm_splits > 1 && !a.split_cnt
                   ? launch_s8_ws<128, 128, 2, 2, 4, 3>(a, s, a.gemm_splits)
                   : launch_s8_ws<128, 128, 2, 2, 4, 3>(a, s);
      }
      // 256 x 192 tiles (six compute waves of 128 x 64, two load waves, two
      // stages) where they make one round and 256 x 128 tiles do not: QKV at
      // M = 2048, 256 against 384 tiles, 69 -> 58.5 us
      const int64_t t192 = ((a.M + 255) / 256) * ((a.N + 191) / 192);
      const bool w192 = tile ? tile[0] == '9' : t256 > 256 && t192 <= 256;
      if (w192) return launch_s8_ws<256, 192, 2, 3, 2, 2>(a, s);
      return launch_s8_ws<256, 128, 2, 2, 4, 3>(a, s);
    }
    if (kind[0] == 'n') {  // 32x32x32 kernel, S stages
      const int st = kind && kind[1] ? kind[1] - '0' : 3;
      if (st == 2) return big ? launch_s8_gemm32<256, 128, 2>(a, s) : launch_s8_gemm32<128, 128, 2>(a, s);
      return big ? launch_s8_gemm32<256, 128, 3>(a, s) : launch_s8_gemm32<128, 128, 3>(a, s);
    }
    if (kind && kind[0] == 'r')
      return big ? launch_s8_tiled<256, 128>(a, s) : launch_s8_tiled<128, 128>(a, s);
    if (kind && kind[0] == '3')
      return big ? launch_s8_dma<256, 128, 3>(a, s) : launch_s8_dma<128, 128, 3>(a, s);
    return big ? launch_s8_dma<256, 128, 2>(a, s) : launch_s8_dma<128, 128, 2>(a, s);
  }
  if (a.M <= 64) {
    dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 63) / 64));
    hipLaunchKernelGGL((s8_gemm_kernel<64, 32>), grid, dim3(256), 0, s, a);
  } else if (a.M <= 128) {
    dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 127) / 128));
    hipLaunchKernelGGL((s8_gemm_kernel<128, 32>), grid, dim3(256), 0, s, a);
  } else {
    dim3 grid((unsigned)((a.N + 127) / 128), (unsigned)((a.M + 127) / 128));
    hipLaunchKernelGGL((s8_gemm_kernel<128, 128>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace zt
