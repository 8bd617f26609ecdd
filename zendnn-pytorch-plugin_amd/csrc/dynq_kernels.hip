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
#include "zt_launch.hpp"

namespace zt {

namespace {

__global__ __launch_bounds__(256) void dyn_quantize_kernel(
    const void *x, int x_dt, int64_t K, int8_t *qx, float *sx) {
  __shared__ float wmax[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t m = blockIdx.x;
  const int64_t base = m * K;
  float amax = 0.f;
  for (int64_t k = tid; k < K; k += 256)
    amax = fmaxf(amax, fabsf(load_elem(x, x_dt, base + k)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if (lane == 0) wmax[wv] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  if (!(amax >= 1e-12f)) amax = 1e-12f;
  const float s = __fdiv_rn(amax, 127.0f);
  if (tid == 0) sx[m] = s;
  for (int64_t k = tid; k < K; k += 256) {
    float r = rintf(__fdiv_rn(load_elem(x, x_dt, base + k), s));
    r = fminf(fmaxf(r, -128.f), 127.f);
    qx[base + k] = (int8_t)(int)r;
  }
}

__device__ __forceinline__ void dyn_epilogue(const DynArgs &a, int64_t m,
                                             int64_t n, int32_t acc) {
  if (a.y_dt == ZT_DT_S32) {
    reinterpret_cast<int32_t *>(a.y)[m * a.N + n] = acc;
    return;
  }
  float v = (float)acc * a.sx[m];
  v = v * load_elem(a.sw, a.sw_dt, n);
  if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
  v = apply_post_ops(v, a.post, m, n);
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

}  // namespace

hipError_t launch_dyn_quantize(const void *x, int x_dt, int64_t M, int64_t K,
                               int8_t *qx, float *sx, hipStream_t s) {
  if (M == 0) return hipSuccess;
  hipLaunchKernelGGL(dyn_quantize_kernel, dim3((unsigned)M), dim3(256), 0, s, x,
                     x_dt, K, qx, sx);
  return hipGetLastError();
}

hipError_t launch_s8_gemm(const DynArgs &a, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  const bool aligned = ((reinterpret_cast<uintptr_t>(a.qx) |
                         reinterpret_cast<uintptr_t>(a.w)) & 15u) == 0;
  if (a.K % 16 != 0 || !aligned) {
    const int64_t blocks = (a.M * a.N + 3) / 4;
    hipLaunchKernelGGL(s8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
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
