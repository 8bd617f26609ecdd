// GPU check of the library's fp32 -> bf16 conversions (zt_common.hpp:
// f32_to_bf16_bits, pack_bf16x2, both gfx950's v_cvt_pk_bf16_f32) against
// round-to-nearest-even written with integer operations, on every one of
// the 2^32 fp32 bit patterns.  Built by zendnn-pytorch-plugin_amd/build.py,
// run by tests/test_bf16_rne_gpu.py.  Prints the mismatch count; exit status
// 0 only when it is zero.
#include <cstdio>

#include "zt_common.hpp"

namespace {

// round to nearest even on the bit pattern; a NaN becomes quiet with its
// sign and top payload bits
__device__ uint32_t rne_bits(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// thread i checks the patterns 2 i and 2 i + 1 of its chunk
__global__ void check_kernel(uint64_t base, unsigned long long *bad, uint32_t *first) {
  const uint64_t i = base + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t u0 = (uint32_t)(2 * i), u1 = u0 + 1;
  const float a = __uint_as_float(u0), b = __uint_as_float(u1);
  const uint32_t want = rne_bits(u0) | (rne_bits(u1) << 16);
  const uint32_t pk = zt::pack_bf16x2(a, b);
  const uint32_t one = zt::f32_to_bf16_bits(a) | (zt::f32_to_bf16_bits(b) << 16);
  if (pk != want || one != want) {
    if (atomicAdd(bad, 1ull) == 0) {
      first[0] = u0;
      first[1] = pk;
      first[2] = one;
      first[3] = want;
    }
  }
}

}  // namespace

int main() {
  unsigned long long *bad = nullptr;
  uint32_t *first = nullptr;
  if (hipMalloc(&bad, sizeof(*bad)) != hipSuccess || hipMalloc(&first, 4 * sizeof(*first)) != hipSuccess) {
    std::printf("hipMalloc failed\n");
    return 2;
  }
  hipMemset(bad, 0, sizeof(*bad));
  hipMemset(first, 0, 4 * sizeof(*first));
  const uint64_t pairs = 1ull << 31, chunk = 1ull << 28;  // 8 launches of 2^20 workgroups
  for (uint64_t b = 0; b < pairs; b += chunk)
    check_kernel<<<dim3((unsigned)(chunk / 256)), dim3(256)>>>(b, bad, first);
  if (hipDeviceSynchronize() != hipSuccess) {
    std::printf("kernel failed\n");
    return 2;
  }
  unsigned long long n = 0;
  uint32_t f[4];
  hipMemcpy(&n, bad, sizeof(n), hipMemcpyDeviceToHost);
  hipMemcpy(f, first, sizeof(f), hipMemcpyDeviceToHost);
  std::printf("bf16 rne: %llu mismatching pairs of 2^31\n", n);
  if (n) std::printf("first: fp32 %08x packed %08x single %08x want %08x\n", f[0], f[1], f[2], f[3]);
  return n ? 1 : 0;
}
