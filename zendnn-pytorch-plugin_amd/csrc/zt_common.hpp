// Shared device helpers for the gfx950 kernels behind include/zentorch_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "zentorch_hip.h"

namespace zt {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Post-op list as a kernel argument (by value).
struct PostOps {
  int count;
  int ids[ZT_MAX_POST_OPS];
  const void *bufs[ZT_MAX_POST_OPS];
  int dts[ZT_MAX_POST_OPS];
  int64_t ld[ZT_MAX_POST_OPS];
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// fp32 -> bf16, IEEE round to nearest even; a NaN keeps its sign and top
// payload bits and becomes quiet ((bits >> 16) | 0x40).  gfx950's
// v_cvt_pk_bf16_f32 does exactly this for every fp32 bit pattern
// (tests/native/bf16_rne_check.hip compares it with the integer form
// ((bits + 0x7fff + lsb) >> 16) on all 2^32 of them), and converts two
// values in one instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float load_elem(const void *p, int dt, int64_t i) {
  switch (dt) {
  case ZT_DT_F32: return reinterpret_cast<const float *>(p)[i];
  case ZT_DT_BF16:
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
  case ZT_DT_S8: return (float)reinterpret_cast<const int8_t *>(p)[i];
  case ZT_DT_U8: return (float)reinterpret_cast<const uint8_t *>(p)[i];
  case ZT_DT_S32: return (float)reinterpret_cast<const int32_t *>(p)[i];
  default: return 0.f;
  }
}

__device__ __forceinline__ void store_elem(void *p, int dt, int64_t i, float v) {
  if (dt == ZT_DT_F32)
    reinterpret_cast<float *>(p)[i] = v;
  else
    reinterpret_cast<uint16_t *>(p)[i] = (uint16_t)f32_to_bf16_bits(v);
}

__device__ __forceinline__ float unary_op(int id, float v) {
  switch (id) {
  case ZT_PO_RELU: return v > 0.f ? v : 0.f;
  case ZT_PO_GELU_TANH: {
    const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
    return 0.5f * v * (1.f + tanhf(k0 * (v + 0.044715f * v * v * v)));
  }
  case ZT_PO_GELU_ERF: return 0.5f * v * (1.f + erff(v * 0.7071067811865476f));
  case ZT_PO_SILU: return v / (1.f + expf(-v));
  case ZT_PO_SIGMOID: return 1.f / (1.f + expf(-v));
  case ZT_PO_TANH: return tanhf(v);
  default: return v;
  }
}

// Post-ops in list order; binary ops consume the buffers in order
// (the reference's matmul_post_ops, MatmulUtils.hpp:36-77).
__device__ __forceinline__ float apply_post_ops(float v, const PostOps &p,
                                                int64_t m, int64_t n) {
  int b = 0;
  for (int i = 0; i < p.count; ++i) {
    const int id = p.ids[i];
    if (id == ZT_PO_ADD || id == ZT_PO_MUL) {
      const float o = load_elem(p.bufs[b], p.dts[b], m * p.ld[b] + n);
      ++b;
      v = (id == ZT_PO_ADD) ? v + o : v * o;
    } else {
      v = unary_op(id, v);
    }
  }
  return v;
}

// gfx9 raw buffer resource: 32-bit offsets from one SGPR base, hardware
// range check (reads at offsets >= bytes return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}

// An offset every raw buffer load treats as out of range (returns 0).
constexpr uint32_t kOobOffset = 0x80000000u;

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs
// on XCD b % 8, each with its own L2).  Map b to a tile index so that each
// XCD works on one contiguous range of the n tiles.
__device__ __forceinline__ int xcd_contiguous_tile(int b, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = b & 7, i = b >> 3;
  return x * q + (x < r ? x : r) + i;
}

}  // namespace zt
