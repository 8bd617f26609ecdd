// int4 -> bf16 dequantisation for the WOQ kernels.
//
// Every kernel produces exactly bf16_rne(w) with w the fp32 dequantised
// weight of the reference's test reference (q*s for signed int4,
// (u-8)*s + z for a float zero point, (u-zp)*s for an integer one), so the
// bf16 MFMA sees the same operand a dequantise-then-bf16-GEMM would.
//
// One packed word holds elements k..k+7 (nibble i = element k+i).  Each
// 16-bit half of a register is turned into the fp16 value 1024 + u (nibble
// in bits 0-3) or 1024 + 16u (nibble in bits 4-7) with a single v_bitop3
// ((t & mask) ^ C: the mask isolates the nibbles, C sets the fp16 exponent
// and, for signed int4, flips bit 3 so u = q + 8).  v_fma_mix_f32 reads an
// fp16 half directly as an fma source:
//   fma(1024 + u,   s,    -1032 s) = (u - 8) s = q s
//   fma(1024 + 16u, s/16, -72 s)   = (u - 8) s = q s
// Both are exact for bf16 scales (q s has at most 12 significant bits and
// 1032 s, 72 s at most 16), so rounding the fp32 result to bf16 with
// v_cvt_pk_bf16_f32 (round to nearest even) gives bf16_rne(q*s).
// Other scale types and zero points first form the exact integer
// (u - 8 or u - zp) the same way and then apply the reference's fp32 steps.
#pragma once

#include "zt_common.hpp"

namespace zt {

// (t & mask) ^ c in one v_bitop3_b32: truth table f(0xF0, 0xCC, 0xAA).
__device__ __forceinline__ uint32_t and_xor(uint32_t t, uint32_t mask, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(t, mask, c, 0x6a);
}

__device__ __forceinline__ float f16_lo(uint32_t p) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(p & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t p) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
}

constexpr uint32_t kNibLo = 0x000F000Fu;   // nibbles at bits 0-3 of each half
constexpr uint32_t kNibHi = 0x00F000F0u;   // nibbles at bits 4-7 of each half
constexpr uint32_t kExpLo = 0x64006400u;   // fp16 1024 in both halves
constexpr uint32_t kXorLo = 0x00080008u;   // flip bit 3 of a low nibble
constexpr uint32_t kXorHi = 0x00800080u;   // flip bit 3 of a high nibble

// Signed int4 with a bf16 scale s: returns 8 bf16 (elements k..k+7 in order,
// two per register).  c0 = -1032 s, c1 = -72 s, s16 = s / 16.
__device__ __forceinline__ u32x4_t dq8_s4_bf16scale(uint32_t w, float s, float s16,
                                                    float c0, float c1) {
  const uint32_t w8 = w >> 8;
  const uint32_t p0 = and_xor(w, kNibLo, kExpLo | kXorLo);   // elements 0, 4
  const uint32_t p1 = and_xor(w, kNibHi, kExpLo | kXorHi);   // elements 1, 5
  const uint32_t p2 = and_xor(w8, kNibLo, kExpLo | kXorLo);  // elements 2, 6
  const uint32_t p3 = and_xor(w8, kNibHi, kExpLo | kXorHi);  // elements 3, 7
  u32x4_t r;
  r[0] = pack_bf16x2(fmaf(f16_lo(p0), s, c0), fmaf(f16_lo(p1), s16, c1));
  r[1] = pack_bf16x2(fmaf(f16_lo(p2), s, c0), fmaf(f16_lo(p3), s16, c1));
  r[2] = pack_bf16x2(fmaf(f16_hi(p0), s, c0), fmaf(f16_hi(p1), s16, c1));
  r[3] = pack_bf16x2(fmaf(f16_hi(p2), s, c0), fmaf(f16_hi(p3), s16, c1));
  return r;
}

// Per-(row, group) constants of the general path.
struct DqGeneral {
  uint32_t xlo, xhi;  // XOR bits (signed int4) or 0 (unsigned)
  float o0, o1;       // 1024 + off, 64 + off: off = 8 (s4, float zp) or zp
  float s, z;         // scale, float zero point (0 if none)
  bool add_z;
};

__device__ __forceinline__ DqGeneral dq_general_params(int zmode, float s, float zp) {
  DqGeneral d;
  d.xlo = zmode == 0 ? kXorLo : 0u;
  d.xhi = zmode == 0 ? kXorHi : 0u;
  const float off = zmode == 2 ? zp : 8.f;
  d.o0 = -(1024.f + off);
  d.o1 = -(64.f + off);
  d.s = s;
  d.z = zmode == 1 ? zp : 0.f;
  d.add_z = zmode == 1;
  return d;
}

__device__ __forceinline__ float dq_general_one(float qf, const DqGeneral &d) {
  float v = qf * d.s;
  if (d.add_z) v = v + d.z;
  return v;
}

// Any scale dtype / zero-point mode: the exact integer first, then the
// reference's fp32 arithmetic.
__device__ __forceinline__ u32x4_t dq8_general(uint32_t w, const DqGeneral &d) {
  const uint32_t w8 = w >> 8;
  const uint32_t p0 = and_xor(w, kNibLo, kExpLo | d.xlo);
  const uint32_t p1 = and_xor(w, kNibHi, kExpLo | d.xhi);
  const uint32_t p2 = and_xor(w8, kNibLo, kExpLo | d.xlo);
  const uint32_t p3 = and_xor(w8, kNibHi, kExpLo | d.xhi);
  auto q0 = [&](float h) { return dq_general_one(fmaf(h, 1.f, d.o0), d); };
  auto q1 = [&](float h) { return dq_general_one(fmaf(h, 0.0625f, d.o1), d); };
  u32x4_t r;
  r[0] = pack_bf16x2(q0(f16_lo(p0)), q1(f16_lo(p1)));
  r[1] = pack_bf16x2(q0(f16_lo(p2)), q1(f16_lo(p3)));
  r[2] = pack_bf16x2(q0(f16_hi(p0)), q1(f16_hi(p1)));
  r[3] = pack_bf16x2(q0(f16_hi(p2)), q1(f16_hi(p3)));
  return r;
}

}  // namespace zt
