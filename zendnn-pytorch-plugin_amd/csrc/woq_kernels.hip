// int4 weight-only linear kernels for gfx950 (zentorch_woq_linear family).
//
// Numerics (every kernel in this file): each weight is dequantised to the bf16 value
// bf16_rne(q*s) (or the zero-point forms, woq_dequant.hpp) and multiplied
// with the bf16 activations on the bf16 MFMA with fp32 accumulation; bias
// and post-ops run in fp32 and the output is rounded once.  That is the
// dequantise-then-bf16-GEMM the reference's own test reference computes
// (test/unittests/op_tests/test_woq_linear.py:118-128) and that its 1e-3
// tolerance pins; an exact sum_g s_g sum_k x q fails that test.
//
// Kernels, in the order zt_woq_linear (capi.hip) tries them:
//  * woq_wide_kernel     17..64 rows with large N * K: row tiles of 32 or 64
//    tokens, K split over workgroups (fp32 partials in the workspace,
//    woq_splitk_reduce_kernel adds them in split order).
//  * woq_wave_kernel / woq_stream_kernel  1..16 rows (and up to 64 on
//    smaller weights): the decode GEMV / skinny GEMM.  Packed int4 weights
//    stream from HBM in 16-byte loads straight into the registers that are
//    the MFMA A operands; x sits in LDS; the waves split K and their partials
//    meet in LDS.  The wave kernel gives every wave its own x slice and no
//    barrier before the reduction; the stream kernel shares one x copy.
//    Rows past what one launch holds go in blocks of 16.
//  * woq_lean_kernel  1..16 rows in the fast mode where it measured faster
//    (the long-K down projection and the widest matrices at few rows, the
//    merged gate_up at 1..2 rows): the stream kernel's work split with each
//    chunk's scales loaded beside its weights, x read only by the lanes of
//    real tokens and two MFMA accumulators.
//  * woq_persist_kernel  the merged gate_up at 3..16 rows and plain calls
//    of 12288 rows or more: one workgroup per CU loops over row units with
//    x in registers and the next units' weights in flight.
//  * woq_decode_kernel   the older decode kernel for shapes the two above do
//    not take (long K split over workgroups, general dequant modes).
//  * woq_gemm32_kernel / woq_gemm_ws_kernel / woq_gemm_dma_kernel  prefill
//    (more rows): LDS tiles moved by DMA, int4 dequantised in registers
//    after the LDS read, bf16 MFMA (32x32x16 for signed int4 with bf16
//    scales -- with load waves of their own when one round of tiles covers
//    the matrix -- 16x16x32 for the other modes); woq_gemm_kernel for group
//    sizes that are not multiples of 128.
//  * woq_generic_kernel  what none of the above takes (K not a multiple of
//    64, odd group sizes): one wave per output element.
//
// Weight layout: [N, K/8] int32, nibble i of word (n, c) is element
// (n, 8c+i) -- the storage of the [K/8, N] view zentorch_woq_linear takes
// (src/cpu/cpp/WOQ_Linear.cpp:31-42, repack :345-350).
#include <algorithm>
#include <type_traits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "woq_dequant.hpp"
#include "zt_launch.hpp"
#include "zt_tuning.hpp"

namespace zt {

namespace {

enum ZpMode { kZpNone = 0, kZpFloat = 1, kZpInt = 2 };

__host__ __device__ inline int zp_mode_of(const void *zp, int zp_dt) {
  if (!zp) return kZpNone;
  return (zp_dt == ZT_DT_F32 || zp_dt == ZT_DT_BF16) ? kZpFloat : kZpInt;
}

// Dequantised weight before rounding to the compute dtype (oracle
// woq_dequant): two fp32 roundings, no contraction (built -ffp-contract=off).
__device__ __forceinline__ float dq_ref(uint32_t nib, float s, int zmode,
                                        float z) {
  if (zmode == kZpNone) {
    const int q = (int)(nib ^ 8u) - 8;
    return (float)q * s;
  }
  if (zmode == kZpFloat) {
    const float w = (float)((int)nib - 8) * s;
    return w + z;
  }
  return ((float)nib - z) * s;
}

__device__ __forceinline__ float round_bf16(float v) {
  return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// ------------------------------------------------------------ generic
__global__ __launch_bounds__(256) void woq_generic_kernel(WoqArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= a.M * a.N) return;
  const int64_t m = wid / a.N, n = wid % a.N;
  const int64_t KW = a.K / 8, gs = a.K / a.G;
  const int zmode = zp_mode_of(a.zp, a.zp_dt);
  const bool round_w = (a.x_dt == ZT_DT_BF16);
  float acc = 0.f;
  for (int64_t c = lane; c < KW; c += kWave) {
    const uint32_t word = a.w[n * KW + c];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = 8 * c + i;
      const int64_t sidx = (k / gs) * a.N + n;
      const float s = load_elem(a.scales, a.s_dt, sidx);
      const float z = zmode ? load_elem(a.zp, a.zp_dt, sidx) : 0.f;
      float w = dq_ref((word >> (4 * i)) & 0xFu, s, zmode, z);
      if (round_w) w = round_bf16(w);
      acc = acc + load_elem(a.x, a.x_dt, m * a.ldx + k) * w;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  if (lane == 0) {
    float v = acc;
    if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
    v = apply_post_ops(v, a.post, m, n);
    store_elem(a.y, a.y_dt, m * a.ldy + n, v);
  }
}

// ------------------------------------------------------------- decode
constexpr unsigned kCounterSlots = 1024;  // 4096-byte counter region

// Dequantisation modes of the decode kernel: signed int4 with bf16 scales
// (the fast path), or the general path with bf16 / fp32 scales.
enum DecodeMode { kDecFast = 0, kDecGenBf16 = 1, kDecGenF32 = 2 };

template <int MODE>
__device__ __forceinline__ float scale_at(const WoqArgs &a, int64_t i) {
  if (MODE == kDecGenF32) return reinterpret_cast<const float *>(a.scales)[i];
  return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(a.scales)[i]);
}

template <int MODE>
__device__ __forceinline__ bf16x8_t dq_word(uint32_t w, float s, float z, int zmode) {
  u32x4_t v;
  if (MODE == kDecFast)
    v = dq8_s4_bf16scale(w, s, s * 0.0625f, -1032.f * s, -72.f * s);
  else
    v = dq8_general(w, dq_general_params(zmode, s, z));
  return __builtin_bit_cast(bf16x8_t, v);
}

// Decode GEMV / skinny GEMM (M <= 32).
//
// Grid (row blocks, K splits).  A workgroup has NT x NK waves: wave (ti, ki)
// takes TPW consecutive 16-row tiles of the row block over K-slice ki of the
// workgroup's split (CPW 128-wide chunks).  Lane (r = lane%16, g = lane/16)
// loads the 16 bytes of row r holding elements [32g, 32g+32) of a chunk --
// exactly its A operands for the chunk's four 16x16x32 MFMAs -- so weights go
// from HBM to registers without touching LDS.  The activations of the wave's
// chunks are loaded once into registers as B operands (L2-resident: every
// workgroup reads the same few KB).  Each wave stores its fp32
// tile partials to its own LDS slab; after one barrier the slabs are added in
// ki order (deterministic), and with more than one split the last workgroup
// of a row block adds the splits' partials from global memory in split order.
template <int CPW>
constexpr int decode_max_threads() {
  return CPW <= 2 ? 1024 : (CPW == 4 ? 512 : 256);
}

// Bytes of the per-wave partial slabs at the start of the dynamic LDS.
__host__ __device__ inline size_t decode_slab_bytes(int NK, int NT, int TPW, int mt) {
  return (size_t)NK * NT * TPW * 16 * (16 * mt + 1) * sizeof(float);
}

// Decode GEMV / skinny GEMM (M <= 32).
//
// Grid: one workgroup per row block of NT*TPW 16-row tiles, covering all of
// K.  Wave (ti, ki) of the NT x NK waves owns the K slice
// [c_wave, c_wave + CW) of 128-wide chunks and walks NI items, fully
// unrolled so every wait on memory is exact:
//  * XR (one phase): item = one of the wave's TPW tiles over the whole
//    slice; the slice's activations are loaded once into registers and
//    reused for every tile.
//  * XG (phased, TPW = 1): item = CPW chunks of the slice; the item's
//    activations are prefetched with its weights.
// Lane (r = lane%16, g = lane/16) loads the 16 bytes of row r holding
// elements [32g, 32g+32) of a chunk -- exactly its A operands for the
// chunk's four 16x16x32 MFMAs -- so weights go from HBM to registers
// without touching LDS, two items ahead.  Each wave stores its fp32 tile
// partials to its own LDS slab; after one barrier the NK slabs of an output
// are added by a fixed shuffle tree (deterministic).  Scale group of chunk
// kc: (kc >> cpg_shift) & gmask (gmask = 0: per channel).
template <int MT, int CPW, int NI, int MODE, bool XR, bool XS>
__global__ __launch_bounds__(decode_max_threads<CPW>()) void woq_decode_kernel(
    WoqArgs a, int NK, int NT, int cpg_shift, int gmask) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int RS = 16 * MT + 1;
  constexpr int PF = NI < 2 ? NI : 2;  // items in flight while one is computed
  constexpr int TPW = XR ? NI : 1;

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int ki = wv % NK, ti = wv / NK;
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N;
  const int KW = (int)(a.K / 8);
  const int C = (int)(a.K / 128);
  const int CW = (C + NK - 1) / NK;
  const int c_wave = ki * CW;
  const int c_hi = min(C, c_wave + CW);
  const int zmode = zp_mode_of(a.zp, a.zp_dt);
  const int tiles = (N + 15) / 16;
  const int t_blk = blockIdx.x * NT * TPW;
  const int t0 = t_blk + ti * TPW;
  // Items that carry work: tiles that exist (XR) or phases (XG).
  const int n_items = XR ? min(NI, max(0, tiles - t0)) : (t0 < tiles ? NI : 0);
  float *slab = reinterpret_cast<float *>(smem);
  const uint16_t *xp = reinterpret_cast<const uint16_t *>(a.x);
  const int s_bytes = MODE == kDecGenF32 ? 4 : 2;
  const auto w_rsrc = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rsrc = make_rsrc(a.scales, (uint32_t)(a.G * N * s_bytes));

  // Raw words and scale bits only: converting at load time would make the
  // compiler wait for the load right there.
  struct ItemRegs {
    u32x4_t w[CPW];
    uint32_t s[CPW];
    float z[CPW];
    u32x4_t x[XR ? 1 : CPW][MT][4];
  };
  auto x_at = [&](int kc, int mt, int i) -> u32x4_t {
    const int m = min(mt * 16 + lr, M - 1);
    return *reinterpret_cast<const u32x4_t *>(xp + (int64_t)m * a.ldx + (int64_t)kc * 128 +
                                              32 * lg + 8 * i);
  };
  // Item it: tile t0 + it over the slice (XR) or chunks it*CPW.. of tile t0
  // (XG).  Indices are clamped, so every item is in bounds.
  auto load_item = [&](ItemRegs &dst, int it) {
    const int tj = XR ? it : 0, ph = XR ? 0 : it;
    const int n = min((t0 + tj) * 16 + lr, N - 1);
    const uint32_t row_off = (uint32_t)n * (uint32_t)KW * 4u + (uint32_t)lg * 16u;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int kc = min(c_wave + ph * CPW + c, C - 1);
      const uint32_t sidx = (uint32_t)((kc >> cpg_shift) & gmask) * (uint32_t)N + (uint32_t)n;
      dst.w[c] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, row_off + (uint32_t)kc * 64u, 0, 0));
      if (MODE == kDecGenF32)
        dst.s[c] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, sidx * 4u, 0, 0);
      else
        dst.s[c] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, sidx * 2u, 0, 0);
      dst.z[c] = (MODE != kDecFast && zmode) ? load_elem(a.zp, a.zp_dt, sidx) : 0.f;
      if (!XR) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst.x[XR ? 0 : c][mt][i] = x_at(kc, mt, i);
      }
    }
  };

  // XS (M <= 8): the wave's activation slice, M rows x CW*128, with
  // full-width coalesced loads issued before the weights, bounced through a
  // wave-private LDS region into the B-operand layout.  A B-operand load
  // straight from global would keep only M of 16 row lanes busy.
  constexpr int XSU = XS ? 8 * CPW * 16 / 64 : 1;  // 16-byte units per lane
  const int xs_upr = CW * 16;                       // units per row
  const int xs_ld = CW * 128 + 8;                   // bf16 per LDS row
  uint16_t *xs_lds = reinterpret_cast<uint16_t *>(
      smem + decode_slab_bytes(NK, NT, TPW, MT) + (size_t)wv * 8 * xs_ld * 2);
  u32x4_t xs_v[XSU];
  if (XS) {
#pragma unroll
    for (int u = 0; u < XSU; ++u) {
      const int idx = lane + 64 * u;
      const int m = min(idx / xs_upr, M - 1), k16 = idx % xs_upr;
      const int kc = min(c_wave + k16 / 16, C - 1);
      xs_v[u] = *reinterpret_cast<const u32x4_t *>(xp + (int64_t)m * a.ldx + (int64_t)kc * 128 +
                                                   (k16 % 16) * 8);
    }
  }

  ItemRegs buf[PF];
#pragma unroll
  for (int p = 0; p < PF; ++p) load_item(buf[p], p);
  // XR: the slice's activations, once (CPW covers the whole slice).
  u32x4_t xr[XR ? CPW : 1][MT][4];
  if (XR && XS) {
#pragma unroll
    for (int u = 0; u < XSU; ++u) {
      const int idx = lane + 64 * u;
      const int m = idx / xs_upr, k16 = idx % xs_upr;
      if (m < M) *reinterpret_cast<u32x4_t *>(xs_lds + m * xs_ld + k16 * 8) = xs_v[u];
    }
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (lr < M && c < CW)
          v = *reinterpret_cast<const u32x4_t *>(xs_lds + lr * xs_ld + c * 128 + 32 * lg + 8 * i);
        xr[XR ? c : 0][0][i] = v;
      }
  } else if (XR) {
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[XR ? c : 0][mt][i] = x_at(min(c_wave + c, C - 1), mt, i);
  }

  f32x4_t acc[MT];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    ItemRegs &cur = buf[it % PF];
    if (it < n_items) {
      const int ph = XR ? 0 : it;
      if (XR || it == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        const int kc = c_wave + ph * CPW + c;
        if (kc < c_hi) {
          const uint32_t sb = cur.s[c];
          const float sc = MODE == kDecGenF32 ? __uint_as_float(sb) : __uint_as_float(sb << 16);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bf16x8_t A = dq_word<MODE>(cur.w[c][i], sc, cur.z[c], zmode);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              u32x4_t v = XR ? xr[XR ? c : 0][mt][i] : cur.x[XR ? 0 : c][mt][i];
              if (mt * 16 + lr >= M) v = u32x4_t{0u, 0u, 0u, 0u};
              acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  A, __builtin_bit_cast(bf16x8_t, v), acc[mt], 0, 0, 0);
            }
          }
        }
      }
      if (XR || it == n_items - 1) {
        // D[row = 4g + r][token = lane % 16] into this wave's slab
        float *sl = slab + ((size_t)(ki * NT + ti) * TPW + (XR ? it : 0)) * 16 * RS;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) sl[(4 * lg + r) * RS + mt * 16 + lr] = acc[mt][r];
      }
    }
    if (it + PF < NI) load_item(cur, it + PF);
  }
  __syncthreads();

  // Add the NK slabs of each output with a fixed shuffle tree: NKP (NK
  // rounded up to a power of two) consecutive lanes hold one output's
  // partials, so the result does not depend on wave timing.
  const int rows = (min(tiles, t_blk + NT * TPW) - t_blk) * 16;
  const int n0 = t_blk * 16;
  const int total = rows * M;
  const int NKP = NK <= 1 ? 1 : (NK <= 2 ? 2 : (NK <= 4 ? 4 : (NK <= 8 ? 8 : 16)));
  const int per_pass = blockDim.x / NKP;
  const int kk = threadIdx.x % NKP;
  for (int pass = 0; pass < total; pass += per_pass) {
    const int idx = pass + threadIdx.x / NKP;
    float v = 0.f;
    int m = 0, nr = 0;
    if (idx < total) {
      m = idx / rows, nr = idx - m * rows;
      if (kk < NK) {
        const int tb = nr >> 4, r16 = nr & 15;
        const int tti = tb / TPW, tj = tb - tti * TPW;
        v = slab[((size_t)(kk * NT + tti) * TPW + tj) * 16 * RS + r16 * RS + m];
      }
    }
    for (int off = 1; off < NKP; off <<= 1) v += __shfl_xor(v, off, kWave);
    const int n = n0 + nr;
    if (kk == 0 && idx < total && n < N) {
      if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
      v = apply_post_ops(v, a.post, m, n);
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
    }
  }
}

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// Weight-streaming decode kernel (M <= 16 and the activations fit in LDS,
// up to kStreamLdsMax with the scales; the partial slabs reuse x's space).
//
// One workgroup per TPW 16-row tiles over all of K; its NW waves split K
// into slices of CPW 128-wide chunks.  The workgroup first starts the copy
// of x [M, K] into LDS by DMA (when the rows are 16-byte aligned) and, in
// the fast mode, of its rows' scales; then a wave issues the weight loads
// of its slice's first chunks (TPW 16-byte fragments per lane per chunk,
// with their scales and zero points in the general modes): ZT_STREAM_DEPTH
// of them, issuing chunk c + depth as it starts computing chunk c, so
// the buffer unit takes the later loads while the wave dequantises instead
// of holding the wave in a long issue phase first.  A wave's loads retire
// in issue order, so x (from L2) lands while its weights are still in
// flight.  The wave then walks its chunks: B operands come from LDS (token
// columns past M repeat row M-1), A operands are the fragments dequantised
// in registers.  K partials meet in LDS and are added in wave order.
constexpr size_t kStreamLdsMax = 160 * 1024;
// chunks (per tile) of weights in flight per wave; the next one is issued
// as each is computed (measured best of 2, 3, 4, 6, 8 and all at once on the
// Llama-3 8B decode shapes)
#ifndef ZT_STREAM_DEPTH
#define ZT_STREAM_DEPTH 2
#endif
// per-wave fp32 partials: TPW row tiles x MT token tiles of 16 x 16 (+1 pad)
__host__ __device__ constexpr size_t stream_slab_bytes(int nw, int tpw, int mt) {
  return (size_t)nw * tpw * mt * 16 * 17 * sizeof(float);
}
// LDS: x [M][XP] (or one phase's range) at offset 0, overlaid after the
// chunk loop by the partial slabs; the fast mode's scales after the larger
// of the two
__host__ __device__ constexpr size_t stream_scale_offset(size_t slab, size_t x) {
  return slab > x ? slab : x;
}
__host__ __device__ inline int stream_x_pitch(int K) { return K + 8; }  // bf16
// row pitch of one K phase of x (kp elements): whole 1 KB DMA pieces, so
// the lanes of a partial last piece land in the row's own padding
__host__ __device__ inline int stream_phase_pitch(int kp) { return (kp + 511) / 512 * 512 + 8; }
// fast mode: the bf16 scales of the workgroup's TPW*16 rows for all G groups,
// [G][TPW*16], moved by 256-byte DMA instructions
__host__ __device__ constexpr size_t stream_scale_bytes(int G, int tpw) {
  return (size_t)((G * tpw + 7) / 8) * 256;
}

// gu > 0 (merged gate_up, fast mode, TPW even, P == MT == 1): weight rows
// [0, gu) are the gate and [gu, 2 gu) the up projection; tile 2i of the
// workgroup is gate tile blockIdx.x * TPW/2 + i and tile 2i + 1 the up tile
// of the same columns, and the workgroup writes silu(gate) * up for its
// TPW/2 * 16 output columns (up rounded to the output dtype first, as the
// two-op composition does).
template <int NW, int CPW, int TPW, int MODE, int P, int MT>
__global__ __launch_bounds__(64 * NW) void woq_stream_kernel(WoqArgs a, int cpg_shift, int gmask,
                                                             int x_dma, int gu) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int KW = K / 8, C = K / 128;
  const int t0 = blockIdx.x * TPW;
  // first weight row of the workgroup's tile t
  auto rowbase = [&](int t) {
    return gu ? (t & 1) * gu + (blockIdx.x * (TPW / 2) + (t >> 1)) * 16 : (t0 + t) * 16;
  };
  const int zmode = zp_mode_of(a.zp, a.zp_dt);
  const int s_bytes = MODE == kDecGenF32 ? 4 : 2;
  const auto w_rsrc = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rsrc = make_rsrc(a.scales, (uint32_t)(a.G * N * s_bytes));
  // Phases (P > 1, when x [M, K] does not fit LDS): K splits into P ranges
  // of CP chunks; x holds one range at a time.  Wave w owns the contiguous
  // chunks [w*CP/NW, (w+1)*CP/NW) of each phase (with P == 1 of all C), so
  // the waves' shares differ by at most one chunk; slots past the share
  // are C, which loads zeros and computes nothing.
  constexpr int CPWP = CPW / P;
  const int CP = C / P;
  const int lo = wv * CP / NW, len = (wv + 1) * CP / NW - lo;
  auto chunk_of = [&](int c) {
    const int p = P == 1 ? 0 : c / CPWP, j = c - p * CPWP;
    return j < len ? p * CP + lo + j : C;
  };

  // 1. x [M, K] (or phase 0's range) -> LDS (row pitch XP bf16).  By DMA
  //    when x_dma (stream_x_dma: every row 16-byte aligned and whole 1 KB
  //    pieces; always for P > 1): instruction i moves 64 16-byte chunks of
  //    one row.
  const int XP = P == 1 ? stream_x_pitch(K) : stream_phase_pitch(K / P);
  uint16_t *xl = reinterpret_cast<uint16_t *>(smem);
  const auto x_rsrc = make_rsrc(a.x, (uint32_t)((int64_t)(M - 1) * a.ldx * 2 + (int64_t)K * 2));
  auto dma_x = [&](int p) {
    // 1 KB pieces per row and phase; with phases the last may be partial:
    // its lanes past the row read nothing and write zeros into the row's
    // padding (stream_phase_pitch)
    const int kp = P == 1 ? K : K / P;
    const int per_row = (kp + 511) / 512;
    for (int i = wv; i < M * per_row; i += NW) {
      const int m = i / per_row, q = i - m * per_row;
      const int e = q * 512 + lane * 8;  // the lane's first element of the row's phase
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          x_rsrc, (lds_ptr_t)(xl + m * XP + q * 512), 16,
          e < kp ? (uint32_t)(m * a.ldx * 2 + p * kp * 2 + e * 2) : kOobOffset, 0, 0, 0);
    }
  };
  if (x_dma) dma_x(0);
  // The fast mode's scales: one DMA instruction moves 64 dwords, i.e. the
  // TPW*16 row scales of 8/TPW groups ([G][TPW*16] bf16 in LDS; N is even,
  // host-checked, so every dword is aligned).  Issued before the weights,
  // so the wait for x below covers them too.
  const uint16_t *sl = reinterpret_cast<const uint16_t *>(
      smem + stream_scale_offset(stream_slab_bytes(NW, TPW, MT), (size_t)M * XP * 2));
  if (MODE == kDecFast) {
    const int G = (int)a.G, gbytes = TPW * 32;
    const int ns = (G * TPW + 7) / 8;
    for (int i = wv; i < ns; i += NW) {
      const int byte = i * 256 + lane * 4, g = byte / gbytes, b = byte - g * gbytes;
      const int q = b >> 1;  // row within the group's TPW*16 (even: both rows in one tile)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          s_rsrc, (lds_ptr_t)(sl + i * 128), 4,
          g < G ? (uint32_t)((g * N + rowbase(q >> 4) + (q & 15)) * 2) : kOobOffset, 0, 0, 0);
    }
  }

  // 2. the slice's weights and (other modes) scales.  Rows past N are
  //    clamped (their results are never stored); chunks past C read zeros.
  u32x4_t wr[TPW][CPW];
  uint32_t sr[TPW][CPW];
  float zr[TPW][CPW];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int n = min(rowbase(t) + lr, N - 1);
      const uint32_t row_off = (uint32_t)n * (uint32_t)KW * 4u + (uint32_t)lg * 16u;
      const int kc = chunk_of(c);
      const int kcs = min(kc, C - 1);
      const uint32_t sidx = (uint32_t)((kcs >> cpg_shift) & gmask) * (uint32_t)N + (uint32_t)n;
      wr[t][c] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                       w_rsrc, kc < C ? row_off + (uint32_t)kc * 64u : kOobOffset, 0, 0));
      if (MODE == kDecGenF32)
        sr[t][c] = __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, sidx * 4u, 0, 0);
      else if (MODE == kDecGenBf16)
        sr[t][c] = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc, sidx * 2u, 0, 0);
      zr[t][c] = (MODE != kDecFast && zmode) ? load_elem(a.zp, a.zp_dt, sidx) : 0.f;
    }
  };
  // the first D chunks now, chunk c + D when chunk c is computed
  constexpr int D = CPW > ZT_STREAM_DEPTH ? ZT_STREAM_DEPTH : CPW;
#pragma unroll
  for (int c = 0; c < D; ++c) load_chunk(c);

  // 3. copy x by loads when the DMA does not apply (P == 1 only), and wait
  //    for it.  With the DMA and the fast mode a wave issued exactly
  //    TPW*CPW weight loads after its x and scale DMAs, so waiting until at
  //    most that many are outstanding (then a bare barrier) leaves the
  //    weights in flight: each chunk is dequantised as its own weights land
  //    instead of after all of them (__syncthreads' fence waits for every
  //    load).  Otherwise the barrier's fence waits for x and the weights.
  if (!x_dma) {
    const uint16_t *xp = reinterpret_cast<const uint16_t *>(a.x);
    const int per_row = K / 8;
    for (int idx = tid; idx < M * per_row; idx += 64 * NW) {
      const int m = idx / per_row, k8 = idx - m * per_row;
      *reinterpret_cast<u32x4_t *>(xl + m * XP + k8 * 8) =
          *reinterpret_cast<const u32x4_t *>(xp + (int64_t)m * a.ldx + k8 * 8);
    }
  }
  if (P == 1 && MODE == kDecFast && x_dma) {
    constexpr int after = TPW * D > 63 ? 63 : TPW * D;
    __builtin_amdgcn_s_waitcnt((after & 15) | ((after >> 4) << 14) | (7 << 4) | (15 << 8));
    asm volatile("s_barrier" ::: "memory");
  } else {
    __syncthreads();
  }

  // 4. the slice's MFMAs; between phases every wave finishes with the
  //    range in LDS before the next one is loaded over it.  A chunk's
  //    weight fragments are dequantised once and feed its MT token tiles.
  f32x4_t acc[TPW][MT];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    if (P > 1 && c > 0 && c % CPWP == 0) {
      __syncthreads();
      dma_x(c / CPWP);
      __syncthreads();
    }
    if (c + D < CPW) load_chunk(c + D);
    const int kc = chunk_of(c);
    if (kc < C) {
      const int kcl = P == 1 ? kc : kc - (c / CPWP) * CP;  // chunk within the LDS range
      bf16x8_t wb[TPW][4];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const uint32_t sb =
            MODE == kDecFast
                ? (uint32_t)sl[((min(kc, C - 1) >> cpg_shift) & gmask) * (TPW * 16) + t * 16 + lr]
                : sr[t][c];
        const float sc = MODE == kDecGenF32 ? __uint_as_float(sb) : __uint_as_float(sb << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) wb[t][i] = dq_word<MODE>(wr[t][c][i], sc, zr[t][c], zmode);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // token columns past M repeat row M-1: their sums are never
        // stored, and an unconditional read keeps the loop free of exec
        // branches and of the zero fills they need
        const int row = min(mt * 16 + lr, M - 1);
        u32x4_t xb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          xb[i] = *reinterpret_cast<const u32x4_t *>(xl + row * XP + kcl * 128 + 32 * lg + 8 * i);
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                wb[t][i], __builtin_bit_cast(bf16x8_t, xb[i]), acc[t][mt], 0, 0, 0);
      }
    }
  }

  // 5. partials D[row = 4g + r][token = lane % 16] -> slab[wave][t][mt]
  //    (over x, once every wave is done with it), then each output adds the
  //    NW partials in wave order
  __syncthreads();
  float *slab = reinterpret_cast<float *>(smem);
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        slab[(((wv * TPW + t) * MT + mt) * 16 + 4 * lg + r) * 17 + lr] = acc[t][mt][r];
  __syncthreads();
  if (gu) {
    constexpr int GT = TPW / 2 > 0 ? TPW / 2 : 1;  // gate tiles (TPW is even here)
    const int j0 = blockIdx.x * GT * 16;
    for (int idx = tid; idx < GT * 16 * M; idx += 64 * NW) {
      const int m = idx / (GT * 16), jr = idx - m * (GT * 16);
      const int i = jr >> 4, r16 = jr & 15;
      const int j = j0 + jr;
      if (j >= gu) continue;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        g += slab[((w * TPW + 2 * i) * MT * 16 + r16) * 17 + m];
        u += slab[((w * TPW + 2 * i + 1) * MT * 16 + r16) * 17 + m];
      }
      if (a.bias) {
        g = g + load_elem(a.bias, a.b_dt, j);
        u = u + load_elem(a.bias, a.b_dt, gu + j);
      }
      if (a.y_dt == ZT_DT_BF16) u = bf16_bits_to_f32(f32_to_bf16_bits(u));
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + j, unary_op(ZT_PO_SILU, g) * u);
    }
    return;
  }
  const int n0 = t0 * 16;
  for (int idx = tid; idx < TPW * 16 * M; idx += 64 * NW) {
    const int m = idx / (TPW * 16), nr = idx - m * (TPW * 16);
    const int t = nr >> 4, r16 = nr & 15, mt = m >> 4;
    const int n = n0 + nr;
    if (n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += slab[(((w * TPW + t) * MT + mt) * 16 + r16) * 17 + (m & 15)];
    if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
    v = apply_post_ops(v, a.post, m, n);
    store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
  }
}

// ----------------------------------------------------- prefill GEMM (DMA)
// BM x BN output tile, 4 waves (2 x 2) of (BM/2) x (BN/2), K in steps of
// 128.  Per step the buffer unit moves straight into LDS:
//  * the x slab [BM, 128] bf16: 256-byte rows whose sixteen 16-byte chunks
//    are XOR-swizzled (chunk c of row r at position c ^ (r & 15)), so the 16
//    rows of a fragment read hit every bank once;
//  * the raw int4 slab [BN, 128] (64-byte rows of packed words).
// A lane's B operand for a step is one 16-byte read (the 32 elements
// [32g, 32g+32) of its row, g = lane / 16), dequantised in registers right
// before its MFMAs -- exactly bf16_rne of the reference's fp32 dequantised
// weight -- and its A operand for sub-step i is the 16 bytes of x at element
// 32g + 8i, the same element order.  Two LDS stages; the step's reads are
// issued before the next step's loads, the MFMAs after, one barrier a step.
// The fp32 tile is staged in LDS for the epilogue (bias, post-ops, 8-byte
// bf16 stores).
constexpr int kXRow = 256;   // bytes of x per row per step
constexpr int kWRow = 64;    // bytes of int4 per weight row per step

template <int BM, int BN>
constexpr size_t woq_dma_lds() {
  const size_t stages = 2 * ((size_t)BM * kXRow + (size_t)BN * kWRow);
  const size_t tile = (size_t)BM * (BN + 4) * 4;
  return stages > tile ? stages : tile;
}

// Epilogue of ROWS x BN fp32 outputs staged in LDS (row pitch BN + 4) for
// rows m0.. and columns n0..: bias, post-ops, then rows of four columns per
// thread (8-byte bf16 stores where the row allows), NT threads.
template <int ROWS, int BN, int NT = 256>
__device__ __forceinline__ void woq_tile_epilogue(const WoqArgs &a, const float *tile, int m0,
                                                  int n0, int tid) {
  constexpr int TP = BN + 4;
  const int M = (int)a.M, N = (int)a.N;
  for (int idx = tid; idx < ROWS * (BN / 4); idx += NT) {
    const int row = idx / (BN / 4), c4 = (idx % (BN / 4)) * 4;
    const int m = m0 + row, n = n0 + c4;
    if (m >= M || n >= N) continue;
    const f32x4_t v4 = *reinterpret_cast<const f32x4_t *>(tile + row * TP + c4);
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = v4[r];
      if (n + r < N) {
        if (a.bias) v = v + load_elem(a.bias, a.b_dt, n + r);
        v = apply_post_ops(v, a.post, m, n + r);
      }
      f[r] = v;
    }
    if (a.y_dt == ZT_DT_BF16 && n + 3 < N && (a.ldy & 3) == 0) {
      u32x2_t pk;
      pk[0] = pack_bf16x2(f[0], f[1]);
      pk[1] = pack_bf16x2(f[2], f[3]);
      *reinterpret_cast<u32x2_t *>(reinterpret_cast<uint16_t *>(a.y) + (int64_t)m * a.ldy + n) = pk;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n + r, f[r]);
    }
  }
}

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void woq_gemm_dma_kernel(WoqArgs a, int tiles_m, int tiles_n, int group_m, int cpg_shift,
                         int gmask) {
  constexpr int WTM = BM / 32, WTN = BN / 32;
  constexpr int STAGE = BM * kXRow + BN * kWRow;
  constexpr int XI = BM * kXRow / 1024;  // 1 KB loads per stage: x
  constexpr int WI = BN * kWRow / 1024;  //                        weights
  static_assert((XI + WI) % 4 == 0, "loads must split over 4 waves");
  constexpr int LPW = (XI + WI) / 4;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 15, lg = lane >> 4;

  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int KW = K / 8;
  const int m0 = tm * BM, n0 = tn * BN;
  const int zmode = zp_mode_of(a.zp, a.zp_dt);
  const int s_bytes = MODE == kDecGenF32 ? 4 : 2;

  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)M * a.ldx * 2));
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * s_bytes));

  // This wave's LPW 1 KB loads per stage: x loads cover 4 rows (16 lanes x
  // 16 B each, chunk positions XOR-swizzled by row), weight loads 16 rows
  // (4 lanes x 16 B each).
  const int ldx2 = (int)a.ldx * 2;
  auto dma = [&](int step) {
    unsigned char *stage = smem + (step & 1) * STAGE;
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      const int li = wv * LPW + q;
      if (li < XI) {
        const int row = li * 4 + (lane >> 4);
        const int chunk = (lane & 15) ^ (row & 15);
        const uint32_t off = m0 + row < M ? (uint32_t)((m0 + row) * ldx2 + step * kXRow + chunk * 16)
                                          : kOobOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rs, (lds_ptr_t)(stage + li * 1024), 16, off, 0, 0, 0);
      } else {
        const int wi = li - XI;
        const int row = wi * 16 + (lane >> 2);
        const uint32_t off = n0 + row < N ? (uint32_t)((n0 + row) * KW * 4 + step * kWRow + (lane & 3) * 16)
                                          : kOobOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (lds_ptr_t)(stage + BM * kXRow + wi * 1024), 16,
                                                 off, 0, 0, 0);
      }
    }
  };

  // this lane's weight rows (clamped: rows past N are computed, never stored)
  uint32_t srow[WTN];
#pragma unroll
  for (int j = 0; j < WTN; ++j) srow[j] = (uint32_t)min(n0 + wn * (BN / 2) + j * 16 + lr, N - 1);

  f32x4_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = K / 128;
  dma(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int ks = 0; ks < nk; ++ks) {
    const unsigned char *stage = smem + (ks & 1) * STAGE;
    // scales (and zero points) of this step, one per weight row
    uint32_t sraw[WTN];
    float zr[WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const uint32_t sidx = (uint32_t)((ks >> cpg_shift) & gmask) * (uint32_t)N + srow[j];
      sraw[j] = MODE == kDecGenF32 ? __builtin_amdgcn_raw_buffer_load_b32(s_rs, sidx * 4u, 0, 0)
                                   : __builtin_amdgcn_raw_buffer_load_b16(s_rs, sidx * 2u, 0, 0);
      zr[j] = (MODE != kDecFast && zmode) ? load_elem(a.zp, a.zp_dt, sidx) : 0.f;
    }
    // raw weight words: row (wn*BN/2 + j*16 + lr), 16 bytes at 16*lg
    u32x4_t wraw[WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j)
      wraw[j] = *reinterpret_cast<const u32x4_t *>(
          stage + BM * kXRow + (wn * (BN / 2) + j * 16 + lr) * kWRow + 16 * lg);
    // x fragments of all four sub-steps: row (wm*BM/2 + i*16 + lr), logical
    // chunk 4*lg + sub (element 32*lg + 8*sub), swizzled by the row
    u32x4_t xf[4][WTM];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const int row = wm * (BM / 2) + i * 16 + lr;
        xf[sub][i] = *reinterpret_cast<const u32x4_t *>(
            stage + row * kXRow + (((4 * lg + sub) ^ (row & 15)) * 16));
      }
    if (ks + 1 < nk) dma(ks + 1);
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      bf16x8_t B[WTN];
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const float sc = MODE == kDecGenF32 ? __uint_as_float(sraw[j]) : __uint_as_float(sraw[j] << 16);
        B[j] = dq_word<MODE>(wraw[j][sub], sc, zr[j], zmode);
      }
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, xf[sub][i]), B[j], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // D[m = 4g + r][n = lane % 16] -> fp32 tile in LDS -> rows of 4 columns
  constexpr int TP = BN + 4;
  float *tile = reinterpret_cast<float *>(smem);
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        tile[(wm * (BM / 2) + i * 16 + 4 * lg + r) * TP + wn * (BN / 2) + j * 16 + lr] = acc[i][j][r];
  __syncthreads();
  woq_tile_epilogue<BM, BN>(a, tile, m0, n0, tid);
}

// ROWS x BN fp32 tile staged in LDS (row pitch BN + 4) -> rows m0.. and
// columns n0.. of a K split's fp32 partial [M][N] (N % 4 == 0: a column
// quad lies wholly inside or past N), NT threads.
template <int ROWS, int BN, int NT = 256>
__device__ __forceinline__ void woq_tile_store_partial(const float *tile, float *pp, int m0,
                                                       int n0, int M, int N, int tid) {
  constexpr int TP = BN + 4, Q = BN / 4;
  for (int idx = tid; idx < ROWS * Q; idx += NT) {
    const int r = idx / Q, c = (idx - r * Q) * 4;
    const int m = m0 + r, n = n0 + c;
    if (m < M && n < N)
      *reinterpret_cast<f32x4_t *>(pp + (size_t)m * N + n) =
          *reinterpret_cast<const f32x4_t *>(tile + r * TP + c);
  }
}

// Prefill int4 GEMM on v_mfma_f32_32x32x16_bf16 (signed int4, bf16 scales):
// BM x BN tiles, 4 waves of (BM/2) x (BN/2), K in steps of 64, two stages
// moved straight into LDS by the buffer unit: the x slab [BM][64] bf16 (128 B
// rows, 16-byte chunk c of row r at position c ^ ((r ^ (r >> 3)) & 7)), the
// int4 slab [BN][64] (32 B rows, 16-byte half h of row r at h ^ ((r >> 3) &
// 1)) and the step's scale row [BN] bf16.  Both swizzles give the 16 rows one
// fragment read touches 16 distinct 16-byte bank groups.  Two workgroups per
// CU (at most 256 registers and 80 KB of LDS each) overlap one another's
// barriers and epilogues.
//
// k order: the MFMA pairs A and B by k position, so any permutation shared
// by both operands leaves the sums unchanged (bit for bit: each MFMA adds
// the same 16 products).  Sub-step s of a step takes, for lane half h, the
// eight k of word 4h + s of each 32-byte weight row, which lets a lane read
// its four weight words of the step in one 16-byte LDS read; its x fragment
// is chunk 4h + s of the row.
//
// A = dequantised W (exactly bf16_rne of the reference's fp32 dequantised
// weight), B = x, so D is [n][m]: register r of lane l holds
// n = 8*(r/4) + 4*(l/32) + r%4 and m = l%32.  The epilogue stages one half of
// the tile (the rows of the waves with wm == h) as fp32 [m][n] at a time.
// With a K split (partial set, grid.y splits of sps steps) a workgroup walks
// its split's steps only and writes its fp32 tile to partial[split][M][N];
// woq_splitk_reduce_kernel then adds the splits in order and applies the
// epilogue.
constexpr int kW32BK = 64;

// s_waitcnt immediate that waits for at most n outstanding vector-memory
// operations (n < 64) and nothing else
__host__ __device__ constexpr int vmcnt_imm_woq(int n) {
  return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

template <int BM, int BN>
constexpr size_t woq_gemm32_stage() {
  return (size_t)BM * 128 + (size_t)BN * 32 + 1024;
}
template <int BM, int BN>
constexpr size_t woq_gemm32_lds() {
  const size_t stages = 2 * woq_gemm32_stage<BM, BN>();
  const size_t half = (size_t)(BM / 2) * (BN + 4) * 4;
  return stages > half ? stages : half;
}

template <int BM, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void woq_gemm32_kernel(WoqArgs a, int tiles_m, int tiles_n, int group_m, int cpg_shift,
                       int gmask, float *partial, int sps) {
  constexpr int WTM = BM / 64, WTN = BN / 64;  // 32 x 32 tiles per wave
  constexpr int STAGE = (int)woq_gemm32_stage<BM, BN>();
  constexpr int XI = BM / 8;                    // 1 KB x loads (8 rows) per stage
  constexpr int WI = BN / 32;                   // 1 KB weight loads (32 rows)
  constexpr int LOADS = XI + WI + 1;            // + the scale row
  constexpr int LPW = (LOADS + 3) / 4;
  static_assert(BN <= 512 && BN % 64 == 0 && BM % 64 == 0, "tile shape");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv >> 1, wn = wv & 1;
  const int hl = lane >> 5, l32 = lane & 31;

  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int m0 = tm * BM, n0 = tn * BN;
  const int ldx2 = (int)a.ldx * 2, KB = K / 2;

  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)M * ldx2));
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KB));
  const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * 2));

  // the wave's loads: index li = wv * LPW + q; x loads first, then the
  // weight loads, then the scale row (lanes 0..BN/8-1, 16 bytes each)
  const int nk = K / kW32BK;
  const int kb = partial ? (int)blockIdx.y * sps : 0;   // this workgroup's steps [kb, ke)
  const int ke = partial ? min(kb + sps, nk) : nk;
  auto dma = [&](int step) {
    const int k0 = step * kW32BK;
    const bool in = step < ke;
    unsigned char *stage = smem + (step & 1) * STAGE;
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
      const int li = wv * LPW + q;
      if (li >= LOADS) break;
      uint32_t off;
      if (li < XI) {
        const int row = li * 8 + (lane >> 3);
        const int chunk = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
        off = in && m0 + row < M ? (uint32_t)((m0 + row) * ldx2 + k0 * 2 + chunk * 16) : kOobOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rs, (lds_ptr_t)(stage + li * 1024), 16, off, 0, 0, 0);
      } else if (li < XI + WI) {
        const int wi = li - XI;
        const int row = wi * 32 + (lane >> 1);
        const int half = (lane & 1) ^ ((row >> 3) & 1);
        off = in && n0 + row < N ? (uint32_t)((n0 + row) * KB + k0 / 2 + half * 16) : kOobOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (lds_ptr_t)(stage + BM * 128 + wi * 1024), 16,
                                                 off, 0, 0, 0);
      } else {
        // N % 8 == 0 (host-checked): a lane's 8 scales lie wholly inside or past N
        const uint32_t grp = (uint32_t)(((k0 >> 7) >> cpg_shift) & gmask);
        off = in && lane < BN / 8 && n0 + 8 * lane < N
                  ? (grp * (uint32_t)N + (uint32_t)(n0 + 8 * lane)) * 2u
                  : kOobOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rs, (lds_ptr_t)(stage + BM * 128 + BN * 32), 16,
                                                 off, 0, 0, 0);
      }
    }
  };

  f32x16_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  dma(kb);
  for (int ks = kb; ks < ke; ++ks) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's loads of step ks
    asm volatile("s_barrier" ::: "memory");
    dma(ks + 1);  // past the last step: zeros into the buffer step ks - 1 used
    const unsigned char *stage = smem + (ks & 1) * STAGE;
    // weight words 4h..4h+3 of rows wn*BN/2 + 32j + l32, and their scales
    u32x4_t wq[WTN];
    float sc[WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int row = wn * (BN / 2) + j * 32 + l32;
      wq[j] = *reinterpret_cast<const u32x4_t *>(stage + BM * 128 + row * 32 +
                                                 ((hl ^ ((row >> 3) & 1)) * 16));
      sc[j] = bf16_bits_to_f32(
          *reinterpret_cast<const uint16_t *>(stage + BM * 128 + BN * 32 + row * 2));
    }
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const int chunk = 4 * hl + sub;
      bf16x8_t xb[WTM];
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const int row = wm * (BM / 2) + i * 32 + l32;
        xb[i] = *reinterpret_cast<const bf16x8_t *>(stage + row * 128 +
                                                    ((chunk ^ ((row ^ (row >> 3)) & 7)) * 16));
      }
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const bf16x8_t wb = dq_word<kDecFast>(wq[j][sub], sc[j], 0.f, 0);
#pragma unroll
        for (int i = 0; i < WTM; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb, xb[i], acc[i][j], 0, 0, 0);
      }
    }
  }

  // epilogue in two halves of BM/2 rows
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_barrier" ::: "memory");
  constexpr int TP = BN + 4;
  float *tile = reinterpret_cast<float *>(smem);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (wm == h) {
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4_t *>(tile + (i * 32 + l32) * TP + wn * (BN / 2) + j * 32 + 8 * q +
                                         4 * hl) =
                f32x4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]};
    }
    __syncthreads();
    if (partial)
      woq_tile_store_partial<BM / 2, BN>(tile, partial + (size_t)blockIdx.y * M * N,
                                         m0 + h * (BM / 2), n0, M, N, tid);
    else
      woq_tile_epilogue<BM / 2, BN>(a, tile, m0 + h * (BM / 2), n0, tid);
    __syncthreads();
  }
}

// The same tile with the loads in waves of their own (as s8_gemm_ws_kernel
// does for int8): four compute waves (128 x 64 each) only read LDS, dequantise
// and issue MFMAs; four load waves move the S-stage [x | W | scales] slabs
// by DMA, S - 1 steps ahead, one workgroup per CU.  A load wave waits only
// for its own loads (in-order vmcnt); one s_barrier per step.  Every load
// wave issues the same number of loads per step (the last ones out of range
// into a spare 1 KB of LDS), so the wait count is one immediate.
template <int BM, int BN, int S>
constexpr size_t woq_gemm_ws_lds() {
  const size_t stages = (size_t)S * woq_gemm32_stage<BM, BN>() + 1024;
  const size_t half = (size_t)(BM / 2) * (BN + 4) * 4;
  return stages > half ? stages : half;
}

template <int BM, int BN, int S>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void woq_gemm_ws_kernel(WoqArgs a, int tiles_m, int tiles_n, int group_m, int cpg_shift,
                        int gmask) {
  constexpr int WTM = BM / 64, WTN = BN / 64;  // 32 x 32 tiles per compute wave
  constexpr int STAGE = (int)woq_gemm32_stage<BM, BN>();
  constexpr int XI = BM / 8;          // 1 KB x loads (8 rows) per stage
  constexpr int WI = BN / 32;         // 1 KB weight loads (32 rows)
  constexpr int LOADS = XI + WI + 1;  // + the scale row
  constexpr int LPW = (LOADS + 3) / 4;
  static_assert((S - 2) * LPW <= 63 && S >= 2 && BN % 64 == 0 && BM % 64 == 0, "tile shape");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = xcd_contiguous_tile(blockIdx.x, tiles_m * tiles_n);
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, tg = t - g * per_group;
  const int gm = min(group_m, tiles_m - g * group_m);
  const int tm = g * group_m + tg % gm, tn = tg / gm;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = K / kW32BK;

  f32x16_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (wv >= 4) {
    // load wave dw issues loads li = dw + 4 q (q < LPW): x rows, weight
    // rows, the scale row, then out-of-range fillers into the spare 1 KB
    const int dw = wv - 4;
    const int ldx2 = (int)a.ldx * 2, KB = K / 2;
    const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)M * ldx2));
    const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KB));
    const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * 2));
    auto dma = [&](int step) {
      const int k0 = step * kW32BK;
      const bool in = step < nk;
      unsigned char *stage = smem + (step % S) * STAGE;
#pragma unroll
      for (int q = 0; q < LPW; ++q) {
        const int li = dw + 4 * q;
        if (li < XI) {
          const int row = li * 8 + (lane >> 3);
          const int chunk = (lane & 7) ^ ((row ^ (row >> 3)) & 7);
          const uint32_t off = in && m0 + row < M
                                   ? (uint32_t)((m0 + row) * ldx2 + k0 * 2 + chunk * 16) : kOobOffset;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rs, (lds_ptr_t)(stage + li * 1024), 16, off, 0, 0, 0);
        } else if (li < XI + WI) {
          const int wi = li - XI;
          const int row = wi * 32 + (lane >> 1);
          const int half = (lane & 1) ^ ((row >> 3) & 1);
          const uint32_t off = in && n0 + row < N
                                   ? (uint32_t)((n0 + row) * KB + k0 / 2 + half * 16) : kOobOffset;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rs, (lds_ptr_t)(stage + BM * 128 + wi * 1024), 16,
                                                   off, 0, 0, 0);
        } else if (li == XI + WI) {
          // N % 8 == 0 (host-checked): a lane's 8 scales lie wholly inside or past N
          const uint32_t grp = (uint32_t)(((k0 >> 7) >> cpg_shift) & gmask);
          const uint32_t off = in && lane < BN / 8 && n0 + 8 * lane < N
                                   ? (grp * (uint32_t)N + (uint32_t)(n0 + 8 * lane)) * 2u
                                   : kOobOffset;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rs, (lds_ptr_t)(stage + BM * 128 + BN * 32), 16,
                                                   off, 0, 0, 0);
        } else {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rs, (lds_ptr_t)(smem + S * STAGE), 16,
                                                   kOobOffset, 0, 0, 0);
        }
      }
    };
#pragma unroll
    for (int p = 0; p < S - 1; ++p) dma(p);
    for (int ks = 0; ks < nk; ++ks) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm_woq((S - 2) * LPW));  // this wave's loads of step ks
      asm volatile("s_barrier" ::: "memory");
      dma(ks + S - 1);  // into the stage step ks - 1 used; past the end: zeros
    }
    __builtin_amdgcn_s_waitcnt(0);
  } else {
    const int wm = wv >> 1, wn = wv & 1;
    const int hl = lane >> 5, l32 = lane & 31;
    for (int ks = 0; ks < nk; ++ks) {
      asm volatile("s_barrier" ::: "memory");
      const unsigned char *stage = smem + (ks % S) * STAGE;
      u32x4_t wq[WTN];
      float sc[WTN];
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const int row = wn * (BN / 2) + j * 32 + l32;
        wq[j] = *reinterpret_cast<const u32x4_t *>(stage + BM * 128 + row * 32 +
                                                   ((hl ^ ((row >> 3) & 1)) * 16));
        sc[j] = bf16_bits_to_f32(
            *reinterpret_cast<const uint16_t *>(stage + BM * 128 + BN * 32 + row * 2));
      }
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const int chunk = 4 * hl + sub;
        bf16x8_t xb[WTM];
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
          const int row = wm * (BM / 2) + i * 32 + l32;
          xb[i] = *reinterpret_cast<const bf16x8_t *>(stage + row * 128 +
                                                      ((chunk ^ ((row ^ (row >> 3)) & 7)) * 16));
        }
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
          const bf16x8_t wb = dq_word<kDecFast>(wq[j][sub], sc[j], 0.f, 0);
#pragma unroll
          for (int i = 0; i < WTM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb, xb[i], acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // epilogue in two halves of BM/2 rows, all eight waves
  __syncthreads();
  constexpr int TP = BN + 4;
  float *tile = reinterpret_cast<float *>(smem);
  const int wm = wv >> 1, wn = wv & 1, hl = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (wv < 4 && wm == h) {
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4_t *>(tile + (i * 32 + l32) * TP + wn * (BN / 2) + j * 32 + 8 * q +
                                         4 * hl) =
                f32x4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]};
    }
    __syncthreads();
    woq_tile_epilogue<BM / 2, BN, 512>(a, tile, m0 + h * (BM / 2), n0, tid);
    __syncthreads();
  }
}

template <int BM, int BN, int S>
static hipError_t launch_woq_gemm_ws_t(const WoqArgs &a, hipStream_t s, int shift, int gmask) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  woq_gemm_ws_kernel<BM, BN, S><<<dim3((unsigned)(tiles_m * tiles_n)), dim3(512),
                                  woq_gemm_ws_lds<BM, BN, S>(), s>>>(a, tiles_m, tiles_n, group_m,
                                                                     shift, gmask);
  return hipGetLastError();
}

// splits > 1: K split into splits ranges of whole steps, fp32 partials to
// `partial` ([splits][M][N]); the caller adds them
template <int BM, int BN>
static hipError_t launch_woq_gemm32_t(const WoqArgs &a, hipStream_t s, int shift, int gmask,
                                      float *partial = nullptr, int splits = 1) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  const int nk = (int)(a.K / kW32BK);
  const int sps = splits > 1 ? (nk + splits - 1) / splits : nk;
  woq_gemm32_kernel<BM, BN><<<dim3((unsigned)(tiles_m * tiles_n), (unsigned)(splits > 1 ? splits : 1)),
                              dim3(256), woq_gemm32_lds<BM, BN>(), s>>>(
      a, tiles_m, tiles_n, group_m, shift, gmask, splits > 1 ? partial : nullptr, sps);
  return hipGetLastError();
}

template <int BM, int BN>
static hipError_t launch_woq_dma_t(const WoqArgs &a, hipStream_t s, int shift, int gmask, int mode) {
  const int tiles_m = (int)((a.M + BM - 1) / BM), tiles_n = (int)((a.N + BN - 1) / BN);
  const int group_m = tiles_m < 4 ? tiles_m : 4;
  dim3 grid((unsigned)(tiles_m * tiles_n)), block(256);
  const size_t lds = woq_dma_lds<BM, BN>();
  if (mode == kDecFast)
    woq_gemm_dma_kernel<BM, BN, kDecFast><<<grid, block, lds, s>>>(a, tiles_m, tiles_n, group_m, shift, gmask);
  else if (mode == kDecGenBf16)
    woq_gemm_dma_kernel<BM, BN, kDecGenBf16><<<grid, block, lds, s>>>(a, tiles_m, tiles_n, group_m, shift, gmask);
  else
    woq_gemm_dma_kernel<BM, BN, kDecGenF32><<<grid, block, lds, s>>>(a, tiles_m, tiles_n, group_m, shift, gmask);
  return hipGetLastError();
}

// --------------------------------------------------------------- GEMM
constexpr int kGemmBK = 64;

template <int BM, int BN>
__global__ __launch_bounds__(256) void woq_gemm_kernel(WoqArgs a) {
  constexpr int LD = kGemmBK + 8;  // bf16 per LDS row, padded by 16 bytes
  constexpr int WTM = BM / 32, WTN = BN / 32;  // 16x16 tiles per wave (2x2 waves)
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LD];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LD];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 15, lg = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t M = a.M, N = a.N, K = a.K, KW = K / 8, gs = K / a.G;
  const int zmode = zp_mode_of(a.zp, a.zp_dt);
  const bool fast = zmode == kZpNone && a.s_dt == ZT_DT_BF16;
  const uint16_t *xp = reinterpret_cast<const uint16_t *>(a.x);

  f32x4_t acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = 0; k0 < K; k0 += kGemmBK) {
    // activations: BM x 64 bf16, 16-byte chunks
    for (int i = tid; i < BM * 8; i += 256) {
      const int r = i >> 3, cc = i & 7;
      const int64_t m = m0 + r;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (m < M)
        v = *reinterpret_cast<const u32x4_t *>(xp + m * a.ldx + k0 + cc * 8);
      *reinterpret_cast<u32x4_t *>(As + r * LD + cc * 8) = v;
    }
    // weights: BN x 64 int4 = two 16-byte chunks per row, dequantised to
    // bf16 as the reference's dequantise-then-GEMM would
    for (int i = tid; i < BN * 2; i += 256) {
      const int r = i >> 1, h = i & 1;
      const int64_t n = min(n0 + r, N - 1);
      const u32x4_t wq =
          *reinterpret_cast<const u32x4_t *>(a.w + n * KW + k0 / 8 + h * 4);
      const int64_t sidx = ((k0 + h * 32) / gs) * N + n;
      const float s = load_elem(a.scales, a.s_dt, sidx);
      u32x4_t o[4];
      if (fast) {
        const float s16 = s * 0.0625f, c0 = -1032.f * s, c1 = -72.f * s;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = dq8_s4_bf16scale(wq[j], s, s16, c0, c1);
      } else {
        const DqGeneral d =
            dq_general_params(zmode, s, zmode ? load_elem(a.zp, a.zp_dt, sidx) : 0.f);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = dq8_general(wq[j], d);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<u32x4_t *>(Bs + r * LD + h * 32 + j * 8) = o[j];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kGemmBK / 32; ++kk) {
      bf16x8_t Af[WTM], Bf[WTN];
#pragma unroll
      for (int i = 0; i < WTM; ++i)
        Af[i] = *reinterpret_cast<const bf16x8_t *>(
            As + (wm * (BM / 2) + i * 16 + lr) * LD + kk * 32 + 8 * lg);
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        Bf[j] = *reinterpret_cast<const bf16x8_t *>(
            Bs + (wn * (BN / 2) + j * 16 + lr) * LD + kk * 32 + 8 * lg);
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(Af[i], Bf[j], acc[i][j], 0, 0, 0);
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
        if (m < M && n < N) {
          float v = acc[i][j][r];
          if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
          v = apply_post_ops(v, a.post, m, n);
          store_elem(a.y, a.y_dt, m * a.ldy + n, v);
        }
      }
}

// ------------------------------------------------------------- repack
__global__ void repack_kernel(const int8_t *w, int64_t N, int64_t K,
                              int32_t *out) {
  const int64_t KW = K / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * KW) return;
  const int64_t n = i / KW, c = i % KW;
  const int8_t *src = w + n * K + 8 * c;
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) word |= ((uint32_t)(uint8_t)src[j] & 0xFu) << (4 * j);
  out[i] = (int32_t)word;
}

// torch CPU int4pack (BLOCK_N = 64): within a 64-row block, column k holds
// 32 bytes; byte d (d<16) has rows d (low nibble) and d+32 (high), byte 16+d
// has rows d+16 (low) and d+48 (high) (WOQ_Linear.cpp:395-426).
__global__ void repack_from_int4pack_kernel(const uint8_t *packed, int64_t N,
                                            int64_t K, int32_t *out) {
  const int64_t KW = K / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * KW) return;
  const int64_t n = i / KW, c = i % KW;
  const int64_t nb = n / 64;
  const int dd = (int)(n % 64), quad = dd / 16, d = dd % 16;
  const uint8_t *src = packed + nb * K * 32;
  const int byte_off = (quad & 1) ? 16 + d : d;
  const int shift = (quad & 2) ? 4 : 0;
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t k = 8 * c + j;
    word |= (((uint32_t)src[k * 32 + byte_off] >> shift) & 0xFu) << (4 * j);
  }
  out[i] = (int32_t)word;
}

}  // namespace

// ------------------------------------------------------------ host side
static bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

WoqKernelKind woq_select_kernel(const WoqArgs &a) {
  if (const char *f = knob(kKnobWoqForceKernel)) {
    if (!std::strcmp(f, "generic")) return kWoqGeneric;
  }
  const bool bf16_ok = a.x_dt == ZT_DT_BF16 && a.ldx % 8 == 0 &&
                       aligned16(a.x) && aligned16(a.w);
  if (!bf16_ok || a.N < 1) return kWoqGeneric;
  const int64_t gs = a.K / a.G;
  const char *f = knob(kKnobWoqForceKernel);
  const int64_t cpg = gs / 128;
  const bool decode_ok = a.K % 128 == 0 &&
                         (a.G == 1 || (gs % 128 == 0 && (cpg & (cpg - 1)) == 0)) &&
                         a.N * (a.K / 2) < ((int64_t)1 << 31) &&  // 32-bit buffer offsets
                         a.M <= 32 && a.N < (int64_t)1 << 30;
  const bool gemm_ok = a.K % kGemmBK == 0 && gs % 32 == 0;
  if (f && !std::strcmp(f, "gemm")) return gemm_ok ? kWoqGemm : kWoqGeneric;
  if (f && !std::strcmp(f, "decode")) return decode_ok ? kWoqDecode : kWoqGeneric;
  if (decode_ok) return kWoqDecode;
  if (gemm_ok) return kWoqGemm;
  return kWoqGeneric;
}

static int env_plan(int *v) {
  const char *p = knob(kKnobWoqDecodePlan);
  if (!p) return 0;
  return std::sscanf(p, "%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3]) == 4;
}

static int max_waves_for(int cpw) { return (cpw <= 2 ? 1024 : (cpw == 4 ? 512 : 256)) / 64; }

// Instantiated (MT, CPW, NI, XR) shapes; the launcher has one case each.
static bool decode_shape_ok(int mt, int cpw, int ni, bool xr) {
  if (cpw != 2) return false;
  if (xr) return ni == 1 || ni == 2 || ni == 3 || ni == 4 || ni == 6 || ni == 8;
  return mt == 1 && (ni == 2 || ni == 4 || ni == 8);
}

static size_t decode_lds(int64_t M, int C, const DecodePlan &p) {
  size_t b = decode_slab_bytes(p.NK, p.NT, p.TPW, p.mt);
  if (p.xs) {
    const int CW = (C + p.NK - 1) / p.NK;
    b += (size_t)p.NK * p.NT * 8 * (CW * 128 + 8) * 2;
  }
  (void)M;
  return b;
}

// Shape of a decode launch (measured on MI355X, graph-replayed):
//  * K slices of 2 chunks per wave (CPW = 2) with up to 16 waves per
//    workgroup splitting K; for longer K the slice is walked in phases and
//    the wave count is the one that leaves no idle chunk (K = 14336:
//    14 waves x 8 chunks);
//  * one row block per workgroup, TPW = ceil(tiles / 256) tiles per wave, so
//    the grid is one round over the 256 CUs and each wave reuses its
//    activations over TPW tiles.
bool woq_decode_plan(int64_t M, int64_t N, int64_t K, DecodePlan *plan) {
  const int C = (int)(K / 128);
  const int tiles = (int)((N + 15) / 16);
  DecodePlan p{};
  p.mt = M <= 16 ? 1 : 2;
  p.S = 1;
  p.CPW = 2;
  p.NT = 1;
  auto finish = [&](DecodePlan &q) {
    const int CW = (C + q.NK - 1) / q.NK;
    const int nphase = (CW + q.CPW - 1) / q.CPW;
    q.xl = nphase == 1;  // XR
    q.xs = q.xl && M <= 8;
    q.ni = q.xl ? q.TPW : nphase;
    if (!q.xl && q.TPW != 1) return false;
    if (!decode_shape_ok(q.mt, q.CPW, q.ni, q.xl)) return false;
    if (q.NK < 1 || q.NT < 1 || q.NK * q.NT > max_waves_for(q.CPW)) return false;
    if (decode_lds(M, C, q) > 160 * 1024) return false;
    q.nrb = (tiles + q.NT * q.TPW - 1) / (q.NT * q.TPW);
    return true;
  };
  int v[4];
  if (env_plan(v)) {
    p.NK = v[0], p.NT = v[1], p.CPW = v[2], p.TPW = v[3];
    if (!finish(p)) return false;
    *plan = p;
    return true;
  }
  if (C <= 32) {
    p.NK = (C + 1) / 2;
    int tpw = std::max(1, (tiles + 255) / 256);
    for (int t : {1, 2, 3, 4, 6, 8})
      if (t >= tpw) { tpw = t; break; }
    p.TPW = std::min(tpw, 8);
    // Keep the slabs of wide row blocks inside LDS.
    while (p.TPW > 1 && !finish(p)) p.TPW = p.TPW == 8 ? 6 : (p.TPW == 6 ? 4 : p.TPW - 1);
  } else {
    // Phased: the largest wave count <= 16 whose slice is a whole number of
    // 2-chunk phases with the fewest idle chunks.
    int best_nk = 16, best_waste = 1 << 30;
    for (int nk = 16; nk >= 1; --nk) {
      int cw = (C + nk - 1) / nk;
      cw = (cw + 1) / 2 * 2;
      const int waste = cw * nk - C;
      if ((cw / 2 == 2 || cw / 2 == 4 || cw / 2 == 8) && waste < best_waste)
        best_nk = nk, best_waste = waste;
    }
    p.NK = best_nk;
    p.TPW = 1;
  }
  if (!finish(p)) return false;
  *plan = p;
  return true;
}

size_t woq_decode_workspace(const DecodePlan &, int64_t, int64_t) { return 0; }

hipError_t launch_woq_generic(const WoqArgs &a, hipStream_t s) {
  const int64_t waves = a.M * a.N;
  if (waves == 0) return hipSuccess;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL(woq_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int MT, int CPW, int NI, bool XR, bool XS>
static hipError_t launch_decode_t(const WoqArgs &a, const DecodePlan &p, hipStream_t s) {
  const size_t lds = decode_lds(a.M, (int)(a.K / 128), p);
  dim3 grid((unsigned)p.nrb), block(64 * p.NK * p.NT);
  const int64_t cpg = a.G == 1 ? 0 : (a.K / a.G) / 128;
  int shift = 0;
  while (cpg > 1 && (1 << shift) < cpg) ++shift;
  const int gmask = a.G == 1 ? 0 : 0x7fffffff;
  const int mode = a.s_dt == ZT_DT_F32 ? kDecGenF32 : (a.zp ? kDecGenBf16 : kDecFast);
  if (mode == kDecFast)
    hipLaunchKernelGGL((woq_decode_kernel<MT, CPW, NI, kDecFast, XR, XS>), grid, block, lds, s, a,
                       p.NK, p.NT, shift, gmask);
  else if (mode == kDecGenBf16)
    hipLaunchKernelGGL((woq_decode_kernel<MT, CPW, NI, kDecGenBf16, XR, XS>), grid, block, lds, s,
                       a, p.NK, p.NT, shift, gmask);
  else
    hipLaunchKernelGGL((woq_decode_kernel<MT, CPW, NI, kDecGenF32, XR, XS>), grid, block, lds, s,
                       a, p.NK, p.NT, shift, gmask);
  return hipGetLastError();
}

// x goes to LDS by DMA when its rows (or each phase's part of them) are
// whole 1 KB pieces, 16-byte aligned, within 32-bit offsets
// ------------------------------------------- wave-independent decode
// One 16-row weight tile per workgroup, K split over NW waves of CPW
// 128-wide chunks each, and no barrier until the final reduction: each wave
// moves its own slice of x (its chunks' columns of the M token rows) into
// its own LDS region by DMA, loads its own row scales per lane and issues
// all its weight loads at once, then computes its chunks as they land.
// (The stream kernel's shared x copy needs one barrier before any wave
// computes; here the waves start as soon as their own loads arrive.)  The
// NW partial tiles meet in LDS and are added in wave order, as the stream
// kernel does.  Fast mode only: signed int4, bf16 scales, bf16 x, M <= 16.
// A wave's region holds its [M][CPW * 256 B] slice rounded up to whole
// 1 KB DMA instructions (each writes 64 lanes x 16 B, the lanes past the
// slice writing zeros), so no DMA reaches the next wave's region.
__host__ __device__ constexpr int wave_region_bytes(int M, int CPW) {
  return (M * CPW * 256 + 1023) / 1024 * 1024;
}
template <int NW, int CPW>
constexpr size_t wave_x_bytes(int M) {
  return (size_t)NW * wave_region_bytes(M, CPW);
}

template <int NW, int CPW, int TPW>
__global__ __launch_bounds__(64 * NW) void woq_wave_kernel(WoqArgs a, int cpg_shift, int gmask,
                                                           int gu) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K, KW = K / 8;
  // tile t's first weight row: TPW consecutive 16-row tiles, or with gu > 0
  // (merged gate_up, TPW == 2) gate rows j0.. and the up rows gu + j0..
  const int j0 = blockIdx.x * 16;
  auto rowbase = [&](int t) { return gu ? t * gu + j0 : (blockIdx.x * TPW + t) * 16; };
  constexpr int RB = CPW * 256;    // bytes of one token row of the wave's slice
  constexpr int UPR = RB / 16;     // 16-byte units per row
  const int c0 = wv * CPW;         // the wave's first chunk (K == NW * CPW * 128)
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * 2));
  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)(M - 1) * a.ldx * 2 + (int64_t)K * 2));
  unsigned char *xw = smem + (size_t)wv * wave_region_bytes(M, CPW);
  // 1. the wave's x slice [M][RB] by DMA: unit u = 64 j + lane is row u / UPR,
  //    16-byte column u % UPR
  const int units = M * UPR;
  for (int j = 0; j * 64 < units; ++j) {
    const int u = j * 64 + lane;
    const int row = u / UPR, col = u - row * UPR;
    const uint32_t off = u < units ? (uint32_t)(row * a.ldx * 2 + c0 * 256 + col * 16) : kOobOffset;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rs, (lds_ptr_t)(xw + j * 1024), 16, off, 0, 0, 0);
  }
  // 2. the row scales of its chunks, 3. all its weights (rows past N, only
  //    in the last workgroup of a plain call, read zeros and are not stored)
  uint32_t sr[TPW][CPW];
  u32x4_t wr[TPW][CPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const uint32_t g = (uint32_t)(((c0 + c) >> cpg_shift) & gmask);
      sr[t][c] = __builtin_amdgcn_raw_buffer_load_b16(
          s_rs, (g * (uint32_t)N + (uint32_t)(rowbase(t) + lr)) * 2u, 0, 0);
    }
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int n = rowbase(t) + lr;
    const uint32_t row_off = n < N ? (uint32_t)n * (uint32_t)KW * 4u + (uint32_t)lg * 16u : kOobOffset;
#pragma unroll
    for (int c = 0; c < CPW; ++c)
      wr[t][c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                 w_rs, row_off + (uint32_t)(c0 + c) * 64u, 0, 0));
  }
  // the x DMA was issued first: once at most the later loads are outstanding
  // it has landed in this wave's region (no other wave writes it)
  constexpr int after = 2 * TPW * CPW > 63 ? 63 : 2 * TPW * CPW;
  __builtin_amdgcn_s_waitcnt((after & 15) | ((after >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");

  f32x4_t acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // token columns past M repeat row M-1: their sums are never stored
  const int row = min(lr, M - 1);
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    u32x4_t xb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xb[i] = *reinterpret_cast<const u32x4_t *>(xw + row * RB + (c * 128 + 32 * lg + 8 * i) * 2);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const float sc = __uint_as_float(sr[t][c] << 16);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(dq_word<kDecFast>(wr[t][c][i], sc, 0.f, 0),
                                                         __builtin_bit_cast(bf16x8_t, xb[i]), acc[t],
                                                         0, 0, 0);
    }
  }
  // 4. partial D[row = 4 lg + r][token = lr] of tile t -> slab[wave][t] (over
  //    x, after every wave is done with its slice), then each output adds the
  //    NW partials in wave order
  __syncthreads();
  float *slab = reinterpret_cast<float *>(smem);
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) slab[((wv * TPW + t) * 16 + 4 * lg + r) * 17 + lr] = acc[t][r];
  __syncthreads();
  if (gu) {
    for (int idx = tid; idx < 16 * M; idx += 64 * NW) {
      const int m = idx / 16, nr = idx - m * 16;
      const int jj = j0 + nr;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        g += slab[((w * TPW) * 16 + nr) * 17 + m];
        u += slab[((w * TPW + 1) * 16 + nr) * 17 + m];
      }
      if (a.bias) {
        g = g + load_elem(a.bias, a.b_dt, jj);
        u = u + load_elem(a.bias, a.b_dt, gu + jj);
      }
      if (a.y_dt == ZT_DT_BF16) u = bf16_bits_to_f32(f32_to_bf16_bits(u));
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + jj, unary_op(ZT_PO_SILU, g) * u);
    }
    return;
  }
  for (int idx = tid; idx < TPW * 16 * M; idx += 64 * NW) {
    const int m = idx / (TPW * 16), nr = idx - m * (TPW * 16);
    const int n = blockIdx.x * TPW * 16 + nr;
    if (n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += slab[((w * TPW + (nr >> 4)) * 16 + (nr & 15)) * 17 + m];
    if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
    v = apply_post_ops(v, a.post, m, n);
    store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
  }
}

template <int NW, int CPW, int TPW>
static hipError_t launch_wave_t(const WoqArgs &a, hipStream_t s, int shift, int gmask, int gu) {
  const size_t slab = (size_t)NW * TPW * 16 * 17 * 4;
  const size_t x = wave_x_bytes<NW, CPW>((int)a.M);
  const unsigned blocks = gu ? (unsigned)(gu / 16) : (unsigned)((a.N + 16 * TPW - 1) / (16 * TPW));
  woq_wave_kernel<NW, CPW, TPW><<<dim3(blocks), dim3(64 * NW), x > slab ? x : slab, s>>>(
      a, shift, gmask, gu);
  return hipGetLastError();
}

// The wave-independent kernel where it applies: fast mode, bf16 x with
// 16-byte rows, M <= 16, K = 16 waves x CPW chunks (CPW 1, 2 or 4) and the
// x slices within 64 KB, more than 4096 rows unless forced; gu > 0 is the
// merged gate_up (I = gu, a multiple of 16, a gate tile and its up tile per
// workgroup; "1" in ZT_WOQ_WAVE takes it below 3 rows and on 4096 rows or
// fewer too).
static bool try_launch_wave(const WoqArgs &a, hipStream_t s, int shift, int gmask, int mode,
                            int gu, hipError_t *err) {
  const char *e = knob(kKnobWoqWave);  // "0" disables
  if (e && e[0] == '0') return false;
  if (mode != kDecFast || a.x_dt != ZT_DT_BF16 || a.M < 1 || a.M > 16 || a.K % (16 * 128) ||
      (gu ? gu % 16 : a.N % 2))
    return false;
  if (((reinterpret_cast<uintptr_t>(a.x) | ((uintptr_t)a.ldx * 2)) & 15u) ||
      (a.M - 1) * a.ldx * 2 + a.K * 2 >= (int64_t)kOobOffset ||
      a.N * (a.K / 2) >= (int64_t)kOobOffset || a.G * a.N * 2 >= (int64_t)kOobOffset)
    return false;
  const int cpw = (int)(a.K / (16 * 128));
  // measured against the stream kernel in the same process (graph replays
  // over rotating weights, Llama-3 8B shapes): QKV 6.3-6.4 us against
  // 6.7-6.9 at M = 2..8, O even; the merged gate_up from M = 3 when the
  // persistent kernel does not take it (16.4-17.1 us at M = 3..8 against
  // 17.1-19.1 on the lean and stream kernels); the down projection (16 x 7
  // chunks, M <= 2) no faster, so CPW 7 is not used
  if (gu && a.M < 3 && !e) return false;
  // at most one tile per CU (N <= 4096), the stream kernel's 8 waves did as
  // well or better on every box measured but one (4096 x 4096 at M = 1..8:
  // 4.96-5.38 us against 5.21-5.42), and its rocprof kernel durations agree
  // with the graph-replay time per call where the wave kernel's run 14 %
  // longer under the tracer
  if (!gu && a.N <= 4096 && !e) return false;
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr, "[zt] woq wave M=%lld N=%lld K=%lld gu=%d: NW=16 CPW=%d\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, gu, cpw);
#define ZT_WAVE_CASE(CPW_)                                                         \
  if (cpw == CPW_ && wave_x_bytes<16, CPW_>((int)a.M) <= 64 * 1024) {              \
    *err = gu ? launch_wave_t<16, CPW_, 2>(a, s, shift, gmask, gu)                 \
              : launch_wave_t<16, CPW_, 1>(a, s, shift, gmask, 0);                 \
    return true;                                                                  \
  }
  ZT_WAVE_CASE(1) ZT_WAVE_CASE(2) ZT_WAVE_CASE(4)
#undef ZT_WAVE_CASE
  return false;
}

// ------------------------------------------------ persistent decode
// The wave kernel's split of K (NW waves of CPW 128-wide chunks, no barrier
// before the reduction) with each workgroup looping over many row units:
// TPW 16-row tiles, or with gu the gate tile and its up tile.  A wave's x
// slice is loaded once into registers as its B operands and serves every
// unit; the weights and scales of the next D units are in flight while a
// unit is computed.  Unit i's partial tiles meet in LDS slab i % 2 after
// one barrier, and its reduction and epilogue run while the next units'
// weights land (slab i % 2 is written again only after the barrier of unit
// i + 1, which every thread reaches after reducing unit i).  Grid: at most
// one workgroup per CU, units dealt round robin, so per-workgroup set-up
// (x, launch) is paid once per CU rather than once per unit.  Fast mode
// only: signed int4, bf16 scales, bf16 x, M <= 16, K == NW * CPW * 128.
template <int NW, int CPW, int TPW>
struct PersistSet {
  u32x4_t w[TPW][CPW];
  uint32_t s[TPW][CPW];
};

template <int NW, int CPW, int TPW, int D>
__global__ __launch_bounds__(64 * NW) void woq_persist_kernel(WoqArgs a, int cpg_shift, int gmask,
                                                              int gu, int units) {
  extern __shared__ __attribute__((aligned(16))) float pslab[];  // [2][NW][TPW][16][17]
  constexpr int SLAB = NW * TPW * 16 * 17;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K, KW = K / 8;
  const int c0 = wv * CPW;
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * 2));
  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)(M - 1) * a.ldx * 2 + (int64_t)K * 2));
  // B operands: token column lr (columns past M repeat row M - 1, whose
  // sums are never stored), elements 32 lg + 8 i .. + 7 of each chunk
  const int xrow = min(lr, M - 1);
  u32x4_t xb[CPW][4];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xb[c][i] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                       x_rs, (uint32_t)(xrow * a.ldx * 2 + ((c0 + c) * 128 + 32 * lg + 8 * i) * 2),
                       0, 0));
  const int G0 = (int)gridDim.x;
  // units of this workgroup: ub + i us, i < nu (>= 1: the grid is <= units).
  // Round robin (ub = blockIdx.x, us = G0), or for the merged gate_up's half
  // tiles on a grid of whole XCD groups, a contiguous range of units per XCD
  // (XCD x = blockIdx.x % 8), dealt round robin over its G0 / 8 workgroups,
  // so the scale lines that neighbouring units share are fetched once into
  // that XCD's L2
  int ub = (int)blockIdx.x, us = G0, nu = (units - (int)blockIdx.x + G0 - 1) / G0;
  if (gu && TPW == 1 && (G0 & 7) == 0) {
    const int x = (int)blockIdx.x & 7, jw = (int)blockIdx.x >> 3, per = G0 >> 3;
    const int q = units >> 3, r = units & 7;
    const int cnt = q + (x < r ? 1 : 0);  // >= per: G0 <= units
    ub = x * q + (x < r ? x : r) + jw;
    us = per;
    nu = (cnt - jw + per - 1) / per;
  }
  // weight row of row r of unit u's tile t: TPW consecutive 16-row tiles;
  // with gu > 0 and TPW == 2 gate rows 16 u.. (t = 0) and their up rows
  // (t = 1); with gu > 0 and TPW == 1 gate rows 8 u .. 8 u + 7, then their
  // up rows (gu / 8 units instead of gu / 16)
  constexpr bool kHalf = TPW == 1;
  auto row_of = [&](int u, int t, int r) {
    if (gu && kHalf) return u * 8 + r + (r < 8 ? 0 : gu - 8);
    return (gu ? t * gu + u * 16 : (u * TPW + t) * 16) + r;
  };
  // unconditional loads (a load under a lane condition becomes a branch,
  // and the compiler then drains every load in flight at it): a unit index
  // past nu re-reads the workgroup's last unit into a set nothing uses, and
  // rows past N (plain calls' last unit) re-read row N - 1, never stored
  auto issue = [&](int i, PersistSet<NW, CPW, TPW> &S) {
    const int u = ub + min(i, nu - 1) * us;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int n = min(row_of(u, t, lr), N - 1);
      const uint32_t row_off = (uint32_t)n * (uint32_t)KW * 4u + (uint32_t)lg * 16u;
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        S.w[t][c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                    w_rs, row_off + (uint32_t)(c0 + c) * 64u, 0, 0));
        const uint32_t g = (uint32_t)(((c0 + c) >> cpg_shift) & gmask);
        S.s[t][c] = __builtin_amdgcn_raw_buffer_load_b16(
            s_rs, (g * (uint32_t)N + (uint32_t)n) * 2u, 0, 0);
      }
    }
  };
  auto unit = [&](int i, const PersistSet<NW, CPW, TPW> &S) {
    f32x4_t acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float sc = __uint_as_float(S.s[t][c] << 16);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              dq_word<kDecFast>(S.w[t][c][q], sc, 0.f, 0), __builtin_bit_cast(bf16x8_t, xb[c][q]),
              acc[t], 0, 0, 0);
      }
    // D[row = 4 lg + r][token = lr] of tile t -> slab (i % 2)[wave][t]
    float *slab = pslab + (i & 1) * SLAB;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) slab[((wv * TPW + t) * 16 + 4 * lg + r) * 17 + lr] = acc[t][r];
    __syncthreads();
    const int u = ub + i * us;
    if (gu && kHalf) {
      for (int idx = tid; idx < 8 * M; idx += 64 * NW) {
        const int m = idx >> 3, r8 = idx & 7;
        const int jj = u * 8 + r8;
        float g = 0.f, up = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          g += slab[(w * 16 + r8) * 17 + m];
          up += slab[(w * 16 + 8 + r8) * 17 + m];
        }
        if (a.bias) {
          g = g + load_elem(a.bias, a.b_dt, jj);
          up = up + load_elem(a.bias, a.b_dt, gu + jj);
        }
        if (a.y_dt == ZT_DT_BF16) up = bf16_bits_to_f32(f32_to_bf16_bits(up));
        store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + jj, unary_op(ZT_PO_SILU, g) * up);
      }
      return;
    }
    if (gu) {
      for (int idx = tid; idx < 16 * M; idx += 64 * NW) {
        const int m = idx / 16, nr = idx - m * 16;
        const int jj = u * 16 + nr;
        float g = 0.f, up = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          g += slab[((w * TPW) * 16 + nr) * 17 + m];
          up += slab[((w * TPW + 1) * 16 + nr) * 17 + m];
        }
        if (a.bias) {
          g = g + load_elem(a.bias, a.b_dt, jj);
          up = up + load_elem(a.bias, a.b_dt, gu + jj);
        }
        if (a.y_dt == ZT_DT_BF16) up = bf16_bits_to_f32(f32_to_bf16_bits(up));
        store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + jj, unary_op(ZT_PO_SILU, g) * up);
      }
      return;
    }
    for (int idx = tid; idx < TPW * 16 * M; idx += 64 * NW) {
      const int m = idx / (TPW * 16), nr = idx - m * (TPW * 16);
      const int n = u * TPW * 16 + nr;
      if (n >= N) continue;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += slab[((w * TPW + (nr >> 4)) * 16 + (nr & 15)) * 17 + m];
      if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
      v = apply_post_ops(v, a.post, m, n);
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
    }
  };

  PersistSet<NW, CPW, TPW> S[D + 1];
#pragma unroll
  for (int p = 0; p < D; ++p) issue(p, S[p]);
  // whole rounds of D + 1 units (fixed register sets), then the rest
  int i0 = 0;
  for (; i0 + D + 1 <= nu; i0 += D + 1) {
#pragma unroll
    for (int p = 0; p <= D; ++p) {
      issue(i0 + p + D, S[(p + D) % (D + 1)]);
      unit(i0 + p, S[p]);
    }
  }
#pragma unroll
  for (int p = 0; p < D; ++p)
    if (i0 + p < nu) {
      issue(i0 + p + D, S[(p + D) % (D + 1)]);
      unit(i0 + p, S[p]);
    }
}

template <int NW, int CPW, int TPW, int D>
static hipError_t launch_persist_t(const WoqArgs &a, hipStream_t s, int shift, int gmask, int gu,
                                   int units) {
  const unsigned grid = (unsigned)(units < 256 ? units : 256);
  const size_t lds = (size_t)2 * NW * TPW * 16 * 17 * 4;
  woq_persist_kernel<NW, CPW, TPW, D><<<dim3(grid), dim3(64 * NW), lds, s>>>(a, shift, gmask, gu,
                                                                           units);
  return hipGetLastError();
}

// The persistent kernel where it applies: fast mode, bf16 x with 16-byte
// rows, M <= 16, K = NW waves x CPW chunks, gu > 0 the merged gate_up (I =
// gu, a multiple of 16; units of 8 gate rows and their 8 up rows), else
// units of one 16-row tile.  Taken by default with 16 waves where it
// measured faster (HIP-graph replays over rotating weights): the merged
// gate_up from M = 3 (28672 x 4096, one box: 16.8 / 17.0 / 17.1 / 17.4 /
// 18.3 / 19.3 us at M = 3 / 6 / 8 / 9 / 12 / 16 against 18.9 / 18.7 / 18.2
// / 17.8 / 18.3 / 19.3 on the wave kernel and 17.7 / 17.8 / 18.2 / 18.2 /
// 18.8 / 20.0 here in gate/up tile pairs, 896 units for 256 workgroups
// where half tiles make 1792, 7 each), and plain calls from 8193 rows,
// more than two units per CU (14336 x 4096: 10.2 / 10.7 / 12.6 us at M = 1
// / 8 / 16 against 10.9 / 11.9 / 13.5 for the stream kernel; 11008 x 4096
// at M = 4 / 8: 9.6 / 10.1 us against 11.0 / 10.7-11.0 on the wave
// kernel); QKV- and O-sized calls (1.5 and 1 unit per CU) are slower on it.  ZT_WOQ_PERSIST: "0" never, "1" / "2"
// force 8 / 16 waves wherever the shape allows ("1p" / "2p": the merged
// gate_up in gate/up tile pairs instead of half tiles).
static bool try_launch_persist(const WoqArgs &a, hipStream_t s, int shift, int gmask, int mode,
                               int gu, hipError_t *err) {
  const char *e = knob(kKnobWoqPersist);
  if (e && e[0] == '0') return false;
  if (!e && !(gu ? a.M >= 3 : a.N > 8192)) return false;
  if (mode != kDecFast || a.x_dt != ZT_DT_BF16 || a.M < 1 || a.M > 16 || (gu && gu % 16))
    return false;
  if (((reinterpret_cast<uintptr_t>(a.x) | ((uintptr_t)a.ldx * 2)) & 15u) ||
      (a.M - 1) * a.ldx * 2 + a.K * 2 >= (int64_t)kOobOffset ||
      a.N * (a.K / 2) >= (int64_t)kOobOffset || a.G * a.N * 2 >= (int64_t)kOobOffset)
    return false;
  const int nw = e && e[0] == '1' ? 8 : 16;
  if (a.K % (nw * 128)) return false;
  const int cpw = (int)(a.K / (nw * 128));
  // units: one 16-row tile of 8 gate rows and their 8 up rows (a "p" in the
  // knob: a gate tile and its up tile), or single 16-row tiles of a plain
  // call (rows past N read row N - 1)
  const bool pairs = gu && e && std::strchr(e, 'p');
  const int units = gu ? (int)(gu / (pairs ? 16 : 8)) : (int)((a.N + 15) / 16);
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr, "[zt] woq persist M=%lld N=%lld K=%lld gu=%d: NW=%d CPW=%d units=%d\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, gu, nw, cpw, units);
  // register budgets: 16 waves hold 128 VGPRs, 8 waves 256 (x slices of
  // 16 CPW, D + 1 sets of 20 TPW CPW)
#define ZT_PERSIST_CASE(NW_, CPW_, D_)                                              \
  if (nw == NW_ && cpw == CPW_) {                                                   \
    *err = pairs ? launch_persist_t<NW_, CPW_, 2, D_>(a, s, shift, gmask, gu, units) \
                 : launch_persist_t<NW_, CPW_, 1, D_>(a, s, shift, gmask, gu, units); \
    return true;                                                                    \
  }
  ZT_PERSIST_CASE(8, 2, 2) ZT_PERSIST_CASE(8, 4, 1) ZT_PERSIST_CASE(16, 1, 2)
  ZT_PERSIST_CASE(16, 2, 1)
#undef ZT_PERSIST_CASE
  return false;
}

// one phase (p == 1): rows of whole 1 KB pieces; several: rows of 16-byte
// pieces (the phase pitch rounds each row up to whole 1 KB pieces)
static bool stream_x_dma(const WoqArgs &a, int p) {
  return (p == 1 ? a.K % 512 == 0 : (a.K / p) % 8 == 0) &&
         ((reinterpret_cast<uintptr_t>(a.x) | ((uintptr_t)a.ldx * 2)) & 15u) == 0 &&
         (a.M - 1) * a.ldx * 2 + a.K * 2 < (int64_t)kOobOffset;
}

template <int NW, int CPW, int TPW, int P = 1, int MT = 1>
static hipError_t launch_stream_t(const WoqArgs &a, hipStream_t s, int shift, int gmask, int mode) {
  const int tiles = (int)((a.N + 15) / 16);
  const int x_dma = stream_x_dma(a, P) ? 1 : 0;
  if (P > 1 && !x_dma) return hipErrorInvalidValue;  // phases need the DMA (host-checked)
  const size_t lds =
      stream_scale_offset(stream_slab_bytes(NW, TPW, MT),
                          (size_t)a.M *
                              (P == 1 ? stream_x_pitch((int)a.K) : stream_phase_pitch((int)(a.K / P))) * 2) +
      (mode == kDecFast ? stream_scale_bytes((int)a.G, TPW) : 0);
  dim3 grid((unsigned)((tiles + TPW - 1) / TPW)), block(64 * NW);
  if (mode == kDecFast)
    woq_stream_kernel<NW, CPW, TPW, kDecFast, P, MT><<<grid, block, lds, s>>>(a, shift, gmask, x_dma, 0);
  else if (P > 1 || MT > 1)
    return hipErrorInvalidValue;  // phases and token tiles are built for the fast mode only
  else if (mode == kDecGenBf16)
    woq_stream_kernel<NW, CPW, TPW, kDecGenBf16, 1, 1><<<grid, block, lds, s>>>(a, shift, gmask, x_dma, 0);
  else
    woq_stream_kernel<NW, CPW, TPW, kDecGenF32, 1, 1><<<grid, block, lds, s>>>(a, shift, gmask, x_dma, 0);
  return hipGetLastError();
}

// ------------------------------------------------------ lean decode
// The fast mode (signed int4, bf16 scales, bf16 x) at M <= 16 when K is
// exactly NW * CPW 128-wide chunks and x [M, K] fits the LDS whole.  One
// workgroup owns TPW 16-row tiles (or, with gu, a gate tile and its up
// tile) over all of K; wave w owns the chunks [w * CPW, (w + 1) * CPW).
//
// Against the stream kernel, three things change and each was measured on
// the Llama-3-8B decode shapes (graph replays over rotating weights):
//  * a chunk's scale is loaded by each lane into a register right before
//    the chunk's weights (one 2-byte load per lane per tile), so a chunk
//    waits only for its own loads.  With the scales staged through LDS the
//    workgroup barrier also waits for them; they come from HBM behind the
//    weight requests of every other resident workgroup, so the dequant of
//    most workgroups started only after nearly all weights had landed.
//  * only the lanes of the M real token columns read x from LDS (the B
//    columns past M keep the zeros they start with; their sums are never
//    stored), so M = 1 reads 1/16 of the LDS bytes the replicated read did.
//  * the four MFMAs of a chunk alternate between two accumulators, so
//    consecutive MFMAs do not wait on each other's results.
// Partials meet in LDS in wave order (deterministic), then the stream
// kernel's epilogue (bias, post-ops, or silu(gate) * round(up) with gu).
// With gu and TPW == 1 a workgroup's one 16-row tile is half gate, half up:
// rows 0-7 are gate rows j0 .. j0 + 7 and rows 8-15 their up rows gu + j0
// .., j0 = 8 * blockIdx.x, so the merged gate_up makes gu / 8 workgroups
// (1792 for the Llama-3-8B gate_up, 7 per CU) where pairs of whole tiles
// make gu / 16 (896, 3.5 per CU: half the CUs then carry a third more).
template <int NW, int CPW, int TPW>
__global__ __launch_bounds__(64 * NW) void woq_lean_kernel(WoqArgs a, int cpg_shift, int gmask,
                                                           int gu) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K, KW = K / 8;
  const int XP = stream_x_pitch(K);
  uint16_t *xl = reinterpret_cast<uint16_t *>(smem);
  // weight row of row r of tile t: TPW consecutive tiles; with gu and
  // TPW == 2 the gate rows j0.. (t = 0) and the up rows gu + j0.. (t = 1);
  // with gu and TPW == 1 gate rows j0 .. j0 + 7, then their up rows
  constexpr bool kHalf = TPW == 1;
  // half tiles: the workgroups of one XCD take consecutive units, so the
  // scale lines that neighbouring units share are fetched once into that
  // XCD's L2 (round robin, every XCD would fetch each line)
  const int hu = gu && kHalf ? xcd_contiguous_tile((int)blockIdx.x, (int)gridDim.x) : 0;
  auto row_of = [&](int t, int r) {
    if (gu && kHalf) return hu * 8 + r + (r < 8 ? 0 : gu - 8);
    return (gu ? t * gu + (int)blockIdx.x * 16 : ((int)blockIdx.x * TPW + t) * 16) + r;
  };
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * 2));
  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)(M - 1) * a.ldx * 2 + (int64_t)K * 2));
  // 1. x [M, K] -> LDS by DMA, instruction i moving 1 KB of one row (the
  //    host checks 16-byte rows and K % 512 == 0)
  const int per_row = K / 512;
  for (int i = wv; i < M * per_row; i += NW) {
    const int m = i / per_row, q = i - m * per_row;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        x_rs, (lds_ptr_t)(xl + m * XP + q * 512), 16,
        (uint32_t)(m * a.ldx * 2 + q * 1024 + lane * 16), 0, 0, 0);
  }
  // 2. per chunk and tile: the row's scale, then its 16 weight bytes (rows
  //    past N are clamped; their results are never stored)
  const int c0 = wv * CPW;
  uint32_t sr[TPW][CPW];
  u32x4_t wr[TPW][CPW];
  auto load_chunk = [&](int c) {
    const uint32_t g = (uint32_t)(((c0 + c) >> cpg_shift) & gmask);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int n = min(row_of(t, lr), N - 1);
      sr[t][c] = __builtin_amdgcn_raw_buffer_load_b16(s_rs, (g * (uint32_t)N + (uint32_t)n) * 2u,
                                                      0, 0);
      wr[t][c] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                       w_rs, (uint32_t)n * (uint32_t)KW * 4u + (uint32_t)lg * 16u +
                                 (uint32_t)(c0 + c) * 64u, 0, 0));
    }
  };
  // chunks in flight per wave: all of them up to 4 (the merged gate_up at M
  // = 2, K = 4096: 16.3-16.8 -> 15.5-15.6 us), else 2 (the down
  // projection's 14 chunks: 9.6 / 10.6 us at M = 1 / 4 against 10.0-10.4 /
  // 11.1-11.6 with 4 or 6)
  constexpr int D = CPW <= 4 ? CPW : 2;
#pragma unroll
  for (int c = 0; c < D; ++c) load_chunk(c);
  // this wave's x DMA was issued before its 2 * TPW * D loads: once at most
  // those are outstanding it has landed; the barrier covers the other waves'
  constexpr int after = 2 * TPW * D > 63 ? 63 : 2 * TPW * D;
  __builtin_amdgcn_s_waitcnt((after & 15) | ((after >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("s_barrier" ::: "memory");

  // 3. the chunks, each as its loads land; chunk c + D is requested first
  u32x4_t xb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xb[i] = u32x4_t{0u, 0u, 0u, 0u};
  f32x4_t acc[TPW][2];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t][0] = acc[t][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    if (c + D < CPW) load_chunk(c + D);
    const int kc = c0 + c;
    if (lr < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xb[i] = *reinterpret_cast<const u32x4_t *>(xl + lr * XP + kc * 128 + 32 * lg + 8 * i);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const float sc = __uint_as_float(sr[t][c] << 16);
      const float s16 = sc * 0.0625f, k0 = -1032.f * sc, k1 = -72.f * sc;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[t][i & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, dq8_s4_bf16scale(wr[t][c][i], sc, s16, k0, k1)),
            __builtin_bit_cast(bf16x8_t, xb[i]), acc[t][i & 1], 0, 0, 0);
    }
  }

  // 4. partial D[row = 4 lg + r][token = lr] of tile t -> slab[wave][t] (over
  //    x, once every wave is done with it), then each output adds the NW
  //    partials in wave order
  __syncthreads();
  float *slab = reinterpret_cast<float *>(smem);
  if (lr < M) {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        slab[((wv * TPW + t) * 16 + 4 * lg + r) * 17 + lr] = acc[t][0][r] + acc[t][1][r];
  }
  __syncthreads();
  if (gu && kHalf) {
    const int j0 = hu * 8;
    for (int idx = tid; idx < 8 * M; idx += 64 * NW) {
      const int m = idx >> 3, r8 = idx & 7;
      const int j = j0 + r8;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        g += slab[(w * 16 + r8) * 17 + m];
        u += slab[(w * 16 + 8 + r8) * 17 + m];
      }
      if (a.bias) {
        g = g + load_elem(a.bias, a.b_dt, j);
        u = u + load_elem(a.bias, a.b_dt, gu + j);
      }
      if (a.y_dt == ZT_DT_BF16) u = bf16_bits_to_f32(f32_to_bf16_bits(u));
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + j, unary_op(ZT_PO_SILU, g) * u);
    }
    return;
  }
  if (gu) {
    const int j0 = blockIdx.x * 16;
    for (int idx = tid; idx < 16 * M; idx += 64 * NW) {
      const int m = idx >> 4, r16 = idx & 15;
      const int j = j0 + r16;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        g += slab[((w * TPW) * 16 + r16) * 17 + m];
        u += slab[((w * TPW + 1) * 16 + r16) * 17 + m];
      }
      if (a.bias) {
        g = g + load_elem(a.bias, a.b_dt, j);
        u = u + load_elem(a.bias, a.b_dt, gu + j);
      }
      if (a.y_dt == ZT_DT_BF16) u = bf16_bits_to_f32(f32_to_bf16_bits(u));
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + j, unary_op(ZT_PO_SILU, g) * u);
    }
    return;
  }
  const int n0 = blockIdx.x * TPW * 16;
  for (int idx = tid; idx < TPW * 16 * M; idx += 64 * NW) {
    const int m = idx / (TPW * 16), nr = idx - m * (TPW * 16);
    const int n = n0 + nr;
    if (n >= N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += slab[((w * TPW + (nr >> 4)) * 16 + (nr & 15)) * 17 + m];
    if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
    v = apply_post_ops(v, a.post, m, n);
    store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
  }
}

template <int NW, int CPW, int TPW>
static hipError_t launch_lean_t(const WoqArgs &a, hipStream_t s, int shift, int gmask, int gu) {
  const size_t x = (size_t)a.M * stream_x_pitch((int)a.K) * 2;
  const size_t slab = (size_t)NW * TPW * 16 * 17 * 4;
  const unsigned blocks = gu ? (unsigned)(gu / (TPW == 1 ? 8 : 16))
                             : (unsigned)((a.N + 16 * TPW - 1) / (16 * TPW));
  woq_lean_kernel<NW, CPW, TPW><<<dim3(blocks), dim3(64 * NW), x > slab ? x : slab, s>>>(
      a, shift, gmask, gu);
  return hipGetLastError();
}

// Whether the lean kernel serves this call by default: the shapes where it
// measured faster than the kernel the dispatch would otherwise take (graph
// replays of the Llama-3-8B decode shapes over rotating weights, same
// process); ZT_WOQ_LEAN "1" forces it wherever it applies, "0" never.
// Measured (default dispatch -> lean kernel, one box): 4096 x 14336 at
// M = 1 / 2 / 4 10.5 -> 9.9, 10.6 -> 10.2, 11.6 -> 10.7 us; 14336 x 4096
// at M = 1 / 2 11.0 -> 9.9, 11.0 -> 10.1 us and at M = 12 / 16 (against
// the persistent kernel) 28672 x 4096 25.2 -> 23.6, 25.3 -> 23.8 us; from
// 8193 rows (11008 x 4096 at M = 1 / 2: 9.1 / 9.5 us against 10.1-10.8 /
// 10.8-10.9 on the wave kernel, which the persistent kernel also replaces
// there from M = 3: 9.6 / 10.1 us against 11.0 / 10.7-11.0 at M = 4 / 8).
// The merged 28672 x 4096 gate_up in half-gate / half-up tiles at M = 1 /
// 2: 15.5 / 16.2 us, against 16.4-16.5 / 16.3 on the stream and wave
// kernels and 17.1 / 17.2 in tile pairs; from M = 3 the wave kernel is
// faster (M = 3 / 4: 16.6 / 16.4 against 17.3 / 18.2 here).  QKV and most
// shapes at M = 8 stay where they are (2-43 % slower on the lean kernel).
static bool lean_preferred(const WoqArgs &a, int gu) {
  // the merged gate_up: 1-2 rows; at K = 8192, where the persistent kernel
  // has no register budget, up to 4 (57344 x 8192 at M = 4: 60.2 us against
  // 65.0 on the wave kernel)
  if (gu) return a.M <= 2 || (a.M <= 4 && a.K >= 8192);
  if (a.K >= 8192) return a.M <= 4;
  if (a.N > 8192) return a.M <= 2 || (a.N >= 28672 && a.M >= 12);
  return false;
}

// The lean kernel where it applies: fast mode, bf16 x with 16-byte rows,
// M <= 16, K = 8 waves x CPW chunks (CPW 2, 4, 8, 14 or 28), x within the LDS,
// the index ranges within 32-bit buffer offsets; gu > 0 is the merged
// gate_up (I = gu, a multiple of 16).
static bool try_launch_lean(const WoqArgs &a, hipStream_t s, int shift, int gmask, int mode,
                            int gu, hipError_t *err) {
  // "0" never, "1" wherever it applies, "p" also, with the merged gate_up in
  // pairs of whole tiles instead of half-gate / half-up tiles
  const char *e = knob(kKnobWoqLean);
  if (e && e[0] == '0') return false;
  const bool pairs = e && e[0] == 'p';
  if (mode != kDecFast || a.x_dt != ZT_DT_BF16 || a.M < 1 || a.M > 16 || a.K % 1024 ||
      (gu && gu % 16) || !stream_x_dma(a, 1) || a.N * (a.K / 2) >= (int64_t)kOobOffset ||
      a.G * a.N * 2 >= (int64_t)kOobOffset)
    return false;
  if ((size_t)a.M * stream_x_pitch((int)a.K) * 2 > kStreamLdsMax) return false;
  if (!(e && (e[0] == '1' || pairs)) && !lean_preferred(a, gu)) return false;
  const int cpw = (int)(a.K / 1024);
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr, "[zt] woq lean M=%lld N=%lld K=%lld gu=%d%s: NW=8 CPW=%d\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, gu,
                 gu ? (pairs ? " (tile pairs)" : " (half tiles)") : "", cpw);
#define ZT_LEAN_CASE(CPW_)                                                         \
  if (cpw == CPW_) {                                                               \
    *err = !gu     ? launch_lean_t<8, CPW_, 1>(a, s, shift, gmask, 0)              \
           : pairs ? launch_lean_t<8, CPW_, 2>(a, s, shift, gmask, gu)             \
                   : launch_lean_t<8, CPW_, 1>(a, s, shift, gmask, gu);            \
    return true;                                                                   \
  }
  ZT_LEAN_CASE(2) ZT_LEAN_CASE(4) ZT_LEAN_CASE(8) ZT_LEAN_CASE(14) ZT_LEAN_CASE(28)
#undef ZT_LEAN_CASE
  return false;
}

// The weight-streaming kernel, when it applies: M <= 64 and x [M, K] (or,
// in the fast mode, a 2-, 4- or 8-phase range of it) in at most
// kStreamLdsMax of LDS.  Returns false when the caller should use another
// kernel.
// With plan_p set nothing is launched: the function returns whether the
// stream kernel itself has a layout for the call and sets *plan_p to its
// K phase count (1: x whole in LDS).
static bool try_launch_stream(const WoqArgs &a, hipStream_t s, int shift, int gmask, int mode,
                              hipError_t *err, int *plan_p = nullptr) {
  const int C = (int)(a.K / 128);
  const int tiles = (int)((a.N + 15) / 16);
  if (a.M > 64) return false;
  // the fast mode moves the scales by 4-byte DMA, aligned for even N; odd
  // N take the general bf16-scale mode (same weights, same results)
  if (mode == kDecFast && a.N % 2 != 0) mode = kDecGenBf16;
  const bool others = !plan_p && !knob(kKnobWoqStream);
  if (others && try_launch_lean(a, s, shift, gmask, mode, 0, err)) return true;
  if (others && try_launch_persist(a, s, shift, gmask, mode, 0, err)) return true;
  if (others && try_launch_wave(a, s, shift, gmask, mode, 0, err)) return true;
  // measured on MI355X (graph-replayed Llama shapes): 8 waves of few chunks
  // each, two tiles per wave once there are two rounds of tiles, or more
  // tiles than CUs when x takes most of the LDS (one workgroup per CU)
  const bool big_x = (size_t)a.M * stream_x_pitch((int)a.K) * 2 > 64 * 1024;
  int nw = 8, tpw = tiles >= 512 || (big_x && tiles > 256) ? 2 : 1, cpw = 0;
  const char *e = knob(kKnobWoqStream);  // "0" disables; "NW,CPW,TPW" forces
  if (e && e[0] == '0') return false;
  if (e) std::sscanf(e, "%d,%d,%d", &nw, &cpw, &tpw);
  const int mt = (int)((a.M + 15) / 16) == 3 ? 4 : (int)((a.M + 15) / 16);
  auto fits = [&](int p) {
    return stream_scale_offset(stream_slab_bytes(nw, tpw, mt),
                               (size_t)a.M *
                                   (p == 1 ? stream_x_pitch((int)a.K) : stream_phase_pitch((int)(a.K / p))) * 2) +
               (mode == kDecFast ? stream_scale_bytes((int)a.G, tpw) : 0) <=
           kStreamLdsMax;
  };
  // x whole would leave room for one workgroup per CU while the grid makes
  // more than one round: K phases first, whose smaller x range fits two or
  // more workgroups per CU (measured: 10240 x 8192 at M = 6 / 8 took
  // 20.4 / 21.3 us with x whole on 320 workgroups of two tiles)
  const int tpw0 = tpw;
  const bool prefer_phases =
      !e && mt == 1 && mode == kDecFast && a.x_dt == ZT_DT_BF16 && fits(1) &&
      (size_t)a.M * stream_x_pitch((int)a.K) * 2 > kStreamLdsMax / 2 && (tiles + tpw - 1) / tpw > 256;
  if (mt > 1 || !fits(1) || prefer_phases) {
    // several token tiles or K phases: 8 waves, one tile each, fast mode,
    // the fewest phases whose x range fits
    if (e || mode != kDecFast || a.x_dt != ZT_DT_BF16) return false;
    nw = 8, tpw = 1;
    for (int p : {1, 2, 4, 8}) {
      const int cp = C / p;
      if (C % p || (p > 1 && !stream_x_dma(a, p)) || !fits(p)) continue;
      if (prefer_phases &&
          (p == 1 || (size_t)a.M * stream_phase_pitch((int)(a.K / p)) * 2 > kStreamLdsMax / 2))
        continue;
      // two phases that leave room for one workgroup per CU under more than
      // a round of tiles: four when they fit two per CU and have a case
      // (cpw_need <= 28 below)
      auto half_x = [&](int q) {
        return (size_t)a.M * stream_phase_pitch((int)(a.K / q)) * 2 <= kStreamLdsMax / 2;
      };
      if (p == 2 && mt == 1 && tiles > 256 && !half_x(2) && C % 4 == 0 && stream_x_dma(a, 4) &&
          fits(4) && half_x(4) && 4 * ((C / 4 + 7) / 8) <= 28)
        continue;
      const int cpw_need = p * ((cp + 7) / 8);  // chunks per wave over all phases
      if (knob(kKnobWoqDebug) && !plan_p)
        std::fprintf(stderr, "[zt] woq stream M=%lld N=%lld K=%lld: MT=%d P=%d CPW>=%d\n",
                     (long long)a.M, (long long)a.N, (long long)a.K, mt, p, cpw_need);
#define ZT_STREAM_PCASE(CPW_, P_, MT_)                                          \
  if (mt == MT_ && p == P_ && cpw_need <= CPW_ && CPW_ % P_ == 0) {            \
    if (plan_p) return *plan_p = P_, true;                                      \
    *err = launch_stream_t<8, CPW_, 1, P_, MT_>(a, s, shift, gmask, mode);      \
    return true;                                                                \
  }
      // smallest CPW first, so that every wave has chunks in each phase
      ZT_STREAM_PCASE(8, 2, 1) ZT_STREAM_PCASE(14, 2, 1) ZT_STREAM_PCASE(16, 2, 1)
      ZT_STREAM_PCASE(16, 4, 1) ZT_STREAM_PCASE(20, 2, 1) ZT_STREAM_PCASE(20, 4, 1)
      ZT_STREAM_PCASE(28, 2, 1) ZT_STREAM_PCASE(28, 4, 1)
      ZT_STREAM_PCASE(4, 1, 2) ZT_STREAM_PCASE(4, 2, 2) ZT_STREAM_PCASE(16, 4, 2)
      ZT_STREAM_PCASE(4, 1, 4) ZT_STREAM_PCASE(4, 4, 4) ZT_STREAM_PCASE(8, 8, 4)
#undef ZT_STREAM_PCASE
    }
    if (!prefer_phases) return false;
    nw = 8, tpw = tpw0;  // no phase case: x whole after all
  }
  // at M <= 4 one tile per wave at any tile count (measured in HIP-graph
  // replays of the Llama-3 8B shapes: gate_up 28672 x 4096 at M = 1 takes
  // 16.0-16.5 us so against 17.4 with two tiles; 16 waves of two chunks or
  // 4 of eight are no faster once the weights are pipelined)
  if (!e && a.M <= 4) tpw = 1;
  // x too large for two workgroups per CU: four tiles per wave while that
  // still leaves most of a round of workgroups (measured: 14336 x 4096 at
  // M = 12 / 16 takes 13.1 / 13.3 us so against 14.0 / 15.1 with two; at
  // M = 8, with two workgroups per CU, four tiles lose)
  if (!e && (size_t)a.M * stream_x_pitch((int)a.K) * 2 > 76 * 1024 && tiles >= 800 && C <= 64)
    tpw = 4;
  const int need = (C + nw - 1) / nw;
  if (cpw == 0)
    for (int c : {2, 4, 8, 12, 14, 16, 28})
      if (c >= need && ((c != 14 && c != 28) || nw == 8)) { cpw = c; break; }
  if (cpw < need) return false;
  if (knob(kKnobWoqDebug) && !plan_p)
    std::fprintf(stderr, "[zt] woq stream M=%lld N=%lld K=%lld: NW=%d CPW=%d TPW=%d\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, nw, cpw, tpw);
#define ZT_STREAM_CASE(NW_, CPW_, TPW_) \
  if (nw == NW_ && cpw == CPW_ && tpw == TPW_) { \
    if (plan_p) return *plan_p = 1, true; \
    *err = launch_stream_t<NW_, CPW_, TPW_>(a, s, shift, gmask, mode); return true; }
  ZT_STREAM_CASE(4, 2, 1) ZT_STREAM_CASE(4, 4, 1) ZT_STREAM_CASE(4, 8, 1) ZT_STREAM_CASE(4, 12, 1)
  ZT_STREAM_CASE(4, 16, 1) ZT_STREAM_CASE(4, 8, 2) ZT_STREAM_CASE(4, 4, 2) ZT_STREAM_CASE(4, 16, 2)
  ZT_STREAM_CASE(8, 4, 1) ZT_STREAM_CASE(8, 8, 1) ZT_STREAM_CASE(8, 12, 1) ZT_STREAM_CASE(8, 14, 1)
  ZT_STREAM_CASE(8, 16, 1) ZT_STREAM_CASE(8, 14, 2) ZT_STREAM_CASE(8, 2, 4) ZT_STREAM_CASE(8, 4, 4)
  ZT_STREAM_CASE(8, 8, 4) ZT_STREAM_CASE(8, 28, 1)
  ZT_STREAM_CASE(8, 4, 2) ZT_STREAM_CASE(8, 8, 2) ZT_STREAM_CASE(8, 16, 2) ZT_STREAM_CASE(2, 16, 1)
  ZT_STREAM_CASE(16, 2, 1) ZT_STREAM_CASE(16, 2, 2) ZT_STREAM_CASE(16, 4, 1) ZT_STREAM_CASE(16, 8, 1)
#undef ZT_STREAM_CASE
  return false;
}

// ------------------------------------------------ wide decode (17..64 rows)
// Weight streaming for 17..64 tokens, where re-reading x per 16-row weight
// tile (the stream kernel) moves up to 16 bytes of x per byte of int4.  A
// workgroup owns 128 weight rows over one K split and keeps x [32*MT][256]
// of each 256-k phase in LDS, shared by its 8 waves, so x costs 4*M/128
// bytes per weight byte.  The waves form 4 row groups of 32; the two waves
// of a group take the two 128-k chunks of each phase (two waves per SIMD,
// so one wave's dequantisation overlaps the other's MFMAs) and add their
// halves in LDS at the end.
//
// Loads, all issued three phases before their use: x and the phase's scales
// move by DMA into four LDS stages; each wave's weights go straight from HBM
// to registers (two 16-row x 64-byte loads per chunk) into four register
// sets.  A wave's loads retire in issue order and every phase issues the
// same loads (past the split out of range, so zeros), so one wait per phase
// -- everything issued for this phase has landed -- and the barrier after it
// cover x, scales and weights; the barrier also retires the stage the new
// DMA overwrites.  The weights are issued at the start of a phase, the DMA
// spread over its first steps.  The phase loop runs whole rounds of four
// phases with the register sets fixed per position and nothing skipped, so
// the compiler's own wait counting stays exact (a remainder or a skipped
// compute makes it wait for every load at each phase).  The PAD form pads a
// split that is not a whole number of rounds and skips the compute of the
// padding; it is the slower fallback.
//
// Compute: a chunk's two 16-row tiles become the 32-row A operands of
// v_mfma_f32_32x32x16_bf16 with one v_permlane16_swap per dword (lanes 0-31
// then hold bytes [0, 16) and [16, 32) of rows 0-31, lanes 32-63 bytes
// [32, 48) and [48, 64)), so MFMA q of the chunk takes k block 8*(l/32) + q
// in both operands.  B is x from LDS: 512-byte token rows, 16-byte column c
// of row t at position c ^ (t & 15) (16 distinct bank groups per read pass).
// A wave reads the phase's eight B fragments first, then dequantises
// (bf16_rne of the exact fp32 product, dq_word) and multiplies.
//
// D is [n][token]: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4
// of the wave's 32 and token 32*j + l%32.  With one K split the workgroup
// applies the epilogue; with several it writes fp32 partials
// [split][M][N], which woq_splitk_reduce_kernel adds in split order.

// sched_barrier mask: everything but vector-memory instructions may cross
constexpr int kSchedAllButVmem = 0x78f;
constexpr int kWideKP = 256;    // k per phase (two 128-k chunks)
constexpr int kWideRows = 128;  // weight rows per workgroup
constexpr int kWideAhead = 3;   // phases between a load's issue and its use
constexpr int kWideRound = kWideAhead + 1;  // LDS stages, register sets, phases per loop round

template <int MT>
constexpr size_t woq_wide_xstage() {
  return (size_t)(32 * MT) * (kWideKP * 2);
}

template <int MT>
constexpr size_t woq_wide_lds() {
  // x stages, scale stages [round][2 chunks][128 rows], and a spare 256-byte
  // block the out-of-range scale DMA of waves 2..7 writes
  const size_t x = kWideRound * woq_wide_xstage<MT>() + kWideRound * 2 * (kWideRows * 2) + 256;
  const size_t tile = (size_t)(32 * MT) * (kWideRows + 4) * 4;
  return x > tile ? x : tile;
}

template <int MT, bool PAD>
__global__ __launch_bounds__(512) void woq_wide_kernel(WoqArgs a, int pps, int cpg_shift, int gmask,
                                                       float *partial, int gu) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int XS = (int)woq_wide_xstage<MT>();
  constexpr int XL = 2 * MT;        // x DMA (two token rows each) per wave per phase
  constexpr int OPS = 3 + XL;       // loads per wave per phase: 2 weight tiles, scales, x
  constexpr int WAIT = vmcnt_imm_woq((kWideAhead - 1) * OPS);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = wv & 3, kh = wv >> 2;  // row group; chunk of each phase
  const int lr = lane & 15, lg = lane >> 4, l32 = lane & 31, hl = lane >> 5;
  const int M = (int)a.M, N = (int)a.N, K = (int)a.K, KW = K / 8;
  const int ldx2 = (int)a.ldx * 2;
  const int n0 = blockIdx.x * kWideRows;
  const int ph0 = blockIdx.y * pps;  // first phase of this K split
  // the last split may be shorter (uneven splits): its phases past K load
  // zeros and add nothing
  const int pend = min(ph0 + pps, (int)(a.K / kWideKP));
  // merged gate_up (gu = N/2, a multiple of 64): local rows [0, 64) are gate
  // rows j0.., local rows [64, 128) the up rows gu + j0..
  const int j0 = blockIdx.x * (kWideRows / 2);
  auto row_of = [&](int r) { return gu ? (r < 64 ? j0 + r : gu + j0 + r - 64) : n0 + r; };

  const auto x_rs = make_rsrc(a.x, (uint32_t)((int64_t)(M - 1) * ldx2 + (int64_t)K * 2));
  const auto w_rs = make_rsrc(a.w, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rs = make_rsrc(a.scales, (uint32_t)(a.G * N * 2));

  // the lane's two load rows (rows past N read zeros, scales past N zeros
  // or another group's; their outputs are never stored)
  const int r_lo = row_of(rw * 32 + lr), r_hi = row_of(rw * 32 + lr + 16);
  const uint32_t off_lo = (uint32_t)r_lo * (uint32_t)KW * 4u + 16u * lg;
  const uint32_t off_hi = (uint32_t)r_hi * (uint32_t)KW * 4u + 16u * lg;
  const uint32_t oob_lo = r_lo < N ? 0u : kOobOffset, oob_hi = r_hi < N ? 0u : kOobOffset;

  u32x4_t wq[kWideRound][2];
  unsigned char *sbuf0 = smem + kWideRound * XS;
  // Load i of phase ph.  The out-of-range bit is ORed into the offsets
  // (valid offsets stay below it): a select on the wave-uniform condition
  // would be compiled into branches around each load.
  //  0, 1: the weight tiles of the lane's low / high row (register set `set`)
  //  2:    the scales: waves 0 and 1 move chunk wv's 128 row scales (one
  //        256-byte DMA; N % 4 == 0 keeps the dwords aligned), the others an
  //        out-of-range DMA into the spare block, so no branch surrounds it
  //  3..:  x token rows 2 (wv + 8 i) and 2 (wv + 8 i) + 1, 512 bytes each
  auto load = [&](int i, int ph, int set) {
    const uint32_t oob = ph < pend ? 0u : kOobOffset;
    if (i < 2) {
      const uint32_t kc = (uint32_t)(ph * 2 + kh);
      const uint32_t off = i == 0 ? (off_lo + kc * 64u) | oob_lo : (off_hi + kc * 64u) | oob_hi;
      wq[set][i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
          w_rs, off | oob, 0, 0));
    } else if (i == 2) {
      const int ch = wv & 1;
      const uint32_t g = ((uint32_t)(ph * 2 + ch) >> cpg_shift) & (uint32_t)gmask;
      const uint32_t soob = wv < 2 ? 0u : kOobOffset;
      const int slot = wv < 2 ? (ph & (kWideRound - 1)) * 2 + ch : 2 * kWideRound;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          s_rs, (lds_ptr_t)(sbuf0 + slot * (kWideRows * 2)), 4,
          ((g * (uint32_t)N + (uint32_t)row_of(2 * lane)) * 2u) | oob | soob, 0, 0, 0);
    } else {
      const int r = 2 * (wv + 8 * (i - 3));
      const int t = r + hl;
      const int c = l32 ^ (t & 15);
      const uint32_t off = (uint32_t)(t * ldx2 + ph * (kWideKP * 2) + c * 16) |
                           (t < M ? 0u : kOobOffset) | oob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          x_rs, (lds_ptr_t)(smem + (ph & (kWideRound - 1)) * XS + r * (kWideKP * 2)), 16, off, 0,
          0, 0);
    }
  };

  f32x16_t acc[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;

  // the compute of phase ph, issuing the DMA loads 2.. of phase ph + 3 one
  // per step (VMEM pinned in place, everything else free to move around it)
  auto compute = [&](int set, int ph) {
    const unsigned char *buf = smem + (ph & (kWideRound - 1)) * XS;
    bf16x8_t xf[8][MT];
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int t = 32 * j + l32;
        const int cc = kh * 16 + 8 * hl + q;
        xf[q][j] = *reinterpret_cast<const bf16x8_t *>(buf + t * (kWideKP * 2) + ((cc ^ (t & 15)) * 16));
      }
    const float sc = __uint_as_float(
        (uint32_t)reinterpret_cast<const uint16_t *>(
            sbuf0 + ((ph & (kWideRound - 1)) * 2 + kh) * (kWideRows * 2))[rw * 32 + l32]
        << 16);
    u32x4_t w0 = wq[set][0], w1 = wq[set][1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const auto sw = __builtin_amdgcn_permlane16_swap(w0[e], w1[e], false, false);
      w0[e] = sw[0];
      w1[e] = sw[1];
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (q < OPS - 2) {
        __builtin_amdgcn_sched_barrier(kSchedAllButVmem);
        load(2 + q, ph + kWideAhead, 0);
        __builtin_amdgcn_sched_barrier(kSchedAllButVmem);
      }
      const bf16x8_t wb = dq_word<kDecFast>(q < 4 ? w0[q] : w1[q - 4], sc, 0.f, 0);
#pragma unroll
      for (int j = 0; j < MT; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb, xf[q][j], acc[j], 0, 0, 0);
    }
  };
  static_assert(OPS - 2 <= 8, "the DMA loads fit the steps of a phase");
  auto phase = [&](int j, int set) {
    const int ph = ph0 + j;
    __builtin_amdgcn_s_waitcnt(WAIT);
    asm volatile("s_barrier" ::: "memory");
    load(0, ph + kWideAhead, (set + kWideAhead) % kWideRound);
    load(1, ph + kWideAhead, (set + kWideAhead) % kWideRound);
    __builtin_amdgcn_sched_barrier(0);
    if (!PAD || ph < pend) {
      compute(set, ph);
    } else {
#pragma unroll
      for (int i = 2; i < OPS; ++i) load(i, ph + kWideAhead, 0);
    }
  };
  // prologue: the loads of phases 0 .. 2, in the order the phases issue them
#pragma unroll
  for (int v = 0; v < kWideAhead; ++v)
#pragma unroll
    for (int i = 0; i < OPS; ++i) load(i, ph0 + v, v);
  // whole rounds (the host gives PAD = false only when pps is a multiple of 4)
  const int jend = PAD ? (pps + kWideRound - 1) / kWideRound * kWideRound : pps;
  int j = 0;
  do {
    static_assert(kWideRound == 4, "one loop round is four phases");
    phase(j, 0);
    phase(j + 1, 1);
    phase(j + 2, 2);
    phase(j + 3, 3);
    j += kWideRound;
  } while (j < jend);

  // the two chunk halves meet in LDS: waves kh = 1 store, kh = 0 add (the
  // out-of-range DMA of the padding phases lands before the stages are reused)
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_barrier" ::: "memory");
  f32x16_t *red = reinterpret_cast<f32x16_t *>(smem) + (rw * MT) * 64 + lane;
  if (kh == 1) {
#pragma unroll
    for (int j = 0; j < MT; ++j) red[j * 64] = acc[j];
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] += red[j * 64];
  }
  __syncthreads();
  if (partial == nullptr) {
    constexpr int TP = kWideRows + 4;
    float *tile = reinterpret_cast<float *>(smem);
    if (kh == 0) {
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4_t *>(tile + (32 * j + l32) * TP + rw * 32 + 8 * q + 4 * hl) =
              f32x4_t{acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]};
    }
    __syncthreads();
    if (tid >= 256) return;
    if (gu) {
      // y[m][j] = silu(gate + bias[j]) * (up + bias[gu + j]), the up value
      // rounded to y's bf16 first (the unfused op's bf16 up output)
      for (int idx = tid; idx < 32 * MT * 16; idx += 256) {
        const int m = idx >> 4, c4 = (idx & 15) * 4;
        if (m >= M) continue;
        const f32x4_t g4 = *reinterpret_cast<const f32x4_t *>(tile + m * TP + c4);
        const f32x4_t u4 = *reinterpret_cast<const f32x4_t *>(tile + m * TP + 64 + c4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = j0 + c4 + r;
          float g = g4[r], u = u4[r];
          if (a.bias) {
            g = g + load_elem(a.bias, a.b_dt, j);
            u = u + load_elem(a.bias, a.b_dt, gu + j);
          }
          if (a.y_dt == ZT_DT_BF16) u = bf16_bits_to_f32(f32_to_bf16_bits(u));
          store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + j, unary_op(ZT_PO_SILU, g) * u);
        }
      }
      return;
    }
    woq_tile_epilogue<32 * MT, kWideRows>(a, tile, 0, n0, tid);
    return;
  }
  if (kh != 0) return;
  float *pp = partial + (size_t)blockIdx.y * M * N;
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int m = 32 * j + l32;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + rw * 32 + 8 * q + 4 * hl;  // N % 4 == 0: n..n+3 all in or out
      if (m < M && n < N)
        *reinterpret_cast<f32x4_t *>(pp + (size_t)m * N + n) =
            f32x4_t{acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]};
    }
  }
}

// y = epilogue(sum over the splits of partial[split][m][n], in split order).
// The partials were written by another kernel, most of them on other XCDs,
// so each load is a round trip to memory: every split's load is issued
// before the first add.  S = 2..8 splits unroll fully; S = 0 (any count)
// issues eight at a time.  The adds run in split order either way.
template <int S>
__global__ __launch_bounds__(256) void woq_splitk_reduce_kernel(WoqArgs a, const float *partial,
                                                                int splits) {
  const int M = (int)a.M, N = (int)a.N;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * (N / 4)) return;
  const int m = (int)(idx / (N / 4)), n = (int)(idx % (N / 4)) * 4;
  const size_t stride = (size_t)M * N;
  const float *p0 = partial + (size_t)m * N + n;
  f32x4_t v;
  if constexpr (S > 0) {
    f32x4_t q[S];
#pragma unroll
    for (int i = 0; i < S; ++i) q[i] = *reinterpret_cast<const f32x4_t *>(p0 + i * stride);
    v = q[0];
#pragma unroll
    for (int i = 1; i < S; ++i) v += q[i];
  } else {
    v = *reinterpret_cast<const f32x4_t *>(p0);
    int s = 1;
    for (; s + 8 <= splits; s += 8) {
      f32x4_t q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = *reinterpret_cast<const f32x4_t *>(p0 + (s + i) * stride);
#pragma unroll
      for (int i = 0; i < 8; ++i) v += q[i];
    }
    for (; s < splits; ++s) v += *reinterpret_cast<const f32x4_t *>(p0 + s * stride);
  }
  float f[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float t = v[r];
    if (a.bias) t = t + load_elem(a.bias, a.b_dt, n + r);
    f[r] = apply_post_ops(t, a.post, m, n + r);
  }
  if (a.y_dt == ZT_DT_BF16 && (a.ldy & 3) == 0) {
    u32x2_t pk;
    pk[0] = pack_bf16x2(f[0], f[1]);
    pk[1] = pack_bf16x2(f[2], f[3]);
    *reinterpret_cast<u32x2_t *>(reinterpret_cast<uint16_t *>(a.y) + (int64_t)m * a.ldy + n) = pk;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n + r, f[r]);
  }
}

// y = epilogue(sum of the `splits` fp32 partials [splits][M][N]), in split order
static hipError_t launch_splitk_reduce(const WoqArgs &a, const float *partial, int splits,
                                       hipStream_t s) {
  const int64_t n4 = a.M * (a.N / 4);
  const dim3 rgrid((unsigned)((n4 + 255) / 256)), rblock(256);
  switch (splits) {
#define ZT_REDUCE_CASE(S_) \
  case S_: woq_splitk_reduce_kernel<S_><<<rgrid, rblock, 0, s>>>(a, partial, splits); break;
    ZT_REDUCE_CASE(2) ZT_REDUCE_CASE(3) ZT_REDUCE_CASE(4) ZT_REDUCE_CASE(5)
    ZT_REDUCE_CASE(6) ZT_REDUCE_CASE(7) ZT_REDUCE_CASE(8)
#undef ZT_REDUCE_CASE
    default: woq_splitk_reduce_kernel<0><<<rgrid, rblock, 0, s>>>(a, partial, splits); break;
  }
  return hipGetLastError();
}

static void launch_wide_t(const WoqArgs &a, const WidePlan &p, dim3 grid, int shift, int gmask,
                          float *partial, int gu, hipStream_t s) {
  if (p.mt == 1 && !p.pad)
    woq_wide_kernel<1, false><<<grid, dim3(512), woq_wide_lds<1>(), s>>>(a, p.pps, shift, gmask, partial, gu);
  else if (p.mt == 1)
    woq_wide_kernel<1, true><<<grid, dim3(512), woq_wide_lds<1>(), s>>>(a, p.pps, shift, gmask, partial, gu);
  else if (!p.pad)
    woq_wide_kernel<2, false><<<grid, dim3(512), woq_wide_lds<2>(), s>>>(a, p.pps, shift, gmask, partial, gu);
  else
    woq_wide_kernel<2, true><<<grid, dim3(512), woq_wide_lds<2>(), s>>>(a, p.pps, shift, gmask, partial, gu);
}

// Whether the stream kernel takes a call of up to 16 rows of this shape
// well (bf16 x and scales, aligned): it has a layout for x (whole in LDS, or
// K phases with a compiled case), and in K phases its grid of one 16-row
// tile per workgroup makes one round while x leaves room for one workgroup
// per CU.  Measured (HIP-graph replays, one box; stream or decode kernel
// against the wide kernel): without a layout 4096 x 11008 at M = 15 / 16
// took 22.8 / 23.6 us against 17.2 / 17.4, 3584 x 18944 at M = 16 32.5
// against 25.7, 8192 x 28672 at M = 9..16 57-81 against 37-39; with a
// layout but 320 tiles on one workgroup per CU, 5120 x 13824 at M = 12 / 16
// 27.9 / 30.8 against 25.6 / 26.2.  With a layout and one round the stream
// kernel was faster (3584 x 18944 at M = 9..15: 17.6-20.7 against 24.9-25.6).
static bool stream_takes_well(int64_t M, int64_t N, int64_t K, int64_t G) {
  WoqArgs a{};
  a.x = reinterpret_cast<const void *>(256);
  a.w = reinterpret_cast<const uint32_t *>(256);
  a.x_dt = ZT_DT_BF16, a.s_dt = ZT_DT_BF16, a.y_dt = ZT_DT_BF16;
  a.M = M, a.N = N, a.K = K, a.G = G, a.ldx = K, a.ldy = N;
  int p = 0;
  hipError_t err = hipSuccess;
  if (!try_launch_stream(a, nullptr, 0, 0, kDecFast, &err, &p)) return false;
  if (p == 1) return true;
  const bool one_per_cu = (size_t)M * stream_phase_pitch((int)(K / p)) * 2 > kStreamLdsMax / 2;
  return !(one_per_cu && (N + 15) / 16 > 256);
}

bool woq_wide_plan(int64_t M, int64_t N, int64_t K, int64_t G, WidePlan *p) {
  const char *e = knob(kKnobWoqWide);  // "0" disables; "KS" forces the split count
  if (e && e[0] == '0') return false;
  if (M < 1 || M > 64 || N < 4 || N % 4 || K % kWideKP || G <= 0 || K % G) return false;
  // up to 32 rows of a matrix of at most 4096 x 4096 the stream kernel is
  // faster (measured: the split-K reduce launch outweighs the x savings)
  const char *f = knob(kKnobWoqForceKernel);
  const bool forced = e || (f && !std::strcmp(f, "wide"));
  // below 8 rows only from 4 rows, where the stream kernel has no good
  // layout (measured: 8192 x 28672 at M = 4 / 6 took 35.9 / 40.8 us on the
  // stream kernel in K phases against 35.2 / 35.2 here; at M = 1 / 2 29.0 /
  // 32.1 against 35.2 / 34.8)
  if (M < 8 && !forced && (M < 4 || stream_takes_well(M, N, K, G))) return false;
  // while x [M, K] leaves room for two stream-kernel workgroups per CU the
  // stream kernel is faster (measured: gate_up 28672 x 4096 at M = 8 / 9
  // takes 18.5 / 18.8 us there against 22.2 / 22.8 us here; 25.1 / 22.9 at
  // M = 10, where x no longer fits twice)
  if (M * (K + 8) * 2 <= 76 * 1024 && !forced) return false;
  // (also up to 64 rows: the 4096 x 4096 O projection at M = 64 takes
  // 12.3 us on the stream kernel against 15.8 us split 8 ways here), while
  // the stream kernel's 16-row tiles make one round (past 4096 rows its
  // second round doubles the call: 4608 x 3584 at M = 32 / 64 took 15.2 /
  // 24.6 us there against 11.8 / 14.4 here)
  if (M <= 64 && N <= 4096 && N * K <= (int64_t)4096 * 4096 && !forced) return false;
  const int64_t gs = K / G, cpg = gs / 128;
  if (G != 1 && (gs % 128 || (cpg & (cpg - 1)))) return false;
  const int phases = (int)(K / kWideKP);
  const int64_t blocks = (N + kWideRows - 1) / kWideRows;
  // the most K splits (a divisor of the phase count) of whole rounds of
  // phases that keep the grid within about 1.25 rounds of 256 CUs.  Without
  // such a divisor: splits of whole rounds with a shorter last split (its
  // phases past K load zeros), as many as keep the grid within 1.25 rounds
  // (a prime phase count left 4096 x 11008 at M = 17..64 unsplit on 32
  // workgroups: 41-52 us)
  int ks = 0, pps = 0;
  for (int d = 1; d <= phases; ++d)
    if (phases % d == 0 && (phases / d) % kWideRound == 0 && blocks * d <= 320) ks = d;
  if (ks > 0) {
    pps = phases / ks;
  } else {
    const int target = (int)std::max<int64_t>(1, std::min<int64_t>(phases, 320 / blocks));
    pps = ((phases + target - 1) / target + kWideRound - 1) / kWideRound * kWideRound;
    ks = (phases + pps - 1) / pps;
  }
  if (e) {
    const int f = std::atoi(e);
    if (f >= 1 && f <= phases) {
      ks = f;
      pps = (phases + f - 1) / f;
      if (phases % f) pps = (pps + kWideRound - 1) / kWideRound * kWideRound;
      ks = (phases + pps - 1) / pps;
    }
  }
  // up to 16 rows: only without a K split (measured: gate_up 28672 x 4096
  // at M = 12 / 16 takes 22.6 / 22.9 us here against 25.9 / 27.2 on the
  // stream kernel, while the split shapes lose the reduce launch), and only
  // with at least half a round of workgroups (a prime phase count leaves no
  // split: 4096 x 11008 at M = 8 took 40.9 us on 32 workgroups) -- unless
  // the stream kernel has no good layout for the call (stream_takes_well)
  if (M < 17 && (ks > 1 || blocks < 128) && !forced && stream_takes_well(M, N, K, G))
    return false;
  p->mt = M <= 32 ? 1 : 2;
  p->splits = ks;
  p->pps = pps;
  p->pad = p->pps % kWideRound != 0;
  return true;
}

size_t woq_wide_workspace(const WidePlan &p, int64_t M, int64_t N) {
  return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
}

bool woq_wide_ok(const WoqArgs &a, WidePlan *p) {
  const char *f = knob(kKnobWoqForceKernel);  // another forced kernel skips this one
  if (f && std::strcmp(f, "wide")) return false;
  if (!woq_wide_plan(a.M, a.N, a.K, a.G, p)) return false;
  return a.x_dt == ZT_DT_BF16 && a.s_dt == ZT_DT_BF16 && !a.zp && a.ldx % 8 == 0 &&
         aligned16(a.x) && aligned16(a.w) &&
         (a.M - 1) * a.ldx * 2 + a.K * 2 < (int64_t)kOobOffset &&
         a.N * (a.K / 2) < (int64_t)kOobOffset && a.G * a.N * 2 < (int64_t)kOobOffset;
}

hipError_t launch_woq_wide(const WoqArgs &a, const WidePlan &p, void *workspace, hipStream_t s) {
  const int64_t cpg = a.G == 1 ? 0 : (a.K / a.G) / 128;
  int shift = 0;
  while (cpg > 1 && (1 << shift) < cpg) ++shift;
  const int gmask = a.G == 1 ? 0 : 0x7fffffff;
  float *partial = p.splits > 1 ? static_cast<float *>(workspace) : nullptr;
  if (p.splits > 1 && !partial) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.N + kWideRows - 1) / kWideRows), (unsigned)p.splits);
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr,
                 "[zt] woq wide M=%lld N=%lld K=%lld: MT=%d splits=%d phases/split=%d%s\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, p.mt, p.splits, p.pps,
                 p.pad ? " (padded)" : "");
  launch_wide_t(a, p, grid, shift, gmask, partial, 0, s);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.splits == 1) return err;
  return launch_splitk_reduce(a, partial, p.splits, s);
}

// Merged gate_up on the wide kernel: one launch writes silu(gate) * up,
// workgroup b computing gate rows [64b, 64b + 64) and the matching up rows.
// Taken when the wide kernel would run the full [M, N] linear without a K
// split and N/2 is a multiple of 64; otherwise returns false.
bool woq_try_wide_gate_up(const WoqArgs &a, hipStream_t s, hipError_t *err) {
  WidePlan p;
  if (a.N % (2 * 64) || a.post.count != 0 || !woq_wide_ok(a, &p) || p.splits != 1) return false;
  const int64_t cpg = a.G == 1 ? 0 : (a.K / a.G) / 128;
  int shift = 0;
  while (cpg > 1 && (1 << shift) < cpg) ++shift;
  const int gmask = a.G == 1 ? 0 : 0x7fffffff;
  const int gu = (int)(a.N / 2);
  const dim3 grid((unsigned)(a.N / kWideRows), 1u);
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr, "[zt] woq wide gate_up M=%lld N=%lld K=%lld: MT=%d\n", (long long)a.M,
                 (long long)a.N, (long long)a.K, p.mt);
  launch_wide_t(a, p, grid, shift, gmask, nullptr, gu, s);
  *err = hipGetLastError();
  return true;
}

// The stream kernel for a call of up to 64 rows whose shape the decode
// kernels accept (capi.hip tries it before splitting 33..64 rows into
// blocks of 16).
bool woq_try_stream(const WoqArgs &a, hipStream_t s, hipError_t *err) {
  const int64_t cpg = a.G == 1 ? 0 : (a.K / a.G) / 128;
  int shift = 0;
  while (cpg > 1 && (1 << shift) < cpg) ++shift;
  const int gmask = a.G == 1 ? 0 : 0x7fffffff;
  const int mode = a.s_dt == ZT_DT_F32 ? kDecGenF32 : (a.zp ? kDecGenBf16 : kDecFast);
  return try_launch_stream(a, s, shift, gmask, mode, err);
}

// The merged gate_up launch of the stream kernel (fast mode, M <= 16, x
// whole in LDS).  Returns false when the caller should take the two-step
// path (the full linear into fp32, then launch_silu_mul_halves).
bool woq_try_stream_gate_up(const WoqArgs &a, hipStream_t s, hipError_t *err) {
  const int64_t I = a.N / 2, gs = a.K / a.G, cpg = gs / 128;
  if (a.x_dt != ZT_DT_BF16 || a.s_dt != ZT_DT_BF16 || a.zp || a.M < 1 || a.M > 16 ||
      a.N % 32 != 0 || a.K % 128 != 0 || (a.G != 1 && (gs % 128 || (cpg & (cpg - 1)))) ||
      a.ldx % 8 != 0 || !aligned16(a.x) || !aligned16(a.w) ||
      a.N * (a.K / 2) >= (int64_t)kOobOffset || a.G * a.N * 2 >= (int64_t)kOobOffset)
    return false;
  int shift = 0;
  while (cpg > 1 && (1 << shift) < cpg) ++shift;
  const int gmask = a.G == 1 ? 0 : 0x7fffffff;
  if (!knob(kKnobWoqStream) && try_launch_lean(a, s, shift, gmask, kDecFast, (int)I, err))
    return true;
  if (!knob(kKnobWoqStream) && try_launch_persist(a, s, shift, gmask, kDecFast, (int)I, err))
    return true;
  if (!knob(kKnobWoqStream) && try_launch_wave(a, s, shift, gmask, kDecFast, (int)I, err))
    return true;
  const int C = (int)(a.K / 128), tiles = (int)(a.N / 16);
  const size_t x_bytes = (size_t)a.M * stream_x_pitch((int)a.K) * 2;
  // as the plain stream kernel: four tiles (two pairs) per wave once x
  // takes a CU's LDS and there are enough tiles, else one pair
  const int tpw = x_bytes > 76 * 1024 && tiles >= 800 ? 4 : 2;
  // x leaving room for one workgroup per CU over more than a round of
  // workgroups: the wide kernel's merged form when it takes the call in one
  // launch (woq_try_wide_gate_up).  Measured: 27648 x 5120 at M = 10 / 12
  // took 29.3 / 30.2 us here against 25.2 / 24.9 there; 16384 x 3072 at
  // M = 16 (one round here, half a round there) 12.2 against 16.2
  if (!knob(kKnobWoqStream) && x_bytes > 76 * 1024 && a.post.count == 0 && a.N % 128 == 0 &&
      (I / 16 + tpw / 2 - 1) / (tpw / 2) > 256) {
    WidePlan wp;
    if (woq_wide_ok(a, &wp) && wp.splits == 1) return false;
  }
  const size_t lds = stream_scale_offset(stream_slab_bytes(8, tpw, 1), x_bytes) +
                     stream_scale_bytes((int)a.G, tpw);
  if (lds > kStreamLdsMax) return false;
  const int need = (C + 7) / 8;
  int cpw = 0;
  for (int c : {2, 4, 8, 12, 14, 16})
    if (c >= need) { cpw = c; break; }
  if (cpw < need) return false;
  const int x_dma = stream_x_dma(a, 1) ? 1 : 0;
  const dim3 grid((unsigned)((I / 16 + tpw / 2 - 1) / (tpw / 2))), block(512);
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr, "[zt] woq gate_up stream M=%lld N=%lld K=%lld: CPW=%d TPW=%d\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, cpw, tpw);
#define ZT_GU_CASE(CPW_, TPW_)                                                              \
  if (cpw == CPW_ && tpw == TPW_) {                                                        \
    woq_stream_kernel<8, CPW_, TPW_, kDecFast, 1, 1><<<grid, block, lds, s>>>(a, shift, gmask, \
                                                                            x_dma, (int)I); \
    *err = hipGetLastError();                                                              \
    return true;                                                                           \
  }
  ZT_GU_CASE(4, 2) ZT_GU_CASE(8, 2) ZT_GU_CASE(14, 2) ZT_GU_CASE(16, 2)
  ZT_GU_CASE(2, 4) ZT_GU_CASE(4, 4) ZT_GU_CASE(8, 4)
#undef ZT_GU_CASE
  return false;
}

// y[m][j] = silu(h[m][j]) * round_y(h[m][I + j]) for the fp32 [M, ld_h]
// result h of the full gate_up linear (the two-step merged path)
__global__ __launch_bounds__(256) void silu_mul_halves_kernel(const float *h, int64_t ld_h,
                                                              int64_t M, int64_t I, void *y,
                                                              int y_dt, int64_t ldy) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * I) return;
  const int64_t m = idx / I, j = idx - m * I;
  float u = h[m * ld_h + I + j];
  if (y_dt == ZT_DT_BF16) u = bf16_bits_to_f32(f32_to_bf16_bits(u));
  store_elem(y, y_dt, m * ldy + j, unary_op(ZT_PO_SILU, h[m * ld_h + j]) * u);
}

hipError_t launch_silu_mul_halves(const float *h, int64_t ld_h, int64_t M, int64_t I, void *y,
                                  int y_dt, int64_t ldy, hipStream_t s) {
  if (M == 0 || I == 0) return hipSuccess;
  const int64_t n = M * I;
  silu_mul_halves_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(h, ld_h, M, I, y,
                                                                                y_dt, ldy);
  return hipGetLastError();
}

hipError_t launch_woq_decode(const WoqArgs &a, const DecodePlan &p, void *workspace,
                             hipStream_t s) {
  (void)workspace;
  if (a.M == 0 || a.N == 0) return hipSuccess;
  {
    const int64_t cpg = a.G == 1 ? 0 : (a.K / a.G) / 128;
    int shift = 0;
    while (cpg > 1 && (1 << shift) < cpg) ++shift;
    const int gmask = a.G == 1 ? 0 : 0x7fffffff;
    const int mode = a.s_dt == ZT_DT_F32 ? kDecGenF32 : (a.zp ? kDecGenBf16 : kDecFast);
    hipError_t err = hipSuccess;
    if (try_launch_stream(a, s, shift, gmask, mode, &err)) return err;
  }
  if (knob(kKnobWoqDebug))
    std::fprintf(stderr,
                 "[zt] woq decode M=%lld N=%lld K=%lld: NK=%d NT=%d CPW=%d TPW=%d NI=%d xr=%d "
                 "xs=%d grid=%d lds=%zu\n",
                 (long long)a.M, (long long)a.N, (long long)a.K, p.NK, p.NT, p.CPW, p.TPW, p.ni,
                 p.xl, p.xs, p.nrb, decode_lds(a.M, (int)(a.K / 128), p));
#define ZT_DECODE_CASE(MT_, NI_, XR_, XS_)                                   \
  if (p.mt == MT_ && p.ni == NI_ && (bool)p.xl == XR_ && (bool)p.xs == XS_) \
    return launch_decode_t<MT_, 2, NI_, XR_, XS_>(a, p, s);
  ZT_DECODE_CASE(1, 1, true, true) ZT_DECODE_CASE(1, 2, true, true)
  ZT_DECODE_CASE(1, 3, true, true) ZT_DECODE_CASE(1, 4, true, true)
  ZT_DECODE_CASE(1, 6, true, true) ZT_DECODE_CASE(1, 8, true, true)
  ZT_DECODE_CASE(1, 1, true, false) ZT_DECODE_CASE(1, 2, true, false)
  ZT_DECODE_CASE(1, 3, true, false) ZT_DECODE_CASE(1, 4, true, false)
  ZT_DECODE_CASE(1, 6, true, false) ZT_DECODE_CASE(1, 8, true, false)
  ZT_DECODE_CASE(2, 1, true, false) ZT_DECODE_CASE(2, 2, true, false)
  ZT_DECODE_CASE(2, 3, true, false) ZT_DECODE_CASE(2, 4, true, false)
  ZT_DECODE_CASE(2, 6, true, false) ZT_DECODE_CASE(2, 8, true, false)
  ZT_DECODE_CASE(1, 2, false, false) ZT_DECODE_CASE(1, 4, false, false)
  ZT_DECODE_CASE(1, 8, false, false)
#undef ZT_DECODE_CASE
  return hipErrorInvalidValue;
}

// K splits of the prefill GEMM when its 128 x 128 tiles (the tile it takes
// at half a round of 256 x 128 tiles or less) make at most one round: up to
// 8, about two workgroups per CU, at least 16 steps of 64 each (1 = no split)
int woq_gemm_splits(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < 1 || knob(kKnobWoqGemm)) return 1;
  const int64_t t256 = ((M + 255) / 256) * ((N + 127) / 128);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (t256 > 128 || t128 > 256) return 1;
  const int64_t sp = std::min<int64_t>(std::min<int64_t>(8, 512 / t128), (K / kW32BK) / 16);
  return sp >= 2 ? (int)sp : 1;
}

size_t woq_gemm_workspace(int64_t M, int64_t N, int64_t K) {
  const int sp = woq_gemm_splits(M, N, K);
  return sp > 1 ? (size_t)sp * (size_t)M * (size_t)N * sizeof(float) : 0;
}

hipError_t launch_woq_gemm(const WoqArgs &a, hipStream_t s) {
  return launch_woq_gemm(a, s, nullptr, 0);
}

hipError_t launch_woq_gemm(const WoqArgs &a, hipStream_t s, void *workspace, size_t workspace_bytes) {
  {
    // the DMA kernel: bf16 x, K % 128 == 0, one scale per 128-chunk, 32-bit
    // byte offsets for x and the weights
    const int64_t gs = a.K / a.G, cpg = gs / 128;
    const bool ok = a.x_dt == ZT_DT_BF16 && a.K % 128 == 0 && a.ldx % 8 == 0 &&
                    aligned16(a.x) && aligned16(a.w) &&
                    (a.G == 1 || (gs % 128 == 0 && (cpg & (cpg - 1)) == 0)) &&
                    a.M * a.ldx * 2 < (int64_t)kOobOffset &&
                    a.N * (a.K / 2) < (int64_t)kOobOffset;
    const char *e = knob(kKnobWoqGemm);  // o: 16x16, d: 16x16 DMA, 1: 128x128, 2, w / v / x: load waves
    if (ok && !(e && e[0] == 'o')) {
      int shift = 0;
      while (cpg > 1 && (1 << shift) < cpg) ++shift;
      const int gmask = a.G == 1 ? 0 : 0x7fffffff;
      const int mode = a.s_dt == ZT_DT_F32 ? kDecGenF32 : (a.zp ? kDecGenBf16 : kDecFast);
      const int64_t t256 = ((a.M + 255) / 256) * ((a.N + 127) / 128);
      // the 32x32 kernel: fast mode, K in 64-steps, scale rows of whole
      // 16-byte pieces
      if (mode == kDecFast && a.N % 8 == 0 && !(e && e[0] == 'd') &&
          (int64_t)a.G * a.N * 2 < (int64_t)kOobOffset) {
        // one round of 256 x 128 tiles (at most one per CU, more than half
        // of them): the load-wave kernel, whose deeper prefetch is then not
        // paid for by an epilogue that a second workgroup per CU would hide
        // (O and down at M = 2048: 104 -> 81 and 327 -> 255 us); when 256 x
        // 192 tiles make one round where 256 x 128 do not, those (QKV: 152 ->
        // 112 us); more rounds: two workgroups per CU (gate_up 508 against 549
        // us with 256 x 128).  At half a round or less the split path below
        // (8192 x 8192 / 8192 x 28672 at M = 384: 106.8 / 338 us on 128
        // load-wave tiles, 87.0 / 265 split in two)
        const bool big32 = e ? e[0] != '1' : t256 > 128;
        const bool ws = e ? e[0] == 'w' || e[0] == 'v' : t256 > 128 && t256 <= 256;
        const int64_t t192 = ((a.M + 255) / 256) * ((a.N + 191) / 192);
        const bool ws192 = e ? e[0] == 'x' : t256 > 256 && t192 <= 256;
        if (ws192) return launch_woq_gemm_ws_t<256, 192, 3>(a, s, shift, gmask);
        if (ws)
          return e && e[0] == 'w' ? launch_woq_gemm_ws_t<256, 128, 4>(a, s, shift, gmask)
                                  : launch_woq_gemm_ws_t<256, 128, 3>(a, s, shift, gmask);
        if (big32) return launch_woq_gemm32_t<256, 128>(a, s, shift, gmask);
        // few tiles: K split over fp32 partials in the workspace when it has
        // room (graph replays over rotating weights, one box, M = 512:
        // 4096 x 11008 148.5 us and 3072 x 8192 113.9 us unsplit, as long as
        // at M = 2048 on twice the tile area)
        const int sp = woq_gemm_splits(a.M, a.N, a.K);
        const size_t need = woq_gemm_workspace(a.M, a.N, a.K);
        if (sp > 1 && workspace && workspace_bytes >= need &&
            (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0) {
          if (knob(kKnobWoqDebug))
            std::fprintf(stderr, "[zt] woq gemm32 M=%lld N=%lld K=%lld: 128x128 tiles, %d K splits\n",
                         (long long)a.M, (long long)a.N, (long long)a.K, sp);
          float *partial = static_cast<float *>(workspace);
          hipError_t err = launch_woq_gemm32_t<128, 128>(a, s, shift, gmask, partial, sp);
          if (err != hipSuccess) return err;
          return launch_splitk_reduce(a, partial, sp, s);
        }
        return launch_woq_gemm32_t<128, 128>(a, s, shift, gmask);
      }
      // 256 x 128 only for the fast mode: the general dequant spills there
      const bool big = mode == kDecFast && (e ? e[0] == '2' : t256 >= 128);
      return big ? launch_woq_dma_t<256, 128>(a, s, shift, gmask, mode)
                 : launch_woq_dma_t<128, 128>(a, s, shift, gmask, mode);
    }
  }
  if (a.M == 0 || a.N == 0) return hipSuccess;
  if (a.M <= 64) {
    dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 63) / 64));
    hipLaunchKernelGGL((woq_gemm_kernel<64, 32>), grid, dim3(256), 0, s, a);
  } else {
    dim3 grid((unsigned)((a.N + 127) / 128), (unsigned)((a.M + 127) / 128));
    hipLaunchKernelGGL((woq_gemm_kernel<128, 128>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_repack(const int8_t *w, int64_t N, int64_t K, int32_t *out,
                         hipStream_t s) {
  const int64_t n = N * (K / 8);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, s, w, N, K, out);
  return hipGetLastError();
}

hipError_t launch_repack_from_int4pack(const uint8_t *packed, int64_t N,
                                       int64_t K, int32_t *out, hipStream_t s) {
  const int64_t n = N * (K / 8);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(repack_from_int4pack_kernel,
                     dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, packed,
                     N, K, out);
  return hipGetLastError();
}

}  // namespace zt
