// int4 weight-only linear kernels for gfx950 (zentorch_woq_linear family).
//
// Numerics (all three kernels): each weight is dequantised to the bf16 value
// bf16_rne(q*s) (or the zero-point forms, woq_dequant.hpp) and multiplied
// with the bf16 activations on the bf16 MFMA with fp32 accumulation; bias
// and post-ops run in fp32 and the output is rounded once.  That is the
// dequantise-then-bf16-GEMM the reference's own test reference computes
// (test/unittests/op_tests/test_woq_linear.py:118-128) and that its 1e-3
// tolerance pins; an exact sum_g s_g sum_k x q fails that test.
//
//  * woq_decode_kernel  M <= 32: the decode GEMV / skinny GEMM.  Packed int4
//    weights stream from HBM in 16-byte loads straight into the registers
//    that are the MFMA A operands; the activations stay in registers for
//    every row tile a wave visits.  Waves split K inside a workgroup
//    (reduced through LDS); long K is split across workgroups too, and the
//    last workgroup of a row block reduces the fp32 partials and runs the
//    epilogue.
//  * woq_gemm_kernel    M > 32: tiled bf16 MFMA GEMM; weight tiles are
//    dequantised into LDS.
//  * woq_generic_kernel any shape/dtype the two above do not take (fp32
//    activations, K not a multiple of 64, odd group sizes): one wave per
//    output element.
//
// Weight layout: [N, K/8] int32, nibble i of word (n, c) is element
// (n, 8c+i) -- the storage of the [K/8, N] view zentorch_woq_linear takes
// (src/cpu/cpp/WOQ_Linear.cpp:31-42, repack :345-350).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "woq_dequant.hpp"
#include "zt_launch.hpp"

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

// Per-(row, group) dequantisation constants for one lane's weight row.
struct RowDq {
  float s, s16, c0, c1;
  DqGeneral g;
};

template <bool FAST>
__device__ __forceinline__ RowDq row_dq(const WoqArgs &a, int zmode, int64_t sidx) {
  RowDq r;
  const float s = load_elem(a.scales, a.s_dt, sidx);
  if (FAST) {
    r.s = s, r.s16 = s * 0.0625f, r.c0 = -1032.f * s, r.c1 = -72.f * s;
  } else {
    const float z = zmode ? load_elem(a.zp, a.zp_dt, sidx) : 0.f;
    r.g = dq_general_params(zmode, s, z);
  }
  return r;
}

template <bool FAST>
__device__ __forceinline__ bf16x8_t dq_word(uint32_t w, const RowDq &r) {
  const u32x4_t v = FAST ? dq8_s4_bf16scale(w, r.s, r.s16, r.c0, r.c1) : dq8_general(w, r.g);
  return __builtin_bit_cast(bf16x8_t, v);
}

// Decode GEMV / skinny GEMM (M <= 32).  Grid (row blocks, K splits); a
// workgroup of NW waves covers TPW 16-row tiles over its K split, wave w
// taking CPW 128-wide chunks of it.  Lane (r = lane%16, g = lane/16) loads
// the 16 bytes of row r holding elements [32g, 32g+32) of a chunk, which are
// exactly its A operands for the chunk's four 16x16x32 MFMAs; the matching
// activations (B operands) are loaded once per wave and reused for every
// tile.  Partial sums meet in LDS; with more than one K split the last
// workgroup of a row block adds the splits' fp32 partials.
template <int MT, int CPW, bool FAST>
__global__ __launch_bounds__(512, 2) void woq_decode_kernel(
    WoqArgs a, int S, int TPW, float *part, unsigned *counters) {
  extern __shared__ float red[];  // [TPW*16 rows][RS]
  constexpr int RS = 16 * MT + 1;
  __shared__ int is_last;

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int rb = blockIdx.x, sp = blockIdx.y;
  const int M = (int)a.M, N = (int)a.N;
  const int64_t KW = a.K / 8;
  const int C = (int)(a.K / 128);
  const int Cs = (C + S - 1) / S;
  const int c_lo = sp * Cs + wv * CPW;
  const int c_hi = min(C, (sp + 1) * Cs);
  const int64_t gs = a.K / a.G;
  const int zmode = zp_mode_of(a.zp, a.zp_dt);

  for (int i = threadIdx.x; i < TPW * 16 * RS; i += blockDim.x) red[i] = 0.f;

  // Activations of this wave's chunks as MFMA B operands: lane (m, g) holds
  // x[m, 128c + 32g + 8i .. +8) for MFMA i of chunk c.
  bf16x8_t xb[CPW][MT][4];
  const uint16_t *xp = reinterpret_cast<const uint16_t *>(a.x);
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int kc = c_lo + c;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (kc < c_hi && m < M)
          v = *reinterpret_cast<const u32x4_t *>(
              xp + (int64_t)m * a.ldx + (int64_t)kc * 128 + 32 * lg + 8 * i);
        xb[c][mt][i] = __builtin_bit_cast(bf16x8_t, v);
      }
    }
  }
  __syncthreads();

  const int tiles = (N + 15) / 16;
  const int t_lo = rb * TPW;
  const int t_hi = min(tiles, t_lo + TPW);

  u32x4_t wcur[CPW], wnxt[CPW];
  auto load_tile = [&](u32x4_t *dst, int t) {
    const int n = min(t * 16 + lr, N - 1);
    const uint32_t *row = a.w + (int64_t)n * KW;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int kc = c_lo + c;
      if (kc < c_hi)
        dst[c] = *reinterpret_cast<const u32x4_t *>(row + (int64_t)kc * 16 + 4 * lg);
      else
        dst[c] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  if (t_lo < t_hi) load_tile(wcur, t_lo);

  for (int t = t_lo; t < t_hi; ++t) {
    if (t + 1 < t_hi) load_tile(wnxt, t + 1);
    const int n_row = min(t * 16 + lr, N - 1);
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int kc = c_lo + c;
      if (kc >= c_hi) break;
      const RowDq rd = row_dq<FAST>(a, zmode, (((int64_t)kc * 128) / gs) * N + n_row);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8_t A = dq_word<FAST>(wcur[c][i], rd);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, xb[c][mt][i], acc[mt], 0, 0, 0);
      }
    }
    // D[row = 4g + r][token = lane % 16]
    float *rt = red + (t - t_lo) * 16 * RS;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        atomicAdd(rt + (4 * lg + r) * RS + mt * 16 + lr, acc[mt][r]);
#pragma unroll
    for (int c = 0; c < CPW; ++c) wcur[c] = wnxt[c];
  }
  __syncthreads();

  const int rows = (t_hi - t_lo) * 16;
  const int n0 = t_lo * 16;
  const int total = rows * M;
  if (S == 1) {
    for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
      const int m = idx / rows, nr = idx - m * rows, n = n0 + nr;
      if (n >= N) continue;
      float v = red[nr * RS + m];
      if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
      v = apply_post_ops(v, a.post, m, n);
      store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
    }
    return;
  }

  // K split across workgroups: publish this split's partial, then the last
  // workgroup of the row block adds all splits and runs the epilogue.
  float *mine = part + (int64_t)sp * M * N;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int m = idx / rows, nr = idx - m * rows, n = n0 + nr;
    if (n < N) mine[(int64_t)m * N + n] = red[nr * RS + m];
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = atomicAdd(counters + rb, 1u);
    is_last = (old == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int m = idx / rows, nr = idx - m * rows, n = n0 + nr;
    if (n >= N) continue;
    float v = 0.f;
    for (int s2 = 0; s2 < S; ++s2)
      v += __hip_atomic_load(part + ((int64_t)s2 * M + m) * N + n, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if (a.bias) v = v + load_elem(a.bias, a.b_dt, n);
    v = apply_post_ops(v, a.post, m, n);
    store_elem(a.y, a.y_dt, (int64_t)m * a.ldy + n, v);
  }
  if (threadIdx.x == 0) counters[rb] = 0u;
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
  if (const char *f = std::getenv("ZT_WOQ_FORCE_KERNEL")) {
    if (!std::strcmp(f, "generic")) return kWoqGeneric;
  }
  const bool bf16_ok = a.x_dt == ZT_DT_BF16 && a.ldx % 8 == 0 &&
                       aligned16(a.x) && aligned16(a.w);
  if (!bf16_ok || a.N < 1) return kWoqGeneric;
  const int64_t gs = a.K / a.G;
  const char *f = std::getenv("ZT_WOQ_FORCE_KERNEL");
  const bool decode_ok = a.K % 128 == 0 && (a.G == 1 || gs % 128 == 0) &&
                         a.M <= 32 && a.N < (int64_t)1 << 30;
  const bool gemm_ok = a.K % kGemmBK == 0 && gs % 32 == 0;
  if (f && !std::strcmp(f, "gemm")) return gemm_ok ? kWoqGemm : kWoqGeneric;
  if (f && !std::strcmp(f, "decode")) return decode_ok ? kWoqDecode : kWoqGeneric;
  if (decode_ok) return kWoqDecode;
  if (gemm_ok) return kWoqGemm;
  return kWoqGeneric;
}

static int env_plan(int *v) {
  const char *p = std::getenv("ZT_WOQ_DECODE_PLAN");
  if (!p) return 0;
  return std::sscanf(p, "%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3]) == 4;
}

bool woq_decode_plan(int64_t M, int64_t N, int64_t K, DecodePlan *plan) {
  const int C = (int)(K / 128);
  const int tiles = (int)((N + 15) / 16);
  const int mt = M <= 16 ? 1 : 2;
  const int cpw_max = mt == 1 ? 4 : 2;
  int v[4];
  DecodePlan p{};
  p.mt = mt;
  if (env_plan(v)) {
    p.S = v[0], p.NW = v[1], p.CPW = v[2], p.TPW = v[3];
  } else {
    // Smallest K split whose chunks fit 8 waves of cpw_max chunks; then as
    // many row tiles per workgroup as keep >= 256 workgroups (one per CU)
    // so the activations held in registers are reused across tiles.
    auto split = [&](int S, int *NW, int *CPW) {
      const int Cs = (C + S - 1) / S;
      *NW = std::min(8, Cs);
      *CPW = (Cs + *NW - 1) / *NW;
      *NW = (Cs + *CPW - 1) / *CPW;
    };
    int S = 1, NW = 1, CPW = 1;
    for (;; ++S) {
      split(S, &NW, &CPW);
      if (CPW <= cpw_max) break;
    }
    // Row-poor problems with more than a few tokens: split K once more so
    // each workgroup covers several row tiles and reuses its activations.
    if (M > 4 && tiles * S < 2 * 256 && 2 * S <= C && S < 4) {
      S *= 2;
      split(S, &NW, &CPW);
    }
    int TPW = std::max(1, (tiles * S) / 256);
    TPW = std::min(TPW, 1024 / (16 * mt + 1));  // reduction buffer <= 64 KB of LDS
    p.S = S, p.NW = NW, p.CPW = CPW, p.TPW = TPW;
  }
  if (p.S < 1 || p.NW < 1 || p.NW > 8 || p.CPW < 1 || p.CPW > (mt == 1 ? 8 : 4) ||
      p.TPW < 1 || p.TPW * 16 * (16 * mt + 1) > 16384)
    return false;
  if ((long)p.S * p.NW * p.CPW < C) return false;  // must cover K
  p.nrb = (tiles + p.TPW - 1) / p.TPW;
  if (p.S > 1 && p.nrb > (int)kCounterSlots) return false;
  *plan = p;
  return true;
}

size_t woq_decode_workspace(const DecodePlan &p, int64_t M, int64_t N) {
  if (p.S <= 1) return 0;
  return kCounterSlots * sizeof(unsigned) + (size_t)p.S * M * N * sizeof(float);
}

hipError_t launch_woq_generic(const WoqArgs &a, hipStream_t s) {
  const int64_t waves = a.M * a.N;
  if (waves == 0) return hipSuccess;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL(woq_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int MT, int CPW>
static hipError_t launch_decode_t(const WoqArgs &a, const DecodePlan &p,
                                  float *part, unsigned *counters,
                                  hipStream_t s) {
  const size_t lds = (size_t)p.TPW * 16 * (16 * MT + 1) * sizeof(float);
  dim3 grid((unsigned)p.nrb, (unsigned)p.S);
  const bool fast = a.zp == nullptr && a.s_dt == ZT_DT_BF16;
  if (fast)
    hipLaunchKernelGGL((woq_decode_kernel<MT, CPW, true>), grid, dim3(64 * p.NW), lds, s,
                       a, p.S, p.TPW, part, counters);
  else
    hipLaunchKernelGGL((woq_decode_kernel<MT, CPW, false>), grid, dim3(64 * p.NW), lds, s,
                       a, p.S, p.TPW, part, counters);
  return hipGetLastError();
}

hipError_t launch_woq_decode(const WoqArgs &a, const DecodePlan &p,
                             void *workspace, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  unsigned *counters = reinterpret_cast<unsigned *>(workspace);
  float *part = workspace ? reinterpret_cast<float *>(
                                reinterpret_cast<char *>(workspace) +
                                kCounterSlots * sizeof(unsigned))
                          : nullptr;
#define ZT_DECODE_CASE(MT_, CPW_)                                   \
  if (p.mt == MT_ && p.CPW == CPW_)                                 \
    return launch_decode_t<MT_, CPW_>(a, p, part, counters, s);
  ZT_DECODE_CASE(1, 1) ZT_DECODE_CASE(1, 2) ZT_DECODE_CASE(1, 3)
  ZT_DECODE_CASE(1, 4) ZT_DECODE_CASE(1, 5) ZT_DECODE_CASE(1, 6)
  ZT_DECODE_CASE(1, 7) ZT_DECODE_CASE(1, 8)
  ZT_DECODE_CASE(2, 1) ZT_DECODE_CASE(2, 2) ZT_DECODE_CASE(2, 3)
  ZT_DECODE_CASE(2, 4)
#undef ZT_DECODE_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_woq_gemm(const WoqArgs &a, hipStream_t s) {
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
