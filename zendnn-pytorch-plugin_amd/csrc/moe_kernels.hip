// Grouped int4 weight-only MoE for gfx950 (zentorch_fused_moe with packed
// int4 expert weights).
//
// The reference (src/cpu/cpp/FusedMoE.cpp:289-433, 508-700) groups the
// (token, k) pairs by expert on the host, runs each active expert's
// w13 GEMM + gated activation and w2 GEMM, and reduces
// out[t] = sum_k topk_weights[t, k] * y[t, k].  Here every step runs on the
// GPU without a host round trip (so the op can be captured in a HIP graph):
//
//  * moe_route_kernel   one workgroup: per-expert counts, a stable order of
//    the pairs by expert (the token of each row in that order: pair_token;
//    ranks from wave ballots),
//    each pair's row in that order (pair_pos, -1 for ids outside [0, E)),
//    expert row offsets, and a table of (expert, first row, end row) for
//    every BM-row tile of the grouped GEMMs.
//  * woq_moe_gemm_kernel<GATED, BN> / woq_moe_gemm_wide_kernel<GATED, BN>
//    an int4 GEMM over that tile table on 32x32x16 bf16 MFMAs (the wide
//    form, 256 weight rows per workgroup, runs the gate_up GEMM).  A rows are gathered (w13: the input row of the
//    pair's token; w2: the pair's row of the intermediate), the weight
//    pointer is the tile's expert.  GATED tiles pair gate rows n with their
//    up rows I + n, so the epilogue writes act(g) * u directly.
//  * moe_combine_kernel out[t] = sum over k (in k order) of
//    w[t, k] * y[pair_pos[t, k]], fp32, rounded once.
#include <cstdio>
#include <cstdlib>

#include "woq_dequant.hpp"
#include "zt_launch.hpp"
#include "zt_tuning.hpp"

namespace zt {

namespace {

typedef __attribute__((address_space(3))) void *lds_ptr_t;

constexpr int kMoeBM = 96;    // grouped-GEMM rows (pairs) per tile
constexpr int kXRowB = 256;   // bytes of A per row per 128-wide K step
constexpr int kWRowB = 64;    // bytes of int4 per weight row per step
constexpr int kXStage = kMoeBM * kXRowB;  // one LDS buffer of A rows
constexpr int kXStages = 3;               // x prefetched two steps ahead
constexpr int kMoeDepth = 2;  // K steps of weights loaded ahead
constexpr int kMoeComputeWaves = 4;
constexpr int kMoeThreads = 64 * (kMoeComputeWaves + 1);  // + the x producer

// Ranks are stable: pair i's row is its expert's offset plus the number of
// earlier pairs with the same expert.  The pairs go in chunks of 1024, one
// per thread; inside a wave a ballot per distinct expert gives each lane its
// rank among the wave's lanes of that expert and the wave's count of it
// (wcnt[wave][e], dynamic LDS of 16 E ints), the waves before it add theirs,
// and base[e] carries the counts of earlier chunks.
__global__ __launch_bounds__(1024) void moe_route_kernel(const int32_t *ids, int P, int E,
                                                          int topk, MoeWork w) {
  __shared__ int cnt[1024];
  __shared__ int base[1024];
  extern __shared__ int wcnt[];  // [16][E]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < P; i += 1024) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int off = 0, nt = 0;
    for (int e = 0; e < E; ++e) {
      w.expert_off[e] = off;
      base[e] = off;
      for (int m0 = 0; m0 < cnt[e]; m0 += kMoeBM) {
        w.mt_info[4 * nt] = e;
        w.mt_info[4 * nt + 1] = off + m0;
        w.mt_info[4 * nt + 2] = off + min(cnt[e], m0 + kMoeBM);
        w.mt_info[4 * nt + 3] = 0;
        ++nt;
      }
      off += cnt[e];
    }
    w.expert_off[E] = off;
    w.num_mt[0] = nt;
  }
  const uint64_t lt = (1ull << lane) - 1;
  for (int c0 = 0; c0 < P; c0 += 1024) {
    for (int j = tid; j < 16 * E; j += 1024) wcnt[j] = 0;
    __syncthreads();  // also orders base[] after tid 0 or the previous chunk
    const int i = c0 + tid;
    int e = i < P ? ids[i] : -1;
    if (e >= E) e = -1;
    // rank among this wave's lanes of the same expert, one ballot per
    // distinct expert of the wave (the loop is wave-uniform)
    int rank = 0;
    uint64_t todo = __ballot(e >= 0);
    while (todo) {
      const int ee = __shfl(e, __ffsll((unsigned long long)todo) - 1);
      const uint64_t m = __ballot(e == ee);
      if (e == ee) {
        rank = __popcll(m & lt);
        if (rank == 0) wcnt[wave * E + e] = __popcll(m);
      }
      todo &= ~m;
    }
    __syncthreads();
    int pos = -1;
    if (e >= 0) {
      for (int v = 0; v < wave; ++v) rank += wcnt[v * E + e];
      pos = base[e] + rank;
      w.pair_token[pos] = i / topk;
    }
    if (i < P) w.pair_pos[i] = pos;
    __syncthreads();  // every base[] read of this chunk is done
    for (int ee = tid; ee < E; ee += 1024) {
      int n = 0;
      for (int v = 0; v < 16; ++v) n += wcnt[v * E + ee];
      base[ee] += n;
    }
    __syncthreads();  // before the next chunk clears wcnt
  }
}

// s_waitcnt immediate that waits for at most n outstanding vector-memory
// loads (n < 64) and nothing else
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// One grouped-GEMM tile: NB 32-row blocks of the expert's pairs (rows
// r0 .. r0 + 32 NB; the blocks of the 96-row tile past the expert's last
// pair cost nothing) times BN weight rows, on v_mfma_f32_32x32x16_bf16
// (the 32x32 shape sustains twice the 16x16x32 shape's rate on gfx950).
//  * kMoeComputeWaves waves split along N only: each owns BN/4 weight rows
//    (WTN 32-column MFMA tiles), so every weight fragment is dequantised
//    once and feeds NB MFMAs.  Their weights and scales go straight from
//    HBM to registers kMoeDepth K steps ahead in rotating register sets.
//  * One more wave only moves the gathered A rows to LDS by DMA (16-byte
//    chunks XOR-swizzled by the row's low 4 bits) into kXStages buffers,
//    two steps ahead (an L2-resident tile still takes about 2 us to land
//    under this load).  A wave's loads retire in issue order, so a wave
//    that waited for its own x DMA would also wait for every weight load
//    issued before it; keeping the x DMA in a wave of its own leaves D
//    steps of weights in flight.  The waves meet at one barrier per step:
//    the producer arrives once x(ks + 1) has landed, the compute waves
//    once step ks is done.
//  * K order inside a 128-wide step: lane (c, kb) of a B fragment holds the
//    row's bytes 32 kb .. 32 kb + 31, and sub-step s (0..7) multiplies its
//    word s, i.e. k = 64 kb + 8 s + 0..7; the A fragment of lane (m, kb)
//    holds x[m][64 kb + 8 s .. + 7] to match.
//  * GATED: every 32-column tile holds 16 gate rows n and their 16 up rows
//    I + n; the epilogue pairs them through the LDS tile.
template <bool GATED, int BN, int NB>
__device__ __forceinline__ void moe_tile(const MoeGemm &g, int e, int r0, int r_end, int tn,
                                         unsigned char *smem) {
  constexpr int WTN = BN / 128;  // 32-column tiles per compute wave
  static_assert(WTN >= 1, "a wave owns at least one 32-column tile");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, kb = lane >> 5;
  const int K = g.K, KW = K / 8, N = g.N;
  const int n0 = GATED ? tn * (BN / 2) : tn * BN;
  const int nk = K / 128;
  // s_waitcnt lgkmcnt(0) alone
  constexpr int kLgkm0 = 15 | (3 << 14) | (7 << 4);

  f32x16_t acc[NB][WTN];
  if (wv == kMoeComputeWaves) {
    // ---- producer: x(0) .. x(nk - 1), one step ahead of the compute waves
    const auto a_rs = make_rsrc(g.a, (uint32_t)((int64_t)g.a_rows * g.lda * 2));
    // load q fills tile rows 4 q .. 4 q + 3, 16 bytes per lane; rows past
    // the expert's last pair start at kOobOffset and so read 0
    // (the token loads are unconditional, clamped to a live row, and the
    // out-of-range bit is ORed in, so the loads issue back to back rather
    // than one round trip each behind a branch)
    uint32_t a_off[8 * NB];
#pragma unroll
    for (int q = 0; q < 8 * NB; ++q) {
      const int row = 4 * q + (lane >> 4);
      const int gr = r0 + row;
      const int src = GATED ? g.w.pair_token[min(gr, r_end - 1)] : gr;
      a_off[q] = (uint32_t)(src * (2 * g.lda) + (((lane & 15) ^ (row & 15)) * 16)) |
                 (gr < r_end ? 0u : kOobOffset);
    }
    auto issue_x = [&](int step) {
      unsigned char *st = smem + (step % kXStages) * kXStage;
#pragma unroll
      for (int q = 0; q < 8 * NB; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, (lds_ptr_t)(st + 4 * q * kXRowB), 16,
                                                 a_off[q], step * kXRowB, 0, 0);
    };
    static_assert(kXStages == 3, "the waits below are written for x two steps ahead");
    issue_x(0);
    if (nk > 1) {
      issue_x(1);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(8 * NB));  // x(0) has landed
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    asm volatile("s_barrier" ::: "memory");
    for (int ks = 0; ks < nk; ++ks) {
      // buffer (ks + 2) % 3 was last read in step ks - 1, which every
      // compute wave finished before the barrier just passed; x(ks + 1)
      // (issued before x(ks + 2)) must land before the next barrier
      if (ks + 2 < nk) {
        issue_x(ks + 2);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(8 * NB));
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      asm volatile("s_barrier" ::: "memory");
    }
  } else {
    // ---- compute waves
    const uint32_t *wexp = g.w_packed + (size_t)e * N * KW;
    const uint16_t *sexp = g.scales + (size_t)e * g.G * N;
    const auto w_rs = make_rsrc(wexp, (uint32_t)((int64_t)N * KW * 4));
    const auto s_rs = make_rsrc(sexp, (uint32_t)(g.G * N * 2));
    // this lane's B column (expert weight row) in each of the wave's tiles;
    // only the last tile of a non-gated GEMM can pass N (not stored)
    uint32_t srow2[WTN], woff[WTN];
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int t = wv * WTN + j;  // 32-column tile of the workgroup
      int n = GATED ? (lc < 16 ? n0 : g.I + n0) + t * 16 + (lc & 15) : n0 + t * 32 + lc;
      n = min(n, N - 1);
      srow2[j] = 2u * (uint32_t)n;
      woff[j] = (uint32_t)n * (uint32_t)(KW * 4) + 32u * (uint32_t)kb;
    }
    // the per-lane offsets are fixed; the step's offset is the uniform
    // soffset.  Steps past the last one re-read step nk - 1 (an L2 hit)
    // into a register set nothing reads again.
    auto issue_w = [&](int step, u32x4_t (&w)[WTN][2], uint32_t (&s)[WTN]) {
      step = min(step, nk - 1);
      const int sb = ((step >> g.cpg_shift) & g.gmask) * N * 2;
#pragma unroll
      for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          w[j][h] = __builtin_bit_cast(
              u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rs, woff[j] + 16u * h,
                                                             step * kWRowB, 0));
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        s[j] = __builtin_amdgcn_raw_buffer_load_b16(s_rs, srow2[j], sb, 0);
    };

#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto dequant = [&](const u32x4_t (&w)[WTN][2], const uint32_t (&s)[WTN], int sub,
                       bf16x8_t (&B)[WTN]) {
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        const float sc = __uint_as_float(s[j] << 16);
        B[j] = __builtin_bit_cast(bf16x8_t, dq8_s4_bf16scale(w[j][sub >> 2][sub & 3], sc,
                                                              sc * 0.0625f, -1032.f * sc,
                                                              -72.f * sc));
      }
    };
    // A fragments of one 16-wide K sub-step: row 32 i + lc, k 64 kb + 8 sub ..
    auto read_x = [&](const unsigned char *st, int sub, u32x4_t (&xf)[NB]) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
        xf[i] = *reinterpret_cast<const u32x4_t *>(st + (32 * i + lc) * kXRowB +
                                                   (((8 * kb + sub) ^ (lc & 15)) * 16));
    };
    auto mfmas = [&](const u32x4_t (&xf)[NB], const bf16x8_t (&B)[WTN]) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, xf[i]), B[j], acc[i][j], 0, 0, 0);
    };
    // Issue order of one sub-step: each MFMA is followed by V VALU
    // instructions (the dequantisation of the next sub-step's B fragments
    // runs in the MFMA shadow) and, while there are any, one LDS read of
    // the next sub-step's A fragments.
    auto interleave = [&](bool reads) {
      constexpr int M = NB * WTN;
      constexpr int V = (16 * WTN + M - 1) / M;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
        if (reads && m < NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    };

    // D + 1 rotating register sets of weights and scales (D = kMoeDepth):
    // step ks computes on set ks % (D + 1), dequantises sub-step 0 of step
    // ks + 1 from the next set during its last sub-step, and loads step
    // ks + D into the set step ks - 1 used.
    constexpr int D = kMoeDepth;
    u32x4_t wq[D + 1][WTN][2];
    uint32_t sq[D + 1][WTN];
    bf16x8_t Bn[WTN];  // B fragments of the next sub-step to run
#pragma unroll
    for (int p = 0; p < D; ++p) issue_w(p, wq[p], sq[p]);
    asm volatile("s_barrier" ::: "memory");  // x(0) has landed
    dequant(wq[0], sq[0], 0, Bn);
    auto step = [&](int ks, const u32x4_t (&wc)[WTN][2], const uint32_t (&sc)[WTN],
                    const u32x4_t (&wx)[WTN][2], const uint32_t (&sx)[WTN],
                    u32x4_t (&wn)[WTN][2], uint32_t (&sn)[WTN]) {
      const unsigned char *st = smem + (ks % kXStages) * kXStage;
      u32x4_t xa[NB], xb[NB];
      read_x(st, 0, xa);
      __builtin_amdgcn_sched_barrier(0);
      issue_w(ks + D, wn, sn);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int sub = 0; sub < 8; ++sub) {
        bf16x8_t Bc[WTN];
#pragma unroll
        for (int j = 0; j < WTN; ++j) Bc[j] = Bn[j];
        if (sub < 7) {
          read_x(st, sub + 1, sub & 1 ? xa : xb);
          dequant(wc, sc, sub + 1, Bn);
        } else {
          dequant(wx, sx, 0, Bn);
        }
        mfmas(sub & 1 ? xb : xa, Bc);
        interleave(sub < 7);
      }
      // every read of buffer ks % 3 has returned before the producer may
      // refill it (after the next barrier).  A bare s_barrier: no fence, so
      // the weight prefetch stays in flight; the memory clobber keeps the
      // compiler from moving LDS accesses across it.
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kLgkm0);
      asm volatile("s_barrier" ::: "memory");
    };
    // whole rounds of D + 1 steps, then the rest outside the loop: a
    // guarded step inside the loop would make the compiler's wait counts at
    // the loop head conservative (a full drain of the prefetch)
    int k0 = 0;
    for (; k0 + D + 1 <= nk; k0 += D + 1) {
#pragma unroll
      for (int p = 0; p <= D; ++p)
        step(k0 + p, wq[p], sq[p], wq[(p + 1) % (D + 1)], sq[(p + 1) % (D + 1)],
             wq[(p + D) % (D + 1)], sq[(p + D) % (D + 1)]);
    }
#pragma unroll
    for (int p = 0; p < D; ++p)
      if (k0 + p < nk)
        step(k0 + p, wq[p], sq[p], wq[(p + 1) % (D + 1)], sq[(p + 1) % (D + 1)],
             wq[(p + D) % (D + 1)], sq[(p + D) % (D + 1)]);
  }

  // epilogue: the fp32 sums (+ bias) go through an LDS tile (the x buffers
  // are free: the producer's last DMA landed before the last barrier); one
  // loop then applies act(g) * u, rounds to bf16 and stores 8 bytes per
  // thread.  Accumulator register r of lane (lc, kb) is row
  // 8 (r / 4) + 4 kb + r % 4 of its 32-row block, column lc.
  constexpr int COLS = GATED ? BN / 2 : BN;           // output columns of the tile
  constexpr int TPF = (GATED ? 2 * COLS : COLS) + 4;  // fp32 pitch
  float *tile = reinterpret_cast<float *>(smem);
  const int NO = GATED ? g.I : N;  // output columns of the GEMM
  if (wv < kMoeComputeWaves) {
    const uint16_t *bexp = g.bias ? g.bias + (size_t)e * N : nullptr;
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const int t = wv * WTN + j;
      // gated: column lc < 16 is gate output t * 16 + lc, lc >= 16 its up row
      const int oc = GATED ? t * 16 + (lc & 15) : t * 32 + lc;
      const int c = GATED && lc >= 16 ? COLS + oc : oc;
      const int n = n0 + oc;
      float b = 0.f;
      if (bexp && n < NO) b = bf16_bits_to_f32(bexp[GATED && lc >= 16 ? g.I + n : n]);
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          tile[(32 * i + 8 * (r >> 2) + 4 * kb + (r & 3)) * TPF + c] = acc[i][j][r] + b;
    }
  }
  __syncthreads();
  const int rows = min(32 * NB, r_end - r0);
  for (int idx = tid; idx < rows * (COLS / 4); idx += kMoeThreads) {
    const int row = idx / (COLS / 4), c4 = (idx % (COLS / 4)) * 4;
    const int n = n0 + c4;
    if (n >= NO) continue;
    const float *t = tile + row * TPF + c4;
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) f[r] = GATED ? unary_op(g.act, t[r]) * t[COLS + r] : t[r];
    u32x2_t pk;
    pk[0] = pack_bf16x2(f[0], f[1]);
    pk[1] = pack_bf16x2(f[2], f[3]);
    *reinterpret_cast<u32x2_t *>(g.out + (size_t)(r0 + row) * g.ldo + n) = pk;
  }
}

// Wide form of moe_tile: BN = 128 WTN weight rows per workgroup, four
// waves that each own WTN 32-column tiles (tile t = 4 j + wave), so every
// A fragment read from LDS feeds WTN MFMAs instead of one.  There is no
// producer wave (its registers would cost the second workgroup per CU):
// each wave moves a quarter of the A rows by DMA together with its own
// weights, both two K steps ahead.  A wave's loads retire in issue order
// and the A rows and weights of a step are issued together, so one vmcnt
// wait per step covers both, and the barrier after it publishes every
// wave's share of the A tile.  Past the last step the DMA still issues,
// out of range (zeros into a stage no one reads), so that every step
// leaves the same number of loads in flight.  The epilogue goes through
// LDS one tile column j at a time (128 fp32 columns, so two workgroups fit
// a CU).
template <bool GATED, int BN, int NB>
__device__ __forceinline__ void moe_tile_wide(const MoeGemm &g, int e, int r0, int r_end, int tn,
                                              unsigned char *smem) {
  constexpr int WTN = BN / 128;  // 32-column tiles per wave
  constexpr int XL = 2 * NB;     // 1 KB A loads (4 rows each) per wave per step
  static_assert(WTN >= 2, "the wide form owns at least two tiles per wave");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, kb = lane >> 5;
  const int K = g.K, KW = K / 8, N = g.N;
  const int n0 = GATED ? tn * (BN / 2) : tn * BN;
  const int nk = K / 128;
  constexpr int kLgkm0 = 15 | (3 << 14) | (7 << 4);  // s_waitcnt lgkmcnt(0) alone

  // A rows 4 q' .. 4 q' + 3, q' = XL wv + q, 16 bytes per lane; rows past
  // the expert's last pair read 0
  const auto a_rs = make_rsrc(g.a, (uint32_t)((int64_t)g.a_rows * g.lda * 2));
  uint32_t a_off[XL];
#pragma unroll
  for (int q = 0; q < XL; ++q) {
    const int row = 4 * (XL * wv + q) + (lane >> 4);
    const int gr = r0 + row;
    const int src = GATED ? g.w.pair_token[min(gr, r_end - 1)] : gr;
    a_off[q] = (uint32_t)(src * (2 * g.lda) + (((lane & 15) ^ (row & 15)) * 16)) |
               (gr < r_end ? 0u : kOobOffset);
  }
  auto issue_x = [&](int step) {
    unsigned char *st = smem + (step % kXStages) * kXStage;
    const uint32_t past = step < nk ? 0u : kOobOffset;
#pragma unroll
    for (int q = 0; q < XL; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, (lds_ptr_t)(st + 4 * (XL * wv + q) * kXRowB),
                                               16, a_off[q] | past, step * kXRowB, 0, 0);
  };

  const uint32_t *wexp = g.w_packed + (size_t)e * N * KW;
  const uint16_t *sexp = g.scales + (size_t)e * g.G * N;
  const auto w_rs = make_rsrc(wexp, (uint32_t)((int64_t)N * KW * 4));
  const auto s_rs = make_rsrc(sexp, (uint32_t)(g.G * N * 2));
  uint32_t srow2[WTN], woff[WTN];
#pragma unroll
  for (int j = 0; j < WTN; ++j) {
    const int t = 4 * j + wv;
    int n = GATED ? (lc < 16 ? n0 : g.I + n0) + t * 16 + (lc & 15) : n0 + t * 32 + lc;
    n = min(n, N - 1);
    srow2[j] = 2u * (uint32_t)n;
    woff[j] = (uint32_t)n * (uint32_t)(KW * 4) + 32u * (uint32_t)kb;
  }
  auto issue_w = [&](int step, u32x4_t (&w)[WTN][2], uint32_t (&s)[WTN]) {
    step = min(step, nk - 1);  // past the end: an L2 hit into a set no one reads
    const int sb = ((step >> g.cpg_shift) & g.gmask) * N * 2;
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        w[j][h] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rs, woff[j] + 16u * h,
                                                           step * kWRowB, 0));
#pragma unroll
    for (int j = 0; j < WTN; ++j)
      s[j] = __builtin_amdgcn_raw_buffer_load_b16(s_rs, srow2[j], sb, 0);
  };

  f32x16_t acc[NB][WTN];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto dequant = [&](const u32x4_t (&w)[WTN][2], const uint32_t (&s)[WTN], int sub,
                     bf16x8_t (&B)[WTN]) {
#pragma unroll
    for (int j = 0; j < WTN; ++j) {
      const float sc = __uint_as_float(s[j] << 16);
      B[j] = __builtin_bit_cast(bf16x8_t, dq8_s4_bf16scale(w[j][sub >> 2][sub & 3], sc,
                                                            sc * 0.0625f, -1032.f * sc,
                                                            -72.f * sc));
    }
  };
  auto read_x = [&](const unsigned char *st, int sub, u32x4_t (&xf)[NB]) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
      xf[i] = *reinterpret_cast<const u32x4_t *>(st + (32 * i + lc) * kXRowB +
                                                 (((8 * kb + sub) ^ (lc & 15)) * 16));
  };
  auto mfmas = [&](const u32x4_t (&xf)[NB], const bf16x8_t (&B)[WTN]) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < WTN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, xf[i]), B[j], acc[i][j], 0, 0, 0);
  };
  auto interleave = [&](bool reads) {
    constexpr int M = NB * WTN;
    constexpr int V = (16 * WTN + M - 1) / M;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
      if (reads && m < NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };

  constexpr int D = kMoeDepth;
  static_assert(D == 2 && kXStages == 3, "A rows and weights travel two steps ahead");
  u32x4_t wq[D + 1][WTN][2];
  uint32_t sq[D + 1][WTN];
  bf16x8_t Bn[WTN];
#pragma unroll
  for (int p = 0; p < D; ++p) {
    issue_x(p);
    issue_w(p, wq[p], sq[p]);
  }
  // step ks: x(ks) and w(ks) landed once only step ks + 1's loads (XL A
  // loads, 2 WTN weight loads, WTN scale loads) are still in flight
  constexpr int kAfter = XL + 3 * WTN;
  dequant(wq[0], sq[0], 0, Bn);
  auto step = [&](int ks, const u32x4_t (&wc)[WTN][2], const uint32_t (&sc)[WTN],
                  const u32x4_t (&wx)[WTN][2], const uint32_t (&sx)[WTN],
                  u32x4_t (&wn)[WTN][2], uint32_t (&sn)[WTN]) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kAfter));
    __builtin_amdgcn_s_waitcnt(kLgkm0);  // this wave's reads of step ks - 1 are done
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char *st = smem + (ks % kXStages) * kXStage;
    u32x4_t xa[NB], xb[NB];
    read_x(st, 0, xa);
    __builtin_amdgcn_sched_barrier(0);
    issue_x(ks + D);
    issue_w(ks + D, wn, sn);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int sub = 0; sub < 8; ++sub) {
      bf16x8_t Bc[WTN];
#pragma unroll
      for (int j = 0; j < WTN; ++j) Bc[j] = Bn[j];
      if (sub < 7) {
        read_x(st, sub + 1, sub & 1 ? xa : xb);
        dequant(wc, sc, sub + 1, Bn);
      } else {
        dequant(wx, sx, 0, Bn);
      }
      mfmas(sub & 1 ? xb : xa, Bc);
      interleave(sub < 7);
    }
  };
  int k0 = 0;
  for (; k0 + D + 1 <= nk; k0 += D + 1) {
#pragma unroll
    for (int p = 0; p <= D; ++p)
      step(k0 + p, wq[p], sq[p], wq[(p + 1) % (D + 1)], sq[(p + 1) % (D + 1)],
           wq[(p + D) % (D + 1)], sq[(p + D) % (D + 1)]);
  }
#pragma unroll
  for (int p = 0; p < D; ++p)
    if (k0 + p < nk)
      step(k0 + p, wq[p], sq[p], wq[(p + 1) % (D + 1)], sq[(p + 1) % (D + 1)],
           wq[(p + D) % (D + 1)], sq[(p + D) % (D + 1)]);

  // epilogue, one tile column j (the waves' tiles 4 j .. 4 j + 3, i.e. 128
  // consecutive weight rows) at a time through an fp32 LDS tile; the
  // in-flight out-of-range DMA must land before the stages are reused
  constexpr int COLS = GATED ? 64 : 128;              // output columns per j
  constexpr int TPF = (GATED ? 2 * COLS : COLS) + 4;  // fp32 pitch
  float *tile = reinterpret_cast<float *>(smem);
  const int NO = GATED ? g.I : N;
  const uint16_t *bexp = g.bias ? g.bias + (size_t)e * N : nullptr;
  const int rows = min(32 * NB, r_end - r0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < WTN; ++j) {
    if (j) __syncthreads();  // the previous column's reads are done
    const int oc = GATED ? wv * 16 + (lc & 15) : wv * 32 + lc;  // within this j
    const int c = GATED && lc >= 16 ? COLS + oc : oc;
    const int n = n0 + j * COLS + oc;
    float b = 0.f;
    if (bexp && n < NO) b = bf16_bits_to_f32(bexp[GATED && lc >= 16 ? g.I + n : n]);
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        tile[(32 * i + 8 * (r >> 2) + 4 * kb + (r & 3)) * TPF + c] = acc[i][j][r] + b;
    __syncthreads();
    for (int idx = tid; idx < rows * (COLS / 4); idx += 256) {
      const int row = idx / (COLS / 4), c4 = (idx % (COLS / 4)) * 4;
      const int nn = n0 + j * COLS + c4;
      if (nn >= NO) continue;
      const float *tp = tile + row * TPF + c4;
      float f[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) f[r] = GATED ? unary_op(g.act, tp[r]) * tp[COLS + r] : tp[r];
      u32x2_t pk;
      pk[0] = pack_bf16x2(f[0], f[1]);
      pk[1] = pack_bf16x2(f[2], f[3]);
      *reinterpret_cast<u32x2_t *>(g.out + (size_t)(r0 + row) * g.ldo + nn) = pk;
    }
  }
}

template <bool GATED, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void woq_moe_gemm_wide_kernel(MoeGemm g, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int live = g.w.num_mt[0] * tiles_n;
  if ((int)blockIdx.x >= live) return;  // uniform: the whole workgroup leaves
  const int t = xcd_contiguous_tile(blockIdx.x, live);
  const int mt = t / tiles_n, tn = t - mt * tiles_n;
  const i32x4_t info = reinterpret_cast<const i32x4_t *>(g.w.mt_info)[mt];
  const int e = info[0], r0 = info[1], r_end = info[2];
  switch ((r_end - r0 + 31) >> 5) {
    case 1: moe_tile_wide<GATED, BN, 1>(g, e, r0, r_end, tn, smem); break;
    case 2: moe_tile_wide<GATED, BN, 2>(g, e, r0, r_end, tn, smem); break;
    default: moe_tile_wide<GATED, BN, 3>(g, e, r0, r_end, tn, smem); break;
  }
}

// Grid: mt_max * tiles_n workgroups (the route kernel's tile count is only
// known on the device).  The first num_mt * tiles_n blocks take the live
// tiles, XCD-contiguously (consecutive column tiles of one row tile share
// an XCD's L2 copy of its A rows); the rest leave at once.
template <bool GATED, int BN>
__global__ __launch_bounds__(kMoeThreads) void woq_moe_gemm_kernel(MoeGemm g, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int live = g.w.num_mt[0] * tiles_n;
  if ((int)blockIdx.x >= live) return;  // uniform: the whole workgroup leaves
  const int t = xcd_contiguous_tile(blockIdx.x, live);
  const int mt = t / tiles_n, tn = t - mt * tiles_n;
  const i32x4_t info = reinterpret_cast<const i32x4_t *>(g.w.mt_info)[mt];
  const int e = info[0], r0 = info[1], r_end = info[2];
  static_assert(kMoeBM == 96, "tiles are 1 to 3 blocks of 32 rows");
  switch ((r_end - r0 + 31) >> 5) {
    case 1: moe_tile<GATED, BN, 1>(g, e, r0, r_end, tn, smem); break;
    case 2: moe_tile<GATED, BN, 2>(g, e, r0, r_end, tn, smem); break;
    default: moe_tile<GATED, BN, 3>(g, e, r0, r_end, tn, smem); break;
  }
}

// out[t, h] = sum_k w[t, k] * y[pair_pos[t*topk + k], h], k in order.
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t *y, int H,
                                                          const int32_t *pair_pos,
                                                          const void *wts, int wts_dt,
                                                          int topk, bool skip_weighted,
                                                          uint16_t *out) {
  const int t = blockIdx.x;
  for (int h = threadIdx.x * 8; h < H; h += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < topk; ++k) {
      const int p = pair_pos[t * topk + k];
      if (p < 0) continue;
      const float wk = skip_weighted ? 1.f : load_elem(wts, wts_dt, (int64_t)t * topk + k);
      const u32x4_t v = *reinterpret_cast<const u32x4_t *>(y + (size_t)p * H + h);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += wk * __uint_as_float(v[i] << 16);
        acc[2 * i + 1] += wk * __uint_as_float(v[i] & 0xffff0000u);
      }
    }
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = pack_bf16x2(acc[2 * i], acc[2 * i + 1]);
    *reinterpret_cast<u32x4_t *>(out + (size_t)t * H + h) = o;
  }
}

// N is a multiple of the tile's column count (host-checked: I, H % 128 == 0)
template <bool GATED, int BN>
hipError_t launch_moe_gemm(const MoeGemm &g, hipStream_t s) {
  const int cols = GATED ? BN / 2 : BN;
  const int tiles_n = (GATED ? g.I : g.N + cols - 1) / cols;
  const dim3 grid((unsigned)(g.mt_max * tiles_n));
  if constexpr (BN > 128) {  // the wide form: 128-column epilogue tiles, no producer wave
    const size_t tile = (size_t)kMoeBM * (128 + 4) * 4;
    const size_t lds = tile > (size_t)kXStages * kXStage ? tile : (size_t)kXStages * kXStage;
    woq_moe_gemm_wide_kernel<GATED, BN><<<grid, dim3(256), lds, s>>>(g, tiles_n);
    return hipGetLastError();
  } else {
    const size_t tile = (size_t)kMoeBM * (BN + 4) * 4;  // fp32 epilogue tile
    const size_t lds = tile > (size_t)kXStages * kXStage ? tile : (size_t)kXStages * kXStage;
    woq_moe_gemm_kernel<GATED, BN><<<grid, dim3(kMoeThreads), lds, s>>>(g, tiles_n);
    return hipGetLastError();
  }
}

// weight rows per workgroup of the gate_up and down GEMMs; ZT_MOE_BN="g,d"
// (each 128 or 256) overrides them for tuning.  Measured on the Mixtral
// layer (256 tokens): gate_up 218 -> 199 us with the wide form; the down
// GEMM (4096 rows) would leave half the CUs idle with 256-row tiles.
void moe_tile_widths(int &bn1, int &bn2) {
  bn1 = 256, bn2 = 128;
  if (const char *v = knob(kKnobMoeBn)) {
    int a = 0, b = 0;
    if (std::sscanf(v, "%d,%d", &a, &b) == 2 && (a == 128 || a == 256) &&
        (b == 128 || b == 256))
      bn1 = a, bn2 = b;
  }
}

}  // namespace

int moe_max_tiles(int64_t P, int64_t E) { return (int)((P + kMoeBM - 1) / kMoeBM + E); }

hipError_t launch_woq_moe(const MoeArgs &a, const MoeWork &w, hipStream_t s) {
  const int P = (int)(a.T * a.topk);
  const int mt_max = moe_max_tiles(P, a.E);
  moe_route_kernel<<<1, 1024, (size_t)16 * a.E * sizeof(int), s>>>(a.ids, P, (int)a.E, (int)a.topk, w);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;

  auto shift_of = [](int64_t K, int64_t G) {
    const int64_t cpg = G == 1 ? 0 : (K / G) / 128;
    int sh = 0;
    while (cpg > 1 && (1 << sh) < cpg) ++sh;
    return sh;
  };
  MoeGemm g1{};
  g1.w = w;
  g1.a = reinterpret_cast<const uint16_t *>(a.x), g1.lda = (int)a.H, g1.a_rows = (int)a.T;
  g1.topk = (int)a.topk, g1.K = (int)a.H, g1.N = (int)(2 * a.I), g1.I = (int)a.I;
  g1.w_packed = a.w13, g1.scales = a.s13, g1.G = (int)a.G13;
  g1.cpg_shift = shift_of(a.H, a.G13), g1.gmask = a.G13 == 1 ? 0 : 0x7fffffff;
  g1.bias = a.b13, g1.act = a.act;
  g1.out = w.h1, g1.ldo = (int)a.I, g1.mt_max = mt_max;
  int bn1, bn2;
  moe_tile_widths(bn1, bn2);
  err = bn1 == 256 ? launch_moe_gemm<true, 256>(g1, s) : launch_moe_gemm<true, 128>(g1, s);
  if (err != hipSuccess) return err;

  MoeGemm g2 = g1;
  g2.a = w.h1, g2.lda = (int)a.I, g2.a_rows = P;
  g2.K = (int)a.I, g2.N = (int)a.H, g2.I = 0;
  g2.w_packed = a.w2, g2.scales = a.s2, g2.G = (int)a.G2;
  g2.cpg_shift = shift_of(a.I, a.G2), g2.gmask = a.G2 == 1 ? 0 : 0x7fffffff;
  g2.bias = a.b2;
  g2.out = w.y, g2.ldo = (int)a.H;
  err = bn2 == 256 ? launch_moe_gemm<false, 256>(g2, s) : launch_moe_gemm<false, 128>(g2, s);
  if (err != hipSuccess) return err;

  moe_combine_kernel<<<dim3((unsigned)a.T), dim3(256), 0, s>>>(
      w.y, (int)a.H, w.pair_pos, a.wts, a.wts_dt, (int)a.topk, a.skip_weighted, a.out);
  return hipGetLastError();
}

}  // namespace zt
