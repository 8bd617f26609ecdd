// Host-side launch interface shared by the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "zt_common.hpp"

namespace zt {

struct WoqArgs {
  const void *x;
  int x_dt;
  int64_t M, K, ldx;
  const uint32_t *w;  // [N, K/8]
  int64_t N;
  const void *scales;
  int s_dt;
  int64_t G;
  const void *zp;
  int zp_dt;
  const void *bias;
  int b_dt;
  PostOps post;
  void *y;
  int y_dt;
  int64_t ldy;
};

// Shape of a decode (M <= 32) launch: S K splits (grid.y); NT x NK waves
// per workgroup, wave (ti, ki) covering TPW 16-row tiles over CPW 128-wide
// K chunks; nrb row blocks of NT*TPW tiles (grid.x).
struct DecodePlan {
  int mt;  // 16-token tiles (1 or 2)
  int S, NK, NT, CPW, TPW;
  int nrb;
  int xl;  // activations held in registers for the whole slice (1) or
           // prefetched per item (0)
  int ni;  // items per wave
  int xs;  // activation slice staged through wave-private LDS (M <= 8)
};

enum WoqKernelKind { kWoqGeneric = 0, kWoqDecode = 1, kWoqGemm = 2 };

WoqKernelKind woq_select_kernel(const WoqArgs &a);
bool woq_decode_plan(int64_t M, int64_t N, int64_t K, DecodePlan *plan);
size_t woq_decode_workspace(const DecodePlan &p, int64_t M, int64_t N);

hipError_t launch_woq_generic(const WoqArgs &a, hipStream_t s);
hipError_t launch_woq_decode(const WoqArgs &a, const DecodePlan &p,
                             void *workspace, hipStream_t s);
hipError_t launch_woq_gemm(const WoqArgs &a, hipStream_t s);
// With a workspace of woq_gemm_workspace(M, N, K) bytes the prefill GEMM
// splits K when its tiles make less than a round (woq_gemm_splits > 1);
// with less it runs unsplit.
hipError_t launch_woq_gemm(const WoqArgs &a, hipStream_t s, void *workspace,
                           size_t workspace_bytes);
int woq_gemm_splits(int64_t M, int64_t N, int64_t K);
size_t woq_gemm_workspace(int64_t M, int64_t N, int64_t K);
// The weight-streaming decode kernel for up to 64 rows, when it applies
// (returns false otherwise; *err holds the launch status when it does).
bool woq_try_stream(const WoqArgs &a, hipStream_t s, hipError_t *err);
// merged gate_up (weight rows [0, N/2) gate, [N/2, N) up): y = silu(gate) * up
bool woq_try_stream_gate_up(const WoqArgs &a, hipStream_t s, hipError_t *err);
hipError_t launch_silu_mul_halves(const float *h, int64_t ld_h, int64_t M, int64_t I, void *y,
                                  int y_dt, int64_t ldy, hipStream_t s);
// 17..64 rows: the wide weight-streaming kernel (bf16 x and scales, no
// zero points), K split over `splits` workgroups per row block whose fp32
// partials take woq_wide_workspace bytes of workspace.
struct WidePlan {
  int mt;      // 32-token tiles (1 or 2)
  int splits;  // K splits
  int pps;     // 256-k phases per split
  bool pad;    // pps not a multiple of 4: the padded kernel form
};
bool woq_wide_plan(int64_t M, int64_t N, int64_t K, int64_t G, WidePlan *p);
size_t woq_wide_workspace(const WidePlan &p, int64_t M, int64_t N);
bool woq_wide_ok(const WoqArgs &a, WidePlan *p);
hipError_t launch_woq_wide(const WoqArgs &a, const WidePlan &p, void *workspace, hipStream_t s);
// merged gate_up on the wide kernel (no K split, N % 128 == 0)
bool woq_try_wide_gate_up(const WoqArgs &a, hipStream_t s, hipError_t *err);

hipError_t launch_repack(const int8_t *w, int64_t N, int64_t K, int32_t *out,
                         hipStream_t s);
hipError_t launch_repack_from_int4pack(const uint8_t *packed, int64_t N,
                                       int64_t K, int32_t *out, hipStream_t s);

struct DynArgs {
  const void *x;
  int x_dt;
  int64_t M, K;
  const int8_t *w;  // [N, K]
  int64_t N;
  const void *sw;
  int sw_dt;
  const void *bias;
  int b_dt;
  PostOps post;
  void *y;
  int y_dt;  // ZT_DT_S32 writes the raw accumulators
  const int8_t *qx;  // [M, K] quantised activations (row-major unless qx_frag)
  const float *sx;   // [M]
  int qx_frag;       // qx in the 32-token fragment order of s8_skinny32_kernel
  // asymmetric activations: qx holds q_u8 - 128 and the accumulator of
  // (m, n) is corrected by - azp[m] * colsum[n] (azp[m] = zp_u8[m] - 128,
  // colsum[n] = sum_k w[n][k]); both null for symmetric s8
  const int32_t *azp;     // [M]
  const int32_t *colsum;  // [N]
  int sw_bcast;           // one weight scale for every column (sw[0])
  // y_dt ZT_DT_U8 / ZT_DT_S8: requantised output clamp(rint(v * (1 / *out_scale))
  // + *out_zp) (out_zp null = 0)
  const float *out_scale;
  const int32_t *out_zp;
  // split-K exchange of s8_splitk_kernel (both null: not used): int32
  // partials of both K halves of every tile, then one counter per tile that
  // the quantise kernel of the same call clears.  Past 128 tokens,
  // split_part with gemm_splits > 1 holds the tiled GEMM's int32 partials
  // [gemm_splits][M][N] instead (no counters).
  int32_t *split_part;
  int32_t *split_cnt;
  int gemm_splits;
};

// frag: write qx in the fragment order (K % 64 == 0; the buffer holds
// ceil(M / 32) * 32 rows)
// azp non-null: per-token asymmetric uint8 (qx = q_u8 - 128, azp = zp - 128)
// zero[0, nzero): the split-K tile counters, cleared by the same launch
hipError_t launch_dyn_quantize(const void *x, int x_dt, int64_t M, int64_t K,
                               int8_t *qx, float *sx, bool frag, hipStream_t s,
                               int32_t *azp = nullptr, int32_t *zero = nullptr, int nzero = 0);
// Static per-tensor quantisation of zentorch_qlinear's activations into qx
// (fragment order when frag), with sx[m] = *scale and, when azp is set,
// azp[m] = the offset o with q - zp = qx - o (see static_quantize_kernel).
hipError_t launch_static_quantize(const void *x, int x_dt, int64_t M, int64_t K, int8_t *qx,
                                  bool frag, const float *scale, const int32_t *zp, float *sx,
                                  int32_t *azp, hipStream_t s, int32_t *zero = nullptr,
                                  int nzero = 0);
// colsum[n] = sum_k w[n][k] of an int8 [N, K] weight
hipError_t launch_s8_colsum(const int8_t *w, int64_t N, int64_t K, int32_t *colsum,
                            hipStream_t s);
// whether launch_s8_gemm takes qx in fragment order for this call (a.qx set)
bool s8_frag_ok(const DynArgs &a);
// Workspace bytes of the split-K exchange for an [M, K] x [N, K] call whose
// shape s8_splitk_kernel takes (0 otherwise), and its tile-counter count;
// the counters follow split_bytes - 4 * counters bytes of partials.
size_t s8_split_bytes(int64_t M, int64_t K, int64_t N);
// K splits of the tiled int8 GEMM past 128 tokens when its 128 x 128 tiles
// make less than one round (1 = none)
int s8_ws_splits(int64_t M, int64_t N, int64_t K);
int s8_split_counters(int64_t N);
hipError_t launch_s8_gemm(const DynArgs &a, hipStream_t s);
// The 16-token skinny GEMM with the per-token quantisation in its prologue
// (symmetric s8, bf16 x): whether it takes this call (a.qx and a.sx unused),
// its LDS bytes, and its launch, which replaces launch_dyn_quantize +
// launch_s8_gemm.
bool s8_fused_ok(const DynArgs &a);
size_t s8_fused_lds(int64_t M, int64_t K, int tpw);
hipError_t launch_s8_skinny_fused(const DynArgs &a, hipStream_t s);

// Grouped int4 MoE (moe_kernels.hip).  Device scratch of one call.
struct MoeWork {
  int32_t *pair_token;  // [P] token of the pair at each row of the expert order
  int32_t *pair_pos;    // [P] row of each pair in that order, -1 if dropped
  int32_t *expert_off;  // [E + 1]
  int32_t *mt_info;     // [tiles][4] per grouped-GEMM row tile: expert, first
                        // row, end row (its expert's end or first + BM), 0
  int32_t *num_mt;      // [1] tiles in use
  uint16_t *h1;         // [P, I] bf16 activated intermediate
  uint16_t *y;          // [P, H] bf16 expert outputs
};

struct MoeArgs {
  const void *x;  // [T, H] bf16
  int64_t T, H, topk, E, I;
  const int32_t *ids;  // [T, topk]
  const void *wts;     // [T, topk] bf16 or fp32
  int wts_dt;
  bool skip_weighted;
  int act;  // ZT_PO_SILU, ZT_PO_GELU_ERF or ZT_PO_GELU_TANH on the gate half
  const uint32_t *w13;  // [E, 2I, H/8] packed int4
  const uint16_t *s13;  // [E, G13, 2I] bf16
  const uint16_t *b13;  // [E, 2I] bf16 or null
  int64_t G13;
  const uint32_t *w2;   // [E, H, I/8]
  const uint16_t *s2;   // [E, G2, H] bf16
  const uint16_t *b2;   // [E, H] bf16 or null
  int64_t G2;
  uint16_t *out;        // [T, H] bf16
};

struct MoeGemm {
  MoeWork w;
  const uint16_t *a;  // A rows (gathered through pair_token when gated)
  int lda, a_rows, topk, K, N, I;
  const uint32_t *w_packed;
  const uint16_t *scales;
  int G, cpg_shift, gmask;
  const uint16_t *bias;
  int act;
  uint16_t *out;
  int ldo, mt_max;
};

int moe_max_tiles(int64_t P, int64_t E);
hipError_t launch_woq_moe(const MoeArgs &a, const MoeWork &w, hipStream_t s);

}  // namespace zt
