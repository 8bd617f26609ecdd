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
  const int8_t *qx;  // [M, K] quantised activations
  const float *sx;   // [M]
};

hipError_t launch_dyn_quantize(const void *x, int x_dt, int64_t M, int64_t K,
                               int8_t *qx, float *sx, hipStream_t s);
hipError_t launch_s8_gemm(const DynArgs &a, hipStream_t s);

}  // namespace zt
