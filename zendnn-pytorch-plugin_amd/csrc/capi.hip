// extern "C" entry points of libzentorch_hip.so (declared in
// include/zentorch_hip.h): argument validation, kernel choice, launch.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include <algorithm>

#include "zt_launch.hpp"
#include "zt_tuning.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return ZT_OK;
  return fail(ZT_EHIP, "%s: HIP error %d (%s)", what, (int)e,
              hipGetErrorString(e));
}

bool is_float_dt(int dt) { return dt == ZT_DT_F32 || dt == ZT_DT_BF16; }

int convert_post_ops(const zt_post_ops *in, zt::PostOps *out, const char *op) {
  std::memset(out, 0, sizeof(*out));
  if (!in) return ZT_OK;
  if (in->count < 0 || in->count > ZT_MAX_POST_OPS)
    return fail(ZT_EINVAL, "%s: post-op count %d outside [0, %d]", op,
                (int)in->count, ZT_MAX_POST_OPS);
  int nbuf = 0;
  out->count = in->count;
  for (int i = 0; i < in->count; ++i) {
    const int id = in->ids[i];
    if (id < ZT_PO_NONE || id > ZT_PO_ADD)
      return fail(ZT_EINVAL, "%s: unknown post-op id %d", op, id);
    out->ids[i] = id;
    if (id == ZT_PO_ADD || id == ZT_PO_MUL) {
      if (!in->bufs[nbuf])
        return fail(ZT_EINVAL, "%s: binary post-op %d has no buffer", op, i);
      if (!is_float_dt(in->buf_dtypes[nbuf]))
        return fail(ZT_EINVAL, "%s: post-op buffer %d must be bf16 or fp32", op,
                    nbuf);
      out->bufs[nbuf] = in->bufs[nbuf];
      out->dts[nbuf] = in->buf_dtypes[nbuf];
      out->ld[nbuf] = in->buf_ld[nbuf];
      ++nbuf;
    }
  }
  return ZT_OK;
}

size_t float_dt_bytes(int dt) { return dt == ZT_DT_F32 ? 4 : 2; }

// 17..64 rows of a decode-sized call: one stream-kernel launch over all
// rows when x fits (in K phases), else blocks of 16 rows on the decode
// kernels.  Each block streams the weights again, which still beats one
// prefill-GEMM launch of so few row tiles (it cannot fill the GPU).  x, y
// and the binary post-op buffers are offset to the block's first row.
constexpr int64_t kWoqRowBlock = 16, kWoqRowBlockMax = 64;

bool woq_use_row_blocks(const zt::WoqArgs &a) {
  if (a.M <= kWoqRowBlock || a.M > kWoqRowBlockMax) return false;
  zt::WoqArgs b = a;
  b.M = kWoqRowBlock;
  zt::DecodePlan p;
  return zt::woq_select_kernel(b) == zt::kWoqDecode &&
         zt::woq_decode_plan(b.M, b.N, b.K, &p) && zt::woq_decode_workspace(p, b.M, b.N) == 0;
}

hipError_t woq_row_blocks(const zt::WoqArgs &a, hipStream_t s) {
  for (int64_t m0 = 0; m0 < a.M; m0 += kWoqRowBlock) {
    zt::WoqArgs b = a;
    b.M = std::min(kWoqRowBlock, a.M - m0);
    b.x = static_cast<const char *>(a.x) + m0 * a.ldx * float_dt_bytes(a.x_dt);
    b.y = static_cast<char *>(a.y) + m0 * a.ldy * float_dt_bytes(a.y_dt);
    for (int i = 0; i < ZT_MAX_POST_OPS; ++i)
      if (b.post.bufs[i])
        b.post.bufs[i] = static_cast<const char *>(b.post.bufs[i]) +
                         m0 * b.post.ld[i] * float_dt_bytes(b.post.dts[i]);
    zt::DecodePlan p;
    if (!zt::woq_decode_plan(b.M, b.N, b.K, &p)) return hipErrorInvalidValue;
    const hipError_t err = zt::launch_woq_decode(b, p, nullptr, s);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace

// ------------------------------------------------------------ tuning knobs
namespace zt {
namespace {

constexpr const char *kKnobNames[kKnobCount] = {
    "ZT_WOQ_FORCE_KERNEL", "ZT_WOQ_DECODE_PLAN", "ZT_WOQ_STREAM", "ZT_WOQ_WIDE",
    "ZT_WOQ_GEMM",         "ZT_WOQ_DEBUG",       "ZT_WOQ_WAVE",    "ZT_WOQ_PERSIST",
    "ZT_S8_SKINNY32",      "ZT_S8_SKINNY",
    "ZT_S8_FRAG",          "ZT_S8_FORCE",        "ZT_S8_TILE",     "ZT_S8_KIND",
    "ZT_S8_SPLIT",         "ZT_MOE_BN",          "ZT_WOQ_LEAN",    "ZT_S8_FUSED"};

// Values are interned copies that are never freed: a reader may hold an old
// pointer while another thread replaces the value.
std::atomic<const char *> g_knobs[kKnobCount];

const char *intern(const char *v) {
  if (!v || !*v) return nullptr;
  static std::mutex mu;
  static std::vector<std::unique_ptr<std::string>> pool;
  std::lock_guard<std::mutex> g(mu);
  pool.emplace_back(new std::string(v));
  return pool.back()->c_str();
}

// Reads the environment once, when the library is loaded.
struct KnobsFromEnv {
  KnobsFromEnv() {
    for (int i = 0; i < kKnobCount; ++i)
      g_knobs[i].store(intern(std::getenv(kKnobNames[i])), std::memory_order_release);
  }
} g_knobs_from_env;

}  // namespace

const char *knob(Knob k) { return g_knobs[k].load(std::memory_order_acquire); }

}  // namespace zt

extern "C" {

const char *zt_last_error_string(void) { return g_last_error.c_str(); }

int zt_set_tuning(const char *name, const char *value) {
  if (!name) return fail(ZT_EINVAL, "zt_set_tuning: null name");
  for (int i = 0; i < zt::kKnobCount; ++i)
    if (!std::strcmp(name, zt::kKnobNames[i])) {
      zt::g_knobs[i].store(zt::intern(value), std::memory_order_release);
      return ZT_OK;
    }
  return fail(ZT_EINVAL, "zt_set_tuning: unknown knob '%s'", name);
}

const char *zt_get_tuning(const char *name) {
  if (!name) return nullptr;
  for (int i = 0; i < zt::kKnobCount; ++i)
    if (!std::strcmp(name, zt::kKnobNames[i])) return zt::knob(static_cast<zt::Knob>(i));
  return nullptr;
}

}  // extern "C"

namespace {

// Byte layout of the MoE workspace (every region 256-byte aligned).
struct MoeLayout {
  size_t pair_token, pair_pos, expert_off, mt_info, num_mt, h1, y, total;
};

MoeLayout moe_layout(int64_t T, int64_t H, int64_t topk, int64_t E, int64_t I) {
  const int64_t P = T * topk;
  const int64_t tiles = zt::moe_max_tiles(P, E);
  MoeLayout l{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) / 256 * 256;
    return at;
  };
  l.pair_token = take(P * 4);
  l.pair_pos = take(P * 4);
  l.expert_off = take((E + 1) * 4);
  l.mt_info = take(tiles * 16);
  l.num_mt = take(4);
  l.h1 = take((size_t)P * I * 2);
  l.y = take((size_t)P * H * 2);
  l.total = off;
  return l;
}

}  // namespace

extern "C" {

size_t zt_woq_moe_workspace_size(int64_t T, int64_t H, int64_t topk, int64_t E, int64_t I) {
  if (T <= 0 || H <= 0 || topk <= 0 || E <= 0 || I <= 0) return 0;
  return moe_layout(T, H, topk, E, I).total;
}

int zt_woq_moe(const void *x, int64_t T, int64_t H, const int32_t *topk_ids,
               const void *topk_weights, int32_t weights_dtype, int64_t topk,
               int32_t skip_weighted, int32_t act, const int32_t *w13,
               const void *w13_scales, int64_t G13, const void *w13_bias,
               const int32_t *w2, const void *w2_scales, int64_t G2,
               const void *w2_bias, int64_t E, int64_t I, void *out,
               void *workspace, size_t workspace_bytes, zt_stream_t stream) {
  static const char *op = "zt_woq_moe";
  if (T < 0 || H <= 0 || I <= 0 || topk <= 0 || E <= 0)
    return fail(ZT_EINVAL, "%s: need T >= 0 and H, I, topk, E > 0", op);
  if (H % 128 || I % 128)
    return fail(ZT_EINVAL, "%s: H=%lld and I=%lld must be multiples of 128", op,
                (long long)H, (long long)I);
  if (E > 1024) return fail(ZT_EUNSUPPORTED, "%s: at most 1024 experts (E=%lld)", op, (long long)E);
  auto groups_ok = [](int64_t K, int64_t G) {
    if (G < 1 || K % G) return false;
    if (G == 1) return true;
    const int64_t gs = K / G, c = gs / 128;
    return gs % 128 == 0 && (c & (c - 1)) == 0;
  };
  if (!groups_ok(H, G13) || !groups_ok(I, G2))
    return fail(ZT_EINVAL, "%s: scale groups must be one group or a power of two times 128 "
                "columns (H=%lld G13=%lld, I=%lld G2=%lld)", op, (long long)H, (long long)G13,
                (long long)I, (long long)G2);
  if (!is_float_dt(weights_dtype))
    return fail(ZT_EINVAL, "%s: topk_weights must be fp32 or bf16", op);
  if (act != ZT_PO_SILU && act != ZT_PO_GELU_ERF && act != ZT_PO_GELU_TANH)
    return fail(ZT_EUNSUPPORTED, "%s: act must be silu, gelu or gelu_tanh", op);
  const int64_t P = T * topk;
  if (P * std::max(H, I) * 2 >= (int64_t)zt::kOobOffset || 2 * I * (H / 8) * 4 >= (int64_t)zt::kOobOffset ||
      H * (I / 8) * 4 >= (int64_t)zt::kOobOffset)
    return fail(ZT_EUNSUPPORTED, "%s: operands exceed 32-bit offsets", op);
  if (T == 0) return ZT_OK;
  if (!x || !topk_ids || !topk_weights || !w13 || !w13_scales || !w2 || !w2_scales || !out)
    return fail(ZT_EINVAL, "%s: null tensor pointer", op);
  const MoeLayout l = moe_layout(T, H, topk, E, I);
  if (!workspace || workspace_bytes < l.total)
    return fail(ZT_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op, l.total,
                workspace ? workspace_bytes : (size_t)0);
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  zt::MoeWork w{};
  w.pair_token = reinterpret_cast<int32_t *>(ws + l.pair_token);
  w.pair_pos = reinterpret_cast<int32_t *>(ws + l.pair_pos);
  w.expert_off = reinterpret_cast<int32_t *>(ws + l.expert_off);
  w.mt_info = reinterpret_cast<int32_t *>(ws + l.mt_info);
  w.num_mt = reinterpret_cast<int32_t *>(ws + l.num_mt);
  w.h1 = reinterpret_cast<uint16_t *>(ws + l.h1);
  w.y = reinterpret_cast<uint16_t *>(ws + l.y);
  zt::MoeArgs a{};
  a.x = x, a.T = T, a.H = H, a.topk = topk, a.E = E, a.I = I;
  a.ids = topk_ids, a.wts = topk_weights, a.wts_dt = weights_dtype;
  a.skip_weighted = skip_weighted != 0, a.act = act;
  a.w13 = reinterpret_cast<const uint32_t *>(w13);
  a.s13 = static_cast<const uint16_t *>(w13_scales), a.G13 = G13;
  a.b13 = static_cast<const uint16_t *>(w13_bias);
  a.w2 = reinterpret_cast<const uint32_t *>(w2);
  a.s2 = static_cast<const uint16_t *>(w2_scales), a.G2 = G2;
  a.b2 = static_cast<const uint16_t *>(w2_bias);
  a.out = static_cast<uint16_t *>(out);
  return hip_status(zt::launch_woq_moe(a, w, reinterpret_cast<hipStream_t>(stream)), op);
}

int32_t zt_version(void) { return 100; }

size_t zt_woq_linear_workspace_size(int64_t M, int64_t K, int64_t N,
                                    int64_t G) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0 || K % G) return 0;
  // the wide kernel's K-split partials (17..64 rows)
  zt::WidePlan wp;
  const size_t wide = zt::woq_wide_plan(M, N, K, G, &wp) ? zt::woq_wide_workspace(wp, M, N) : 0;
  zt::WoqArgs a{};
  a.x_dt = ZT_DT_BF16;
  a.M = M, a.K = K, a.N = N, a.G = G, a.ldx = K;
  // Assume aligned pointers: the workspace a call needs is never larger.
  a.x = reinterpret_cast<const void *>(256);
  a.w = reinterpret_cast<const uint32_t *>(256);
  // the prefill GEMM's K-split partials (few tiles)
  const size_t gemm = zt::woq_gemm_workspace(M, N, K);
  if (zt::woq_select_kernel(a) != zt::kWoqDecode) return std::max(wide, gemm);
  zt::DecodePlan p;
  if (!zt::woq_decode_plan(M, N, K, &p)) return std::max(wide, gemm);
  return std::max(wide, zt::woq_decode_workspace(p, M, N));
}

// Argument checks shared by zt_woq_linear and zt_woq_linear_gate_up (ZT_OK
// or the error code, with the message set); y_cols is the output width.
static int check_woq_args(const char *op, const void *x, int32_t x_dtype, int64_t M,
                          int64_t K, int64_t ldx, const int32_t *w_packed, int64_t N,
                          const void *scales, int32_t scales_dtype, int64_t G, const void *zp,
                          int32_t zp_dtype, const void *bias, int32_t bias_dtype, void *y,
                          int32_t y_dtype, int64_t ldy, int64_t y_cols) {
  if (M < 0 || N < 0 || K < 8 || K % 8)
    return fail(ZT_EINVAL, "%s: need M,N >= 0 and K >= 8 with K %% 8 == 0 "
                "(M=%lld N=%lld K=%lld)", op, (long long)M, (long long)N,
                (long long)K);
  if (G < 1 || K % G)
    return fail(ZT_EINVAL, "%s: scale groups G=%lld must divide K=%lld", op,
                (long long)G, (long long)K);
  if (!is_float_dt(x_dtype) || !is_float_dt(y_dtype) || !is_float_dt(scales_dtype))
    return fail(ZT_EINVAL, "%s: input, output and scales must be bf16 or fp32", op);
  if (zp && !(is_float_dt(zp_dtype) || zp_dtype == ZT_DT_S8 ||
              zp_dtype == ZT_DT_U8 || zp_dtype == ZT_DT_S32))
    return fail(ZT_EINVAL, "%s: zero points must be bf16, fp32, int8, uint8 or int32", op);
  if (bias && !is_float_dt(bias_dtype))
    return fail(ZT_EINVAL, "%s: bias must be bf16 or fp32", op);
  if (ldx < K || ldy < y_cols)
    return fail(ZT_EINVAL, "%s: leading dimensions too small", op);
  if (M > 0 && N > 0 && (!x || !w_packed || !scales || !y))
    return fail(ZT_EINVAL, "%s: null tensor pointer", op);
  return ZT_OK;
}

int zt_woq_linear(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                  int64_t ldx, const int32_t *w_packed, int64_t N,
                  const void *scales, int32_t scales_dtype, int64_t G,
                  const void *zp, int32_t zp_dtype, const void *bias,
                  int32_t bias_dtype, const zt_post_ops *post, void *y,
                  int32_t y_dtype, int64_t ldy, void *workspace,
                  size_t workspace_bytes, zt_stream_t stream) {
  static const char *op = "zt_woq_linear";
  int rc0 = check_woq_args(op, x, x_dtype, M, K, ldx, w_packed, N, scales, scales_dtype, G, zp,
                           zp_dtype, bias, bias_dtype, y, y_dtype, ldy, N);
  if (rc0) return rc0;
  if (M == 0 || N == 0) return ZT_OK;

  zt::WoqArgs a{};
  a.x = x, a.x_dt = x_dtype, a.M = M, a.K = K, a.ldx = ldx;
  a.w = reinterpret_cast<const uint32_t *>(w_packed), a.N = N;
  a.scales = scales, a.s_dt = scales_dtype, a.G = G;
  a.zp = zp, a.zp_dt = zp ? zp_dtype : ZT_DT_NONE;
  a.bias = bias, a.b_dt = bias ? bias_dtype : ZT_DT_NONE;
  a.y = y, a.y_dt = y_dtype, a.ldy = ldy;
  int rc = convert_post_ops(post, &a.post, op);
  if (rc) return rc;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  zt::WidePlan wp;
  if (zt::woq_wide_ok(a, &wp)) {
    const size_t need = zt::woq_wide_workspace(wp, M, N);
    if (need && (!workspace || workspace_bytes < need))
      return fail(ZT_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op, need,
                  workspace ? workspace_bytes : (size_t)0);
    return hip_status(zt::launch_woq_wide(a, wp, workspace, s), op);
  }
  if (woq_use_row_blocks(a)) {
    // one stream-kernel launch over all rows when x (in K phases) fits, else
    // blocks of 16 rows
    hipError_t err = hipSuccess;
    if (zt::woq_try_stream(a, s, &err)) return hip_status(err, op);
    return hip_status(woq_row_blocks(a, s), op);
  }
  switch (zt::woq_select_kernel(a)) {
  case zt::kWoqDecode: {
    zt::DecodePlan p;
    if (!zt::woq_decode_plan(M, N, K, &p)) {
      const int64_t gs = K / G;
      if (K % 64 == 0 && gs % 32 == 0)
        return hip_status(zt::launch_woq_gemm(a, s, workspace, workspace_bytes), op);
      return hip_status(zt::launch_woq_generic(a, s), op);
    }
    const size_t need = zt::woq_decode_workspace(p, M, N);
    if (need > 0 && (!workspace || workspace_bytes < need))
      return fail(ZT_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op,
                  need, workspace ? workspace_bytes : (size_t)0);
    return hip_status(zt::launch_woq_decode(a, p, workspace, s), op);
  }
  case zt::kWoqGemm:
    return hip_status(zt::launch_woq_gemm(a, s, workspace, workspace_bytes), op);
  default:
    return hip_status(zt::launch_woq_generic(a, s), op);
  }
}

size_t zt_woq_linear_gate_up_workspace_size(int64_t M, int64_t K, int64_t N,
                                            int64_t G) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0 || K % G) return 0;
  const size_t h = ((size_t)M * (size_t)N * sizeof(float) + 255) / 256 * 256;
  return h + zt_woq_linear_workspace_size(M, K, N, G);
}

int zt_woq_linear_gate_up(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                          int64_t ldx, const int32_t *w_packed, int64_t N,
                          const void *scales, int32_t scales_dtype, int64_t G,
                          const void *zp, int32_t zp_dtype, const void *bias,
                          int32_t bias_dtype, void *y, int32_t y_dtype, int64_t ldy,
                          void *workspace, size_t workspace_bytes, zt_stream_t stream) {
  static const char *op = "zt_woq_linear_gate_up";
  if (N % 2)
    return fail(ZT_EINVAL, "%s: N=%lld must be even (gate rows, then up rows)", op,
                (long long)N);
  int rc0 = check_woq_args(op, x, x_dtype, M, K, ldx, w_packed, N, scales, scales_dtype, G, zp,
                           zp_dtype, bias, bias_dtype, y, y_dtype, ldy, N / 2);
  if (rc0) return rc0;
  if (M == 0 || N == 0) return ZT_OK;
  zt::WoqArgs a{};
  a.x = x, a.x_dt = x_dtype, a.M = M, a.K = K, a.ldx = ldx;
  a.w = reinterpret_cast<const uint32_t *>(w_packed), a.N = N;
  a.scales = scales, a.s_dt = scales_dtype, a.G = G;
  a.zp = zp, a.zp_dt = zp ? zp_dtype : ZT_DT_NONE;
  a.bias = bias, a.b_dt = bias ? bias_dtype : ZT_DT_NONE;
  a.y = y, a.y_dt = y_dtype, a.ldy = ldy;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = hipSuccess;
  if (zt::woq_try_stream_gate_up(a, s, &err)) return hip_status(err, op);
  if (zt::woq_try_wide_gate_up(a, s, &err)) return hip_status(err, op);
  // two steps: the full [M, N] linear in fp32 into the workspace, then
  // silu(gate) * up over its halves
  const size_t h = ((size_t)M * (size_t)N * sizeof(float) + 255) / 256 * 256;
  if (!workspace || workspace_bytes < h)
    return fail(ZT_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op,
                zt_woq_linear_gate_up_workspace_size(M, K, N, G),
                workspace ? workspace_bytes : (size_t)0);
  float *hbuf = static_cast<float *>(workspace);
  int rc = zt_woq_linear(x, x_dtype, M, K, ldx, w_packed, N, scales, scales_dtype, G, zp,
                         zp_dtype, bias, bias_dtype, nullptr, hbuf, ZT_DT_F32, N,
                         static_cast<unsigned char *>(workspace) + h, workspace_bytes - h,
                         stream);
  if (rc) return rc;
  return hip_status(zt::launch_silu_mul_halves(hbuf, N, M, N / 2, y, y_dtype, ldy, s), op);
}

// qx region of the dynamic-qlinear workspace: whole 32-row tiles (the
// fragment order of the skinny int8 kernel), rounded to 256 bytes
static size_t dyn_qx_bytes(int64_t M, int64_t K) {
  return ((size_t)((M + 31) / 32 * 32) * (size_t)K + 255) & ~(size_t)255;
}

// Bytes of qx, the row scales and (asym) the row offsets, rounded to 256:
// the least workspace a dynamic or static qlinear call takes.  The split-K
// exchange of the skinny int8 GEMM (zt::s8_split_bytes) follows it; a call
// whose workspace has no room for it runs the unsplit kernel.
static size_t dyn_base_bytes(int64_t M, int64_t K, bool asym) {
  return (dyn_qx_bytes(M, K) + (size_t)M * 4 * (asym ? 2 : 1) + 255) & ~(size_t)255;
}

size_t zt_dynamic_qlinear_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0) return 0;
  return dyn_base_bytes(M, K, false) + zt::s8_split_bytes(M, K, N);
}

// Points a at the split-K exchange when the workspace holds it; returns the
// tile-counter count the quantise kernel must clear (0: no split).
// Past 128 tokens the same room holds the tiled GEMM's K-split partials
// (gemm_splits > 1, no counters).
static int attach_split(zt::DynArgs &a, char *ws, size_t ws_bytes, size_t base) {
  const size_t sb = zt::s8_split_bytes(a.M, a.K, a.N);
  if (!sb || ws_bytes < base + sb) return 0;
  if (a.M > 128) {
    a.split_part = reinterpret_cast<int32_t *>(ws + base);
    a.gemm_splits = zt::s8_ws_splits(a.M, a.N, a.K);
    return 0;
  }
  const int nc = zt::s8_split_counters(a.N);
  a.split_part = reinterpret_cast<int32_t *>(ws + base);
  a.split_cnt = reinterpret_cast<int32_t *>(ws + base + sb - (((size_t)nc * 4 + 255) & ~(size_t)255));
  return nc;
}

int zt_dynamic_quantize(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                        int8_t *qx, float *sx, zt_stream_t stream) {
  static const char *op = "zt_dynamic_quantize";
  if (!is_float_dt(x_dtype))
    return fail(ZT_EINVAL, "%s: input must be bf16 or fp32", op);
  if (M < 0 || K < 1) return fail(ZT_EINVAL, "%s: need M >= 0, K >= 1", op);
  if (M == 0) return ZT_OK;
  if (!x || !qx || !sx) return fail(ZT_EINVAL, "%s: null pointer", op);
  return hip_status(zt::launch_dyn_quantize(x, x_dtype, M, K, qx, sx, false,
                                            reinterpret_cast<hipStream_t>(stream)),
                    op);
}

int zt_s8s8s32_gemm(const int8_t *qa, const int8_t *w, int64_t M, int64_t N,
                    int64_t K, int32_t *acc, zt_stream_t stream) {
  static const char *op = "zt_s8s8s32_gemm";
  if (M < 0 || N < 0 || K < 1) return fail(ZT_EINVAL, "%s: bad sizes", op);
  if (M == 0 || N == 0) return ZT_OK;
  if (!qa || !w || !acc) return fail(ZT_EINVAL, "%s: null pointer", op);
  zt::DynArgs a{};
  a.M = M, a.N = N, a.K = K, a.w = w, a.qx = qa;
  a.y = acc, a.y_dt = ZT_DT_S32;
  return hip_status(zt::launch_s8_gemm(a, reinterpret_cast<hipStream_t>(stream)), op);
}

// The dynamic qlinear of both quantisation schemes: symmetric s8 when
// colsum is null, per-token asymmetric u8 otherwise (the azp row offsets
// then follow sx in the workspace).
static int dynamic_qlinear_common(const char *op, const void *x, int32_t x_dtype, int64_t M,
                                  int64_t K, const int8_t *w, int64_t N, const void *w_scales,
                                  int32_t w_scales_dtype, const int32_t *colsum,
                                  const void *bias, int32_t bias_dtype, const zt_post_ops *post,
                                  void *y, int32_t y_dtype, void *workspace,
                                  size_t workspace_bytes, zt_stream_t stream) {
  const bool asym = colsum != nullptr;
  if (!is_float_dt(x_dtype) || !(is_float_dt(y_dtype) || (asym && y_dtype == ZT_DT_S32)))
    return fail(ZT_EINVAL, "%s: input and output must be bf16 or fp32", op);
  if (!is_float_dt(w_scales_dtype))
    return fail(ZT_EINVAL, "%s: weight_scales must be float32 or bfloat16", op);
  if (bias && !is_float_dt(bias_dtype))
    return fail(ZT_EINVAL, "%s: bias must be float32 or bfloat16", op);
  if (M < 0 || N < 0 || K < 1) return fail(ZT_EINVAL, "%s: bad sizes", op);
  if (M == 0 || N == 0) return ZT_OK;
  if (!x || !w || !w_scales || !y) return fail(ZT_EINVAL, "%s: null pointer", op);
  if (asym && (reinterpret_cast<uintptr_t>(colsum) & 15u))
    return fail(ZT_EINVAL, "%s: weight_colsum must be 16-byte aligned", op);
  const size_t need = dyn_base_bytes(M, K, asym);
  if (!workspace || workspace_bytes < need)
    return fail(ZT_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op,
                need, workspace ? workspace_bytes : (size_t)0);
  zt::DynArgs a{};
  a.x = x, a.x_dt = x_dtype, a.M = M, a.K = K, a.w = w, a.N = N;
  a.sw = w_scales, a.sw_dt = w_scales_dtype;
  a.bias = bias, a.b_dt = bias ? bias_dtype : ZT_DT_NONE;
  a.y = y, a.y_dt = y_dtype;
  int rc = convert_post_ops(post, &a.post, op);
  if (rc) return rc;
  char *ws = reinterpret_cast<char *>(workspace);
  int8_t *qx = reinterpret_cast<int8_t *>(ws);
  float *sx = reinterpret_cast<float *>(ws + dyn_qx_bytes(M, K));
  int32_t *azp = asym ? reinterpret_cast<int32_t *>(ws + dyn_qx_bytes(M, K) + M * 4) : nullptr;
  a.qx = qx, a.sx = sx, a.azp = azp, a.colsum = colsum;
  a.qx_frag = zt::s8_frag_ok(a) ? 1 : 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // few tokens: one launch that quantises x in the GEMM's prologue
  if (zt::s8_fused_ok(a)) return hip_status(zt::launch_s8_skinny_fused(a, s), op);
  const int nc = a.qx_frag || a.M > 128 ? attach_split(a, ws, workspace_bytes, need) : 0;
  rc = hip_status(zt::launch_dyn_quantize(x, x_dtype, M, K, qx, sx, a.qx_frag != 0, s, azp,
                                          a.split_cnt, nc),
                  op);
  if (rc) return rc;
  return hip_status(zt::launch_s8_gemm(a, s), op);
}

int zt_dynamic_qlinear(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                       const int8_t *w, int64_t N, const void *w_scales,
                       int32_t w_scales_dtype, const void *bias,
                       int32_t bias_dtype, const zt_post_ops *post, void *y,
                       int32_t y_dtype, void *workspace, size_t workspace_bytes,
                       zt_stream_t stream) {
  return dynamic_qlinear_common("zt_dynamic_qlinear", x, x_dtype, M, K, w, N, w_scales,
                                w_scales_dtype, nullptr, bias, bias_dtype, post, y, y_dtype,
                                workspace, workspace_bytes, stream);
}

size_t zt_qlinear_workspace_size(int64_t M, int64_t K, int64_t N) {
  return zt_dynamic_qlinear_asym_workspace_size(M, K, N);
}

int zt_qlinear(const void *x, int32_t x_dtype, int64_t M, int64_t K, const float *x_scale,
               const int32_t *x_zero_point, const int8_t *w, int64_t N, const float *w_scales,
               int64_t n_w_scales, const int32_t *w_colsum, const void *bias,
               int32_t bias_dtype, const zt_post_ops *post, void *y, int32_t y_dtype,
               const float *y_scale, const int32_t *y_zero_point, void *workspace,
               size_t workspace_bytes, zt_stream_t stream) {
  static const char *op = "zt_qlinear";
  if (!(is_float_dt(x_dtype) || x_dtype == ZT_DT_S8 || x_dtype == ZT_DT_U8))
    return fail(ZT_EINVAL, "%s: input must be float32, bfloat16, uint8 or int8", op);
  if (y_scale) {
    if (y_dtype != (y_zero_point ? ZT_DT_U8 : ZT_DT_S8))
      return fail(ZT_EINVAL,
                  "%s: a requantised output is uint8 with an output zero point, int8 without",
                  op);
  } else if (!is_float_dt(y_dtype)) {
    return fail(ZT_EINVAL, "%s: output must be float32 or bfloat16 without output scales", op);
  }
  if (bias && !is_float_dt(bias_dtype))
    return fail(ZT_EINVAL, "%s: bias must be float32 or bfloat16", op);
  if (M < 0 || N < 0 || K < 1) return fail(ZT_EINVAL, "%s: bad sizes", op);
  if (n_w_scales != 1 && n_w_scales != N)
    return fail(ZT_EINVAL, "%s: %lld weight scales for %lld output channels", op,
                (long long)n_w_scales, (long long)N);
  if (M == 0 || N == 0) return ZT_OK;
  if (!x || !x_scale || !w || !w_scales || !y) return fail(ZT_EINVAL, "%s: null pointer", op);
  // activations carry an offset (u8, or an s8 zero point): the epilogue
  // subtracts offset * colsum[n]
  const bool offset = x_dtype == ZT_DT_U8 || x_zero_point != nullptr;
  if (offset && !w_colsum)
    return fail(ZT_EINVAL, "%s: weight_colsum is required for uint8 / zero-point activations",
                op);
  if (offset && (reinterpret_cast<uintptr_t>(w_colsum) & 15u))
    return fail(ZT_EINVAL, "%s: weight_colsum must be 16-byte aligned", op);
  const size_t need = dyn_base_bytes(M, K, true);
  if (!workspace || workspace_bytes < need)
    return fail(ZT_EINVAL, "%s: workspace of %zu bytes needed, %zu given", op, need,
                workspace ? workspace_bytes : (size_t)0);
  zt::DynArgs a{};
  a.x = x, a.x_dt = x_dtype, a.M = M, a.K = K, a.w = w, a.N = N;
  a.sw = w_scales, a.sw_dt = ZT_DT_F32, a.sw_bcast = n_w_scales == 1 && N > 1;
  a.bias = bias, a.b_dt = bias ? bias_dtype : ZT_DT_NONE;
  a.y = y, a.y_dt = y_dtype, a.out_scale = y_scale, a.out_zp = y_zero_point;
  int rc = convert_post_ops(post, &a.post, op);
  if (rc) return rc;
  char *ws = reinterpret_cast<char *>(workspace);
  int8_t *qx = reinterpret_cast<int8_t *>(ws);
  float *sx = reinterpret_cast<float *>(ws + dyn_qx_bytes(M, K));
  int32_t *azp = offset ? reinterpret_cast<int32_t *>(ws + dyn_qx_bytes(M, K) + M * 4) : nullptr;
  a.qx = qx, a.sx = sx, a.azp = azp, a.colsum = offset ? w_colsum : nullptr;
  a.qx_frag = zt::s8_frag_ok(a) ? 1 : 0;
  const int nc = a.qx_frag || a.M > 128 ? attach_split(a, ws, workspace_bytes, need) : 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  rc = hip_status(zt::launch_static_quantize(x, x_dtype, M, K, qx, a.qx_frag != 0, x_scale,
                                             x_zero_point, sx, azp, s, a.split_cnt, nc),
                  op);
  if (rc) return rc;
  return hip_status(zt::launch_s8_gemm(a, s), op);
}

size_t zt_dynamic_qlinear_asym_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= 0 || K <= 0) return 0;
  return dyn_base_bytes(M, K, true) + zt::s8_split_bytes(M, K, N);
}

int zt_dynamic_quantize_asym(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                             int8_t *qx, float *sx, int32_t *azp, zt_stream_t stream) {
  static const char *op = "zt_dynamic_quantize_asym";
  if (!is_float_dt(x_dtype))
    return fail(ZT_EINVAL, "%s: input must be bf16 or fp32", op);
  if (M < 0 || K < 1) return fail(ZT_EINVAL, "%s: need M >= 0, K >= 1", op);
  if (M == 0) return ZT_OK;
  if (!x || !qx || !sx || !azp) return fail(ZT_EINVAL, "%s: null pointer", op);
  return hip_status(zt::launch_dyn_quantize(x, x_dtype, M, K, qx, sx, false,
                                            reinterpret_cast<hipStream_t>(stream), azp),
                    op);
}

int zt_s8_weight_colsum(const int8_t *w, int64_t N, int64_t K, int32_t *colsum,
                        zt_stream_t stream) {
  static const char *op = "zt_s8_weight_colsum";
  if (N < 0 || K < 1) return fail(ZT_EINVAL, "%s: bad sizes", op);
  if (N == 0) return ZT_OK;
  if (!w || !colsum) return fail(ZT_EINVAL, "%s: null pointer", op);
  return hip_status(zt::launch_s8_colsum(w, N, K, colsum, reinterpret_cast<hipStream_t>(stream)),
                    op);
}

int zt_dynamic_qlinear_asym(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                            const int8_t *w, int64_t N, const void *w_scales,
                            int32_t w_scales_dtype, const int32_t *w_colsum,
                            const void *bias, int32_t bias_dtype, const zt_post_ops *post,
                            void *y, int32_t y_dtype, void *workspace,
                            size_t workspace_bytes, zt_stream_t stream) {
  if (!w_colsum && M > 0 && N > 0)
    return fail(ZT_EINVAL, "zt_dynamic_qlinear_asym: null weight_colsum");
  return dynamic_qlinear_common("zt_dynamic_qlinear_asym", x, x_dtype, M, K, w, N, w_scales,
                                w_scales_dtype, w_colsum, bias, bias_dtype, post, y, y_dtype,
                                workspace, workspace_bytes, stream);
}

}  // extern "C"

// ------------------------------------------ allocation-free dynamic qlinear
// Scratch of zt_dynamic_qlinear_scratch: the quantised activations and row
// scales of one call, in a device array each GPU holds for the life of the
// process.  In host code `scratch` names a host-side stand-in, never the
// device memory: the device address comes from hipGetSymbolAddress, once
// per device (g_scratch_ptr), and only that address reaches a kernel.
static __device__ __align__(256) unsigned char scratch[ZT_DYN_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The array's address on device `dev`, which must be the current device.
int scratch_address(const char *op, int dev, void **out) {
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ZT_EHIP, "%s: device id %d out of range (at most %d devices)", op, dev,
                kMaxDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(ZT_EHIP, "%s: hipGetSymbolAddress(scratch) on device %d: HIP error %d (%s)",
                  op, dev, (int)e, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ZT_OK;
}

}  // namespace

extern "C" {

size_t zt_dynamic_qlinear_scratch_max(void) { return ZT_DYN_SCRATCH_BYTES; }

int zt_dynamic_qlinear_scratch(const void *x, int32_t x_dtype, int64_t M, int64_t K,
                               const int8_t *w, int64_t N, const void *w_scales,
                               int32_t w_scales_dtype, const void *bias, int32_t bias_dtype,
                               const zt_post_ops *post, void *y, int32_t y_dtype,
                               zt_stream_t stream) {
  static const char *op = "zt_dynamic_qlinear_scratch";
  if (M < 0 || N < 0 || K < 1) return fail(ZT_EINVAL, "%s: bad sizes", op);
  if (M == 0 || N == 0) return ZT_OK;
  const size_t need = dyn_base_bytes(M, K, false);
  if (need > (size_t)ZT_DYN_SCRATCH_BYTES)
    return fail(ZT_EINVAL, "%s: M=%lld x K=%lld needs %zu bytes of scratch, more than the "
                "%zu this entry point holds (use zt_dynamic_qlinear with a workspace)",
                op, (long long)M, (long long)K, need, (size_t)ZT_DYN_SCRATCH_BYTES);
  // the stream's device holds the array this call uses; it is made current
  // for the call (and the caller's current device restored) when it is not
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int cur = -1, dev = -1;
  if (hipGetDevice(&cur) != hipSuccess)
    return fail(ZT_EHIP, "%s: no current HIP device", op);
  if (s == nullptr) {
    dev = cur;
  } else if (hipStreamGetDevice(s, &dev) != hipSuccess) {
    return fail(ZT_EHIP, "%s: cannot query the stream's device", op);
  }
  if (dev != cur && hipSetDevice(dev) != hipSuccess)
    return fail(ZT_EHIP, "%s: cannot make the stream's device %d current", op, dev);
  void *ws = nullptr;
  int rc = scratch_address(op, dev, &ws);
  if (rc == ZT_OK)
    rc = zt_dynamic_qlinear(x, x_dtype, M, K, w, N, w_scales, w_scales_dtype, bias, bias_dtype,
                            post, y, y_dtype, ws, (size_t)ZT_DYN_SCRATCH_BYTES, stream);
  if (dev != cur && hipSetDevice(cur) != hipSuccess && rc == ZT_OK)
    return fail(ZT_EHIP, "%s: cannot restore the current device %d", op, cur);
  return rc;
}

int zt_woq_repack_weight(const int8_t *w, int64_t N, int64_t K, int32_t *out,
                         zt_stream_t stream) {
  static const char *op = "zt_woq_repack_weight";
  if (K < 8 || K % 8)
    return fail(ZT_EINVAL, "%s: K must be at least 8 and divisible by 8, got %lld",
                op, (long long)K);
  if (N < 0) return fail(ZT_EINVAL, "%s: N must be >= 0", op);
  if (N == 0) return ZT_OK;
  if (!w || !out) return fail(ZT_EINVAL, "%s: null pointer", op);
  return hip_status(zt::launch_repack(w, N, K, out, reinterpret_cast<hipStream_t>(stream)), op);
}

int zt_woq_repack_from_int4pack(const uint8_t *packed, int64_t N, int64_t K,
                                int32_t *out, zt_stream_t stream) {
  static const char *op = "zt_woq_repack_from_int4pack";
  if (N % 64)
    return fail(ZT_EINVAL, "%s: packed_weight row count (%lld) must be a multiple "
                "of 64", op, (long long)N);
  if (K < 8 || K % 8)
    return fail(ZT_EINVAL, "%s: K must be at least 8 and divisible by 8, got %lld",
                op, (long long)K);
  if (N == 0) return ZT_OK;
  if (!packed || !out) return fail(ZT_EINVAL, "%s: null pointer", op);
  return hip_status(zt::launch_repack_from_int4pack(
                        packed, N, K, out, reinterpret_cast<hipStream_t>(stream)),
                    op);
}

}  // extern "C"
