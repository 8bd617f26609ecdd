// TORCH_LIBRARY(zentorch) for PyTorch-ROCm: the reference's quantized-linear
// operator schemas, implemented for the CUDA (= HIP) dispatch key on top of
// the C-ABI in include/zentorch_hip.h, plus the AOTInductor C shims
// (include/shim_cuda_zentorch.h).
//
// Schemas are kept character-for-character with the reference
// (src/cpu/cpp/WOQ_Linear.cpp:435-480, DynamicQLinear.cpp:184-189) so graphs,
// the compile pass and callers such as vLLM's torchao patch bind unchanged.
// zentorch_woq_linear_silu_mul is an extension (no reference op; the
// reference's closest is zentorch_mm_silu_mul, Matmul.cpp:440-441), and so is
// its merged-weight form zentorch_woq_linear_gate_up_silu_mul.
//
// There is no CPU kernel: a CPU tensor reaching these ops is an error, not a
// fallback.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <rocprofiler-sdk-roctx/roctx.h>

#include <algorithm>
#include <deque>
#include <mutex>
#include <utility>
#include <vector>

#include "ops.hpp"
#include "zentorch_hip.h"

namespace zentorch_hip {

namespace {

int32_t zt_dtype_of(const at::Tensor &t) {
  switch (t.scalar_type()) {
  case at::kFloat: return ZT_DT_F32;
  case at::kBFloat16: return ZT_DT_BF16;
  case at::kHalf: return ZT_DT_F16;
  case at::kChar: return ZT_DT_S8;
  case at::kByte: return ZT_DT_U8;
  case at::kInt: return ZT_DT_S32;
  default: return ZT_DT_NONE;
  }
}

void check_device(const at::Tensor &t, const at::Tensor &ref, const char *op,
                  const char *name) {
  TORCH_CHECK(t.is_cuda(), op, ": ", name,
              " must be a GPU tensor (zentorch-mi355x has no CPU kernels), got ",
              t.device());
  TORCH_CHECK(t.device() == ref.device(), op, ": ", name, " is on ", t.device(),
              " but input is on ", ref.device());
}

hipStream_t current_stream() {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
}

// Device workspace of one call, from torch's stream-ordered caching
// allocator.  It is released when the call returns; the allocator hands the
// block to later work on the same stream only, and inside a HIP graph
// capture it comes from the graph's private pool, so a captured call keeps
// its own workspace on every replay.
at::Tensor call_workspace(const at::Tensor &like, size_t bytes) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

std::vector<int64_t> out_sizes(const at::Tensor &input, int64_t N) {
  auto s = input.sizes().vec();
  s.back() = N;
  return s;
}

at::Tensor as_2d(const at::Tensor &t) {
  const int64_t last = t.size(-1);
  return t.contiguous().view({t.numel() / std::max<int64_t>(last, 1), last});
}

// [rows, K] view of t with unit column stride and row stride *ld, sharing
// t's storage when its leading dimensions collapse into one (a contiguous
// tensor, or a 2-D tensor whose rows are strided, such as a column slice);
// otherwise a contiguous copy with *ld = K.
at::Tensor rows_view(const at::Tensor &t, int64_t *ld) {
  const int64_t d = t.dim(), K = t.size(-1);
  bool ok = t.stride(d - 1) == 1 || K == 1;
  for (int64_t i = 0; ok && i + 2 < d; ++i)
    ok = t.size(i) == 1 || t.stride(i) == t.stride(i + 1) * t.size(i + 1);
  const int64_t rows = t.numel() / std::max<int64_t>(K, 1);
  if (ok && rows > 0) {
    const int64_t rs = d >= 2 ? t.stride(d - 2) : K;
    if (rs >= K || rows == 1) {
      *ld = rows == 1 ? K : rs;
      return t.as_strided({rows, K}, {*ld, 1});
    }
  }
  *ld = K;
  return as_2d(t);
}

// The reference hands zentorch_op_name to ZenDNNL's profiler
// (MatmulUtils.hpp:763); here it names a ROCTx range around the launches,
// which rocprofv3 --marker-trace records.
struct OpRange {
  explicit OpRange(const std::string &name) { roctxRangePushA(name.c_str()); }
  ~OpRange() { roctxRangePop(); }
};

// Shared body of every zentorch_woq_linear* op.  post_ids follow the
// reference's post-op numbering; binary ops take binary_inputs in order.
at::Tensor woq_linear_impl(const at::Tensor &input, const at::Tensor &weight,
                           const at::Tensor &weight_scales,
                           const c10::optional<at::Tensor> &weight_zero_points,
                           const c10::optional<at::Tensor> &bias,
                           const std::vector<int32_t> &post_ids,
                           const std::vector<at::Tensor> &binary_inputs,
                           const std::string &op_name, bool gate_up = false) {
  const char *op = op_name.c_str();
  check_device(input, input, op, "input");
  check_device(weight, input, op, "weight");
  check_device(weight_scales, input, op, "weight_scales");
  // Same checks and messages as WOQ_Linear.cpp:35-42.
  TORCH_CHECK(weight.dtype() == at::kInt, "weight must have dtype int32, got ",
              weight.dtype());
  TORCH_CHECK(weight.dim() == 2, "weight must be 2D, got ", weight.dim(), "D");
  TORCH_CHECK(weight_scales.dim() == 2, "weight_scales must be 2D [G, N], got ",
              weight_scales.dim(), "D");
  TORCH_CHECK(weight_scales.size(1) == weight.size(1), "weight_scales dim 1 (",
              weight_scales.size(1), ") must match weight dim 1 (",
              weight.size(1), ")");
  const int64_t K = weight.size(0) * 8;
  const int64_t N = weight.size(1);
  TORCH_CHECK(input.dim() >= 2, op, ": input must be at least 2D");
  TORCH_CHECK(input.size(-1) == K, op, ": input last dim (", input.size(-1),
              ") must equal 8 * weight.size(0) (", K, ")");
  TORCH_CHECK(input.scalar_type() == at::kBFloat16 ||
                  input.scalar_type() == at::kFloat,
              op, ": input must be bfloat16 or float32, got ",
              input.scalar_type());
  const int64_t G = weight_scales.size(0);
  TORCH_CHECK(G >= 1 && K % G == 0, op, ": weight_scales groups (", G,
              ") must divide K (", K, ")");

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(input.device());
  const OpRange range(op_name);
  int64_t ldx = K;
  const at::Tensor x2 = rows_view(input, &ldx);
  const int64_t M = x2.size(0);
  // The op's weight is the [K/8, N] view of [N, K/8] storage
  // (_op_replacements_new.py:376-379), which the kernels stream row by row.
  // A weight in any other layout is transposed into that one on every call.
  at::Tensor w_nk = weight.t();
  if (!w_nk.is_contiguous()) {
    TORCH_WARN_ONCE(op, ": weight is not the [K/8, N] transposed view of a contiguous "
                    "[N, K/8] tensor (zentorch_woq_repack_weight(...).t()); it is copied into "
                    "that layout on every call");
    w_nk = w_nk.contiguous();
  }
  at::Tensor s = weight_scales.contiguous();
  at::Tensor zp, b;
  if (weight_zero_points.has_value() && weight_zero_points->defined()) {
    check_device(*weight_zero_points, input, op, "weight_zero_points");
    TORCH_CHECK(weight_zero_points->sizes() == weight_scales.sizes(), op,
                ": weight_zero_points must have the shape of weight_scales");
    zp = weight_zero_points->contiguous();
  }
  if (bias.has_value() && bias->defined()) {
    check_device(*bias, input, op, "bias");
    TORCH_CHECK(bias->numel() == N, op, ": bias must have N = ", N,
                " elements, got ", bias->numel());
    b = bias->contiguous();
  }
  if (gate_up)
    TORCH_CHECK(N % 2 == 0, op, ": the merged gate_up weight needs an even N (gate rows, "
                "then up rows), got ", N);
  at::Tensor result = at::empty(out_sizes(input, gate_up ? N / 2 : N), input.options());
  if (result.numel() == 0) return result;
  const zt_stream_t stream = reinterpret_cast<zt_stream_t>(current_stream());
  if (gate_up) {
    const size_t ws = zt_woq_linear_gate_up_workspace_size(M, K, N, G);
    const at::Tensor wsp = call_workspace(input, ws);
    const int rc = zt_woq_linear_gate_up(
        x2.data_ptr(), zt_dtype_of(x2), M, K, ldx,
        reinterpret_cast<const int32_t *>(w_nk.data_ptr()), N, s.data_ptr(),
        zt_dtype_of(s), G, zp.defined() ? zp.data_ptr() : nullptr,
        zp.defined() ? zt_dtype_of(zp) : ZT_DT_NONE,
        b.defined() ? b.data_ptr() : nullptr,
        b.defined() ? zt_dtype_of(b) : ZT_DT_NONE, result.data_ptr(),
        zt_dtype_of(result), N / 2, wsp.data_ptr(), ws, stream);
    TORCH_CHECK(rc == ZT_OK, op, ": ", zt_last_error_string());
    return result;
  }

  zt_post_ops post{};
  post.count = (int32_t)post_ids.size();
  TORCH_CHECK(post.count <= ZT_MAX_POST_OPS, op, ": too many post-ops");
  std::vector<at::Tensor> keep;
  size_t nb = 0;
  for (size_t i = 0; i < post_ids.size(); ++i) {
    post.ids[i] = post_ids[i];
    if (post_ids[i] == ZT_PO_ADD || post_ids[i] == ZT_PO_MUL) {
      TORCH_CHECK(nb < binary_inputs.size(), op, ": missing binary input");
      const at::Tensor &bi = binary_inputs[nb];
      check_device(bi, input, op, "binary post-op input");
      TORCH_CHECK(bi.numel() == M * N, op, ": binary post-op input has ",
                  bi.numel(), " elements, expected ", M * N);
      TORCH_CHECK(bi.size(-1) == N, op, ": binary post-op input must have N = ", N,
                  " columns, got ", bi.size(-1));
      at::Tensor bc = bi;
      if (bc.scalar_type() != at::kBFloat16 && bc.scalar_type() != at::kFloat)
        bc = bc.to(input.scalar_type());
      int64_t ld = N;
      bc = rows_view(bc, &ld);
      keep.push_back(bc);
      post.bufs[nb] = bc.data_ptr();
      post.buf_dtypes[nb] = zt_dtype_of(bc);
      post.buf_ld[nb] = ld;
      ++nb;
    }
  }
  const size_t ws = zt_woq_linear_workspace_size(M, K, N, G);
  const at::Tensor wsp = call_workspace(input, ws);
  const int rc = zt_woq_linear(
      x2.data_ptr(), zt_dtype_of(x2), M, K, ldx,
      reinterpret_cast<const int32_t *>(w_nk.data_ptr()), N, s.data_ptr(),
      zt_dtype_of(s), G, zp.defined() ? zp.data_ptr() : nullptr,
      zp.defined() ? zt_dtype_of(zp) : ZT_DT_NONE,
      b.defined() ? b.data_ptr() : nullptr,
      b.defined() ? zt_dtype_of(b) : ZT_DT_NONE, &post, result.data_ptr(),
      zt_dtype_of(result), N, wsp.data_ptr(), ws, stream);
  TORCH_CHECK(rc == ZT_OK, op, ": ", zt_last_error_string());
  return result;
}

}  // namespace

template <int32_t UNARY>
at::Tensor woq_linear_unary(const at::Tensor &input, const at::Tensor &weight,
                            const at::Tensor &weight_scales,
                            const c10::optional<at::Tensor> &weight_zero_points,
                            const c10::optional<at::Tensor> &bias,
                            c10::string_view zentorch_op_name) {
  std::vector<int32_t> ids;
  if (UNARY != ZT_PO_NONE) ids.push_back(UNARY);
  return woq_linear_impl(input, weight, weight_scales, weight_zero_points, bias,
                         ids, {}, std::string(zentorch_op_name));
}

template at::Tensor woq_linear_unary<ZT_PO_NONE>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
template at::Tensor woq_linear_unary<ZT_PO_RELU>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
template at::Tensor woq_linear_unary<ZT_PO_SIGMOID>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
template at::Tensor woq_linear_unary<ZT_PO_GELU_TANH>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);
template at::Tensor woq_linear_unary<ZT_PO_GELU_ERF>(
    const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,
    c10::string_view);

at::Tensor woq_linear_add(const at::Tensor &input, const at::Tensor &weight,
                          const at::Tensor &weight_scales,
                          const c10::optional<at::Tensor> &weight_zero_points,
                          const at::Tensor &add_input,
                          const c10::optional<at::Tensor> &bias,
                          c10::string_view zentorch_op_name) {
  return woq_linear_impl(input, weight, weight_scales, weight_zero_points, bias,
                         {ZT_PO_ADD}, {add_input}, std::string(zentorch_op_name));
}

at::Tensor woq_linear_mul_add(const at::Tensor &input, const at::Tensor &weight,
                              const at::Tensor &weight_scales,
                              const c10::optional<at::Tensor> &weight_zero_points,
                              const at::Tensor &mul_input,
                              const at::Tensor &add_input,
                              const c10::optional<at::Tensor> &bias,
                              c10::string_view zentorch_op_name) {
  return woq_linear_impl(input, weight, weight_scales, weight_zero_points, bias,
                         {ZT_PO_MUL, ZT_PO_ADD}, {mul_input, add_input},
                         std::string(zentorch_op_name));
}

at::Tensor woq_linear_add_add(const at::Tensor &input, const at::Tensor &weight,
                              const at::Tensor &weight_scales,
                              const c10::optional<at::Tensor> &weight_zero_points,
                              const at::Tensor &add_input,
                              const at::Tensor &add_input_2,
                              const c10::optional<at::Tensor> &bias,
                              c10::string_view zentorch_op_name) {
  return woq_linear_impl(input, weight, weight_scales, weight_zero_points, bias,
                         {ZT_PO_ADD, ZT_PO_ADD}, {add_input, add_input_2},
                         std::string(zentorch_op_name));
}

at::Tensor woq_linear_silu_mul(const at::Tensor &input, const at::Tensor &weight,
                               const at::Tensor &weight_scales,
                               const c10::optional<at::Tensor> &weight_zero_points,
                               const at::Tensor &mul_input,
                               const c10::optional<at::Tensor> &bias,
                               c10::string_view zentorch_op_name) {
  return woq_linear_impl(input, weight, weight_scales, weight_zero_points, bias,
                         {ZT_PO_SILU, ZT_PO_MUL}, {mul_input},
                         std::string(zentorch_op_name));
}

at::Tensor woq_linear_gate_up_silu_mul(const at::Tensor &input, const at::Tensor &weight,
                                       const at::Tensor &weight_scales,
                                       const c10::optional<at::Tensor> &weight_zero_points,
                                       const c10::optional<at::Tensor> &bias,
                                       c10::string_view zentorch_op_name) {
  return woq_linear_impl(input, weight, weight_scales, weight_zero_points, bias, {}, {},
                         std::string(zentorch_op_name), /*gate_up=*/true);
}

at::Tensor woq_repack_weight(const at::Tensor &unpacked_weight) {
  // Checks and messages of WOQ_Linear.cpp:295-310.
  TORCH_CHECK(unpacked_weight.dtype() == at::kChar,
              "unpacked_weight must have dtype int8, got ",
              unpacked_weight.dtype());
  TORCH_CHECK(unpacked_weight.dim() == 2, "unpacked_weight must be 2D, got ",
              unpacked_weight.dim(), "D");
  TORCH_CHECK(unpacked_weight.is_cuda(),
              "zentorch_woq_repack_weight: unpacked_weight must be a GPU tensor, "
              "got ", unpacked_weight.device());
  const int64_t N = unpacked_weight.size(0), K = unpacked_weight.size(1);
  TORCH_CHECK(K >= 8, "K must be at least ", 8, ", got ", K);
  TORCH_CHECK(K % 8 == 0, "K must be divisible by ", 8, ", got ", K);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(unpacked_weight.device());
  at::Tensor w = unpacked_weight.contiguous();
  at::Tensor out = at::empty({N, K / 8}, w.options().dtype(at::kInt));
  const int rc = zt_woq_repack_weight(
      reinterpret_cast<const int8_t *>(w.data_ptr()), N, K,
      reinterpret_cast<int32_t *>(out.data_ptr()),
      reinterpret_cast<zt_stream_t>(current_stream()));
  TORCH_CHECK(rc == ZT_OK, "zentorch_woq_repack_weight: ", zt_last_error_string());
  return out;
}

at::Tensor woq_repack_from_int4pack(const at::Tensor &packed_weight) {
  TORCH_CHECK(packed_weight.dtype() == at::kByte,
              "packed_weight must have dtype uint8, got ", packed_weight.dtype());
  TORCH_CHECK(packed_weight.dim() == 2, "packed_weight must be 2D, got ",
              packed_weight.dim(), "D");
  TORCH_CHECK(packed_weight.is_cuda(),
              "zentorch_woq_repack_from_int4pack: packed_weight must be a GPU "
              "tensor, got ", packed_weight.device());
  const int64_t N = packed_weight.size(0), K = packed_weight.size(1) * 2;
  TORCH_CHECK(N % 64 == 0, "packed_weight row count (", N,
              ") must be a multiple of ", 64,
              ". The int4pack format from PyTorch pads N to BLOCK_N; "
              "receiving an unpadded tensor indicates a packing mismatch.");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(packed_weight.device());
  at::Tensor p = packed_weight.contiguous();
  at::Tensor out = at::empty({N, K / 8}, p.options().dtype(at::kInt));
  const int rc = zt_woq_repack_from_int4pack(
      reinterpret_cast<const uint8_t *>(p.data_ptr()), N, K,
      reinterpret_cast<int32_t *>(out.data_ptr()),
      reinterpret_cast<zt_stream_t>(current_stream()));
  TORCH_CHECK(rc == ZT_OK, "zentorch_woq_repack_from_int4pack: ",
              zt_last_error_string());
  return out;
}

namespace {

// Shared body of zentorch_dynamic_qlinear and its fused-epilogue
// extensions: post_ids in list order, binary operands [*, N] in order.
at::Tensor dynamic_qlinear_impl(const at::Tensor &input, const at::Tensor &weight,
                                const at::Tensor &weight_scales,
                                const c10::optional<at::Tensor> &bias,
                                const std::vector<int32_t> &post_ids,
                                const std::vector<at::Tensor> &binary_inputs,
                                const std::string &name,
                                const at::Tensor &colsum = at::Tensor()) {
  // dtype / size checks with the messages of DynamicQLinear.cpp:15-70.
  TORCH_CHECK(input.scalar_type() == at::kBFloat16 ||
                  input.scalar_type() == at::kFloat,
              "zentorch_dynamic_qlinear: input must be bfloat16 or float32, got ",
              input.scalar_type());
  TORCH_CHECK(weight_scales.scalar_type() == at::kFloat ||
                  weight_scales.scalar_type() == at::kBFloat16,
              "zentorch_dynamic_qlinear: weight_scales must be float32, "
              "bfloat16, got ", weight_scales.scalar_type());
  TORCH_CHECK(weight.scalar_type() == at::kChar,
              "zentorch_dynamic_qlinear: weight must be int8 (c10::kChar), got ",
              weight.scalar_type());
  at::Tensor b;
  if (bias.has_value() && bias->defined()) {
    TORCH_CHECK(bias->scalar_type() == at::kFloat ||
                    bias->scalar_type() == at::kBFloat16,
                "zentorch_dynamic_qlinear: bias must be float32 or bfloat16, got ",
                bias->scalar_type());
    b = *bias;
  }
  TORCH_CHECK(input.dim() >= 2,
              "zentorch_dynamic_qlinear: input must be at least 2D");
  TORCH_CHECK(weight.dim() == 2,
              "zentorch_dynamic_qlinear: weight must be 2D [N, K], got ",
              weight.dim(), "D");
  const int64_t N = weight.size(0), K = weight.size(1);
  TORCH_CHECK(input.size(input.dim() - 1) == K,
              "zentorch_dynamic_qlinear: input last dim (", input.size(-1),
              ") must match weight dim 1 (", K, ")");
  if (b.defined())
    TORCH_CHECK(b.dim() == 1 && b.size(0) == N,
                "zentorch_dynamic_qlinear: bias must be 1D with size N (", N, ")");
  TORCH_CHECK(weight_scales.numel() == N,
              "zentorch_dynamic_qlinear: weight_scales must hold one scale per "
              "output channel (", N, "), got ", weight_scales.numel());
  const char *op = "zentorch_dynamic_qlinear";
  check_device(input, input, op, "input");
  check_device(weight, input, op, "weight");
  check_device(weight_scales, input, op, "weight_scales");
  if (b.defined()) check_device(b, input, op, "bias");
  at::Tensor cs;
  if (colsum.defined()) {
    TORCH_CHECK(colsum.scalar_type() == at::kInt && colsum.numel() == N, name,
                ": weight_colsum must be int32 with one entry per output channel (", N,
                "), got ", colsum.scalar_type(), " ", colsum.sizes());
    check_device(colsum, input, op, "weight_colsum");
    cs = colsum.contiguous();
    if (reinterpret_cast<uintptr_t>(cs.data_ptr()) & 15u) cs = cs.clone();
  }

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(input.device());
  const OpRange range(name);
  at::Tensor result = at::empty(out_sizes(input, N), input.options());
  if (result.numel() == 0) return result;
  // the reference quantises a contiguous copy of a strided input
  // (DynamicQLinear.cpp:163-165); so does the kernel here
  at::Tensor x2 = as_2d(input);
  const int64_t M = x2.size(0);
  at::Tensor wc = weight.contiguous();
  at::Tensor sc = weight_scales.contiguous();
  at::Tensor bc = b.defined() ? b.contiguous() : b;
  zt_post_ops post{};
  post.count = (int32_t)post_ids.size();
  std::vector<at::Tensor> keep;
  size_t nb = 0;
  for (size_t i = 0; i < post_ids.size(); ++i) {
    post.ids[i] = post_ids[i];
    if (post_ids[i] == ZT_PO_ADD || post_ids[i] == ZT_PO_MUL) {
      const at::Tensor &bi = binary_inputs[nb];
      check_device(bi, input, op, "binary post-op input");
      TORCH_CHECK(bi.numel() == M * N && bi.size(-1) == N, name,
                  ": binary post-op input must have the output's shape [*, ", N, "], got ",
                  bi.sizes());
      at::Tensor bt = bi;
      if (bt.scalar_type() != at::kBFloat16 && bt.scalar_type() != at::kFloat)
        bt = bt.to(input.scalar_type());
      int64_t ld = N;
      bt = rows_view(bt, &ld);
      keep.push_back(bt);
      post.bufs[nb] = bt.data_ptr();
      post.buf_dtypes[nb] = zt_dtype_of(bt);
      post.buf_ld[nb] = ld;
      ++nb;
    }
  }
  const int8_t *wp = reinterpret_cast<const int8_t *>(wc.data_ptr());
  const void *bp = bc.defined() ? bc.data_ptr() : nullptr;
  const int32_t bdt = bc.defined() ? zt_dtype_of(bc) : ZT_DT_NONE;
  const zt_stream_t st = reinterpret_cast<zt_stream_t>(current_stream());
  int rc;
  if (cs.defined()) {
    const size_t ws_bytes = zt_dynamic_qlinear_asym_workspace_size(M, K, N);
    const at::Tensor ws = call_workspace(input, ws_bytes);
    rc = zt_dynamic_qlinear_asym(x2.data_ptr(), zt_dtype_of(x2), M, K, wp, N, sc.data_ptr(),
                                 zt_dtype_of(sc), cs.data_ptr<int32_t>(), bp, bdt,
                                 post.count ? &post : nullptr, result.data_ptr(),
                                 zt_dtype_of(result), ws.data_ptr(), ws_bytes, st);
  } else {
    const size_t ws_bytes = zt_dynamic_qlinear_workspace_size(M, K, N);
    const at::Tensor ws = call_workspace(input, ws_bytes);
    rc = zt_dynamic_qlinear(x2.data_ptr(), zt_dtype_of(x2), M, K, wp, N, sc.data_ptr(),
                            zt_dtype_of(sc), bp, bdt, post.count ? &post : nullptr,
                            result.data_ptr(), zt_dtype_of(result), ws.data_ptr(), ws_bytes, st);
  }
  TORCH_CHECK(rc == ZT_OK, name, ": ", zt_last_error_string());
  return result;
}

}  // namespace

at::Tensor dynamic_qlinear(const at::Tensor &input, const at::Tensor &weight,
                           const at::Tensor &weight_scales,
                           const c10::optional<at::Tensor> &bias,
                           c10::string_view zentorch_op_name) {
  return dynamic_qlinear_impl(input, weight, weight_scales, bias, {}, {},
                              std::string(zentorch_op_name));
}

// Extensions: the reference's dynamic qlinear has no fused post-ops
// (docs/zentorch_dynamic_qlinear.md:99).  silu(linear) * mul_input (the gate
// of a gated MLP) and linear + add_input (a residual), in fp32 before the one
// rounding, as zentorch_woq_linear_silu_mul / _add do.
at::Tensor dynamic_qlinear_silu_mul(const at::Tensor &input, const at::Tensor &weight,
                                    const at::Tensor &weight_scales, const at::Tensor &mul_input,
                                    const c10::optional<at::Tensor> &bias,
                                    c10::string_view zentorch_op_name) {
  return dynamic_qlinear_impl(input, weight, weight_scales, bias, {ZT_PO_SILU, ZT_PO_MUL},
                              {mul_input}, std::string(zentorch_op_name));
}

at::Tensor dynamic_qlinear_add(const at::Tensor &input, const at::Tensor &weight,
                               const at::Tensor &weight_scales, const at::Tensor &add_input,
                               const c10::optional<at::Tensor> &bias,
                               c10::string_view zentorch_op_name) {
  return dynamic_qlinear_impl(input, weight, weight_scales, bias, {ZT_PO_ADD}, {add_input},
                              std::string(zentorch_op_name));
}

// Extension: per-token asymmetric uint8 activations (the reference's dynamic
// qlinear is symmetric s8, DynamicQLinear.cpp:94-110).  weight_colsum is
// zentorch_s8_weight_colsum(weight), computed once per weight.
at::Tensor dynamic_qlinear_asym(const at::Tensor &input, const at::Tensor &weight,
                                const at::Tensor &weight_scales, const at::Tensor &weight_colsum,
                                const c10::optional<at::Tensor> &bias,
                                c10::string_view zentorch_op_name) {
  return dynamic_qlinear_impl(input, weight, weight_scales, bias, {}, {},
                              std::string(zentorch_op_name), weight_colsum);
}

// sum_k weight[n][k] in int32 for an int8 [N, K] weight.
at::Tensor s8_weight_colsum(const at::Tensor &weight) {
  TORCH_CHECK(weight.scalar_type() == at::kChar && weight.dim() == 2,
              "zentorch_s8_weight_colsum: weight must be int8 [N, K], got ",
              weight.scalar_type(), " ", weight.sizes());
  check_device(weight, weight, "zentorch_s8_weight_colsum", "weight");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(weight.device());
  const at::Tensor wc = weight.contiguous();
  at::Tensor out = at::empty({weight.size(0)}, weight.options().dtype(at::kInt));
  if (out.numel() == 0) return out;
  const int rc = zt_s8_weight_colsum(reinterpret_cast<const int8_t *>(wc.data_ptr()),
                                     wc.size(0), wc.size(1), out.data_ptr<int32_t>(),
                                     reinterpret_cast<zt_stream_t>(current_stream()));
  TORCH_CHECK(rc == ZT_OK, "zentorch_s8_weight_colsum: ", zt_last_error_string());
  return out;
}

// ----------------------------------------------------------- static qlinear
// zentorch_qlinear / _relu / _sigmoid / _mul_add and the .out forms
// (src/cpu/cpp/QLinear.cpp:367-573), with the argument checks and messages of
// check_valid_dtypes_for_quantized_matmul / _sizes_ (MatmulUtils.hpp:325-518).
namespace {

void qlinear_checks(const at::Tensor &input, const at::Tensor &weight, const at::Tensor &result,
                    const at::Tensor &bias, const at::Tensor &input_scales,
                    const at::Tensor &input_zero_points, const at::Tensor &weight_scales,
                    const at::Tensor &weight_zero_points, const at::Tensor &output_scales,
                    const at::Tensor &output_zero_points,
                    const std::vector<at::Tensor> &post_bufs) {
  const auto it = input.scalar_type();
  TORCH_CHECK(it == at::kFloat || it == at::kBFloat16 || it == at::kByte || it == at::kChar,
              "unsupported dtype for input tensor, only float32/bfloat16/uint8/int8 is supported");
  TORCH_CHECK(weight.scalar_type() == at::kChar,
              "unsupported dtype for weight tensor, only int8 is supported");
  const auto rt = result.scalar_type();
  TORCH_CHECK(rt == at::kFloat || rt == at::kBFloat16 || rt == at::kByte || rt == at::kChar,
              "unsupported dtype for result tensor, only float32/bfloat16/uint8/int8 is supported");
  if (bias.defined())
    TORCH_CHECK(bias.scalar_type() == at::kFloat || bias.scalar_type() == at::kBFloat16,
                "unsupported dtype for bias tensor, only float32 or bfloat16 is supported");
  TORCH_CHECK(input_scales.scalar_type() == at::kFloat,
              "unsupported dtype for input_scales, only float32 is supported");
  if (input_zero_points.defined())
    TORCH_CHECK(input_zero_points.scalar_type() == at::kInt,
                "unsupported dtype for input_zero_points, only int32 supported");
  TORCH_CHECK(weight_scales.scalar_type() == at::kFloat,
              "unsupported dtype for weight_scales, only float32 is supported");
  if (weight_zero_points.defined())
    TORCH_CHECK(weight_zero_points.scalar_type() == at::kInt,
                "unsupported dtype for weight_zero_points, only int32 is supported");
  if (output_scales.defined()) {
    TORCH_CHECK(output_scales.scalar_type() == at::kFloat,
                "unsupported dtype for output_scales, only float32 is supported");
    if (output_zero_points.defined()) {
      TORCH_CHECK(output_zero_points.scalar_type() == at::kInt,
                  "unsupported dtype for output_zero_points, only int32 is supported");
      TORCH_CHECK(rt == at::kByte,
                  "unsupported dtype for result tensor when output_zero_points are defined, "
                  "uint8 are supported dtype");
    } else {
      TORCH_CHECK(rt == at::kChar,
                  "unsupported dtype for result tensor when output_zero_points are not "
                  "defined while output_scales are defined, int8 are supported dtype");
    }
  } else {
    TORCH_CHECK(rt == at::kFloat || rt == at::kBFloat16,
                "unsupported dtype for result tensor, only float32/bfloat16 is supported "
                "when output_scales are not defined");
  }
  for (const auto &b : post_bufs)
    TORCH_CHECK(b.scalar_type() == at::kFloat || b.scalar_type() == at::kBFloat16,
                "unsupported dtype for post_ops, only float32/bfloat16 is supported");
  // sizes (check_valid_sizes_for_matmul + the quantised ones)
  TORCH_CHECK(input.dim() >= 2 && weight.dim() == 2,
              "unsupported dims for input and weight");
  TORCH_CHECK(input.size(-1) == weight.size(1),
              "unsupported sizes for input and weight: input last dim (", input.size(-1),
              ") must match weight dim 1 (", weight.size(1), ")");
  const int64_t N = weight.size(0);
  if (bias.defined())
    TORCH_CHECK(bias.dim() == 1 && bias.size(0) == N, "unsupported sizes for bias");
  TORCH_CHECK(input_scales.dim() <= 1, "unsupported dims for input_scales with respect to input "
                                       "tensor");
  if (input_zero_points.defined()) {
    TORCH_CHECK(input_zero_points.dim() <= 1,
                "only scalar and 1-d input_zero_points are supported");
    TORCH_CHECK(input_zero_points.numel() == 1,
                "only supporting per-tensor quantization for input");
  }
  TORCH_CHECK(input_scales.numel() == 1,
              "unsupported number of elements for input_scales with respect to input tensor");
  TORCH_CHECK(weight_scales.dim() <= 1,
              "unsupported dims for weight_scales with respect to weight tensor");
  TORCH_CHECK(weight_scales.numel() == 1 || weight_scales.numel() == N,
              "unsupported number of elements for weight_scales with respect to weight tensor");
  if (weight_zero_points.defined()) {
    TORCH_CHECK(weight_zero_points.dim() <= 1,
                "only scalar and 1-d weight_zero_points are supported");
    TORCH_CHECK(weight_zero_points.numel() == 1 || weight_zero_points.numel() == N,
                "only supporting per-tensor and per-channel quantization for weight");
  }
  if (output_scales.defined() && output_zero_points.defined()) {
    TORCH_CHECK(output_scales.dim() <= 1,
                "unsupported dims for output_scales with respect to output tensor");
    TORCH_CHECK(output_zero_points.dim() <= 1,
                "unsupported dims for output_zero_points with respect to output tensor");
    TORCH_CHECK(output_scales.numel() == 1,
                "unsupported number of elements for output_scales with respect to output tensor");
    TORCH_CHECK(output_zero_points.numel() == 1,
                "unsupported number of elements for output_zero_points with respect to output "
                "tensor");
  }
  const auto osz = out_sizes(input, N);
  for (const auto &b : post_bufs) {
    TORCH_CHECK(b.dim() == input.dim(), "unsupported dims for post op buffers for input and "
                                        "weight");
    TORCH_CHECK(b.sizes() == c10::IntArrayRef(osz),
                "unsupported shapes for post op buffers for input and weight");
  }
  TORCH_CHECK(result.sizes() == c10::IntArrayRef(osz), "unsupported shape for the result tensor");
}

// sum_k weight[n][k] (int32) of a static qlinear's int8 weight, computed
// once per weight: the weights of a quantised model are constant, as the
// reference's first-call weight reorder assumes (is_weights_const,
// QLinear.cpp:290-300).  An entry holds a weak reference to the weight's
// storage (so its address cannot be taken by another storage while the
// entry exists) and the version counter it was computed at; an in-place
// update of the weight recomputes it.  Under HIP-graph capture the sums are
// computed inside the captured work instead, so replays after an in-place
// update still see the current weight.
struct ColsumEntry {
  c10::weak_intrusive_ptr<c10::StorageImpl> storage;
  const void *data;
  std::vector<int64_t> sizes, strides;
  uint32_t version;
  at::Tensor colsum;
};
constexpr size_t kColsumCacheMax = 4096;
std::mutex g_colsum_mu;
std::deque<ColsumEntry> g_colsum;

at::Tensor compute_colsum(const at::Tensor &wc, zt_stream_t st, const std::string &name) {
  at::Tensor cs = at::empty({wc.size(0)}, wc.options().dtype(at::kInt));
  const int rc = zt_s8_weight_colsum(reinterpret_cast<const int8_t *>(wc.data_ptr()), wc.size(0),
                                     wc.size(1), cs.data_ptr<int32_t>(), st);
  TORCH_CHECK(rc == ZT_OK, name, ": ", zt_last_error_string());
  return cs;
}

at::Tensor weight_colsum_cached(const at::Tensor &weight, const at::Tensor &wc, hipStream_t st,
                                const std::string &name) {
  const zt_stream_t zst = reinterpret_cast<zt_stream_t>(st);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
    return compute_colsum(wc, zst, name);
  c10::StorageImpl *impl = weight.storage().unsafeGetStorageImpl();
  const uint32_t version = weight._version();
  {
    std::lock_guard<std::mutex> lock(g_colsum_mu);
    for (auto it = g_colsum.begin(); it != g_colsum.end();) {
      if (it->storage.expired()) {
        it = g_colsum.erase(it);
        continue;
      }
      if (it->storage._unsafe_get_target() == impl && it->data == weight.data_ptr() &&
          it->sizes == weight.sizes().vec() && it->strides == weight.strides().vec()) {
        if (it->version == version) return it->colsum;
        it = g_colsum.erase(it);  // the weight changed in place
        continue;
      }
      ++it;
    }
  }
  at::Tensor cs = compute_colsum(wc, zst, name);
  std::lock_guard<std::mutex> lock(g_colsum_mu);
  if (g_colsum.size() >= kColsumCacheMax) g_colsum.pop_front();
  g_colsum.push_back({c10::weak_intrusive_ptr<c10::StorageImpl>(
                          weight.storage().getWeakStorageImpl()),
                      weight.data_ptr(), weight.sizes().vec(), weight.strides().vec(), version, cs});
  return cs;
}

void qlinear_into(at::Tensor &result, const at::Tensor &input, const at::Tensor &weight,
                  const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                  const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                  const c10::optional<at::Tensor> &bias_opt,
                  const c10::optional<at::Tensor> &output_scales_opt,
                  const c10::optional<at::Tensor> &output_zero_points_opt,
                  const std::vector<int32_t> &post_ids,
                  const std::vector<at::Tensor> &post_bufs, const std::string &name) {
  const at::Tensor bias = bias_opt.has_value() ? *bias_opt : at::Tensor();
  const at::Tensor os = output_scales_opt.has_value() ? *output_scales_opt : at::Tensor();
  const at::Tensor oz = output_zero_points_opt.has_value() ? *output_zero_points_opt : at::Tensor();
  qlinear_checks(input, weight, result, bias, input_scales, input_zero_points, weight_scales,
                 weight_zero_points, os, oz, post_bufs);
  const char *op = "zentorch_qlinear";
  for (const at::Tensor *t : std::initializer_list<const at::Tensor *>{
           &weight, &input_scales, &weight_scales, &result})
    check_device(*t, input, op, "argument");
  for (const at::Tensor *t :
       std::initializer_list<const at::Tensor *>{&input_zero_points, &bias, &os, &oz})
    if (t->defined()) check_device(*t, input, op, "argument");
  for (const auto &b : post_bufs) check_device(b, input, op, "post-op buffer");

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(input.device());
  const OpRange range(name);
  if (result.numel() == 0) return;
  const at::Tensor x2 = as_2d(input);
  const int64_t M = x2.size(0), K = x2.size(1), N = weight.size(0);
  const at::Tensor wc = weight.contiguous();
  const at::Tensor sx = input_scales.contiguous(), sw = weight_scales.contiguous();
  const at::Tensor zx = input_zero_points.defined() ? input_zero_points.contiguous() : at::Tensor();
  const at::Tensor bc = bias.defined() ? bias.contiguous() : at::Tensor();
  const at::Tensor osc = os.defined() ? os.contiguous() : at::Tensor();
  const at::Tensor ozc = oz.defined() ? oz.contiguous() : at::Tensor();
  const hipStream_t st = current_stream();
  const zt_stream_t zst = reinterpret_cast<zt_stream_t>(st);
  // activations with an offset (u8, or a zero point) need sum_k w[n][k],
  // kept per weight (the op's input_zero_points is always given, so this is
  // every call of the reference's schema)
  at::Tensor colsum;
  if (x2.scalar_type() == at::kByte || zx.defined()) colsum = weight_colsum_cached(weight, wc, st, name);
  zt_post_ops post{};
  post.count = (int32_t)post_ids.size();
  std::vector<at::Tensor> keep;
  for (size_t i = 0, nb = 0; i < post_ids.size(); ++i) {
    post.ids[i] = post_ids[i];
    if (post_ids[i] == ZT_PO_ADD || post_ids[i] == ZT_PO_MUL) {
      int64_t ld = N;
      at::Tensor bt = rows_view(post_bufs[nb], &ld);
      keep.push_back(bt);
      post.bufs[nb] = bt.data_ptr();
      post.buf_dtypes[nb] = zt_dtype_of(bt);
      post.buf_ld[nb] = ld;
      ++nb;
    }
  }
  // the result may be a strided .out tensor: compute into a contiguous one
  at::Tensor y = result.is_contiguous() ? result : at::empty_like(result, at::MemoryFormat::Contiguous);
  const size_t ws_bytes = zt_qlinear_workspace_size(M, K, N);
  const at::Tensor ws = call_workspace(input, ws_bytes);
  const int rc = zt_qlinear(
      x2.data_ptr(), zt_dtype_of(x2), M, K, sx.data_ptr<float>(),
      zx.defined() ? zx.data_ptr<int32_t>() : nullptr,
      reinterpret_cast<const int8_t *>(wc.data_ptr()), N, sw.data_ptr<float>(), sw.numel(),
      colsum.defined() ? colsum.data_ptr<int32_t>() : nullptr,
      bc.defined() ? bc.data_ptr() : nullptr, bc.defined() ? zt_dtype_of(bc) : ZT_DT_NONE,
      post.count ? &post : nullptr, y.data_ptr(), zt_dtype_of(y),
      osc.defined() ? osc.data_ptr<float>() : nullptr,
      ozc.defined() ? ozc.data_ptr<int32_t>() : nullptr, ws.data_ptr(), ws_bytes, zst);
  TORCH_CHECK(rc == ZT_OK, name, ": ", zt_last_error_string());
  if (!y.is_same(result)) result.copy_(y);
}

at::Tensor qlinear_alloc(const at::Tensor &input, const at::Tensor &weight,
                         c10::optional<c10::ScalarType> output_dtype) {
  TORCH_CHECK(weight.dim() == 2, "unsupported dims for input and weight");
  const auto dt = output_dtype.has_value() ? *output_dtype : at::kFloat;
  TORCH_CHECK(dt == at::kFloat || dt == at::kBFloat16 || dt == at::kByte || dt == at::kChar,
              "output_dtype received is not yet supported, only float32/bfloat16/uint8/int8 is "
              "supported");
  return at::empty(out_sizes(input, weight.size(0)), input.options().dtype(dt));
}

}  // namespace

template <int32_t PO>
at::Tensor qlinear_unary(const at::Tensor &input, const at::Tensor &weight,
                         const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                         const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                         const c10::optional<at::Tensor> &bias,
                         const c10::optional<at::Tensor> &output_scales,
                         const c10::optional<at::Tensor> &output_zero_points,
                         c10::optional<c10::ScalarType> output_dtype,
                         c10::string_view zentorch_op_name) {
  at::Tensor result = qlinear_alloc(input, weight, output_dtype);
  std::vector<int32_t> ids;
  if (PO != ZT_PO_NONE) ids.push_back(PO);
  qlinear_into(result, input, weight, input_scales, input_zero_points, weight_scales,
               weight_zero_points, bias, output_scales, output_zero_points, ids, {},
               std::string(zentorch_op_name));
  return result;
}

template <int32_t PO>
void qlinear_unary_out(at::Tensor &out, const at::Tensor &input, const at::Tensor &weight,
                       const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                       const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                       const c10::optional<at::Tensor> &bias,
                       const c10::optional<at::Tensor> &output_scales,
                       const c10::optional<at::Tensor> &output_zero_points,
                       c10::optional<c10::ScalarType> output_dtype,
                       c10::string_view zentorch_op_name) {
  TORCH_CHECK(output_dtype.has_value() && *output_dtype == out.scalar_type(),
              "output_dtype received does not match the dtype of the output tensor");
  TORCH_CHECK(out.scalar_type() == at::kFloat || out.scalar_type() == at::kBFloat16 ||
                  out.scalar_type() == at::kByte || out.scalar_type() == at::kChar,
              "output_dtype received is not yet supported, only float32/bfloat16/uint8/int8 is "
              "supported");
  std::vector<int32_t> ids;
  if (PO != ZT_PO_NONE) ids.push_back(PO);
  qlinear_into(out, input, weight, input_scales, input_zero_points, weight_scales,
               weight_zero_points, bias, output_scales, output_zero_points, ids, {},
               std::string(zentorch_op_name));
}

at::Tensor qlinear_mul_add(const at::Tensor &input, const at::Tensor &weight,
                           const at::Tensor &input_scales, const at::Tensor &input_zero_points,
                           const at::Tensor &weight_scales, const at::Tensor &weight_zero_points,
                           const at::Tensor &mul_input, const at::Tensor &add_input,
                           const c10::optional<at::Tensor> &bias,
                           const c10::optional<at::Tensor> &output_scales,
                           const c10::optional<at::Tensor> &output_zero_points,
                           c10::optional<c10::ScalarType> output_dtype,
                           c10::string_view zentorch_op_name) {
  at::Tensor result = qlinear_alloc(input, weight, output_dtype);
  qlinear_into(result, input, weight, input_scales, input_zero_points, weight_scales,
               weight_zero_points, bias, output_scales, output_zero_points,
               {ZT_PO_MUL, ZT_PO_ADD}, {mul_input, add_input}, std::string(zentorch_op_name));
  return result;
}

#define ZT_QLIN_INST(PO_)                                                                       \
  template at::Tensor qlinear_unary<PO_>(                                                       \
      const at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &,           \
      const at::Tensor &, const at::Tensor &, const c10::optional<at::Tensor> &,                \
      const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,                     \
      c10::optional<c10::ScalarType>, c10::string_view);                                        \
  template void qlinear_unary_out<PO_>(                                                         \
      at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &,                 \
      const at::Tensor &, const at::Tensor &, const at::Tensor &,                               \
      const c10::optional<at::Tensor> &, const c10::optional<at::Tensor> &,                     \
      const c10::optional<at::Tensor> &, c10::optional<c10::ScalarType>, c10::string_view);
ZT_QLIN_INST(ZT_PO_NONE)
ZT_QLIN_INST(ZT_PO_RELU)
ZT_QLIN_INST(ZT_PO_SIGMOID)
#undef ZT_QLIN_INST

// The reference's own expert formats (FusedMoE.cpp:470-718,
// docs/zentorch_fused_moe.md:80-101): bf16 / fp32 experts in the input's
// dtype, or int8 experts with per-output-channel scales whose activations
// are quantised per token inside each GEMM.  As the reference, the (token, k)
// pairs are grouped by expert with the per-expert counts on the host
// (FusedMoE.cpp:289-433; here one device-to-host copy of E + 2 counts, so
// these formats are not capturable in a HIP graph, as the reference's host
// grouping is not).  Each active expert then runs
//   h = act(x . W13[e, :I]^T + b13[e, :I]) * (x . W13[e, I:]^T + b13[e, I:])
//   y = h . W2[e]^T + b2[e]
// as the reference's per-expert fallback does (vllm/_int8_moe_patch.py:
// 149-206): int8 experts on zentorch_dynamic_qlinear's kernels (the gate's
// activation and the product with the up half in its fused epilogue, on the
// fp32 accumulator with one rounding, as the int4 path computes h), float
// experts on the plain library
// GEMM (hipBLASLt through at::matmul).  out[t] = sum_k w[t, k] * y[t, k] in
// fp32 (k in order), rounded once; pairs whose id is outside [0, E) are
// dropped.
void fused_moe_dense(at::Tensor &output, const at::Tensor &input, const at::Tensor &w13,
                     const at::Tensor &w2, const at::Tensor &b13, const at::Tensor &b2,
                     const at::Tensor &topk_weights, const at::Tensor &topk_id,
                     bool skip_weighted, int32_t act_id,
                     const c10::optional<at::Tensor> &w13_scales,
                     const c10::optional<at::Tensor> &w2_scales, const std::string &name) {
  const char *op = "zentorch_fused_moe";
  const int64_t T = input.size(0), H = input.size(1), E = w13.size(0);
  const int64_t I = w13.size(1) / 2, topk = topk_id.size(1), P = T * topk;
  const bool int8 = w13.scalar_type() == at::kChar;
  at::Tensor s13, s2;
  if (int8) {
    TORCH_CHECK(w2.scalar_type() == at::kChar, op, ": w13 is int8, so w2 must be int8 too, got ",
                w2.scalar_type());
    TORCH_CHECK(w13_scales.has_value() && w13_scales->defined() && w2_scales.has_value() &&
                    w2_scales->defined(),
                op, ": int8 experts need w13_scales and w2_scales");
    s13 = *w13_scales;
    s2 = *w2_scales;
    TORCH_CHECK(s13.numel() == E * 2 * I && s2.numel() == E * H, op,
                ": int8 experts take per-output-channel scales [E, 2I] and [E, H] (per-group "
                "int8 scales are not supported by this build); got ", s13.sizes(), " and ",
                s2.sizes());
    TORCH_CHECK((s13.scalar_type() == at::kFloat || s13.scalar_type() == at::kBFloat16) &&
                    (s2.scalar_type() == at::kFloat || s2.scalar_type() == at::kBFloat16),
                op, ": int8 expert scales must be float32 or bfloat16");
    s13 = s13.reshape({E, 2 * I});
    s2 = s2.reshape({E, H});
    check_device(s13, input, op, "w13_scales");
    check_device(s2, input, op, "w2_scales");
  } else {
    TORCH_CHECK(w13.scalar_type() == input.scalar_type() && w2.scalar_type() == input.scalar_type(),
                op, ": float experts must have the input's dtype (", input.scalar_type(),
                "), got w13 ", w13.scalar_type(), " and w2 ", w2.scalar_type());
    TORCH_CHECK(!(w13_scales.has_value() && w13_scales->defined()) &&
                    !(w2_scales.has_value() && w2_scales->defined()),
                op, ": scales are only taken with int8 or int4 experts");
  }
  TORCH_CHECK(w13.dim() == 3 && w13.size(1) == 2 * I && w13.size(2) == H, op,
              ": w13 must be [E, 2I, H] for H=", H, ", got ", w13.sizes());
  TORCH_CHECK(w2.dim() == 3 && w2.size(0) == E && w2.size(1) == H && w2.size(2) == I, op,
              ": w2 must be [E, H, I] = [", E, ", ", H, ", ", I, "], got ", w2.sizes());
  if (T == 0) return;
  // group the pairs by expert: a stable sort of the ids, and the counts of
  // ids below 0, of each expert and of ids >= E in one host copy
  const at::Tensor flat = topk_id.reshape({-1}).to(at::kLong);
  const at::Tensor order = std::get<1>(at::sort(flat, /*stable=*/true, 0, false));
  const at::Tensor bins = (flat.clamp(-1, E) + 1);
  const at::Tensor counts = at::bincount(bins, {}, E + 2).cpu();
  const int64_t *cnt = counts.data_ptr<int64_t>();
  const at::Tensor tokens = input.index_select(0, at::div(order, topk, "floor"));
  at::Tensor y = at::zeros({P, H}, input.options());
  int64_t cursor = cnt[0];  // the ids below 0 sort first and stay zero
  for (int64_t e = 0; e < E; ++e) {
    const int64_t n = cnt[e + 1];
    if (n == 0) continue;
    const at::Tensor xe = tokens.narrow(0, cursor, n);
    const at::Tensor we = w13[e];
    const c10::optional<at::Tensor> bg =
        b13.defined() ? c10::optional<at::Tensor>(b13[e].narrow(0, 0, I)) : c10::nullopt;
    const c10::optional<at::Tensor> bu =
        b13.defined() ? c10::optional<at::Tensor>(b13[e].narrow(0, I, I)) : c10::nullopt;
    const c10::optional<at::Tensor> bd =
        b2.defined() ? c10::optional<at::Tensor>(b2[e]) : c10::nullopt;
    at::Tensor h, ye;
    if (int8) {
      // the gate's activation runs on its fp32 accumulator in the GEMM
      // epilogue, times the rounded up half, with one rounding (the int4
      // path's convention); h is then quantised per token for W2
      const at::Tensor up = dynamic_qlinear_impl(xe, we.narrow(0, I, I), s13[e].narrow(0, I, I),
                                                 bu, {}, {}, name);
      h = dynamic_qlinear_impl(xe, we.narrow(0, 0, I), s13[e].narrow(0, 0, I), bg,
                               {act_id, ZT_PO_MUL}, {up}, name);
      ye = dynamic_qlinear_impl(h, w2[e], s2[e], bd, {}, {}, name);
    } else {
      at::Tensor gu = at::matmul(xe, we.t());
      if (b13.defined()) gu = gu + b13[e];
      const at::Tensor g = gu.narrow(1, 0, I), u = gu.narrow(1, I, I);
      h = (act_id == ZT_PO_SILU ? at::silu(g)
                                : at::gelu(g, act_id == ZT_PO_GELU_TANH ? "tanh" : "none")) * u;
      ye = at::matmul(h, w2[e].t());
      if (b2.defined()) ye = ye + b2[e];
    }
    y.narrow(0, cursor, n).copy_(ye);
    cursor += n;
  }
  // back to (token, k) order, then the weighted sum over k in fp32
  at::Tensor yu = at::empty_like(y);
  yu.index_copy_(0, order, y);
  at::Tensor acc = yu.view({T, topk, H}).to(at::kFloat);
  if (!skip_weighted) acc = acc * topk_weights.to(at::kFloat).unsqueeze(-1);
  output.copy_(acc.sum(1));
}

// zentorch_fused_moe (src/cpu/cpp/FusedMoE.cpp:443-700, schema :728-736).
// int4-packed expert weights (an extension: w13 int32 [E, 2I, H/8], w2
// int32 [E, H, I/8], each expert packed by zentorch_woq_repack_weight, with
// bf16 group scales w13_scales [E, G13, 2I], w2_scales [E, G2, H]) run the
// grouped HIP kernels of zt_woq_moe, routing included, with no host
// synchronisation; the reference's bf16 / fp32 / int8 experts take
// fused_moe_dense above.  `output` ([T, H], the input's dtype) is
// overwritten with the result, which equals the reference's accumulation
// into its zero-initialised output.
void fused_moe(at::Tensor &output, const at::Tensor &input, const at::Tensor &w13,
               const at::Tensor &w2, const c10::optional<at::Tensor> &w13_bias,
               const c10::optional<at::Tensor> &w2_bias, const at::Tensor &topk_weights,
               const at::Tensor &topk_id, bool skip_weighted, c10::string_view act,
               const c10::optional<at::Tensor> &w13_scales,
               const c10::optional<at::Tensor> &w2_scales, c10::string_view zentorch_op_name) {
  const char *op = "zentorch_fused_moe";
  const OpRange range{std::string(zentorch_op_name)};
  TORCH_CHECK(input.dim() == 2 && (input.scalar_type() == at::kBFloat16 ||
                                   input.scalar_type() == at::kFloat),
              op, ": input must be a 2D bfloat16 or float32 tensor [T, H]");
  TORCH_CHECK(w13.dim() == 3 && w2.dim() == 3, op, ": w13 and w2 must be 3D");
  if (w13.scalar_type() != at::kInt) {
    TORCH_CHECK(topk_id.dim() == 2 && topk_id.size(0) == input.size(0), op,
                ": topk_id must be [T, K]");
    TORCH_CHECK(topk_weights.sizes() == topk_id.sizes(), op,
                ": topk_weights must have topk_id's shape ", topk_id.sizes());
    TORCH_CHECK(!skip_weighted || topk_id.size(1) == 1, op,
                ": skip_weighted requires K == 1 (got K=", topk_id.size(1), ")");
    TORCH_CHECK(w13.size(1) % 2 == 0, op, ": w13 must be [E, 2I, H]");
    TORCH_CHECK(output.sizes() == input.sizes() && output.scalar_type() == input.scalar_type(),
                op, ": output must be a tensor like input");
    int32_t act_id = 0;
    if (act == "silu") act_id = ZT_PO_SILU;
    else if (act == "gelu") act_id = ZT_PO_GELU_ERF;
    else if (act == "gelu_tanh") act_id = ZT_PO_GELU_TANH;
    else TORCH_CHECK(false, op, ": activation '", std::string(act), "' is not supported here "
                     "(silu, gelu, gelu_tanh)");
    at::Tensor b13, b2;
    if (w13_bias.has_value() && w13_bias->defined()) b13 = w13_bias->reshape({w13.size(0), -1});
    if (w2_bias.has_value() && w2_bias->defined()) b2 = w2_bias->reshape({w13.size(0), -1});
    for (const at::Tensor *t : std::initializer_list<const at::Tensor *>{
             &input, &w13, &w2, &topk_id, &topk_weights, &output})
      check_device(*t, input, op, "argument");
    if (b13.defined()) check_device(b13, input, op, "w13_bias");
    if (b2.defined()) check_device(b2, input, op, "w2_bias");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(input.device());
    fused_moe_dense(output, input.contiguous(), w13, w2, b13, b2, topk_weights, topk_id,
                    skip_weighted, act_id, w13_scales, w2_scales, std::string(zentorch_op_name));
    return;
  }
  TORCH_CHECK(input.scalar_type() == at::kBFloat16, op,
              ": int4-packed experts take a bfloat16 input");
  TORCH_CHECK(w2.scalar_type() == at::kInt, op, ": w13 is int4-packed (int32), so w2 must be "
              "too, got ", w2.scalar_type());
  const int64_t T = input.size(0), H = input.size(1);
  const int64_t E = w13.size(0), I = w13.size(1) / 2;
  TORCH_CHECK(w13.size(1) == 2 * I && w13.size(2) * 8 == H, op,
              ": w13 must be [E, 2I, H/8] for H=", H, ", got ", w13.sizes());
  TORCH_CHECK(w2.size(0) == E && w2.size(1) == H && w2.size(2) * 8 == I, op,
              ": w2 must be [E, H, I/8] = [", E, ", ", H, ", ", I / 8, "], got ", w2.sizes());
  TORCH_CHECK(w13_scales.has_value() && w13_scales->defined() && w2_scales.has_value() &&
                  w2_scales->defined(),
              op, ": int4 experts need w13_scales and w2_scales");
  const at::Tensor s13 = w13_scales->contiguous(), s2 = w2_scales->contiguous();
  TORCH_CHECK(s13.scalar_type() == at::kBFloat16 && s2.scalar_type() == at::kBFloat16,
              op, ": scales must be bfloat16");
  TORCH_CHECK(s13.dim() == 3 && s13.size(0) == E && s13.size(2) == 2 * I, op,
              ": w13_scales must be [E, G13, 2I], got ", s13.sizes());
  TORCH_CHECK(s2.dim() == 3 && s2.size(0) == E && s2.size(2) == H, op,
              ": w2_scales must be [E, G2, H], got ", s2.sizes());
  TORCH_CHECK(topk_id.dim() == 2 && topk_id.size(0) == T, op, ": topk_id must be [T, K]");
  const int64_t topk = topk_id.size(1);
  TORCH_CHECK(topk_weights.sizes() == topk_id.sizes(), op,
              ": topk_weights must have topk_id's shape ", topk_id.sizes());
  TORCH_CHECK(topk_weights.scalar_type() == at::kFloat || topk_weights.scalar_type() == at::kBFloat16,
              op, ": topk_weights must be float32 or bfloat16");
  TORCH_CHECK(!skip_weighted || topk == 1, op, ": skip_weighted requires K == 1 (got K=", topk, ")");
  int32_t act_id;
  if (act == "silu") act_id = ZT_PO_SILU;
  else if (act == "gelu") act_id = ZT_PO_GELU_ERF;
  else if (act == "gelu_tanh") act_id = ZT_PO_GELU_TANH;
  else TORCH_CHECK(false, op, ": activation '", std::string(act), "' is not supported here "
                   "(silu, gelu, gelu_tanh)");
  TORCH_CHECK(output.sizes() == input.sizes() && output.scalar_type() == input.scalar_type() &&
                  output.is_contiguous(),
              op, ": output must be a contiguous tensor like input");
  at::Tensor b13, b2;
  if (w13_bias.has_value() && w13_bias->defined()) {
    b13 = w13_bias->contiguous();
    TORCH_CHECK(b13.scalar_type() == at::kBFloat16 && b13.numel() == E * 2 * I, op,
                ": w13_bias must be bfloat16 [E, 2I]");
  }
  if (w2_bias.has_value() && w2_bias->defined()) {
    b2 = w2_bias->contiguous();
    TORCH_CHECK(b2.scalar_type() == at::kBFloat16 && b2.numel() == E * H, op,
                ": w2_bias must be bfloat16 [E, H]");
  }
  for (const at::Tensor *t : std::initializer_list<const at::Tensor *>{
           &input, &w13, &w2, &s13, &s2, &topk_id, &topk_weights, &output})
    check_device(*t, input, op, "argument");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(input.device());
  if (T == 0) return;
  const at::Tensor x = input.contiguous();
  const at::Tensor ids = topk_id.to(at::kInt).contiguous();
  const at::Tensor wts = topk_weights.contiguous();
  const at::Tensor w13c = w13.contiguous(), w2c = w2.contiguous();
  const size_t ws_bytes = zt_woq_moe_workspace_size(T, H, topk, E, I);
  at::Tensor ws = at::empty({(int64_t)ws_bytes}, input.options().dtype(at::kByte));
  const int rc = zt_woq_moe(
      x.data_ptr(), T, H, ids.data_ptr<int32_t>(), wts.data_ptr(), zt_dtype_of(wts), topk,
      skip_weighted ? 1 : 0, act_id, w13c.data_ptr<int32_t>(), s13.data_ptr(), s13.size(1),
      b13.defined() ? b13.data_ptr() : nullptr, w2c.data_ptr<int32_t>(), s2.data_ptr(),
      s2.size(1), b2.defined() ? b2.data_ptr() : nullptr, E, I, output.data_ptr(),
      ws.data_ptr(), ws_bytes, reinterpret_cast<zt_stream_t>(current_stream()));
  TORCH_CHECK(rc == ZT_OK, op, ": ", zt_last_error_string());
}

// The reference drops its per-expert weight-view caches here
// (FusedMoE.cpp:726); this build keeps no such cache.
void flush_moe_weight_cache() {}

}  // namespace zentorch_hip

TORCH_LIBRARY(zentorch, m) {
  m.def("zentorch_woq_linear(Tensor input, Tensor weight, "
        "Tensor weight_scales, Tensor? weight_zero_points, "
        "Tensor? bias=None, "
        "*, str zentorch_op_name='zentorch::zentorch_woq_linear') -> Tensor");
  m.def("zentorch_woq_linear_relu(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, "
        "*, str zentorch_op_name="
        "'zentorch::zentorch_woq_linear_relu') -> Tensor");
  m.def("zentorch_woq_linear_sigmoid(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, "
        "Tensor? bias=None, *, str "
        "zentorch_op_name='zentorch::zentorch_woq_linear_sigmoid') -> Tensor");
  m.def("zentorch_woq_linear_gelu_tanh(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, "
        "*, str zentorch_op_name="
        "'zentorch::zentorch_woq_linear_gelu_tanh') -> Tensor");
  m.def("zentorch_woq_linear_gelu_erf(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, "
        "*, str zentorch_op_name="
        "'zentorch::zentorch_woq_linear_gelu_erf') -> Tensor");
  m.def("zentorch_woq_linear_add(Tensor input, Tensor weight, "
        "Tensor weight_scales, Tensor? weight_zero_points, "
        "Tensor add_input, Tensor? bias=None, *, str zentorch_op_name="
        "'zentorch::zentorch_woq_linear_add') -> Tensor",
        {at::Tag::needs_contiguous_strides});
  m.def("zentorch_woq_linear_mul_add(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, "
        "Tensor mul_input, Tensor add_input, Tensor? bias=None, *, str "
        "zentorch_op_name= 'zentorch::zentorch_woq_linear_mul_add') -> Tensor",
        {at::Tag::needs_fixed_stride_order});
  m.def("zentorch_woq_linear_add_add(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, "
        "Tensor add_input, Tensor add_input_2, Tensor? bias=None, *, str "
        "zentorch_op_name='zentorch::zentorch_woq_linear_add_add') -> Tensor",
        {at::Tag::needs_fixed_stride_order});
  // Extension: silu(linear) * mul_input, the gate of a gated MLP.
  m.def("zentorch_woq_linear_silu_mul(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, "
        "Tensor mul_input, Tensor? bias=None, *, str "
        "zentorch_op_name='zentorch::zentorch_woq_linear_silu_mul') -> Tensor",
        {at::Tag::needs_fixed_stride_order});
  // Extension: the merged gate_up weight [K/8, 2I] (gate columns, then up
  // columns) with silu(gate) * up as its epilogue; output [*, I].
  m.def("zentorch_woq_linear_gate_up_silu_mul(Tensor input, Tensor weight,"
        "Tensor weight_scales, Tensor? weight_zero_points, Tensor? bias=None, *, str "
        "zentorch_op_name='zentorch::zentorch_woq_linear_gate_up_silu_mul') -> Tensor");
  m.def("zentorch_woq_repack_weight(Tensor unpacked_weight) -> Tensor");
  m.def("zentorch_woq_repack_from_int4pack(Tensor "
        "packed_weight) -> Tensor");
  m.def("zentorch_dynamic_qlinear(Tensor input, Tensor weight, "
        "Tensor weight_scales, Tensor? bias=None, *, "
        "str zentorch_op_name="
        "'zentorch::zentorch_dynamic_qlinear') -> Tensor");
  // Extensions: dynamic qlinear with fused silu * mul and residual add.
  m.def("zentorch_dynamic_qlinear_silu_mul(Tensor input, Tensor weight, "
        "Tensor weight_scales, Tensor mul_input, Tensor? bias=None, *, "
        "str zentorch_op_name='zentorch::zentorch_dynamic_qlinear_silu_mul') -> Tensor",
        {at::Tag::needs_fixed_stride_order});
  m.def("zentorch_dynamic_qlinear_add(Tensor input, Tensor weight, "
        "Tensor weight_scales, Tensor add_input, Tensor? bias=None, *, "
        "str zentorch_op_name='zentorch::zentorch_dynamic_qlinear_add') -> Tensor",
        {at::Tag::needs_fixed_stride_order});
  // Extension: per-token asymmetric uint8 activations (opt-in).
  m.def("zentorch_dynamic_qlinear_asym(Tensor input, Tensor weight, "
        "Tensor weight_scales, Tensor weight_colsum, Tensor? bias=None, *, "
        "str zentorch_op_name='zentorch::zentorch_dynamic_qlinear_asym') -> Tensor",
        {at::Tag::needs_fixed_stride_order});
  m.def("zentorch_s8_weight_colsum(Tensor weight) -> Tensor");
  // Static int8 qlinear (QLinear.cpp:525-573).
  m.def("zentorch_qlinear(Tensor input, Tensor weight, "
        "Tensor input_scales, Tensor input_zero_points, "
        "Tensor weight_scales, Tensor weight_zero_points, Tensor? bias, "
        "Tensor? output_scales, Tensor? output_zero_points, "
        "ScalarType? output_dtype=None, str zentorch_op_name="
        "'zentorch::zentorch_qlinear') -> Tensor");
  m.def("zentorch_qlinear_relu(Tensor input, Tensor weight, "
        "Tensor input_scales, Tensor input_zero_points, "
        "Tensor weight_scales, Tensor weight_zero_points, Tensor? bias, "
        "Tensor? output_scales, Tensor? output_zero_points, "
        "ScalarType? output_dtype=None, str zentorch_op_name="
        "'zentorch::zentorch_qlinear_relu') -> Tensor");
  m.def("zentorch_qlinear_sigmoid(Tensor input, Tensor weight, "
        "Tensor input_scales, Tensor input_zero_points, "
        "Tensor weight_scales, Tensor weight_zero_points, Tensor? bias, "
        "Tensor? output_scales, Tensor? output_zero_points, "
        "ScalarType? output_dtype=None, str zentorch_op_name="
        "'zentorch::zentorch_qlinear_sigmoid') -> Tensor");
  m.def("zentorch_qlinear_mul_add(Tensor input, Tensor weight, "
        "Tensor input_scales, Tensor input_zero_points, "
        "Tensor weight_scales, Tensor weight_zero_points, Tensor mul_input, "
        "Tensor add_input, Tensor? bias, Tensor? output_scales, "
        "Tensor? output_zero_points, ScalarType? output_dtype=None, str "
        "zentorch_op_name='zentorch::zentorch_qlinear_mul_add') -> Tensor");
  m.def("zentorch_qlinear.out(Tensor(a!) out, Tensor input, Tensor weight, "
        "Tensor input_scales, Tensor input_zero_points, "
        "Tensor weight_scales, Tensor weight_zero_points, Tensor? bias, "
        "Tensor? output_scales, Tensor? output_zero_points, "
        "ScalarType? output_dtype=None, "
        "str zentorch_op_name='zentorch::zentorch_qlinear.out') -> ()");
  m.def("zentorch_qlinear_relu.out(Tensor(a!) out, Tensor input, Tensor weight, "
        "Tensor input_scales, Tensor input_zero_points, "
        "Tensor weight_scales, Tensor weight_zero_points, Tensor? bias, "
        "Tensor? output_scales, Tensor? output_zero_points, "
        "ScalarType? output_dtype=None, "
        "str zentorch_op_name='zentorch::zentorch_qlinear_relu.out') -> ()");
  m.def("zentorch_fused_moe(Tensor(a!) output, Tensor input, "
        "Tensor w13, Tensor w2, "
        "Tensor? w13_bias, Tensor? w2_bias, "
        "Tensor topk_weights, Tensor topk_id, "
        "bool skip_weighted, str act, "
        "Tensor? w13_scales=None, Tensor? w2_scales=None, "
        "*, str zentorch_op_name='zentorch::zentorch_fused_moe') -> ()");
  m.def("zentorch_flush_moe_weight_cache() -> ()", &zentorch_hip::flush_moe_weight_cache);
}

TORCH_LIBRARY_IMPL(zentorch, CUDA, m) {
  using namespace zentorch_hip;
  m.impl("zentorch_woq_linear", woq_linear_unary<ZT_PO_NONE>);
  m.impl("zentorch_woq_linear_relu", woq_linear_unary<ZT_PO_RELU>);
  m.impl("zentorch_woq_linear_sigmoid", woq_linear_unary<ZT_PO_SIGMOID>);
  m.impl("zentorch_woq_linear_gelu_tanh", woq_linear_unary<ZT_PO_GELU_TANH>);
  m.impl("zentorch_woq_linear_gelu_erf", woq_linear_unary<ZT_PO_GELU_ERF>);
  m.impl("zentorch_woq_linear_add", woq_linear_add);
  m.impl("zentorch_woq_linear_mul_add", woq_linear_mul_add);
  m.impl("zentorch_woq_linear_add_add", woq_linear_add_add);
  m.impl("zentorch_woq_linear_silu_mul", woq_linear_silu_mul);
  m.impl("zentorch_woq_linear_gate_up_silu_mul", woq_linear_gate_up_silu_mul);
  m.impl("zentorch_woq_repack_weight", woq_repack_weight);
  m.impl("zentorch_woq_repack_from_int4pack", woq_repack_from_int4pack);
  m.impl("zentorch_dynamic_qlinear", dynamic_qlinear);
  m.impl("zentorch_dynamic_qlinear_silu_mul", dynamic_qlinear_silu_mul);
  m.impl("zentorch_dynamic_qlinear_add", dynamic_qlinear_add);
  m.impl("zentorch_dynamic_qlinear_asym", dynamic_qlinear_asym);
  m.impl("zentorch_s8_weight_colsum", s8_weight_colsum);
  m.impl("zentorch_qlinear", qlinear_unary<ZT_PO_NONE>);
  m.impl("zentorch_qlinear_relu", qlinear_unary<ZT_PO_RELU>);
  m.impl("zentorch_qlinear_sigmoid", qlinear_unary<ZT_PO_SIGMOID>);
  m.impl("zentorch_qlinear_mul_add", qlinear_mul_add);
  m.impl("zentorch_qlinear.out", qlinear_unary_out<ZT_PO_NONE>);
  m.impl("zentorch_qlinear_relu.out", qlinear_unary_out<ZT_PO_RELU>);
  m.impl("zentorch_fused_moe", fused_moe);
}
