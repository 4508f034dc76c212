// PyTorch-ROCm operator registration over the C ABI of librlm_hip.so.
//
// Registers the reference's operator names and schemas
//   relation_lm::relation_select_packed      (relation_select.py:311)
//   relationlex::anchor_select               (triton_select.py:255)
//   relationlex::partner_topk                (triton_select.py:298)
//   relation_lm::relation_hidden_cached      (relation_reduce.py:149)
//   relation_lm::relation_hidden_cache_update(relation_reduce.py:312)
//   relation_lm::relation_norm_reduce        (relation_reduce.py:420)
//   relation_lm::router_cache_update         (router_cache.py:181)
// plus the sequence forms, the fused reduce, the packed sparse-cache
// projection and the linear.
// Every op has a CUDA-key (ROCm device) implementation over the C ABI.  The
// one exception to "CPU tensors raise" is packed_sparse_cache_projection: the
// reference's project() is F.linear and runs on any device, so its CPU-key
// implementation is at::linear (device tensors never reach it).
// Outputs are allocated with the caching allocator on the input device and
// every kernel is enqueued on the current HIP stream, so the ops compose
// with graph capture.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <initializer_list>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>

#include "relation_lm_hip.h"

namespace {

int32_t dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kFloat: return RLM_F32;
    case at::kBFloat16: return RLM_BF16;
    case at::kHalf: return RLM_F16;
    case at::kInt: return RLM_I32;
    case at::kLong: return RLM_I64;
    default: return -1;
  }
}

rlm_tensor desc(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.defined(), name, ": tensor is undefined");
  TORCH_CHECK(t.dim() <= RLM_MAX_DIMS, name, ": at most ", RLM_MAX_DIMS, " dims supported");
  const int32_t code = dtype_code(t.scalar_type());
  TORCH_CHECK(code >= 0, name, ": unsupported dtype ", t.scalar_type());
  rlm_tensor d{};
  d.data = t.data_ptr();
  d.dtype = code;
  d.ndim = static_cast<int32_t>(t.dim());
  for (int64_t i = 0; i < t.dim(); ++i) {
    d.shape[i] = t.size(i);
    d.stride[i] = t.stride(i);
  }
  return d;
}

// All tensors must live on one ROCm device; returns its current stream.
hipStream_t device_stream(const char* op, std::initializer_list<const at::Tensor*> tensors) {
  const at::Tensor* first = *tensors.begin();
  TORCH_CHECK(first->is_cuda(), op, ": relation_lm HIP ops need tensors on a ROCm device, got ",
              first->device());
  for (const at::Tensor* t : tensors) {
    if (!t->defined()) continue;
    TORCH_CHECK(t->is_cuda() && t->device() == first->device(), op,
                ": all tensors must be on ", first->device(), ", found one on ", t->device());
  }
  return c10::hip::getCurrentHIPStream(first->device().index()).stream();
}

void check(hipError_t err, const char* op) {
  TORCH_CHECK(err == hipSuccess, op, " failed (hipError ", static_cast<int>(err), "): ",
              rlm_last_error());
}

at::TensorOptions f32(const at::Tensor& like) { return like.options().dtype(at::kFloat); }
at::TensorOptions i32(const at::Tensor& like) { return like.options().dtype(at::kInt); }

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> select_packed_common(
    bool seq, const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid,
    bool ring = false) {
  const char* op = ring  ? "relation_lm::relation_select_packed_ring"
                   : seq ? "relation_lm::relation_select_packed_seq"
                         : "relation_lm::relation_select_packed";
  c10::DeviceGuard guard(anchor_query.device());
  hipStream_t stream = device_stream(
      op, {&anchor_query, &anchor_keys, &anchor_router_query, &anchor_block_mean,
           &anchor_block_std, &anchor_gamma, &anchor_bias, &partner_base, &partner_anchor_cache,
           &partner_keys, &partner_block_mean, &partner_block_std, &partner_gamma, &partner_bias,
           &position});
  TORCH_CHECK(anchor_query.dim() == (seq ? 3 : 2), op, ": anchor_query must be ",
              seq ? "[B,Tq,E]" : "[B,E]");
  TORCH_CHECK(k_out >= 0, op, ": k_out must be non-negative");
  std::vector<int64_t> qshape{anchor_query.size(0)};
  if (seq) qshape.push_back(anchor_query.size(1));
  std::vector<int64_t> kshape = qshape;
  kshape.push_back(k_out);
  at::Tensor out_anchor = at::empty(qshape, i32(anchor_query));
  at::Tensor out_anchor_score = at::empty(qshape, f32(anchor_query));
  at::Tensor out_partner = at::empty(kshape, i32(anchor_query));
  at::Tensor out_partner_score = at::empty(kshape, f32(anchor_query));
  rlm_tensor d[19] = {
      desc(anchor_query, "anchor_query"), desc(anchor_keys, "anchor_keys"),
      desc(anchor_router_query, "anchor_router_query"),
      desc(anchor_block_mean, "anchor_block_mean"), desc(anchor_block_std, "anchor_block_std"),
      desc(anchor_gamma, "anchor_gamma"), desc(anchor_bias, "anchor_bias"),
      desc(partner_base, "partner_base"), desc(partner_anchor_cache, "partner_anchor_cache"),
      desc(partner_keys, "partner_keys"), desc(partner_block_mean, "partner_block_mean"),
      desc(partner_block_std, "partner_block_std"), desc(partner_gamma, "partner_gamma"),
      desc(partner_bias, "partner_bias"), desc(position, "position"),
      desc(out_anchor, "out_anchor"), desc(out_anchor_score, "out_anchor_score"),
      desc(out_partner, "out_partner"), desc(out_partner_score, "out_partner_score")};
  auto fn = ring ? rlm_relation_select_packed_ring
                 : seq ? rlm_relation_select_packed_seq : rlm_relation_select_packed;
  check(fn(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8], &d[9], &d[10], &d[11],
           &d[12], &d[13], &d[14], local_window, top_blocks, k_out, strict_valid ? 1 : 0, &d[15],
           &d[16], &d[17], &d[18], stream),
        op);
  return {out_anchor, out_anchor_score, out_partner, out_partner_score};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> relation_select_packed(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid) {
  return select_packed_common(false, anchor_query, anchor_keys, anchor_router_query,
                              anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                              partner_base, partner_anchor_cache, partner_keys,
                              partner_block_mean, partner_block_std, partner_gamma, partner_bias,
                              position, local_window, top_blocks, k_out, strict_valid);
}

// Ring-buffer caches (no reference op): position p in cache row p mod T.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> relation_select_packed_ring(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid) {
  return select_packed_common(false, anchor_query, anchor_keys, anchor_router_query,
                              anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                              partner_base, partner_anchor_cache, partner_keys,
                              partner_block_mean, partner_block_std, partner_gamma, partner_bias,
                              position, local_window, top_blocks, k_out, strict_valid, true);
}

// relation_select_packed(_ring) with the token's expanded-cache row written
// into expanded_cache by the same launch (no reference op).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> relation_select_packed_expand_row(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid,
    const at::Tensor& operand_cache, const at::Tensor& expanded_weight,
    const c10::optional<at::Tensor>& expanded_bias, at::Tensor& expanded_cache, bool ring) {
  const char* op = "relation_lm::relation_select_packed_expand_row";
  c10::DeviceGuard guard(anchor_query.device());
  const at::Tensor xb = expanded_bias.has_value() ? *expanded_bias : at::Tensor();
  hipStream_t stream = device_stream(
      op, {&anchor_query, &anchor_keys, &anchor_router_query, &anchor_block_mean,
           &anchor_block_std, &anchor_gamma, &anchor_bias, &partner_base, &partner_anchor_cache,
           &partner_keys, &partner_block_mean, &partner_block_std, &partner_gamma, &partner_bias,
           &position, &operand_cache, &expanded_weight, &xb, &expanded_cache});
  TORCH_CHECK(anchor_query.dim() == 2, op, ": anchor_query must be [B,E]");
  TORCH_CHECK(k_out >= 0, op, ": k_out must be non-negative");
  const std::vector<int64_t> qshape{anchor_query.size(0)};
  const std::vector<int64_t> kshape{anchor_query.size(0), k_out};
  at::Tensor out_anchor = at::empty(qshape, i32(anchor_query));
  at::Tensor out_anchor_score = at::empty(qshape, f32(anchor_query));
  at::Tensor out_partner = at::empty(kshape, i32(anchor_query));
  at::Tensor out_partner_score = at::empty(kshape, f32(anchor_query));
  rlm_tensor d[23] = {
      desc(anchor_query, "anchor_query"), desc(anchor_keys, "anchor_keys"),
      desc(anchor_router_query, "anchor_router_query"),
      desc(anchor_block_mean, "anchor_block_mean"), desc(anchor_block_std, "anchor_block_std"),
      desc(anchor_gamma, "anchor_gamma"), desc(anchor_bias, "anchor_bias"),
      desc(partner_base, "partner_base"), desc(partner_anchor_cache, "partner_anchor_cache"),
      desc(partner_keys, "partner_keys"), desc(partner_block_mean, "partner_block_mean"),
      desc(partner_block_std, "partner_block_std"), desc(partner_gamma, "partner_gamma"),
      desc(partner_bias, "partner_bias"), desc(position, "position"),
      desc(operand_cache, "operand_cache"), desc(expanded_weight, "expanded_weight"),
      rlm_tensor{}, desc(expanded_cache, "expanded_cache"), desc(out_anchor, "out_anchor"),
      desc(out_anchor_score, "out_anchor_score"), desc(out_partner, "out_partner"),
      desc(out_partner_score, "out_partner_score")};
  if (xb.defined()) d[17] = desc(xb, "expanded_bias");
  check(rlm_relation_select_packed_expand_row(
            &d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8], &d[9], &d[10], &d[11],
            &d[12], &d[13], &d[14], local_window, top_blocks, k_out, strict_valid ? 1 : 0, &d[15],
            &d[16], xb.defined() ? &d[17] : nullptr, &d[18], ring ? 1 : 0, &d[19], &d[20],
            &d[21], &d[22], stream),
        op);
  return {out_anchor, out_anchor_score, out_partner, out_partner_score};
}

// relation_select_packed_seq with the whole expanded cache written into
// expanded_cache by the same launch where the shapes allow (no reference op).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> relation_select_packed_seq_expand(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid,
    const at::Tensor& operand_cache, const at::Tensor& expanded_weight,
    const c10::optional<at::Tensor>& expanded_bias, at::Tensor& expanded_cache) {
  const char* op = "relation_lm::relation_select_packed_seq_expand";
  c10::DeviceGuard guard(anchor_query.device());
  const at::Tensor xb = expanded_bias.has_value() ? *expanded_bias : at::Tensor();
  hipStream_t stream = device_stream(
      op, {&anchor_query, &anchor_keys, &anchor_router_query, &anchor_block_mean,
           &anchor_block_std, &anchor_gamma, &anchor_bias, &partner_base, &partner_anchor_cache,
           &partner_keys, &partner_block_mean, &partner_block_std, &partner_gamma, &partner_bias,
           &positions, &operand_cache, &expanded_weight, &xb, &expanded_cache});
  TORCH_CHECK(anchor_query.dim() == 3, op, ": anchor_query must be [B,Tq,E]");
  TORCH_CHECK(k_out >= 0, op, ": k_out must be non-negative");
  const std::vector<int64_t> qshape{anchor_query.size(0), anchor_query.size(1)};
  const std::vector<int64_t> kshape{anchor_query.size(0), anchor_query.size(1), k_out};
  at::Tensor out_anchor = at::empty(qshape, i32(anchor_query));
  at::Tensor out_anchor_score = at::empty(qshape, f32(anchor_query));
  at::Tensor out_partner = at::empty(kshape, i32(anchor_query));
  at::Tensor out_partner_score = at::empty(kshape, f32(anchor_query));
  rlm_tensor d[23] = {
      desc(anchor_query, "anchor_query"), desc(anchor_keys, "anchor_keys"),
      desc(anchor_router_query, "anchor_router_query"),
      desc(anchor_block_mean, "anchor_block_mean"), desc(anchor_block_std, "anchor_block_std"),
      desc(anchor_gamma, "anchor_gamma"), desc(anchor_bias, "anchor_bias"),
      desc(partner_base, "partner_base"), desc(partner_anchor_cache, "partner_anchor_cache"),
      desc(partner_keys, "partner_keys"), desc(partner_block_mean, "partner_block_mean"),
      desc(partner_block_std, "partner_block_std"), desc(partner_gamma, "partner_gamma"),
      desc(partner_bias, "partner_bias"), desc(positions, "positions"),
      desc(operand_cache, "operand_cache"), desc(expanded_weight, "expanded_weight"),
      rlm_tensor{}, desc(expanded_cache, "expanded_cache"), desc(out_anchor, "out_anchor"),
      desc(out_anchor_score, "out_anchor_score"), desc(out_partner, "out_partner"),
      desc(out_partner_score, "out_partner_score")};
  if (xb.defined()) d[17] = desc(xb, "expanded_bias");
  check(rlm_relation_select_packed_seq_expand(
            &d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8], &d[9], &d[10], &d[11],
            &d[12], &d[13], &d[14], local_window, top_blocks, k_out, strict_valid ? 1 : 0, &d[15],
            &d[16], xb.defined() ? &d[17] : nullptr, &d[18], &d[19], &d[20], &d[21], &d[22],
            stream),
        op);
  return {out_anchor, out_anchor_score, out_partner, out_partner_score};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> relation_select_packed_seq(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid) {
  return select_packed_common(true, anchor_query, anchor_keys, anchor_router_query,
                              anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                              partner_base, partner_anchor_cache, partner_keys,
                              partner_block_mean, partner_block_std, partner_gamma, partner_bias,
                              positions, local_window, top_blocks, k_out, strict_valid);
}

// Routed multi-anchor selection: no reference op (its semantics are the
// dense MultiAnchorRelationBlock's, multi_relation_blocks.py:69-147).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> multi_relation_select_seq(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys,
    const at::Tensor& anchor_router_query, const at::Tensor& anchor_block_mean,
    const at::Tensor& anchor_block_std, const at::Tensor& anchor_gamma,
    const at::Tensor& anchor_bias, const at::Tensor& partner_base,
    const at::Tensor& partner_anchor_cache, const at::Tensor& partner_keys,
    const at::Tensor& partner_block_mean, const at::Tensor& partner_block_std,
    const at::Tensor& partner_gamma, const at::Tensor& partner_bias, const at::Tensor& positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, bool strict_valid) {
  const char* op = "relation_lm::multi_relation_select_seq";
  c10::DeviceGuard guard(anchor_query.device());
  hipStream_t stream = device_stream(
      op, {&anchor_query, &anchor_keys, &anchor_router_query, &anchor_block_mean,
           &anchor_block_std, &anchor_gamma, &anchor_bias, &partner_base, &partner_anchor_cache,
           &partner_keys, &partner_block_mean, &partner_block_std, &partner_gamma, &partner_bias,
           &positions});
  TORCH_CHECK(anchor_query.dim() == 4, op, ": anchor_query must be [B,Tq,S,E]");
  TORCH_CHECK(k_out >= 0, op, ": k_out must be non-negative");
  std::vector<int64_t> qshape{anchor_query.size(0), anchor_query.size(1), anchor_query.size(2)};
  std::vector<int64_t> kshape = qshape;
  kshape.push_back(k_out);
  at::Tensor out_anchor = at::empty(qshape, i32(anchor_query));
  at::Tensor out_anchor_score = at::empty(qshape, f32(anchor_query));
  at::Tensor out_partner = at::empty(kshape, i32(anchor_query));
  at::Tensor out_partner_score = at::empty(kshape, f32(anchor_query));
  rlm_tensor d[19] = {
      desc(anchor_query, "anchor_query"), desc(anchor_keys, "anchor_keys"),
      desc(anchor_router_query, "anchor_router_query"),
      desc(anchor_block_mean, "anchor_block_mean"), desc(anchor_block_std, "anchor_block_std"),
      desc(anchor_gamma, "anchor_gamma"), desc(anchor_bias, "anchor_bias"),
      desc(partner_base, "partner_base"), desc(partner_anchor_cache, "partner_anchor_cache"),
      desc(partner_keys, "partner_keys"), desc(partner_block_mean, "partner_block_mean"),
      desc(partner_block_std, "partner_block_std"), desc(partner_gamma, "partner_gamma"),
      desc(partner_bias, "partner_bias"), desc(positions, "positions"),
      desc(out_anchor, "out_anchor"), desc(out_anchor_score, "out_anchor_score"),
      desc(out_partner, "out_partner"), desc(out_partner_score, "out_partner_score")};
  check(rlm_multi_relation_select_seq(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7],
                                      &d[8], &d[9], &d[10], &d[11], &d[12], &d[13], &d[14],
                                      local_window, top_blocks, k_out, strict_valid ? 1 : 0,
                                      &d[15], &d[16], &d[17], &d[18], stream),
        op);
  return {out_anchor, out_anchor_score, out_partner, out_partner_score};
}

std::tuple<at::Tensor, at::Tensor> anchor_select(
    const at::Tensor& anchor_query, const at::Tensor& anchor_keys, const at::Tensor& router_query,
    const at::Tensor& block_mean, const at::Tensor& block_std, const at::Tensor& gamma,
    const at::Tensor& bias, const at::Tensor& position, int64_t local_window, int64_t top_blocks,
    bool strict_valid) {
  const char* op = "relationlex::anchor_select";
  c10::DeviceGuard guard(anchor_query.device());
  hipStream_t stream = device_stream(op, {&anchor_query, &anchor_keys, &router_query,
                                          &block_mean, &block_std, &gamma, &bias, &position});
  TORCH_CHECK(anchor_query.dim() == 2, op, ": anchor_query must be [B,E]");
  at::Tensor out_index = at::empty({anchor_query.size(0)}, i32(anchor_query));
  at::Tensor out_score = at::empty({anchor_query.size(0)}, f32(anchor_query));
  rlm_tensor d[10] = {desc(anchor_query, "anchor_query"), desc(anchor_keys, "anchor_keys"),
                      desc(router_query, "router_query"), desc(block_mean, "block_mean"),
                      desc(block_std, "block_std"),       desc(gamma, "gamma"),
                      desc(bias, "bias"),                 desc(position, "position"),
                      desc(out_index, "out_index"),       desc(out_score, "out_score")};
  check(rlm_anchor_select(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], local_window,
                          top_blocks, strict_valid ? 1 : 0, &d[8], &d[9], stream),
        op);
  return {out_index, out_score};
}

std::tuple<at::Tensor, at::Tensor> partner_topk(
    const at::Tensor& partner_query, const at::Tensor& partner_keys,
    const at::Tensor& router_query, const at::Tensor& block_mean, const at::Tensor& block_std,
    const at::Tensor& gamma, const at::Tensor& bias, const at::Tensor& position,
    const at::Tensor& anchor_index, int64_t local_window, int64_t top_blocks, int64_t k_out,
    bool strict_valid) {
  const char* op = "relationlex::partner_topk";
  c10::DeviceGuard guard(partner_query.device());
  hipStream_t stream =
      device_stream(op, {&partner_query, &partner_keys, &router_query, &block_mean, &block_std,
                         &gamma, &bias, &position, &anchor_index});
  TORCH_CHECK(partner_query.dim() == 2, op, ": partner_query must be [B,E]");
  TORCH_CHECK(k_out >= 0, op, ": k_out must be non-negative");
  at::Tensor out_index = at::empty({partner_query.size(0), k_out}, i32(partner_query));
  at::Tensor out_score = at::empty({partner_query.size(0), k_out}, f32(partner_query));
  rlm_tensor d[11] = {desc(partner_query, "partner_query"), desc(partner_keys, "partner_keys"),
                      desc(router_query, "router_query"),   desc(block_mean, "block_mean"),
                      desc(block_std, "block_std"),         desc(gamma, "gamma"),
                      desc(bias, "bias"),                   desc(position, "position"),
                      desc(anchor_index, "anchor_index"),   desc(out_index, "out_index"),
                      desc(out_score, "out_score")};
  check(rlm_partner_topk(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8],
                         local_window, top_blocks, k_out, strict_valid ? 1 : 0, &d[9], &d[10],
                         stream),
        op);
  return {out_index, out_score};
}

at::Tensor hidden_common(bool seq, const at::Tensor& expanded_cache,
                         const at::Tensor& operand_cache, const at::Tensor& anchor_index,
                         const at::Tensor& partner_index, const at::Tensor& product_weight,
                         bool ring = false) {
  const char* op = ring  ? "relation_lm::relation_hidden_cached_ring"
                   : seq ? "relation_lm::relation_hidden_cached_seq"
                         : "relation_lm::relation_hidden_cached";
  c10::DeviceGuard guard(operand_cache.device());
  hipStream_t stream = device_stream(
      op, {&operand_cache, &expanded_cache, &anchor_index, &partner_index, &product_weight});
  TORCH_CHECK(partner_index.dim() == (seq ? 3 : 2), op, ": partner_index must be ",
              seq ? "[B,Tq,K]" : "[B,K]");
  TORCH_CHECK(product_weight.dim() == 2, op, ": product_weight must be [H,R]");
  std::vector<int64_t> shape = partner_index.sizes().vec();
  shape.push_back(product_weight.size(0));
  at::Tensor out = at::empty(shape, f32(operand_cache));
  rlm_tensor d[6] = {desc(expanded_cache, "expanded_cache"), desc(operand_cache, "operand_cache"),
                     desc(anchor_index, "anchor_index"),     desc(partner_index, "partner_index"),
                     desc(product_weight, "product_weight"), desc(out, "out")};
  auto fn = ring ? rlm_relation_hidden_cached_ring
                 : seq ? rlm_relation_hidden_cached_seq : rlm_relation_hidden_cached;
  check(fn(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], stream), op);
  return out;
}

at::Tensor relation_hidden_cached(const at::Tensor& expanded_cache,
                                  const at::Tensor& operand_cache,
                                  const at::Tensor& anchor_index,
                                  const at::Tensor& partner_index,
                                  const at::Tensor& product_weight) {
  return hidden_common(false, expanded_cache, operand_cache, anchor_index, partner_index,
                       product_weight);
}

at::Tensor relation_hidden_cached_ring(const at::Tensor& expanded_cache,
                                       const at::Tensor& operand_cache,
                                       const at::Tensor& anchor_index,
                                       const at::Tensor& partner_index,
                                       const at::Tensor& product_weight) {
  return hidden_common(false, expanded_cache, operand_cache, anchor_index, partner_index,
                       product_weight, true);
}

at::Tensor relation_hidden_cached_seq(const at::Tensor& expanded_cache,
                                      const at::Tensor& operand_cache,
                                      const at::Tensor& anchor_index,
                                      const at::Tensor& partner_index,
                                      const at::Tensor& product_weight) {
  return hidden_common(true, expanded_cache, operand_cache, anchor_index, partner_index,
                       product_weight);
}

// relation_hidden_cached_seq into a caller's [B,Tq,K,H] tensor, fp32 or bf16
// (bf16: the value a bf16 consumer rounds the fp32 hidden to).  No reference
// counterpart: the multi-anchor relation MLP feeds it to a bf16 Linear.
void relation_hidden_cached_seq_out(const at::Tensor& expanded_cache,
                                    const at::Tensor& operand_cache,
                                    const at::Tensor& anchor_index,
                                    const at::Tensor& partner_index,
                                    const at::Tensor& product_weight, at::Tensor& out) {
  const char* op = "relation_lm::relation_hidden_cached_seq_out";
  c10::DeviceGuard guard(operand_cache.device());
  hipStream_t stream = device_stream(
      op, {&operand_cache, &expanded_cache, &anchor_index, &partner_index, &product_weight, &out});
  TORCH_CHECK(out.is_contiguous(), op, ": out must be contiguous");
  rlm_tensor d[6] = {desc(expanded_cache, "expanded_cache"), desc(operand_cache, "operand_cache"),
                     desc(anchor_index, "anchor_index"),     desc(partner_index, "partner_index"),
                     desc(product_weight, "product_weight"), desc(out, "out")};
  check(rlm_relation_hidden_cached_seq(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], stream), op);
}

void relation_hidden_linear_seq_out(const at::Tensor& expanded_cache,
                                    const at::Tensor& operand_cache,
                                    const at::Tensor& anchor_index,
                                    const at::Tensor& partner_index,
                                    const at::Tensor& product_weight,
                                    const at::Tensor& second_weight, at::Tensor& out) {
  const char* op = "relation_lm::relation_hidden_linear_seq_out";
  c10::DeviceGuard guard(operand_cache.device());
  hipStream_t stream =
      device_stream(op, {&operand_cache, &expanded_cache, &anchor_index, &partner_index,
                         &product_weight, &second_weight, &out});
  TORCH_CHECK(out.is_contiguous(), op, ": out must be contiguous");
  rlm_tensor d[7] = {desc(expanded_cache, "expanded_cache"), desc(operand_cache, "operand_cache"),
                     desc(anchor_index, "anchor_index"),     desc(partner_index, "partner_index"),
                     desc(product_weight, "product_weight"), desc(second_weight, "second_weight"),
                     desc(out, "out")};
  check(rlm_relation_hidden_linear_seq(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], stream),
        op);
}

at::Tensor mfma_fragments(const at::Tensor& weight) {
  const char* op = "relation_lm::mfma_fragments";
  c10::DeviceGuard guard(weight.device());
  hipStream_t stream = device_stream(op, {&weight});
  TORCH_CHECK(weight.dim() == 2, op, ": weight must be 2-d");
  TORCH_CHECK(weight.size(0) % 32 == 0 && weight.size(1) % 16 == 0, op,
              ": weight rows must be a multiple of 32 and columns of 16");
  at::Tensor out = at::empty({weight.size(0) / 32, weight.size(1) / 16, 64, 8}, weight.options());
  rlm_tensor d[2] = {desc(weight, "weight"), desc(out, "out")};
  check(rlm_mfma_fragments(&d[0], &d[1], stream), op);
  return out;
}

at::Tensor hidden_update_common(bool ring, at::Tensor& expanded_cache,
                                const at::Tensor& operand_cache, const at::Tensor& anchor_index,
                                const at::Tensor& partner_index, const at::Tensor& anchor_weight,
                                const at::Tensor& partner_weight,
                                const at::Tensor& product_weight, const at::Tensor& first_bias,
                                const at::Tensor& position) {
  const char* op = ring ? "relation_lm::relation_hidden_cache_update_ring"
                        : "relation_lm::relation_hidden_cache_update";
  c10::DeviceGuard guard(operand_cache.device());
  hipStream_t stream = device_stream(
      op, {&operand_cache, &expanded_cache, &anchor_index, &partner_index, &anchor_weight,
           &partner_weight, &product_weight, &first_bias, &position});
  TORCH_CHECK(partner_index.dim() == 2, op, ": partner_index must be [B,K]");
  TORCH_CHECK(product_weight.dim() == 2, op, ": product_weight must be [H,R]");
  at::Tensor out = at::empty({partner_index.size(0), partner_index.size(1),
                              product_weight.size(0)},
                             f32(operand_cache));
  rlm_tensor d[10] = {desc(expanded_cache, "expanded_cache"), desc(operand_cache, "operand_cache"),
                      desc(anchor_index, "anchor_index"),     desc(partner_index, "partner_index"),
                      desc(anchor_weight, "anchor_weight"),   desc(partner_weight, "partner_weight"),
                      desc(product_weight, "product_weight"), desc(first_bias, "first_bias"),
                      desc(position, "position"),             desc(out, "out")};
  auto fn = ring ? rlm_relation_hidden_cache_update_ring : rlm_relation_hidden_cache_update;
  check(fn(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8], &d[9], stream), op);
  return out;
}

at::Tensor relation_hidden_cache_update(at::Tensor& expanded_cache,
                                        const at::Tensor& operand_cache,
                                        const at::Tensor& anchor_index,
                                        const at::Tensor& partner_index,
                                        const at::Tensor& anchor_weight,
                                        const at::Tensor& partner_weight,
                                        const at::Tensor& product_weight,
                                        const at::Tensor& first_bias,
                                        const at::Tensor& position) {
  return hidden_update_common(false, expanded_cache, operand_cache, anchor_index, partner_index,
                              anchor_weight, partner_weight, product_weight, first_bias,
                              position);
}

at::Tensor relation_hidden_cache_update_ring(at::Tensor& expanded_cache,
                                             const at::Tensor& operand_cache,
                                             const at::Tensor& anchor_index,
                                             const at::Tensor& partner_index,
                                             const at::Tensor& anchor_weight,
                                             const at::Tensor& partner_weight,
                                             const at::Tensor& product_weight,
                                             const at::Tensor& first_bias,
                                             const at::Tensor& position) {
  return hidden_update_common(true, expanded_cache, operand_cache, anchor_index, partner_index,
                              anchor_weight, partner_weight, product_weight, first_bias,
                              position);
}

at::Tensor norm_common(bool seq, const at::Tensor& raw, const at::Tensor& partner_scores,
                       const at::Tensor& norm_weight, const at::Tensor& norm_bias,
                       const at::Tensor& position, double norm_eps) {
  const char* op = seq ? "relation_lm::relation_norm_reduce_seq"
                       : "relation_lm::relation_norm_reduce";
  c10::DeviceGuard guard(raw.device());
  hipStream_t stream =
      device_stream(op, {&raw, &partner_scores, &norm_weight, &norm_bias, &position});
  TORCH_CHECK(raw.dim() == (seq ? 4 : 3), op, ": raw must be ", seq ? "[B,Tq,K,D]" : "[B,K,D]");
  std::vector<int64_t> shape{raw.size(0)};
  if (seq) shape.push_back(raw.size(1));
  shape.push_back(raw.size(raw.dim() - 1));
  at::Tensor out = at::empty(shape, f32(raw));
  rlm_tensor d[6] = {desc(raw, "raw"),           desc(partner_scores, "partner_scores"),
                     desc(norm_weight, "norm_weight"), desc(norm_bias, "norm_bias"),
                     desc(position, "position"), desc(out, "out")};
  auto fn = seq ? rlm_relation_norm_reduce_seq : rlm_relation_norm_reduce;
  check(fn(&d[0], &d[1], &d[2], &d[3], &d[4], norm_eps, &d[5], stream), op);
  return out;
}

at::Tensor relation_norm_reduce(const at::Tensor& raw, const at::Tensor& partner_scores,
                                const at::Tensor& norm_weight, const at::Tensor& norm_bias,
                                const at::Tensor& position, double norm_eps) {
  return norm_common(false, raw, partner_scores, norm_weight, norm_bias, position, norm_eps);
}

at::Tensor relation_norm_reduce_seq(const at::Tensor& raw, const at::Tensor& partner_scores,
                                    const at::Tensor& norm_weight, const at::Tensor& norm_bias,
                                    const at::Tensor& positions, double norm_eps) {
  return norm_common(true, raw, partner_scores, norm_weight, norm_bias, positions, norm_eps);
}

std::tuple<at::Tensor, at::Tensor> norm_output_common(
    bool seq, const at::Tensor& raw, const at::Tensor& partner_scores,
    const at::Tensor& norm_weight, const at::Tensor& norm_bias, const at::Tensor& position,
    double norm_eps, const at::Tensor& query, const at::Tensor& mix_logit,
    const at::Tensor& output_weight, const at::Tensor& output_bias, double output_eps) {
  const char* op = seq ? "relation_lm::relation_norm_reduce_output_seq"
                       : "relation_lm::relation_norm_reduce_output";
  c10::DeviceGuard guard(raw.device());
  hipStream_t stream =
      device_stream(op, {&raw, &partner_scores, &norm_weight, &norm_bias, &position, &query,
                         &mix_logit, &output_weight, &output_bias});
  TORCH_CHECK(raw.dim() == (seq ? 4 : 3), op, ": raw must be ", seq ? "[B,Tq,K,D]" : "[B,K,D]");
  std::vector<int64_t> shape{raw.size(0)};
  if (seq) shape.push_back(raw.size(1));
  shape.push_back(raw.size(raw.dim() - 1));
  at::Tensor context = at::empty(shape, f32(raw));
  at::Tensor final = at::empty(shape, query.options().memory_format(at::MemoryFormat::Contiguous));
  rlm_tensor d[11] = {desc(raw, "raw"),
                      desc(partner_scores, "partner_scores"),
                      desc(norm_weight, "norm_weight"),
                      desc(norm_bias, "norm_bias"),
                      desc(position, "position"),
                      desc(query, "query"),
                      desc(mix_logit, "mix_logit"),
                      desc(output_weight, "output_weight"),
                      desc(output_bias, "output_bias"),
                      desc(context, "out_context"),
                      desc(final, "out_final")};
  auto fn = seq ? rlm_relation_norm_reduce_output_seq : rlm_relation_norm_reduce_output;
  check(fn(&d[0], &d[1], &d[2], &d[3], &d[4], norm_eps, &d[5], &d[6], &d[7], &d[8], output_eps,
           &d[9], &d[10], stream),
        op);
  return {context, final};
}

std::tuple<at::Tensor, at::Tensor> relation_norm_reduce_output(
    const at::Tensor& raw, const at::Tensor& partner_scores, const at::Tensor& norm_weight,
    const at::Tensor& norm_bias, const at::Tensor& position, double norm_eps,
    const at::Tensor& query, const at::Tensor& mix_logit, const at::Tensor& output_weight,
    const at::Tensor& output_bias, double output_eps) {
  return norm_output_common(false, raw, partner_scores, norm_weight, norm_bias, position,
                            norm_eps, query, mix_logit, output_weight, output_bias, output_eps);
}

std::tuple<at::Tensor, at::Tensor> relation_norm_reduce_output_seq(
    const at::Tensor& raw, const at::Tensor& partner_scores, const at::Tensor& norm_weight,
    const at::Tensor& norm_bias, const at::Tensor& positions, double norm_eps,
    const at::Tensor& query, const at::Tensor& mix_logit, const at::Tensor& output_weight,
    const at::Tensor& output_bias, double output_eps) {
  return norm_output_common(true, raw, partner_scores, norm_weight, norm_bias, positions,
                            norm_eps, query, mix_logit, output_weight, output_bias, output_eps);
}

// The decode step's second linear and norm-reduce with the output-head
// preparation (no reference op): split-K partial products in a workspace, summed
// by the per-query norm kernel; other shapes run relation_linear then
// relation_norm_reduce_output.
std::tuple<at::Tensor, at::Tensor> relation_linear_norm_reduce_output(
    const at::Tensor& hidden, const at::Tensor& second_weight, const at::Tensor& second_bias,
    const at::Tensor& partner_scores, const at::Tensor& norm_weight, const at::Tensor& norm_bias,
    const at::Tensor& position, double norm_eps, const at::Tensor& query,
    const at::Tensor& mix_logit, const at::Tensor& output_weight, const at::Tensor& output_bias,
    double output_eps) {
  const char* op = "relation_lm::relation_linear_norm_reduce_output";
  c10::DeviceGuard guard(hidden.device());
  hipStream_t stream = device_stream(
      op, {&hidden, &second_weight, &second_bias, &partner_scores, &norm_weight, &norm_bias,
           &position, &query, &mix_logit, &output_weight, &output_bias});
  TORCH_CHECK(hidden.dim() == 3, op, ": hidden must be [B,K,H]");
  TORCH_CHECK(second_weight.dim() == 2, op, ": second_weight must be [D,H]");
  const int64_t B = hidden.size(0), K = hidden.size(1), H = hidden.size(2);
  const int64_t D = second_weight.size(0);
  at::Tensor context = at::empty({B, D}, f32(hidden));
  at::Tensor final = at::empty({B, D}, query.options().memory_format(at::MemoryFormat::Contiguous));
  const bool fused = B * K <= 64 && B <= 256 && K <= 16 && D % 4 == 0 && D <= 1024 &&
                     H <= 4 * 72 * 32 && second_weight.scalar_type() != at::kFloat &&
                     hidden.is_contiguous();
  if (!fused) {
    at::Tensor raw = at::empty({B, K, D}, f32(hidden));
    at::Tensor h2 = hidden.reshape({B * K, H});
    at::Tensor r2 = raw.view({B * K, D});
    rlm_tensor l[4] = {desc(h2, "input"), desc(second_weight, "weight"),
                       desc(second_bias, "bias"), desc(r2, "out")};
    check(rlm_linear(&l[0], &l[1], &l[2], &l[3], stream), op);
    rlm_tensor d[11] = {desc(raw, "raw"),          desc(partner_scores, "partner_scores"),
                        desc(norm_weight, "norm_weight"), desc(norm_bias, "norm_bias"),
                        desc(position, "position"), desc(query, "query"),
                        desc(mix_logit, "mix_logit"), desc(output_weight, "output_weight"),
                        desc(output_bias, "output_bias"), desc(context, "out_context"),
                        desc(final, "out_final")};
    check(rlm_relation_norm_reduce_output(&d[0], &d[1], &d[2], &d[3], &d[4], norm_eps, &d[5],
                                          &d[6], &d[7], &d[8], output_eps, &d[9], &d[10], stream),
          op);
    return {context, final};
  }
  // Splits of the hidden dim (at most four): enough that each split's 32-wide
  // slices fit the short load batch (24), then one more while the grid stays
  // within one workgroup per CU (256).
  const int64_t slices = (H + 31) / 32;
  const int64_t tiles = ((D + 15) / 16) * ((B * K + 15) / 16);
  int64_t splits = std::min<int64_t>(4, (slices + 23) / 24);
  while (splits < 4 && tiles * (splits + 1) <= 256 && slices >= 8 * (splits + 1)) ++splits;
  splits = std::max<int64_t>(1, splits);
  at::Tensor partials = at::empty({splits, B * K, D}, f32(hidden));
  rlm_tensor d[16] = {desc(hidden, "hidden"),
                      desc(second_weight, "second_weight"),
                      desc(second_bias, "second_bias"),
                      desc(partner_scores, "partner_scores"),
                      desc(norm_weight, "norm_weight"),
                      desc(norm_bias, "norm_bias"),
                      desc(position, "position"),
                      desc(query, "query"),
                      desc(mix_logit, "mix_logit"),
                      desc(output_weight, "output_weight"),
                      desc(output_bias, "output_bias"),
                      desc(partials, "partials"),
                      desc(context, "out_context"),
                      desc(final, "out_final")};
  check(rlm_relation_linear_norm_reduce_output(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6],
                                               norm_eps, &d[7], &d[8], &d[9], &d[10], output_eps,
                                               &d[11], &d[12], &d[13], stream),
        op);
  return {context, final};
}

at::Tensor relation_linear(const at::Tensor& input, const at::Tensor& weight,
                           const c10::optional<at::Tensor>& bias,
                           c10::optional<at::ScalarType> out_dtype);
// Counters of the one-launch decode tail: int32, zero before a launch and left
// zero by it (the last workgroup of each level resets its counter).  Each device
// has one buffer, zeroed once when it is created (outside graph capture), cut
// into fixed slots; a stream takes a slot at its first call (no kernel, so a
// capture stream gets one without recording a fill into the graph) and keeps
// it.  Launches on one stream are ordered, so they never share a counter
// concurrently.
constexpr int64_t kCounterSlots = 64;
constexpr int64_t kCounterSlot = 4096;  // int32 counters per stream: B * (groups + 1)

at::Tensor decode_counters(const char* op, const at::Tensor& like, hipStream_t stream) {
  static std::mutex mu;
  static std::map<int, at::Tensor> buffers;
  static std::map<int, int64_t> used;
  static std::map<std::pair<int, hipStream_t>, int64_t> slots;
  std::lock_guard<std::mutex> lock(mu);
  const int dev = static_cast<int>(like.device().index());
  auto buf = buffers.find(dev);
  if (buf == buffers.end()) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    check(hipStreamIsCapturing(stream, &status), op);
    TORCH_CHECK(status == hipStreamCaptureStatusNone, op,
                ": the first call on a device must run outside graph capture (it creates and "
                "zeroes the device's counter buffer)");
    buf = buffers.emplace(dev, at::zeros({kCounterSlots * kCounterSlot}, i32(like))).first;
    check(hipStreamSynchronize(stream), op);  // zeroed before any stream uses a slot
  }
  const auto key = std::make_pair(dev, stream);
  auto slot = slots.find(key);
  if (slot == slots.end()) {
    TORCH_CHECK(used[dev] < kCounterSlots, op, ": more than ", kCounterSlots,
                " streams on one device");
    slot = slots.emplace(key, used[dev]++).first;
  }
  return buf->second.narrow(0, slot->second * kCounterSlot, kCounterSlot);
}

std::tuple<at::Tensor, at::Tensor> relation_hidden_linear_norm_reduce_output(
    const at::Tensor& expanded_cache, const at::Tensor& operand_cache,
    const at::Tensor& anchor_index, const at::Tensor& partner_index,
    const at::Tensor& product_weight, const at::Tensor& second_weight,
    const at::Tensor& second_bias, const at::Tensor& partner_scores,
    const at::Tensor& norm_weight, const at::Tensor& norm_bias, const at::Tensor& position,
    double norm_eps, const at::Tensor& query, const at::Tensor& mix_logit,
    const at::Tensor& output_weight, const at::Tensor& output_bias, double output_eps,
    bool ring) {
  const char* op = "relation_lm::relation_hidden_linear_norm_reduce_output";
  c10::DeviceGuard guard(operand_cache.device());
  hipStream_t stream = device_stream(
      op, {&operand_cache, &expanded_cache, &anchor_index, &partner_index, &product_weight,
           &second_weight, &second_bias, &partner_scores, &norm_weight, &norm_bias, &position,
           &query, &mix_logit, &output_weight, &output_bias});
  TORCH_CHECK(partner_index.dim() == 2 && second_weight.dim() == 2 && product_weight.dim() == 2,
              op, ": partner_index must be [B,K], product_weight [H,R], second_weight [D,H]");
  bool fits;
  {
    const rlm_tensor e = desc(expanded_cache, "expanded_cache");
    const rlm_tensor o = desc(operand_cache, "operand_cache");
    const rlm_tensor pi = desc(partner_index, "partner_index");
    const rlm_tensor wm = desc(product_weight, "product_weight");
    const rlm_tensor w2 = desc(second_weight, "second_weight");
    fits = rlm_relation_hidden_linear_norm_reduce_output_fits(&e, &o, &pi, &wm, &w2) != 0;
  }
  const int64_t B = operand_cache.size(0), K = partner_index.size(1);
  const int64_t H = product_weight.size(0), D = second_weight.size(0);
  int64_t ws = 0, nctr = 0;
  if (fits) {
    check(rlm_relation_hidden_linear_norm_reduce_output_workspace(B, K, H, D, &ws, &nctr), op);
    fits = nctr <= kCounterSlot;
  }
  if (!fits) {
    // Shapes and dtypes the one-launch kernel does not take (fp32 caches, K > 8,
    // d_model > 768, more than 819 queries, ...) run the two-op form: the fp32
    // hidden, then the second linear with the norm-reduce and output head.
    at::Tensor hidden = ring ? relation_hidden_cached_ring(expanded_cache, operand_cache,
                                                           anchor_index, partner_index,
                                                           product_weight)
                             : relation_hidden_cached(expanded_cache, operand_cache, anchor_index,
                                                      partner_index, product_weight);
    return relation_linear_norm_reduce_output(hidden, second_weight, second_bias, partner_scores,
                                              norm_weight, norm_bias, position, norm_eps, query,
                                              mix_logit, output_weight, output_bias, output_eps);
  }
  at::Tensor workspace = at::empty({std::max<int64_t>(ws, 1)}, f32(operand_cache));
  at::Tensor counters = decode_counters(op, operand_cache, stream);
  at::Tensor context = at::empty({B, D}, f32(operand_cache));
  at::Tensor final = at::empty({B, D}, query.options().memory_format(at::MemoryFormat::Contiguous));
  rlm_tensor d[21] = {desc(expanded_cache, "expanded_cache"),
                      desc(operand_cache, "operand_cache"),
                      desc(anchor_index, "anchor_index"),
                      desc(partner_index, "partner_index"),
                      desc(product_weight, "product_weight"),
                      desc(second_weight, "second_weight"),
                      desc(second_bias, "second_bias"),
                      desc(partner_scores, "partner_scores"),
                      desc(norm_weight, "norm_weight"),
                      desc(norm_bias, "norm_bias"),
                      desc(position, "position"),
                      desc(query, "query"),
                      desc(mix_logit, "mix_logit"),
                      desc(output_weight, "output_weight"),
                      desc(output_bias, "output_bias"),
                      desc(workspace, "workspace"),
                      desc(counters, "counters"),
                      desc(context, "out_context"),
                      desc(final, "out_final")};
  check(rlm_relation_hidden_linear_norm_reduce_output(
            &d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8], &d[9], &d[10],
            norm_eps, &d[11], &d[12], &d[13], &d[14], output_eps, ring ? 1 : 0, &d[15], &d[16],
            &d[17], &d[18], stream),
        op);
  return {context, final};
}


at::Tensor relation_reduce_fused_seq(const at::Tensor& expanded_cache,
                                     const at::Tensor& operand_cache,
                                     const at::Tensor& anchor_index,
                                     const at::Tensor& partner_index,
                                     const at::Tensor& product_weight,
                                     const at::Tensor& second_weight,
                                     const at::Tensor& second_bias,
                                     const at::Tensor& partner_scores,
                                     const at::Tensor& norm_weight, const at::Tensor& norm_bias,
                                     const at::Tensor& positions, double norm_eps) {
  const char* op = "relation_lm::relation_reduce_fused_seq";
  c10::DeviceGuard guard(operand_cache.device());
  hipStream_t stream = device_stream(
      op, {&operand_cache, &expanded_cache, &anchor_index, &partner_index, &product_weight,
           &second_weight, &second_bias, &partner_scores, &norm_weight, &norm_bias, &positions});
  const bool frag = second_weight.dim() == 4;
  TORCH_CHECK(partner_index.dim() == 3 && (second_weight.dim() == 2 || frag), op,
              ": partner_index must be [B,Tq,K] and second_weight [D,H] or in MFMA fragment "
              "order [D/32,H/16,64,8]");
  const int64_t d_model = frag ? second_weight.size(0) * 32 : second_weight.size(0);
  {
    const rlm_tensor e = desc(expanded_cache, "expanded_cache");
    const rlm_tensor o = desc(operand_cache, "operand_cache");
    const rlm_tensor pi = desc(partner_index, "partner_index");
    const rlm_tensor wm = desc(product_weight, "product_weight");
    const rlm_tensor w2 = desc(second_weight, "second_weight");
    if (!rlm_relation_reduce_fused_seq_fits(&e, &o, &pi, &wm, &w2)) {
      TORCH_CHECK(!frag, op, ": a second_weight in fragment order needs the fused kernel's "
                  "shapes (bf16, d_model 128/256/384/512, K <= 16, relation dim 32/64/128); "
                  "pass the [D,H] weight for other shapes");
      // Shapes or dtypes the fused kernel does not take (fp32, d_model 576, ...):
      // the same result from the three-op chain it fuses, every step on HIP.
      const at::Tensor hidden = relation_hidden_cached_seq(expanded_cache, operand_cache,
                                                           anchor_index, partner_index,
                                                           product_weight);
      const at::Tensor raw = relation_linear(hidden, second_weight, second_bias, at::kFloat);
      return relation_norm_reduce_seq(raw, partner_scores, norm_weight, norm_bias, positions,
                                      norm_eps);
    }
  }
  at::Tensor out = at::empty({partner_index.size(0), partner_index.size(1), d_model},
                             f32(operand_cache));
  rlm_tensor d[12] = {desc(expanded_cache, "expanded_cache"), desc(operand_cache, "operand_cache"),
                      desc(anchor_index, "anchor_index"), desc(partner_index, "partner_index"),
                      desc(product_weight, "product_weight"), desc(second_weight, "second_weight"),
                      desc(second_bias, "second_bias"), desc(partner_scores, "partner_scores"),
                      desc(norm_weight, "norm_weight"), desc(norm_bias, "norm_bias"),
                      desc(positions, "positions"), desc(out, "out")};
  check(rlm_relation_reduce_fused_seq(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7],
                                      &d[8], &d[9], &d[10], norm_eps, &d[11], stream),
        op);
  return out;
}

at::Tensor linear_common(const char* op, const at::Tensor& input, const at::Tensor& weight,
                         const c10::optional<at::Tensor>& bias, at::ScalarType out_dtype,
                         bool packed) {
  c10::DeviceGuard guard(input.device());
  at::Tensor b = bias.has_value() ? *bias : at::Tensor();
  hipStream_t stream = device_stream(op, {&input, &weight, &b});
  TORCH_CHECK(weight.dim() == 2, op, ": weight must be 2-D");
  TORCH_CHECK(input.dim() >= 1 && input.size(-1) == weight.size(1), op,
              ": input width does not match weight");
  // Row-strided 2-d views (a cache column such as cache[:, t]) pass through
  // as they are; anything else is compacted first.
  at::Tensor x = input.reshape({-1, input.size(-1)});
  if ((x.size(1) > 1 && x.stride(1) != 1) || (x.size(0) > 1 && x.stride(0) % 8 != 0))
    x = x.contiguous();
  std::vector<int64_t> shape = input.sizes().vec();
  shape.back() = weight.size(0);
  at::Tensor out = at::empty({x.size(0), weight.size(0)}, input.options().dtype(out_dtype));
  rlm_tensor dx = desc(x, "input"), dw = desc(weight, "weight"), dout = desc(out, "out");
  hipError_t err;
  if (packed) {
    err = rlm_packed_sparse_cache_projection(&dx, &dw, &dout, stream);
  } else {
    rlm_tensor db{};
    if (b.defined()) db = desc(b, "bias");
    err = rlm_linear(&dx, &dw, b.defined() ? &db : nullptr, &dout, stream);
  }
  check(err, op);
  return out.view(shape);
}

// out = input @ weight^T (+ bias) written into a caller-provided 2-d view whose
// rows may be strided (a cache column such as expanded_cache[:, t]).
void relation_linear_out(const at::Tensor& input, const at::Tensor& weight,
                         const c10::optional<at::Tensor>& bias, at::Tensor& out) {
  const char* op = "relation_lm::relation_linear_out";
  c10::DeviceGuard guard(input.device());
  at::Tensor b = bias.has_value() ? *bias : at::Tensor();
  hipStream_t stream = device_stream(op, {&input, &weight, &b, &out});
  TORCH_CHECK(input.dim() == 2 && weight.dim() == 2 && out.dim() == 2, op,
              ": input, weight and out must be 2-D");
  rlm_tensor dx = desc(input, "input"), dw = desc(weight, "weight"), dout = desc(out, "out");
  rlm_tensor db{};
  if (b.defined()) db = desc(b, "bias");
  check(rlm_linear(&dx, &dw, b.defined() ? &db : nullptr, &dout, stream), op);
}

at::Tensor packed_sparse_cache_projection(const at::Tensor& memory, const at::Tensor& weight) {
  return linear_common("relation_lm::packed_sparse_cache_projection", memory, weight,
                       c10::nullopt, memory.scalar_type(), true);
}

at::Tensor relation_linear(const at::Tensor& input, const at::Tensor& weight,
                           const c10::optional<at::Tensor>& bias,
                           c10::optional<at::ScalarType> out_dtype) {
  return linear_common("relation_lm::relation_linear", input, weight, bias,
                       out_dtype.value_or(input.scalar_type()), false);
}

at::Tensor router_common(bool ring, const at::Tensor& anchor_raw, const at::Tensor& partner_raw,
                         at::Tensor& anchor_raw_cache, at::Tensor& partner_raw_cache,
                         at::Tensor& anchor_conv_cache, at::Tensor& partner_conv_cache,
                         at::Tensor& anchor_mean, at::Tensor& anchor_std,
                         at::Tensor& partner_mean, at::Tensor& partner_std,
                         const at::Tensor& anchor_conv_weight,
                         const at::Tensor& partner_conv_weight, const at::Tensor& position,
                         int64_t block_size) {
  const char* op = ring ? "relation_lm::router_cache_update_ring"
                        : "relation_lm::router_cache_update";
  c10::DeviceGuard guard(anchor_raw.device());
  hipStream_t stream = device_stream(
      op, {&anchor_raw, &partner_raw, &anchor_raw_cache, &partner_raw_cache, &anchor_conv_cache,
           &partner_conv_cache, &anchor_mean, &anchor_std, &partner_mean, &partner_std,
           &anchor_conv_weight, &partner_conv_weight, &position});
  TORCH_CHECK(anchor_raw.dim() == 2, op, ": anchor_raw must be [B,D]");
  at::Tensor out = at::empty({anchor_raw.size(0), 2, anchor_raw.size(1)}, f32(anchor_raw));
  rlm_tensor d[14] = {desc(anchor_raw, "anchor_raw"),
                      desc(partner_raw, "partner_raw"),
                      desc(anchor_raw_cache, "anchor_raw_cache"),
                      desc(partner_raw_cache, "partner_raw_cache"),
                      desc(anchor_conv_cache, "anchor_conv_cache"),
                      desc(partner_conv_cache, "partner_conv_cache"),
                      desc(anchor_mean, "anchor_mean"),
                      desc(anchor_std, "anchor_std"),
                      desc(partner_mean, "partner_mean"),
                      desc(partner_std, "partner_std"),
                      desc(anchor_conv_weight, "anchor_conv_weight"),
                      desc(partner_conv_weight, "partner_conv_weight"),
                      desc(position, "position"),
                      desc(out, "out")};
  auto fn = ring ? rlm_router_cache_update_ring : rlm_router_cache_update;
  check(fn(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7], &d[8], &d[9], &d[10], &d[11],
           &d[12], block_size, &d[13], stream),
        op);
  return out;
}

#define RLM_ROUTER_ARGS                                                                        \
  const at::Tensor &anchor_raw, const at::Tensor &partner_raw, at::Tensor &anchor_raw_cache,  \
      at::Tensor &partner_raw_cache, at::Tensor &anchor_conv_cache,                           \
      at::Tensor &partner_conv_cache, at::Tensor &anchor_mean, at::Tensor &anchor_std,        \
      at::Tensor &partner_mean, at::Tensor &partner_std,                                      \
      const at::Tensor &anchor_conv_weight, const at::Tensor &partner_conv_weight,            \
      const at::Tensor &position, int64_t block_size
#define RLM_ROUTER_PASS                                                                       \
  anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache, anchor_conv_cache,            \
      partner_conv_cache, anchor_mean, anchor_std, partner_mean, partner_std,                 \
      anchor_conv_weight, partner_conv_weight, position, block_size

at::Tensor router_cache_update(RLM_ROUTER_ARGS) { return router_common(false, RLM_ROUTER_PASS); }
at::Tensor router_cache_update_ring(RLM_ROUTER_ARGS) { return router_common(true, RLM_ROUTER_PASS); }
#undef RLM_ROUTER_ARGS
#undef RLM_ROUTER_PASS

// Packed projection plus the token's cache-row writes (no reference op).
at::Tensor packed_projection_to_caches(const at::Tensor& memory, const at::Tensor& weight,
                                       at::Tensor& anchor_keys, at::Tensor& partner_keys,
                                       at::Tensor& operand_cache, at::Tensor& partner_anchor_cache,
                                       const at::Tensor& position, bool ring) {
  const char* op = "relation_lm::packed_projection_to_caches";
  c10::DeviceGuard guard(memory.device());
  hipStream_t stream = device_stream(op, {&memory, &weight, &anchor_keys, &partner_keys,
                                          &operand_cache, &partner_anchor_cache, &position});
  TORCH_CHECK(memory.dim() == 2, op, ": memory must be [B, Din]");
  TORCH_CHECK(weight.dim() == 2, op, ": weight must be [Dout, Din]");
  at::Tensor out = at::empty({memory.size(0), weight.size(0)}, memory.options());
  rlm_tensor d[8] = {desc(memory, "memory"),       desc(weight, "weight"),
                     desc(out, "out"),             desc(anchor_keys, "anchor_keys"),
                     desc(partner_keys, "partner_keys"), desc(operand_cache, "operand_cache"),
                     desc(partner_anchor_cache, "partner_anchor_cache"),
                     desc(position, "position")};
  check(rlm_packed_projection_to_caches(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7],
                                        ring ? 1 : 0, stream),
        op);
  return out;
}

// Packed projection with its cache-row writes and the router cache update as
// one launch (the reference's roadmap item, README.md:148-149; no reference op).
std::tuple<at::Tensor, at::Tensor> packed_projection_router_update(
    const at::Tensor& memory, const at::Tensor& weight, at::Tensor& anchor_keys,
    at::Tensor& partner_keys, at::Tensor& operand_cache, at::Tensor& partner_anchor_cache,
    const at::Tensor& position, bool ring, at::Tensor& anchor_raw_cache,
    at::Tensor& partner_raw_cache, at::Tensor& anchor_conv_cache, at::Tensor& partner_conv_cache,
    at::Tensor& anchor_mean, at::Tensor& anchor_std, at::Tensor& partner_mean,
    at::Tensor& partner_std, const at::Tensor& anchor_conv_weight,
    const at::Tensor& partner_conv_weight, int64_t block_size) {
  const char* op = "relation_lm::packed_projection_router_update";
  c10::DeviceGuard guard(memory.device());
  hipStream_t stream = device_stream(
      op, {&memory, &weight, &anchor_keys, &partner_keys, &operand_cache, &partner_anchor_cache,
           &position, &anchor_raw_cache, &partner_raw_cache, &anchor_conv_cache,
           &partner_conv_cache, &anchor_mean, &anchor_std, &partner_mean, &partner_std,
           &anchor_conv_weight, &partner_conv_weight});
  TORCH_CHECK(memory.dim() == 2, op, ": memory must be [B, Din]");
  TORCH_CHECK(weight.dim() == 2, op, ": weight must be [Dout, Din]");
  TORCH_CHECK(anchor_raw_cache.dim() == 3, op, ": router caches must be [B, T, D]");
  at::Tensor out = at::empty({memory.size(0), weight.size(0)}, memory.options());
  at::Tensor rout = at::empty({memory.size(0), 2, anchor_raw_cache.size(2)}, f32(memory));
  rlm_tensor d[19] = {desc(memory, "memory"),
                      desc(weight, "weight"),
                      desc(out, "out"),
                      desc(anchor_keys, "anchor_keys"),
                      desc(partner_keys, "partner_keys"),
                      desc(operand_cache, "operand_cache"),
                      desc(partner_anchor_cache, "partner_anchor_cache"),
                      desc(position, "position"),
                      desc(anchor_raw_cache, "anchor_raw_cache"),
                      desc(partner_raw_cache, "partner_raw_cache"),
                      desc(anchor_conv_cache, "anchor_conv_cache"),
                      desc(partner_conv_cache, "partner_conv_cache"),
                      desc(anchor_mean, "anchor_mean"),
                      desc(anchor_std, "anchor_std"),
                      desc(partner_mean, "partner_mean"),
                      desc(partner_std, "partner_std"),
                      desc(anchor_conv_weight, "anchor_conv_weight"),
                      desc(partner_conv_weight, "partner_conv_weight"),
                      desc(rout, "router_out")};
  check(rlm_packed_projection_router_update(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6],
                                            &d[7], ring ? 1 : 0, &d[8], &d[9], &d[10], &d[11],
                                            &d[12], &d[13], &d[14], &d[15], &d[16], &d[17],
                                            block_size, &d[18], stream),
        op);
  return {out, rout};
}

at::Tensor multi_relation_reduce_seq(const at::Tensor& raw, const at::Tensor& partner_scores,
                                    const at::Tensor& norm_weight, const at::Tensor& norm_bias,
                                    const at::Tensor& slot_mix_logits,
                                    const at::Tensor& residual_gate, const at::Tensor& hidden,
                                    const at::Tensor& positions, double norm_eps,
                                    const c10::optional<at::Tensor>& raw_bias) {
  const char* op = "relation_lm::multi_relation_reduce_seq";
  const at::Tensor rb = raw_bias.has_value() ? *raw_bias : at::Tensor();
  c10::DeviceGuard guard(raw.device());
  hipStream_t stream = device_stream(op, {&raw, &partner_scores, &norm_weight, &norm_bias,
                                          &slot_mix_logits, &residual_gate, &hidden, &positions,
                                          &rb});
  TORCH_CHECK(raw.dim() == 5 && partner_scores.dim() == 4, op,
              ": raw must be [B,Tq,S,K,D] and partner_scores [B,Tq,S,K]");
  const at::Tensor rows = raw.reshape({raw.size(0), raw.size(1), raw.size(2) * raw.size(3),
                                       raw.size(4)});
  at::Tensor out = at::empty_like(hidden, hidden.options().memory_format(at::MemoryFormat::Contiguous));
  rlm_tensor d[10] = {desc(rows, "raw"),
                     desc(partner_scores, "partner_scores"),
                     desc(norm_weight, "norm_weight"),
                     desc(norm_bias, "norm_bias"),
                     desc(slot_mix_logits, "slot_mix_logits"),
                     desc(residual_gate, "residual_gate"),
                     desc(hidden, "hidden"),
                     desc(positions, "positions"),
                     desc(out, "out"),
                     rlm_tensor{}};
  if (rb.defined()) d[9] = desc(rb, "raw_bias");
  check(rlm_multi_relation_reduce_seq(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7],
                                      norm_eps, &d[8], nullptr, rb.defined() ? &d[9] : nullptr,
                                      stream),
        op);
  return out;
}

// multi_relation_reduce_seq into caller tensors: out (hidden's shape and
// dtype; a batch-row slice of a larger output) and, when given, the fp32
// relation context.
void multi_relation_reduce_seq_out(const at::Tensor& raw, const at::Tensor& partner_scores,
                                   const at::Tensor& norm_weight, const at::Tensor& norm_bias,
                                   const at::Tensor& slot_mix_logits,
                                   const at::Tensor& residual_gate, const at::Tensor& hidden,
                                   const at::Tensor& positions, double norm_eps,
                                   const c10::optional<at::Tensor>& raw_bias, at::Tensor& out,
                                   const c10::optional<at::Tensor>& context) {
  const char* op = "relation_lm::multi_relation_reduce_seq_out";
  const at::Tensor rb = raw_bias.has_value() ? *raw_bias : at::Tensor();
  const at::Tensor ctx = context.has_value() ? *context : at::Tensor();
  c10::DeviceGuard guard(raw.device());
  hipStream_t stream = device_stream(op, {&raw, &partner_scores, &norm_weight, &norm_bias,
                                          &slot_mix_logits, &residual_gate, &hidden, &positions,
                                          &rb, &out, &ctx});
  TORCH_CHECK(raw.dim() == 5 && partner_scores.dim() == 4, op,
              ": raw must be [B,Tq,S,K,D] and partner_scores [B,Tq,S,K]");
  const at::Tensor rows = raw.reshape({raw.size(0), raw.size(1), raw.size(2) * raw.size(3),
                                       raw.size(4)});
  rlm_tensor d[11] = {desc(rows, "raw"),
                      desc(partner_scores, "partner_scores"),
                      desc(norm_weight, "norm_weight"),
                      desc(norm_bias, "norm_bias"),
                      desc(slot_mix_logits, "slot_mix_logits"),
                      desc(residual_gate, "residual_gate"),
                      desc(hidden, "hidden"),
                      desc(positions, "positions"),
                      desc(out, "out"),
                      rlm_tensor{},
                      rlm_tensor{}};
  if (ctx.defined()) d[9] = desc(ctx, "context");
  if (rb.defined()) d[10] = desc(rb, "raw_bias");
  check(rlm_multi_relation_reduce_seq(&d[0], &d[1], &d[2], &d[3], &d[4], &d[5], &d[6], &d[7],
                                      norm_eps, &d[8], ctx.defined() ? &d[9] : nullptr,
                                      rb.defined() ? &d[10] : nullptr, stream),
        op);
}

at::Tensor layer_norm(const at::Tensor& input, const at::Tensor& weight, const at::Tensor& bias,
                      double eps) {
  const char* op = "relation_lm::layer_norm";
  c10::DeviceGuard guard(input.device());
  hipStream_t stream = device_stream(op, {&input, &weight, &bias});
  TORCH_CHECK(input.dim() >= 1, op, ": input must have at least one dimension");
  const at::Tensor x = input.reshape({-1, input.size(-1)});
  at::Tensor out = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  rlm_tensor d[4] = {desc(x, "input"), desc(weight, "weight"), desc(bias, "bias"),
                     desc(out, "out")};
  check(rlm_layer_norm(&d[0], &d[1], &d[2], eps, &d[3], stream), op);
  return out.view(input.sizes());
}

std::tuple<at::Tensor, at::Tensor> block_statistics(const at::Tensor& keys, int64_t block_size) {
  const char* op = "relation_lm::block_statistics";
  c10::DeviceGuard guard(keys.device());
  hipStream_t stream = device_stream(op, {&keys});
  TORCH_CHECK(keys.dim() == 3 && block_size > 0, op,
              ": keys must be [B,T,C] and block_size positive");
  const int64_t nb = keys.size(1) / block_size;
  at::Tensor mean = at::empty({keys.size(0), nb, keys.size(2)}, f32(keys));
  at::Tensor std_ = at::empty({keys.size(0), nb, keys.size(2)}, f32(keys));
  rlm_tensor d[3] = {desc(keys, "keys"), desc(mean, "out_mean"), desc(std_, "out_std")};
  check(rlm_block_statistics(&d[0], block_size, &d[1], &d[2], stream), op);
  return {mean, std_};
}

}  // namespace

TORCH_LIBRARY(relation_lm, m) {
  m.def(
      "relation_select_packed(Tensor anchor_query, Tensor anchor_keys, Tensor "
      "anchor_router_query, Tensor anchor_block_mean, Tensor anchor_block_std, Tensor "
      "anchor_gamma, Tensor anchor_bias, Tensor partner_base, Tensor partner_anchor_cache, "
      "Tensor partner_keys, Tensor partner_block_mean, Tensor partner_block_std, Tensor "
      "partner_gamma, Tensor partner_bias, Tensor position, SymInt local_window, SymInt "
      "top_blocks, SymInt k_out, bool strict_valid) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def(
      "relation_select_packed_seq(Tensor anchor_query, Tensor anchor_keys, Tensor "
      "anchor_router_query, Tensor anchor_block_mean, Tensor anchor_block_std, Tensor "
      "anchor_gamma, Tensor anchor_bias, Tensor partner_base, Tensor partner_anchor_cache, "
      "Tensor partner_keys, Tensor partner_block_mean, Tensor partner_block_std, Tensor "
      "partner_gamma, Tensor partner_bias, Tensor positions, SymInt local_window, SymInt "
      "top_blocks, SymInt k_out, bool strict_valid) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def(
      "relation_select_packed_seq_expand(Tensor anchor_query, Tensor anchor_keys, Tensor "
      "anchor_router_query, Tensor anchor_block_mean, Tensor anchor_block_std, Tensor "
      "anchor_gamma, Tensor anchor_bias, Tensor partner_base, Tensor partner_anchor_cache, "
      "Tensor partner_keys, Tensor partner_block_mean, Tensor partner_block_std, Tensor "
      "partner_gamma, Tensor partner_bias, Tensor positions, SymInt local_window, SymInt "
      "top_blocks, SymInt k_out, bool strict_valid, Tensor operand_cache, Tensor "
      "expanded_weight, Tensor? expanded_bias, Tensor(a!) expanded_cache) -> "
      "(Tensor, Tensor, Tensor, Tensor)");
  m.def(
      "relation_select_packed_expand_row(Tensor anchor_query, Tensor anchor_keys, Tensor "
      "anchor_router_query, Tensor anchor_block_mean, Tensor anchor_block_std, Tensor "
      "anchor_gamma, Tensor anchor_bias, Tensor partner_base, Tensor partner_anchor_cache, "
      "Tensor partner_keys, Tensor partner_block_mean, Tensor partner_block_std, Tensor "
      "partner_gamma, Tensor partner_bias, Tensor position, SymInt local_window, SymInt "
      "top_blocks, SymInt k_out, bool strict_valid, Tensor operand_cache, Tensor "
      "expanded_weight, Tensor? expanded_bias, Tensor(a!) expanded_cache, bool ring=False) -> "
      "(Tensor, Tensor, Tensor, Tensor)");
  m.def(
      "multi_relation_select_seq(Tensor anchor_query, Tensor anchor_keys, Tensor "
      "anchor_router_query, Tensor anchor_block_mean, Tensor anchor_block_std, Tensor "
      "anchor_gamma, Tensor anchor_bias, Tensor partner_base, Tensor partner_anchor_cache, "
      "Tensor partner_keys, Tensor partner_block_mean, Tensor partner_block_std, Tensor "
      "partner_gamma, Tensor partner_bias, Tensor positions, SymInt local_window, SymInt "
      "top_blocks, SymInt k_out, bool strict_valid) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def(
      "relation_hidden_cached(Tensor expanded_cache, Tensor operand_cache, Tensor anchor_index, "
      "Tensor partner_index, Tensor product_weight) -> Tensor");
  m.def(
      "relation_hidden_cached_seq(Tensor expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor product_weight) -> Tensor");
  m.def(
      "relation_hidden_cache_update(Tensor(a!) expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor anchor_weight, Tensor partner_weight, Tensor "
      "product_weight, Tensor first_bias, Tensor position) -> Tensor");
  m.def(
      "relation_norm_reduce(Tensor raw, Tensor partner_scores, Tensor norm_weight, Tensor "
      "norm_bias, Tensor position, float norm_eps) -> Tensor");
  m.def(
      "relation_norm_reduce_seq(Tensor raw, Tensor partner_scores, Tensor norm_weight, Tensor "
      "norm_bias, Tensor positions, float norm_eps) -> Tensor");
  m.def(
      "relation_reduce_fused_seq(Tensor expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor product_weight, Tensor second_weight, Tensor "
      "second_bias, Tensor partner_scores, Tensor norm_weight, Tensor norm_bias, Tensor "
      "positions, float norm_eps) -> Tensor");
  m.def(
      "router_cache_update(Tensor anchor_raw, Tensor partner_raw, Tensor(a!) anchor_raw_cache, "
      "Tensor(b!) partner_raw_cache, Tensor(c!) anchor_conv_cache, Tensor(d!) partner_conv_cache, "
      "Tensor(e!) anchor_mean, Tensor(f!) anchor_std, Tensor(g!) partner_mean, Tensor(h!) "
      "partner_std, Tensor anchor_conv_weight, Tensor partner_conv_weight, Tensor position, "
      "SymInt block_size) -> Tensor");
  // Ring-buffer forms (no reference op): the schemas of the linear ops.
  m.def(
      "relation_select_packed_ring(Tensor anchor_query, Tensor anchor_keys, Tensor "
      "anchor_router_query, Tensor anchor_block_mean, Tensor anchor_block_std, Tensor "
      "anchor_gamma, Tensor anchor_bias, Tensor partner_base, Tensor partner_anchor_cache, "
      "Tensor partner_keys, Tensor partner_block_mean, Tensor partner_block_std, Tensor "
      "partner_gamma, Tensor partner_bias, Tensor position, SymInt local_window, SymInt "
      "top_blocks, SymInt k_out, bool strict_valid) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def(
      "relation_hidden_cached_ring(Tensor expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor product_weight) -> Tensor");
  m.def(
      "relation_hidden_cache_update_ring(Tensor(a!) expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor anchor_weight, Tensor partner_weight, Tensor "
      "product_weight, Tensor first_bias, Tensor position) -> Tensor");
  m.def(
      "router_cache_update_ring(Tensor anchor_raw, Tensor partner_raw, Tensor(a!) "
      "anchor_raw_cache, Tensor(b!) partner_raw_cache, Tensor(c!) anchor_conv_cache, Tensor(d!) "
      "partner_conv_cache, Tensor(e!) anchor_mean, Tensor(f!) anchor_std, Tensor(g!) "
      "partner_mean, Tensor(h!) partner_std, Tensor anchor_conv_weight, Tensor "
      "partner_conv_weight, Tensor position, SymInt block_size) -> Tensor");
  m.def("packed_sparse_cache_projection(Tensor memory, Tensor weight) -> Tensor");
  m.def(
      "packed_projection_to_caches(Tensor memory, Tensor weight, Tensor(a!) anchor_keys, "
      "Tensor(b!) partner_keys, Tensor(c!) operand_cache, Tensor(d!) partner_anchor_cache, "
      "Tensor position, bool ring=False) -> Tensor");
  m.def(
      "packed_projection_router_update(Tensor memory, Tensor weight, Tensor(a!) anchor_keys, "
      "Tensor(b!) partner_keys, Tensor(c!) operand_cache, Tensor(d!) partner_anchor_cache, "
      "Tensor position, bool ring, Tensor(e!) anchor_raw_cache, Tensor(f!) partner_raw_cache, "
      "Tensor(g!) anchor_conv_cache, Tensor(h!) partner_conv_cache, Tensor(i!) anchor_block_mean, "
      "Tensor(j!) anchor_block_std, Tensor(k!) partner_block_mean, Tensor(l!) partner_block_std, "
      "Tensor anchor_conv_weight, Tensor partner_conv_weight, SymInt block_size) -> (Tensor, Tensor)");
  m.def(
      "relation_linear_norm_reduce_output(Tensor hidden, Tensor second_weight, Tensor "
      "second_bias, Tensor partner_scores, Tensor norm_weight, Tensor norm_bias, Tensor "
      "position, float norm_eps, Tensor query, Tensor mix_logit, Tensor output_weight, Tensor "
      "output_bias, float output_eps) -> (Tensor, Tensor)");
  m.def(
      "relation_hidden_linear_norm_reduce_output(Tensor expanded_cache, Tensor operand_cache, "
      "Tensor anchor_index, Tensor partner_index, Tensor product_weight, Tensor second_weight, "
      "Tensor second_bias, Tensor partner_scores, Tensor norm_weight, Tensor norm_bias, Tensor "
      "position, float norm_eps, Tensor query, Tensor mix_logit, Tensor output_weight, Tensor "
      "output_bias, float output_eps, bool ring=False) -> (Tensor, Tensor)");
  m.def(
      "relation_linear(Tensor input, Tensor weight, Tensor? bias=None, ScalarType? "
      "out_dtype=None) -> Tensor");
  m.def(
      "relation_linear_out(Tensor input, Tensor weight, Tensor? bias, Tensor(a!) out) -> ()");
  m.def(
      "relation_hidden_cached_seq_out(Tensor expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor product_weight, Tensor(a!) out) -> ()");
  // The relation MLP's hidden and bias-free second Linear in one launch (the
  // reference runs nn.Linear -> GELU -> nn.Linear, multi_relation_blocks.py:47-52).
  m.def(
      "relation_hidden_linear_seq_out(Tensor expanded_cache, Tensor operand_cache, Tensor "
      "anchor_index, Tensor partner_index, Tensor product_weight, Tensor second_weight, "
      "Tensor(a!) out) -> ()");
  m.def("mfma_fragments(Tensor weight) -> Tensor");
  // Multi-anchor relation block (no reference op: the reference runs these in
  // eager torch inside MultiAnchorRelationBlock / DistilledBlockRouter).
  m.def(
      "multi_relation_reduce_seq(Tensor raw, Tensor partner_scores, Tensor norm_weight, Tensor "
      "norm_bias, Tensor slot_mix_logits, Tensor residual_gate, Tensor hidden, Tensor positions, "
      "float norm_eps, Tensor? raw_bias=None) -> Tensor");
  m.def(
      "multi_relation_reduce_seq_out(Tensor raw, Tensor partner_scores, Tensor norm_weight, "
      "Tensor norm_bias, Tensor slot_mix_logits, Tensor residual_gate, Tensor hidden, Tensor "
      "positions, float norm_eps, Tensor? raw_bias, Tensor(a!) out, Tensor(b!)? context=None) "
      "-> ()");
  m.def("layer_norm(Tensor input, Tensor weight, Tensor bias, float eps) -> Tensor");
  // Norm-reduce with the last-token output preparation as its epilogue
  // (roadmap item of the reference, README.md:150-151; relation_lm.py:203-206).
  m.def(
      "relation_norm_reduce_output(Tensor raw, Tensor partner_scores, Tensor norm_weight, Tensor "
      "norm_bias, Tensor position, float norm_eps, Tensor query, Tensor mix_logit, Tensor "
      "output_weight, Tensor output_bias, float output_eps) -> (Tensor, Tensor)");
  m.def(
      "relation_norm_reduce_output_seq(Tensor raw, Tensor partner_scores, Tensor norm_weight, "
      "Tensor norm_bias, Tensor positions, float norm_eps, Tensor query, Tensor mix_logit, Tensor "
      "output_weight, Tensor output_bias, float output_eps) -> (Tensor, Tensor)");
  m.def("block_statistics(Tensor keys, SymInt block_size) -> (Tensor, Tensor)");
}

TORCH_LIBRARY(relationlex, m) {
  m.def(
      "anchor_select(Tensor anchor_query, Tensor anchor_keys, Tensor router_query, Tensor "
      "block_mean, Tensor block_std, Tensor gamma, Tensor bias, Tensor position, SymInt "
      "local_window, SymInt top_blocks, bool strict_valid) -> (Tensor, Tensor)");
  m.def(
      "partner_topk(Tensor partner_query, Tensor partner_keys, Tensor router_query, Tensor "
      "block_mean, Tensor block_std, Tensor gamma, Tensor bias, Tensor position, Tensor "
      "anchor_index, SymInt local_window, SymInt top_blocks, SymInt k_out, bool strict_valid) "
      "-> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(relation_lm, CUDA, m) {
  m.impl("relation_select_packed", TORCH_FN(relation_select_packed));
  m.impl("relation_select_packed_seq", TORCH_FN(relation_select_packed_seq));
  m.impl("relation_select_packed_expand_row", TORCH_FN(relation_select_packed_expand_row));
  m.impl("relation_select_packed_seq_expand", TORCH_FN(relation_select_packed_seq_expand));
  m.impl("multi_relation_select_seq", TORCH_FN(multi_relation_select_seq));
  m.impl("relation_hidden_cached", TORCH_FN(relation_hidden_cached));
  m.impl("relation_hidden_cached_seq", TORCH_FN(relation_hidden_cached_seq));
  m.impl("relation_hidden_cache_update", TORCH_FN(relation_hidden_cache_update));
  m.impl("relation_norm_reduce", TORCH_FN(relation_norm_reduce));
  m.impl("relation_norm_reduce_seq", TORCH_FN(relation_norm_reduce_seq));
  m.impl("relation_reduce_fused_seq", TORCH_FN(relation_reduce_fused_seq));
  m.impl("router_cache_update", TORCH_FN(router_cache_update));
  m.impl("relation_select_packed_ring", TORCH_FN(relation_select_packed_ring));
  m.impl("relation_hidden_cached_ring", TORCH_FN(relation_hidden_cached_ring));
  m.impl("relation_hidden_cache_update_ring", TORCH_FN(relation_hidden_cache_update_ring));
  m.impl("router_cache_update_ring", TORCH_FN(router_cache_update_ring));
  m.impl("packed_sparse_cache_projection", TORCH_FN(packed_sparse_cache_projection));
  m.impl("packed_projection_to_caches", TORCH_FN(packed_projection_to_caches));
  m.impl("packed_projection_router_update", TORCH_FN(packed_projection_router_update));
  m.impl("relation_linear_norm_reduce_output", TORCH_FN(relation_linear_norm_reduce_output));
  m.impl("relation_hidden_linear_norm_reduce_output",
         TORCH_FN(relation_hidden_linear_norm_reduce_output));
  m.impl("relation_linear", TORCH_FN(relation_linear));
  m.impl("relation_linear_out", TORCH_FN(relation_linear_out));
  m.impl("relation_hidden_cached_seq_out", TORCH_FN(relation_hidden_cached_seq_out));
  m.impl("relation_hidden_linear_seq_out", TORCH_FN(relation_hidden_linear_seq_out));
  m.impl("mfma_fragments", TORCH_FN(mfma_fragments));
  m.impl("multi_relation_reduce_seq", TORCH_FN(multi_relation_reduce_seq));
  m.impl("multi_relation_reduce_seq_out", TORCH_FN(multi_relation_reduce_seq_out));
  m.impl("layer_norm", TORCH_FN(layer_norm));
  m.impl("relation_norm_reduce_output", TORCH_FN(relation_norm_reduce_output));
  m.impl("relation_norm_reduce_output_seq", TORCH_FN(relation_norm_reduce_output_seq));
  m.impl("block_statistics", TORCH_FN(block_statistics));
}

// CPU tensors: the reference's PackedSparseCacheProjection.project is F.linear
// (src/relation_lm/inference/packed_cache.py:52-57), which runs on the CPU.
TORCH_LIBRARY_IMPL(relation_lm, CPU, m) {
  m.impl("packed_sparse_cache_projection", [](const at::Tensor& memory, const at::Tensor& weight) {
    TORCH_CHECK(weight.device() == memory.device(),
                "relation_lm::packed_sparse_cache_projection: memory and weight must share a device");
    return at::linear(memory, weight);
  });
}

TORCH_LIBRARY_IMPL(relationlex, CUDA, m) {
  m.impl("anchor_select", TORCH_FN(anchor_select));
  m.impl("partner_topk", TORCH_FN(partner_topk));
}
