// PyTorch-ROCm operator boundary for libtrianglemix.so.
//
// Registers the reference adapter's schemas
// (operator/torch_adapter/triangle_paged_attention_torch.cpp:265-304) for
// ROCm device tensors (PyTorch's CUDA dispatch key on ROCm builds):
//
//   trianglemix_reference::triangle_paged_sparse_attention(...) -> Tensor
//   trianglemix_reference::triangle_paged_sparse_attention_workspace_size(...) -> int
//   trianglemix::triangle_paged_sparse_attention.out(..., *, Tensor(a!) out) -> Tensor(a!)
//
// plus the README's in-tree name as a positional-out alias
//
//   trianglemix::npu_triangle_paged_sparse_attention(..., Tensor(a!) out) -> Tensor(a!)
//
// and the dense paged causal companion (same tiles, no sparse rows):
//
//   trianglemix::dense_paged_causal_attention.out(q, k, v, bt, query_start, seq_len, scale, *, out)
//   trianglemix_reference::dense_paged_causal_attention(q, k, v, bt, query_start, seq_len, scale)
//
// and the paged KV write upstream of them (vLLM's reshape_and_cache on this
// page layout, bf16 only):
//
//   trianglemix::reshape_and_cache(key, value, key_cache!, value_cache!, slot_mapping) -> ()
//
// Input and output checks restate check_inputs / check_output (:29-97) with
// the same predicates and messages ("GPU" for "NPU").  Launches go on the
// current HIP stream of the query's device under a device guard, with no
// host synchronisation.  When the library reports a non-zero split-KV
// workspace (at most TM_MAX_WORKSPACE_BYTES), it comes from PyTorch's caching
// allocator, as the reference's EXEC_NPU_CMD takes the aclnn workspace from
// torch_npu's.  Its contents do not matter (the library tags each arrival
// word for its workspace), so no buffer is ever cleared.  Outside stream
// capture one buffer is kept per (device, stream) and shared by the launches
// on that stream, which run in order; a call that needs more replaces it,
// and the old buffer goes back to the caching allocator, which hands its
// memory out again only in stream order.  Under stream capture every call
// takes a buffer of its own from the capture's private pool, which the
// graph keeps for its replays, so no graph depends on a buffer this file
// may release.

#include <ATen/ATen.h>
#include <ATen/MemoryOverlap.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime.h>
#include <torch/extension.h>
#include <torch/library.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/trianglemix.h"

namespace trianglemix_rocm {
namespace {

void check_inputs(const at::Tensor& query, const at::Tensor& key_cache, const at::Tensor& value_cache,
                  const at::Tensor& block_table) {
  TORCH_CHECK(query.is_cuda(), "query must be a GPU tensor");
  TORCH_CHECK(key_cache.is_cuda() && value_cache.is_cuda() && block_table.is_cuda(),
              "key_cache, value_cache, and block_table must be GPU tensors");
  TORCH_CHECK(query.scalar_type() == at::ScalarType::BFloat16, "query must be BF16");
  TORCH_CHECK(key_cache.scalar_type() == at::ScalarType::BFloat16 &&
                  value_cache.scalar_type() == at::ScalarType::BFloat16,
              "key_cache and value_cache must be BF16");
  TORCH_CHECK(block_table.scalar_type() == at::ScalarType::Int, "block_table must be INT32");
  TORCH_CHECK(query.device() == key_cache.device() && query.device() == value_cache.device() &&
                  query.device() == block_table.device(),
              "all inputs must be on the same GPU device");
  TORCH_CHECK(query.is_contiguous() && key_cache.is_contiguous() && value_cache.is_contiguous() &&
                  block_table.is_contiguous(),
              "all inputs must be contiguous");
  TORCH_CHECK(query.dim() == 3 && query.size(1) == 32 && query.size(2) == 128, "query must be [Tq, 32, 128]");
  TORCH_CHECK(key_cache.dim() == 4 && key_cache.size(1) == 128 && key_cache.size(2) == 8 &&
                  key_cache.size(3) == 128,
              "key_cache must be [pages, 128, 8, 128]");
  TORCH_CHECK(value_cache.sizes() == key_cache.sizes(), "value_cache shape must equal key_cache shape");
  TORCH_CHECK(block_table.dim() == 2 && block_table.size(0) == 1, "block_table must be [1, max_pages]");
}

void check_output(const at::Tensor& query, const at::Tensor& key_cache, const at::Tensor& value_cache,
                  const at::Tensor& block_table, const at::Tensor& output) {
  TORCH_CHECK(output.is_cuda(), "out must be a GPU tensor");
  TORCH_CHECK(output.device() == query.device(), "out must be on the same GPU device as query");
  TORCH_CHECK(output.scalar_type() == at::ScalarType::BFloat16, "out must be BF16");
  TORCH_CHECK(output.sizes() == query.sizes(), "out shape must exactly match query");
  TORCH_CHECK(output.is_contiguous(), "out must be contiguous");
  at::assert_no_internal_overlap(output);
  at::assert_no_overlap(output, query);
  at::assert_no_overlap(output, key_cache);
  at::assert_no_overlap(output, value_cache);
  at::assert_no_overlap(output, block_table);
}

// Split-KV workspace for a launch on `stream` (see the file comment).
at::Tensor workspace_for(const at::Tensor& like, int64_t bytes, void* stream) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  TORCH_CHECK(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &capture) == hipSuccess,
              "hipStreamIsCapturing failed");
  const auto options = like.options().dtype(at::kByte);
  if (capture != hipStreamCaptureStatusNone) return at::empty({bytes}, options);
  static std::mutex mutex;
  static std::map<std::pair<int, void*>, at::Tensor> cache;  // the buffer of each (device, stream)
  std::lock_guard<std::mutex> lock(mutex);
  at::Tensor& held = cache[{like.device().index(), stream}];
  if (!held.defined() || held.numel() < bytes) {
    held = at::Tensor();  // released first, so that its memory may serve the larger buffer
    held = at::empty({bytes}, options);
  }
  return held;
}

void check_status(int status, const char* what) {
  TORCH_CHECK(status == TM_OK, what, " failed (", tm_status_string(status), "): ", tm_last_error());
}

// Launch one chunk; `prompt_len < 0` selects the dense causal companion.
void run(const at::Tensor& query, const at::Tensor& key_cache, const at::Tensor& value_cache,
         const at::Tensor& block_table, int64_t query_start, int64_t seq_len, int64_t prompt_len, double scale,
         at::Tensor& output) {
  const bool sparse = prompt_len >= 0;
  const int64_t tq = query.size(0);
  const int64_t ws = sparse ? tm_triangle_paged_sparse_attention_workspace_size(tq, query_start, seq_len, prompt_len)
                            : tm_dense_paged_causal_attention_workspace_size(tq, query_start, seq_len);
  TORCH_CHECK(ws >= 0, "invalid attention attributes: ", tm_last_error());
  void* stream = c10::hip::getCurrentHIPStream(query.device().index()).stream();
  at::Tensor ws_tensor;
  if (ws > 0) ws_tensor = workspace_for(query, ws, stream);
  void* workspace = ws > 0 ? ws_tensor.data_ptr() : nullptr;
  const int status =
      sparse ? tm_triangle_paged_sparse_attention(
                   query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                   block_table.data_ptr<int32_t>(), output.data_ptr(), tq, key_cache.size(0), block_table.size(1),
                   query_start, seq_len, prompt_len, static_cast<float>(scale),
                   workspace, ws, stream)
             : tm_dense_paged_causal_attention(
                   query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                   block_table.data_ptr<int32_t>(), output.data_ptr(), tq, key_cache.size(0), block_table.size(1),
                   query_start, seq_len, static_cast<float>(scale), workspace, ws,
                   stream);
  check_status(status, sparse ? "triangle_paged_sparse_attention" : "dense_paged_causal_attention");
}

}  // namespace

at::Tensor triangle_paged_sparse_attention(const at::Tensor& query, const at::Tensor& key_cache,
                                           const at::Tensor& value_cache, const at::Tensor& block_table,
                                           int64_t query_start, int64_t seq_len, int64_t prompt_len, double scale) {
  check_inputs(query, key_cache, value_cache, block_table);
  TORCH_CHECK(prompt_len >= 0, "invalid query_start/seq_len/prompt_len/scale attributes");
  c10::OptionalDeviceGuard guard(query.device());
  at::Tensor output = at::empty_like(query);
  run(query, key_cache, value_cache, block_table, query_start, seq_len, prompt_len, scale, output);
  return output;
}

at::Tensor& triangle_paged_sparse_attention_out(const at::Tensor& query, const at::Tensor& key_cache,
                                                const at::Tensor& value_cache, const at::Tensor& block_table,
                                                int64_t query_start, int64_t seq_len, int64_t prompt_len,
                                                double scale, at::Tensor& output) {
  check_inputs(query, key_cache, value_cache, block_table);
  check_output(query, key_cache, value_cache, block_table, output);
  TORCH_CHECK(prompt_len >= 0, "invalid query_start/seq_len/prompt_len/scale attributes");
  c10::OptionalDeviceGuard guard(query.device());
  run(query, key_cache, value_cache, block_table, query_start, seq_len, prompt_len, scale, output);
  return output;
}

int64_t triangle_paged_sparse_attention_workspace_size(const at::Tensor& query, const at::Tensor& key_cache,
                                                       const at::Tensor& value_cache, const at::Tensor& block_table,
                                                       int64_t query_start, int64_t seq_len, int64_t prompt_len,
                                                       double scale) {
  check_inputs(query, key_cache, value_cache, block_table);
  TORCH_CHECK(std::isfinite(scale) && scale > 0.0, "invalid query_start/seq_len/prompt_len/scale attributes");
  const int64_t ws = tm_triangle_paged_sparse_attention_workspace_size(query.size(0), query_start, seq_len, prompt_len);
  TORCH_CHECK(ws >= 0, "triangle_paged_sparse_attention_workspace_size failed: ", tm_last_error());
  return ws;
}

at::Tensor dense_paged_causal_attention(const at::Tensor& query, const at::Tensor& key_cache,
                                        const at::Tensor& value_cache, const at::Tensor& block_table,
                                        int64_t query_start, int64_t seq_len, double scale) {
  check_inputs(query, key_cache, value_cache, block_table);
  c10::OptionalDeviceGuard guard(query.device());
  at::Tensor output = at::empty_like(query);
  run(query, key_cache, value_cache, block_table, query_start, seq_len, -1, scale, output);
  return output;
}

at::Tensor& dense_paged_causal_attention_out(const at::Tensor& query, const at::Tensor& key_cache,
                                             const at::Tensor& value_cache, const at::Tensor& block_table,
                                             int64_t query_start, int64_t seq_len, double scale, at::Tensor& output) {
  check_inputs(query, key_cache, value_cache, block_table);
  check_output(query, key_cache, value_cache, block_table, output);
  c10::OptionalDeviceGuard guard(query.device());
  run(query, key_cache, value_cache, block_table, query_start, seq_len, -1, scale, output);
  return output;
}

// Paged KV write: token i's K / V rows go to cache slot slot_mapping[i]
// (negative = padding, skipped).  key / value may be row-strided views (a
// slice of a fused QKV buffer); their [8, 128] part must be contiguous.
void reshape_and_cache(const at::Tensor& key, const at::Tensor& value, at::Tensor& key_cache, at::Tensor& value_cache,
                       const at::Tensor& slot_mapping) {
  TORCH_CHECK(key.is_cuda() && value.is_cuda() && key_cache.is_cuda() && value_cache.is_cuda() &&
                  slot_mapping.is_cuda(),
              "key, value, key_cache, value_cache and slot_mapping must be GPU tensors");
  TORCH_CHECK(key.device() == value.device() && key.device() == key_cache.device() &&
                  key.device() == value_cache.device() && key.device() == slot_mapping.device(),
              "all inputs must be on the same GPU device");
  TORCH_CHECK(key.scalar_type() == at::ScalarType::BFloat16 && value.scalar_type() == at::ScalarType::BFloat16 &&
                  key_cache.scalar_type() == at::ScalarType::BFloat16 &&
                  value_cache.scalar_type() == at::ScalarType::BFloat16,
              "key, value, key_cache and value_cache must be BF16");
  TORCH_CHECK(slot_mapping.scalar_type() == at::ScalarType::Long && slot_mapping.dim() == 1 &&
                  slot_mapping.is_contiguous(),
              "slot_mapping must be a contiguous INT64 [num_tokens] tensor");
  TORCH_CHECK(key.dim() == 3 && key.size(1) == 8 && key.size(2) == 128 && value.sizes() == key.sizes(),
              "key and value must be [num_tokens, 8, 128]");
  TORCH_CHECK(key.size(0) == slot_mapping.size(0), "slot_mapping must hold one slot per token");
  TORCH_CHECK(key.stride(2) == 1 && key.stride(1) == 128 && value.stride(2) == 1 && value.stride(1) == 128,
              "the [8, 128] part of each key / value row must be contiguous");
  TORCH_CHECK(key_cache.dim() == 4 && key_cache.size(1) == 128 && key_cache.size(2) == 8 &&
                  key_cache.size(3) == 128 && key_cache.is_contiguous(),
              "key_cache must be a contiguous [pages, 128, 8, 128] tensor");
  TORCH_CHECK(value_cache.sizes() == key_cache.sizes() && value_cache.is_contiguous(),
              "value_cache must be contiguous with the shape of key_cache");
  at::assert_no_overlap(key_cache, value_cache);
  at::assert_no_overlap(key_cache, key);
  at::assert_no_overlap(key_cache, value);
  at::assert_no_overlap(value_cache, key);
  at::assert_no_overlap(value_cache, value);
  const int64_t num_tokens = key.size(0);
  if (num_tokens == 0) return;
  c10::OptionalDeviceGuard guard(key.device());
  void* stream = c10::hip::getCurrentHIPStream(key.device().index()).stream();
  const int status =
      tm_reshape_and_cache(key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                           slot_mapping.data_ptr<int64_t>(), num_tokens, key.stride(0), value.stride(0),
                           key_cache.size(0), stream);
  check_status(status, "reshape_and_cache");
}

void meta_reshape_and_cache(const at::Tensor&, const at::Tensor&, at::Tensor&, at::Tensor&, const at::Tensor&) {}

// Shape-only implementations (the reference's InferShape: out = query shape,
// operator/op_host/triangle_paged_sparse_attention.cpp:332-346).
at::Tensor meta_functional(const at::Tensor& query, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t,
                           int64_t, int64_t, double) {
  return at::empty_like(query);
}
at::Tensor& meta_out(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t, int64_t,
                     int64_t, double, at::Tensor& output) {
  return output;
}
at::Tensor meta_dense(const at::Tensor& query, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t,
                      int64_t, double) {
  return at::empty_like(query);
}
at::Tensor& meta_dense_out(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t,
                           int64_t, double, at::Tensor& output) {
  return output;
}

// ---- routed-call fast path (the Python module trianglemix._trianglemix_torch) ----
// The routing layer pays its tensor gates and the op call on every selected
// layer of every step, and an eager prefill waits for that host time.  These
// entry points give it the same gates in one native call and the .out
// launches without the dispatcher's Python argument handling; the launches
// run the ops' own checks, device guard and workspace code above.

// First failing tensor gate of a routed call whose query is on a GPU: 0 none,
// 1 query / output, 2 KV cache, 3 block table.  The predicates and their order
// are the routing layer's (trianglemix/router.py, _tensor_reason), which
// restate the reference plugin's _validate_query / _validate_static_kv /
// _validate_block_table (package/src/vllm_ascend_trianglemix/plugin.py:1106-1192).
int64_t tensor_gate(const at::Tensor& query, const at::Tensor& output, const at::Tensor& key_cache,
                    const at::Tensor& value_cache, const at::Tensor& block_table, int64_t query_len,
                    int64_t seq_len) {
  constexpr auto kBf16 = at::ScalarType::BFloat16;
  if (query.dim() != 3 || query.size(1) != 32 || query.size(2) != 128 || query.size(0) != query_len ||
      query.scalar_type() != kBf16 || !query.is_contiguous()) {
    return 1;
  }
  const auto device = query.get_device();
  if (output.dim() == 0 || output.size(0) < query.size(0) || output.scalar_type() != kBf16 ||
      output.get_device() != device || !output.is_contiguous()) {
    return 1;
  }
  if (key_cache.dim() != 4 || key_cache.size(1) != 128 || key_cache.size(2) != 8 || key_cache.size(3) != 128 ||
      value_cache.sizes() != key_cache.sizes() || key_cache.scalar_type() != kBf16 ||
      value_cache.scalar_type() != kBf16 || key_cache.get_device() != device || value_cache.get_device() != device ||
      !key_cache.is_contiguous() || !value_cache.is_contiguous()) {
    return 2;
  }
  if (block_table.dim() != 2 || block_table.size(0) != 1 || block_table.size(1) < (seq_len + 127) / 128 ||
      block_table.scalar_type() != at::ScalarType::Int || block_table.get_device() != device ||
      !block_table.is_contiguous()) {
    return 3;
  }
  return 0;
}

// The routed launches: rows [seq_len - Tq, seq_len) into the first Tq rows of
// `output` (an engine's output buffer may hold padding rows past them).
void launch_sparse(const at::Tensor& query, const at::Tensor& key_cache, const at::Tensor& value_cache,
                   const at::Tensor& block_table, int64_t seq_len, int64_t prompt_len, double scale,
                   const at::Tensor& output) {
  const int64_t rows = query.size(0);
  at::Tensor out = output.size(0) == rows ? output : output.narrow(0, 0, rows);
  triangle_paged_sparse_attention_out(query, key_cache, value_cache, block_table, seq_len - rows, seq_len, prompt_len,
                                      scale, out);
}

// tensor_gate, then -- when every gate passes (result 0) -- launch_sparse: one
// native call for a routed direct layer whose engine runs nothing between the
// gates and the launch.
int64_t route_sparse(const at::Tensor& query, const at::Tensor& output, const at::Tensor& key_cache,
                     const at::Tensor& value_cache, const at::Tensor& block_table, int64_t query_len, int64_t seq_len,
                     int64_t prompt_len, double scale) {
  const int64_t gate = tensor_gate(query, output, key_cache, value_cache, block_table, query_len, seq_len);
  if (gate == 0) launch_sparse(query, key_cache, value_cache, block_table, seq_len, prompt_len, scale, output);
  return gate;
}

void launch_dense(const at::Tensor& query, const at::Tensor& key_cache, const at::Tensor& value_cache,
                  const at::Tensor& block_table, int64_t seq_len, double scale, const at::Tensor& output) {
  const int64_t rows = query.size(0);
  at::Tensor out = output.size(0) == rows ? output : output.narrow(0, 0, rows);
  dense_paged_causal_attention_out(query, key_cache, value_cache, block_table, seq_len - rows, seq_len, scale, out);
}

}  // namespace trianglemix_rocm

PYBIND11_MODULE(_trianglemix_torch, m) {
  m.doc() = "Routed-call fast path of the TriangleMix torch adapter (the ops themselves are under torch.ops)";
  m.def("tensor_gate", &trianglemix_rocm::tensor_gate);
  m.def("launch_sparse", &trianglemix_rocm::launch_sparse);
  m.def("route_sparse", &trianglemix_rocm::route_sparse);
  m.def("launch_dense", &trianglemix_rocm::launch_dense);
}

TORCH_LIBRARY(trianglemix_reference, ops) {
  ops.def(
      "triangle_paged_sparse_attention(Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, int query_start, int seq_len, int prompt_len, float scale) -> Tensor");
  ops.def(
      "triangle_paged_sparse_attention_workspace_size(Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, int query_start, int seq_len, int prompt_len, float scale) -> int");
  ops.def(
      "dense_paged_causal_attention(Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, int query_start, int seq_len, float scale) -> Tensor");
}

TORCH_LIBRARY_IMPL(trianglemix_reference, CUDA, ops) {
  ops.impl("triangle_paged_sparse_attention", &trianglemix_rocm::triangle_paged_sparse_attention);
  ops.impl("triangle_paged_sparse_attention_workspace_size",
           &trianglemix_rocm::triangle_paged_sparse_attention_workspace_size);
  ops.impl("dense_paged_causal_attention", &trianglemix_rocm::dense_paged_causal_attention);
}

TORCH_LIBRARY_IMPL(trianglemix_reference, Meta, ops) {
  ops.impl("triangle_paged_sparse_attention", &trianglemix_rocm::meta_functional);
  ops.impl("dense_paged_causal_attention", &trianglemix_rocm::meta_dense);
}

TORCH_LIBRARY_FRAGMENT(trianglemix, ops) {
  ops.def(
      "triangle_paged_sparse_attention.out(Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, int query_start, int seq_len, int prompt_len, float scale, *, "
      "Tensor(a!) out) -> Tensor(a!)");
  ops.def(
      "npu_triangle_paged_sparse_attention(Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, int query_start, int seq_len, int prompt_len, float scale, "
      "Tensor(a!) out) -> Tensor(a!)");
  ops.def(
      "dense_paged_causal_attention.out(Tensor query, Tensor key_cache, Tensor value_cache, "
      "Tensor block_table, int query_start, int seq_len, float scale, *, Tensor(a!) out) -> Tensor(a!)");
  ops.def(
      "reshape_and_cache(Tensor key, Tensor value, Tensor(a!) key_cache, Tensor(b!) value_cache, "
      "Tensor slot_mapping) -> ()");
}

TORCH_LIBRARY_IMPL(trianglemix, CUDA, ops) {
  ops.impl("triangle_paged_sparse_attention.out", &trianglemix_rocm::triangle_paged_sparse_attention_out);
  ops.impl("npu_triangle_paged_sparse_attention", &trianglemix_rocm::triangle_paged_sparse_attention_out);
  ops.impl("dense_paged_causal_attention.out", &trianglemix_rocm::dense_paged_causal_attention_out);
  ops.impl("reshape_and_cache", &trianglemix_rocm::reshape_and_cache);
}

TORCH_LIBRARY_IMPL(trianglemix, Meta, ops) {
  ops.impl("triangle_paged_sparse_attention.out", &trianglemix_rocm::meta_out);
  ops.impl("npu_triangle_paged_sparse_attention", &trianglemix_rocm::meta_out);
  ops.impl("dense_paged_causal_attention.out", &trianglemix_rocm::meta_dense_out);
  ops.impl("reshape_and_cache", &trianglemix_rocm::meta_reshape_and_cache);
}
