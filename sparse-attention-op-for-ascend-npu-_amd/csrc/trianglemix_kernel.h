// Internal interface between the C ABI host code and the gfx950 kernels.
#ifndef TRIANGLEMIX_KERNEL_H
#define TRIANGLEMIX_KERNEL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tmx {

// Fixed geometry of the reference operator's compiled ABI
// (operator/op_host/triangle_paged_sparse_attention.cpp:29-37).
constexpr int kQueryHeads = 32;
constexpr int kKvHeads = 8;
constexpr int kGroup = kQueryHeads / kKvHeads;
constexpr int kHeadDim = 128;
constexpr int kPageSize = 128;
constexpr int kQueryTile = 32;
constexpr int kSinkTokens = 8;
constexpr int kLocalWindow = 512;
constexpr int kDenseTail = 128;
constexpr int kSparseBegin = kSinkTokens + kLocalWindow + 1;  // 521
constexpr int kKvTile = 64;  // keys per LDS tile (divides the 128-token page)

// Largest seq_len / prompt_len the 32-bit position arithmetic accepts.
constexpr int64_t kMaxPositions = (int64_t(1) << 30);

struct KernelParams {
  const __bf16* query;        // [tq, 32, 128]
  const __bf16* key_cache;    // [num_pages, 128, 8, 128]
  const __bf16* value_cache;  // [num_pages, 128, 8, 128]
  const int32_t* block_table; // [>= ceil(seq_len/128)]
  __bf16* out;                // [tq, 32, 128]
  int num_pages;
  int query_start;
  int seq_len;
  int sparse_begin;  // 521 for TriangleMix, 0 for dense causal
  int sparse_end;    // max(0, prompt_len-128) for TriangleMix, 0 for dense causal
  int num_row_blocks;
  float scale_log2;  // softmax scale * log2(e)
};

hipError_t launch_triangle_paged_attention(const KernelParams& p, hipStream_t stream);

}  // namespace tmx

#endif  // TRIANGLEMIX_KERNEL_H
