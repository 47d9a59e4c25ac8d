// C ABI of libtrianglemix.so: host-side validation and launch geometry.
//
// Validation restates the reference's boundary checks
// (operator/torch_adapter/triangle_paged_attention_torch.cpp:29-97 and
// operator/op_host/triangle_paged_sparse_attention.cpp:122-237) on plain
// pointers and sizes.  Every check runs before any HIP call.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/trianglemix.h"
#include "trianglemix_kernel.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

struct Range {
  uintptr_t lo, hi;
};

bool overlaps(Range a, Range b) { return a.lo < b.hi && b.lo < a.hi; }

constexpr int64_t kQueryRowBytes = int64_t(tmx::kQueryHeads) * tmx::kHeadDim * 2;
constexpr int64_t kPageBytes = int64_t(tmx::kPageSize) * tmx::kKvHeads * tmx::kHeadDim * 2;

// Attribute checks shared by the launch and workspace-size entry points.
int check_attributes(int64_t query_tokens, int64_t query_start, int64_t seq_len,
                     int64_t prompt_len, bool check_prompt) {
  if (query_tokens <= 0) {
    return fail(TM_ERR_INVALID_ARGUMENT, "query must be [Tq, 32, 128] with Tq > 0");
  }
  if (query_start < 0 || seq_len <= 0 || (check_prompt && prompt_len < seq_len)) {
    return fail(TM_ERR_INVALID_ARGUMENT, "invalid query_start/seq_len/prompt_len/scale attributes");
  }
  if (query_start + query_tokens != seq_len) {
    return fail(TM_ERR_INVALID_ARGUMENT, "batch-one prefill requires query_start + Tq == seq_len");
  }
  if (seq_len > tmx::kMaxPositions || (check_prompt && prompt_len > tmx::kMaxPositions)) {
    return fail(TM_ERR_UNSUPPORTED, "seq_len and prompt_len must not exceed %lld",
                (long long)tmx::kMaxPositions);
  }
  return TM_OK;
}

// Split-KV sizing: cut long row blocks so that the chunk's tiles spread
// evenly over kTargetItemsPerHead items per KV head -- each item runs as two
// workgroups of one CU each, so 16 items per head give every one of the 256
// CUs about the same number of tiles in one round -- and never cut a row block
// into pieces of fewer than kMinSplitTiles tiles (1024 keys): a split's fp32
// partial (66 KB) must stay small next to the K/V it reads (16 KB per 32-key
// tile).  The heaviest items are issued first.
constexpr int kTargetItemsPerHead = 16;
constexpr int kMinSplitTiles = 1024 / tmx::kKvTile;

// Work items per KV head beyond which a launch is refused (its grid would
// exceed 2^30 workgroups).
constexpr int64_t kMaxItemsPerHead = int64_t(1) << 26;

struct Geometry {
  int sparse_begin, sparse_end, num_row_blocks, tiles_per_split;
  int64_t items_per_head;
  bool any_split;
  int64_t workspace_bytes;
};

Geometry make_geometry(bool sparse, int64_t query_tokens, int64_t query_start, int64_t seq_len, int64_t prompt_len) {
  Geometry g{};
  g.sparse_begin = sparse ? tmx::kSparseBegin : 0;
  g.sparse_end = sparse ? (int)(prompt_len > tmx::kDenseTail ? prompt_len - tmx::kDenseTail : 0) : 0;
  g.num_row_blocks = (int)((query_tokens + tmx::kRowBlock - 1) / tmx::kRowBlock);
  int64_t total_tiles = 0;
  for (int o = 0; o < g.num_row_blocks; ++o) {
    total_tiles += tmx::row_block_splits(o, g.num_row_blocks, (int)query_start, (int)seq_len, g.sparse_begin,
                                         g.sparse_end, 1);
  }
  const int64_t per_item = (total_tiles + kTargetItemsPerHead - 1) / kTargetItemsPerHead;
  g.tiles_per_split = (int)(per_item > kMinSplitTiles ? per_item : kMinSplitTiles);
  if (g.tiles_per_split > tmx::kMaxItemTiles) g.tiles_per_split = tmx::kMaxItemTiles;
  bool any_split = false;
  int64_t items = 0;
  for (int o = 0; o < g.num_row_blocks; ++o) {
    const int s = tmx::row_block_splits(o, g.num_row_blocks, (int)query_start, (int)seq_len, g.sparse_begin,
                                        g.sparse_end, g.tiles_per_split);
    items += s;
    any_split = any_split || s > 1;
  }
  g.items_per_head = items;
  g.any_split = any_split;
  g.workspace_bytes = any_split ? int64_t(tmx::kKvHeads) * items * tmx::kPartialBytes : 0;
  return g;
}

int launch(bool sparse, const void* query, const void* key_cache, const void* value_cache,
           const int32_t* block_table, void* out, int64_t query_tokens, int64_t num_pages,
           int64_t block_table_cols, int64_t query_start, int64_t seq_len, int64_t prompt_len,
           float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  g_last_error[0] = '\0';
  if (!query || !key_cache || !value_cache || !block_table || !out) {
    return fail(TM_ERR_INVALID_ARGUMENT, "query, key_cache, value_cache, block_table and out must be non-null");
  }
  int st = check_attributes(query_tokens, query_start, seq_len, prompt_len, sparse);
  if (st != TM_OK) return st;
  if (!std::isfinite(scale) || scale <= 0.0f) {
    return fail(TM_ERR_INVALID_ARGUMENT, "invalid query_start/seq_len/prompt_len/scale attributes");
  }
  if (num_pages <= 0) {
    return fail(TM_ERR_INVALID_ARGUMENT, "key_cache must be [pages, 128, 8, 128] with pages > 0");
  }
  if (num_pages > tmx::kMaxPages) {
    return fail(TM_ERR_UNSUPPORTED, "key_cache has %lld pages; the limit is %lld", (long long)num_pages,
                (long long)tmx::kMaxPages);
  }
  const int64_t required_pages = (seq_len + tmx::kPageSize - 1) / tmx::kPageSize;
  if (block_table_cols < required_pages) {
    return fail(TM_ERR_INVALID_ARGUMENT, "block_table lacks logical pages required by seq_len");
  }
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace)) {
    return fail(TM_ERR_WORKSPACE, "workspace pointer/size are inconsistent");
  }
  // out must not overlap any input (at::assert_no_overlap, adapter.cpp:92-96).
  const Range r_out{(uintptr_t)out, (uintptr_t)out + uintptr_t(query_tokens * kQueryRowBytes)};
  const Range r_q{(uintptr_t)query, (uintptr_t)query + uintptr_t(query_tokens * kQueryRowBytes)};
  const Range r_k{(uintptr_t)key_cache, (uintptr_t)key_cache + uintptr_t(num_pages * kPageBytes)};
  const Range r_v{(uintptr_t)value_cache, (uintptr_t)value_cache + uintptr_t(num_pages * kPageBytes)};
  const Range r_bt{(uintptr_t)block_table, (uintptr_t)block_table + uintptr_t(block_table_cols * 4)};
  if (overlaps(r_out, r_q) || overlaps(r_out, r_k) || overlaps(r_out, r_v) || overlaps(r_out, r_bt)) {
    return fail(TM_ERR_INVALID_ARGUMENT, "out must not overlap query, key_cache, value_cache or block_table");
  }

  const Geometry g = make_geometry(sparse, query_tokens, query_start, seq_len, prompt_len);
  if (g.items_per_head > kMaxItemsPerHead) {
    return fail(TM_ERR_UNSUPPORTED, "chunk needs %lld work items per KV head; the limit is %lld",
                (long long)g.items_per_head, (long long)kMaxItemsPerHead);
  }
  if (workspace_bytes < g.workspace_bytes) {
    return fail(TM_ERR_WORKSPACE, "workspace of %lld bytes is smaller than the %lld bytes this call needs",
                (long long)workspace_bytes, (long long)g.workspace_bytes);
  }
  if (g.workspace_bytes > 0) {
    const Range r_ws{(uintptr_t)workspace, (uintptr_t)workspace + uintptr_t(g.workspace_bytes)};
    if (overlaps(r_ws, r_out) || overlaps(r_ws, r_q) || overlaps(r_ws, r_k) || overlaps(r_ws, r_v) ||
        overlaps(r_ws, r_bt)) {
      return fail(TM_ERR_WORKSPACE, "workspace must not overlap the inputs or out");
    }
  }

  tmx::KernelParams p{};
  p.query = static_cast<const __bf16*>(query);
  p.key_cache = static_cast<const __bf16*>(key_cache);
  p.value_cache = static_cast<const __bf16*>(value_cache);
  p.block_table = block_table;
  p.out = static_cast<__bf16*>(out);
  p.partials = g.any_split ? static_cast<float*>(workspace) : nullptr;
  p.num_pages = (int)num_pages;
  p.query_start = (int)query_start;
  p.seq_len = (int)seq_len;
  p.sparse_begin = g.sparse_begin;
  p.sparse_end = g.sparse_end;
  p.num_row_blocks = g.num_row_blocks;
  p.tiles_per_split = g.tiles_per_split;
  p.items_per_head = (int)g.items_per_head;
  p.any_split = g.any_split ? 1 : 0;
  p.scale_log2 = scale * 1.4426950408889634f;
  const hipError_t err =
      tmx::launch_triangle_paged_attention(p, sparse, g.any_split, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    return fail(TM_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  }
  return TM_OK;
}

}  // namespace

extern "C" {

int tm_abi_version(void) { return TM_ABI_VERSION; }

const char* tm_status_string(int status) {
  switch (status) {
    case TM_OK: return "TM_OK";
    case TM_ERR_INVALID_ARGUMENT: return "TM_ERR_INVALID_ARGUMENT";
    case TM_ERR_UNSUPPORTED: return "TM_ERR_UNSUPPORTED";
    case TM_ERR_WORKSPACE: return "TM_ERR_WORKSPACE";
    case TM_ERR_LAUNCH: return "TM_ERR_LAUNCH";
    default: return "TM_ERR_UNKNOWN";
  }
}

const char* tm_last_error(void) { return g_last_error; }

int tm_triangle_paged_sparse_attention(const void* query, const void* key_cache, const void* value_cache,
                                       const int32_t* block_table, void* out, int64_t query_tokens,
                                       int64_t num_pages, int64_t block_table_cols, int64_t query_start,
                                       int64_t seq_len, int64_t prompt_len, float scale, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  return launch(true, query, key_cache, value_cache, block_table, out, query_tokens, num_pages,
                block_table_cols, query_start, seq_len, prompt_len, scale, workspace, workspace_bytes, stream);
}

int64_t tm_triangle_paged_sparse_attention_workspace_size(int64_t query_tokens, int64_t query_start,
                                                          int64_t seq_len, int64_t prompt_len) {
  g_last_error[0] = '\0';
  if (check_attributes(query_tokens, query_start, seq_len, prompt_len, true) != TM_OK) return -1;
  return make_geometry(true, query_tokens, query_start, seq_len, prompt_len).workspace_bytes;
}

int tm_dense_paged_causal_attention(const void* query, const void* key_cache, const void* value_cache,
                                    const int32_t* block_table, void* out, int64_t query_tokens,
                                    int64_t num_pages, int64_t block_table_cols, int64_t query_start,
                                    int64_t seq_len, float scale, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  return launch(false, query, key_cache, value_cache, block_table, out, query_tokens, num_pages,
                block_table_cols, query_start, seq_len, seq_len, scale, workspace, workspace_bytes, stream);
}

int64_t tm_dense_paged_causal_attention_workspace_size(int64_t query_tokens, int64_t query_start,
                                                       int64_t seq_len) {
  g_last_error[0] = '\0';
  if (check_attributes(query_tokens, query_start, seq_len, seq_len, false) != TM_OK) return -1;
  return make_geometry(false, query_tokens, query_start, seq_len, seq_len).workspace_bytes;
}

}  // extern "C"
