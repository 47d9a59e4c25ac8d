// Internal interface between the C ABI host code and the gfx950 kernels:
// fixed geometry, the row-block tile schedule (shared by host and device so
// the grid and the kernel agree exactly) and the launch parameters.
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

// Kernel tiling.
constexpr int kKvTile = 32;    // keys per LDS tile (divides the 128-token page)
constexpr int kRowBlock = 32;  // query tokens per work item
// One split-KV partial per (KV head, work item), fp32, for each of the 4
// query heads and 64 lanes: 64 O values, the row max and the lane's partial
// row sum.
constexpr int64_t kPartialFloats = int64_t(kGroup) * 64 * (64 + 2);
constexpr int64_t kPartialBytes = kPartialFloats * 4;
// Workspace of a launch with split row blocks: a block of arrival words (one
// 64-bit word per split row block, KV head and workgroup position), then the
// partials of the split row blocks' items.  A word holds the launch's 48-bit
// epoch above a 16-bit arrival count; a word carrying another epoch counts as
// zero, so the workspace may hold anything before a launch (the reference's
// workspace is plain scratch).  The host keeps one epoch per workspace
// address, and the workgroup that completes a row block leaves its word at
// (epoch, 0): the next launch on that workspace, or the next replay of a
// captured one, finds its words clean.  The counter block has a fixed size,
// so the partials start at the same offset for every geometry.
constexpr int64_t kCounterBytes = 65536;
constexpr int kMaxSplitRowBlocks = int(kCounterBytes / 8 / (kKvHeads * 2));  // 512
constexpr int kEpochShift = 16;
constexpr unsigned long long kEpochMask = (1ull << 48) - 1;
// Largest workspace any call needs: the planner keeps every plan's counters
// and partials within it (at most 124 split items per KV head), and a plan
// with no split at all needs none.
constexpr int64_t kMaxWorkspaceBytes = int64_t(64) << 20;
constexpr int kMaxSplitItems = int((kMaxWorkspaceBytes - kCounterBytes) / (kKvHeads * kPartialBytes));  // 124
static_assert(kMaxSplitItems < (1 << kEpochShift), "an arrival count fits below the epoch");
// Split-KV scratch held per GPU for the no-allocation entry point (counter
// block + partials): the largest workspace of any call.
constexpr int64_t kNoAllocScratchBytes = kMaxWorkspaceBytes;
// A work item may hold any number of tiles: the kernel keeps the page numbers
// of 128 of them in two 64-lane registers and refills the one it has used up
// while the other serves, 64 tiles at a time.
constexpr int kTableTiles = 64;
// Most cache pages a launch accepts: the kernel addresses a key row of one KV
// head by a 32-bit row index (page * 128 + slot) * 8 + head.  2^22 pages of
// 256 KB per K or V cache are more than one GPU's memory.
constexpr int64_t kMaxPages = int64_t(1) << 22;

// Largest seq_len / prompt_len the 32-bit position arithmetic accepts.
constexpr int64_t kMaxPositions = (int64_t(1) << 30);

// Tile schedule of one row block [tb, te): up to two runs of kKvTile-key tiles.
// A block whose rows are all sparse visits the sink tile plus the tiles of
// [tb - 512, te); any other block visits [0, te).
struct TileRuns {
  int first0, count0, first1, count1;
  __host__ __device__ int count() const { return count0 + count1; }
  __host__ __device__ int tile(int i) const { return i < count0 ? first0 + i : first1 + (i - count0); }
};

__host__ __device__ inline TileRuns row_block_tiles(int tb, int te, int sparse_begin, int sparse_end) {
  TileRuns r{0, 0, 0, 0};
  const int last = (te - 1) / kKvTile;
  const bool all_sparse = tb >= sparse_begin && te <= sparse_end;
  const int local_first = all_sparse ? (tb - kLocalWindow) / kKvTile : 0;  // tb >= 521 when all sparse
  if (local_first <= 0) {
    r.count0 = last + 1;
  } else {
    r.count0 = 1;  // sink tile [0, kKvTile)
    r.first1 = local_first;
    r.count1 = last - local_first + 1;
  }
  return r;
}

// Row blocks are issued last-first (later rows attend more keys): order
// index o is row block num_row_blocks - 1 - o.
__host__ __device__ inline int row_block_splits(int o, int num_row_blocks, int query_start, int seq_len,
                                                int sparse_begin, int sparse_end, int tiles_per_split) {
  const int rb = num_row_blocks - 1 - o;
  const int tb = query_start + rb * kRowBlock;
  const int te = tb + kRowBlock < seq_len ? tb + kRowBlock : seq_len;
  const int n = row_block_tiles(tb, te, sparse_begin, sparse_end).count();
  return (n + tiles_per_split - 1) / tiles_per_split;
}

struct KernelParams {
  const __bf16* query;        // [tq, 32, 128]
  const __bf16* key_cache;    // [num_pages, 128, 8, 128]
  const __bf16* value_cache;  // [num_pages, 128, 8, 128]
  const int32_t* block_table; // [>= ceil(seq_len/128)]
  __bf16* out;                // [tq, 32, 128]
  float* partials;            // [8][split_items] split-KV partials, or null
  unsigned long long* counters;  // [8][split_row_blocks][workgroups per item] arrival words, or null
  unsigned long long epoch;   // this launch's arrival tag: nonzero, below 2^48
  int num_pages;
  int query_start;
  int seq_len;
  int sparse_begin;    // 521 for TriangleMix, 0 for dense causal
  int sparse_end;      // max(0, prompt_len-128) for TriangleMix, 0 for dense causal
  int num_row_blocks;
  int tiles_per_split; // max tiles per work item
  int items_per_head;  // sum over row blocks of their split counts
  // The first split_row_blocks row blocks in issue order hold every split
  // one (0 when none splits); their items, the first split_items, are
  // decoded from the split counts.  Every later row block is one item:
  // item split_items + j is row block split_row_blocks + j in issue order.
  int split_row_blocks;
  int split_items;
  float scale_log2;    // softmax scale * log2(e)
};

// Enqueues the attention kernel (TriangleMix mask when `sparse`, plain causal
// otherwise): one launch, split row blocks included.  kv_parts picks the
// workgroup shape: 4 (two query heads x KV quarters, items_per_head x 16
// workgroups of eight waves), 2 (the four heads of the GQA group x KV halves,
// items_per_head x 8 of eight waves) or 1 (the four heads x the whole KV
// range, items_per_head x 8 of four waves, two per CU).
hipError_t launch_triangle_paged_attention(const KernelParams& p, bool sparse, int kv_parts, hipStream_t stream);

// Device address of this GPU's no-allocation scratch (kNoAllocScratchBytes,
// 256-byte aligned), looked up once per device with the device current.
hipError_t noalloc_scratch(void** ptr);

// Enqueues the paged KV write: token i's K and V rows ([8, 128] bf16, row
// strides key_stride / value_stride in elements, multiples of 8) go to cache
// slot slot_mapping[i] (page slot / 128, offset slot % 128); negative slots
// and slots past num_pages * 128 are skipped.
hipError_t launch_paged_kv_write(const void* key, const void* value, void* key_cache, void* value_cache,
                                 const int64_t* slot_mapping, int64_t num_tokens, int64_t key_stride,
                                 int64_t value_stride, int64_t num_pages, hipStream_t stream);

}  // namespace tmx

#endif  // TRIANGLEMIX_KERNEL_H
