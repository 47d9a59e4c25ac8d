// C ABI of libtrianglemix.so: host-side validation and launch geometry.
//
// Validation restates the reference's boundary checks
// (operator/torch_adapter/triangle_paged_attention_torch.cpp:29-97 and
// operator/op_host/triangle_paged_sparse_attention.cpp:122-237) on plain
// pointers and sizes.  Every check runs before any HIP call.

#include <hip/hip_runtime.h>

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <vector>
#include <cstring>
#include <initializer_list>
#include <limits>
#include <mutex>

#include "../../include/trianglemix.h"
#include "trianglemix_kernel.h"

static_assert(TM_WORKSPACE_COUNTER_BYTES == tmx::kCounterBytes, "the public counter block size is the kernel's");
static_assert(TM_MAX_WORKSPACE_BYTES == tmx::kMaxWorkspaceBytes, "the public workspace bound is the planner's");

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

// Workgroup shapes.  KV quarters (P = 4): two query heads per workgroup over
// four KV parts, 16 workgroups per work item, one per CU.  KV halves (P = 2):
// the four heads of a GQA group over two KV parts, 8 workgroups per item, one
// per CU; each K/V tile then serves four heads.  KV whole (P = 1): four waves,
// one per head, over every tile of the item, 8 workgroups per item, two per
// CU; no KV-part merge.  Per KV head the 256 CUs hold 16 quarters, 32 halves
// or 64 KV-whole workgroups at once: a shape's slots.
//
// A plan is a shape and T, the most tiles an item takes: a row block of n
// tiles is cut into ceil(n / T) near-equal items (an item may hold any number
// of tiles, so rows split only for load balance).  A plan is costed by
// simulating the greedy dispatch of its items, issued heaviest row block first
// as the grid lists them, each onto the least loaded slot.  An item costs a
// fixed part (start-up, KV-part merge, output store) plus a part per loop
// iteration (ceil(tiles / P) iterations).  A split row block completes when
// its last piece has finished plus the in-launch merge: a fixed part and a
// part per piece, whose partials the last arriving workgroup reads back.  The
// plan's time is its latest slot or split row block.  The candidate with the
// shortest simulated time is taken (ties: the larger T, fewer partials).
//
// Three regimes, with costs fitted on MI355X to sweeps of forced plans (every
// candidate plan of each geometry timed as 20 launches, fastest of three
// passes, HIP events): 87 TriangleMix and dense-companion chunks of 64 to
// 12288 rows at prompts of 1024 to 131072 tokens, 35 of them held out of the
// first fit to check it.  The fit minimised the time the planned plans lose
// to each geometry's fastest measured plan.  On the committed sweep
// (tests/plan_sweep_mi355x.json) the planned plans lose 43.5 us of the
// 6,533 us the 87 chunks take at their fastest (0.67 %); the previous
// planner, which charged the merge to the whole chunk instead of the split
// rows and never split KV-whole items, lost 212 us (3.2 %).
//  * TriangleMix chunks of up to 16 row blocks: quarters (T from the ladder,
//    32-128 tiles) or halves (T of 24 tiles and more).  Quarters stay on the
//    ladder: their longer items move twice the K/V of halves ones per head.
//    Config 1's chunk: quarters over 84-tile items, 17.9 us (halves over
//    28-tile items: 19.1 us).
//  * Chunks of 17 row blocks or more, TriangleMix and dense companion:
//    halves or KV whole, T of 16 tiles and more.  KV whole fills the GPU
//    with two workgroups per CU, pays no KV-part merge, and split into pieces
//    it also serves the long dense-tail rows of a prompt's last chunks: the
//    last 2048 rows of a 131072-token prompt take 311 us as KV whole over
//    256-tile pieces against 346 us as halves over 512-tile ones.
//  * Dense-companion chunks of up to 16 row blocks: halves when their plan
//    splits a row block and the chunk holds at least kHalvesDenseMinTiles
//    tiles per KV head, quarters otherwise (over whole dense prefills in
//    chunks of 128-512 at L = 4096-16384 the fastest rule, or within 1 % of
//    it), each with the T its simulation picks.
// A candidate is taken only if its split row blocks' counters and partials
// fit the workspace bound (tmx::kMaxSplitRowBlocks, tmx::kMaxSplitItems); the
// no-split plan always does, so every chunk has a plan.
struct PlanModel {
  int slots;               // workgroups of one KV head resident at once
  int parts;               // KV parts: tiles per workgroup and loop iteration
  double item_fixed;       // an item's fixed part ...
  double per_iteration;    // ... plus this much per loop iteration
  double merge_fixed;      // a split row block's merge ...
  double merge_per_piece;  // ... plus this much per piece
};
// Relative costs (only their ratios matter).
constexpr PlanModel kSmallQuarters{16, 4, 5.351, 1.239, 0.040, 0.749};
constexpr PlanModel kSmallHalves{32, 2, 8.112, 0.841, 2.298, 1.084};
constexpr PlanModel kLargeHalves{32, 2, 5.307, 0.483, 0.875, 1.489};
constexpr PlanModel kLargeWhole{64, 1, 4.908, 0.456, 0.555, 1.027};
constexpr PlanModel kDenseQuarters{16, 4, 6, 1, 1, 1};
constexpr PlanModel kDenseHalves{32, 2, 5, 1, 3, 1};
constexpr int kMaxSlots = 64;
static_assert(kSmallQuarters.slots <= kMaxSlots && kSmallHalves.slots <= kMaxSlots &&
                  kLargeHalves.slots <= kMaxSlots && kLargeWhole.slots <= kMaxSlots &&
                  kDenseQuarters.slots <= kMaxSlots && kDenseHalves.slots <= kMaxSlots,
              "simulated_time's slot heap");
constexpr int kLargeMinRowBlocks = 17;
constexpr int kHalvesSplitMinRowBlocks = 4;
constexpr int64_t kHalvesDenseMinTiles = 2048;
// Smallest T per regime: 1024 keys (quarters, dense companion), 768 keys
// (halves of small TriangleMix chunks), 512 keys (chunks of 17+ row blocks).
constexpr int kMinSplitTiles = 1024 / tmx::kKvTile;
constexpr int kFineSplitTiles = 768 / tmx::kKvTile;
constexpr int kLargeSplitTiles = 512 / tmx::kKvTile;
// A chunk of more than this many items at T = kMinSplitTiles is not
// simulated (its host cost would show): T then spreads the chunk's tiles over
// one KV-halves item per slot.
constexpr int64_t kMaxSimulatedItems = 4096;
constexpr int kLadderTop = 128;  // candidate T: kLadderTop, kLadderTop - 4, ..., down to the floor
constexpr int kSplitStep = 4;

// The row blocks (in issue order, row_tiles[o] tiles each) up to the last one
// that T splits, and the items they make: the arrival words and partials a
// launch with this T needs.
struct SplitLayout {
  int split_row_blocks;
  int64_t split_items;
  int64_t items;
};

SplitLayout split_layout(const std::vector<int>& row_tiles, int T) {
  SplitLayout s{0, 0, 0};
  int64_t before = 0;  // items of the row blocks before o
  for (size_t o = 0; o < row_tiles.size(); ++o) {
    const int pieces = (row_tiles[o] + T - 1) / T;
    before += pieces;
    if (pieces > 1) {
      s.split_row_blocks = (int)o + 1;
      s.split_items = before;
    }
  }
  s.items = before;
  return s;
}

bool layout_fits(const SplitLayout& s) {
  return s.split_row_blocks <= tmx::kMaxSplitRowBlocks && s.split_items <= tmx::kMaxSplitItems;
}

// The simulated time of a plan (see above): a min-heap of slot loads.  Slot
// loads and merge completions only grow, so the simulation stops, returning
// a time above `limit`, as soon as either exceeds it: such a plan cannot beat
// the best one so far.
double simulated_time(const std::vector<int>& row_tiles, int T, const PlanModel& m, double limit) {
  double heap[kMaxSlots] = {};  // all zero: a valid min-heap
  auto add_to_least = [&](double cost) {
    const double v = heap[0] + cost;  // replace the root, sift down
    int i = 0;
    for (;;) {
      const int l = 2 * i + 1, r = l + 1;
      int k = i;
      double kv = v;
      if (l < m.slots && heap[l] < kv) k = l, kv = heap[l];
      if (r < m.slots && heap[r] < kv) k = r, kv = heap[r];
      if (k == i) break;
      heap[i] = heap[k];
      i = k;
    }
    heap[i] = v;
    return v;
  };
  double merged = 0.0;  // the latest split row block's merge
  for (const int n : row_tiles) {
    const int pieces = (n + T - 1) / T;
    double last = 0.0;
    for (int i = 0; i < pieces; ++i) {
      const int size = (int)((int64_t)(i + 1) * n / pieces - (int64_t)i * n / pieces);
      const double cost = m.item_fixed + m.per_iteration * (double)((size + m.parts - 1) / m.parts);
      last = std::max(last, add_to_least(cost));
    }
    if (pieces > 1) merged = std::max(merged, last + m.merge_fixed + m.merge_per_piece * pieces);
    if (last > limit || merged > limit) return std::max(last, merged);
  }
  double end = merged;
  for (int k = 0; k < m.slots; ++k) end = std::max(end, heap[k]);
  return end;
}

// Candidate T, largest first: for rows longer than kLadderTop tiles every T
// that cuts the longest row into whole pieces above the ladder (down to one
// piece, no split) unless ladder_only, then the ladder kLadderTop,
// kLadderTop - 4, ... down to min_tiles.
std::vector<int> split_candidates(int longest, int min_tiles, bool ladder_only) {
  std::vector<int> t;
  if (longest > kLadderTop && !ladder_only) {
    for (int k = 1;; ++k) {
      const int tk = (longest + k - 1) / k;
      if (tk <= kLadderTop) break;
      if (t.empty() || tk != t.back()) t.push_back(tk);
    }
  }
  for (int tk = kLadderTop; tk >= min_tiles; tk -= kSplitStep) t.push_back(tk);
  return t;
}

struct ChunkPlan {
  int kv_parts, tiles_per_split;
};

// The best (shape, T) among the shapes' candidates, in the order given
// (earlier shapes and larger T win ties).  Each shape's candidates include a
// plan that splits nothing (T at or above the longest row), which always fits
// the workspace bound; should no candidate fit, the first shape runs every
// row unsplit.
struct ShapeCandidates {
  int kv_parts;
  const PlanModel* model;
  int min_tiles;
  bool ladder_only;
};

ChunkPlan best_plan(const std::vector<int>& row_tiles, std::initializer_list<ShapeCandidates> shapes) {
  int longest = 0;
  for (const int n : row_tiles) longest = std::max(longest, n);
  ChunkPlan best{0, 0};
  double best_time = 0.0;
  for (const ShapeCandidates& s : shapes) {
    bool unsplit_done = false;  // every T >= longest is the same plan: simulate the first only
    for (const int tk : split_candidates(longest, s.min_tiles, s.ladder_only)) {
      if (tk >= longest) {
        if (unsplit_done) continue;
        unsplit_done = true;
      }
      if (!layout_fits(split_layout(row_tiles, tk))) continue;
      const double t = simulated_time(row_tiles, tk, *s.model,
                                      best.kv_parts == 0 ? std::numeric_limits<double>::infinity() : best_time);
      if (best.kv_parts == 0 || t < best_time) {
        best = {s.kv_parts, tk};
        best_time = t;
      }
    }
  }
  if (best.kv_parts == 0) best = {shapes.begin()->kv_parts, std::max(longest, 1)};
  return best;
}

ChunkPlan choose_plan(const std::vector<int>& row_tiles, bool sparse) {
  const int num_row_blocks = (int)row_tiles.size();
  int64_t total = 0;
  int longest = 0;
  for (const int n : row_tiles) {
    total += n;
    longest = std::max(longest, n);
  }
  if (total / kMinSplitTiles > kMaxSimulatedItems) {
    // Spread the tiles over one KV-halves item per slot: the largest
    // candidate that does not go below that share and fits the workspace
    // bound (one piece always does).  Such chunks have so many row blocks, or
    // rows so long, that this rarely splits.
    const int64_t per_item = (total + kLargeHalves.slots - 1) / kLargeHalves.slots;
    const std::vector<int> cands = split_candidates(longest, kMinSplitTiles, false);
    int pick = cands.front();
    for (const int tk : cands) {
      if (tk < per_item || !layout_fits(split_layout(row_tiles, tk))) break;
      pick = tk;
    }
    return {2, pick};
  }
  if (num_row_blocks >= kLargeMinRowBlocks) {
    return best_plan(row_tiles, {{2, &kLargeHalves, kLargeSplitTiles, false},
                                 {1, &kLargeWhole, kLargeSplitTiles, false}});
  }
  if (sparse) {
    return best_plan(row_tiles, {{4, &kSmallQuarters, kMinSplitTiles, true},
                                 {2, &kSmallHalves, kFineSplitTiles, false}});
  }
  const ChunkPlan halves = best_plan(row_tiles, {{2, &kDenseHalves, kMinSplitTiles, false}});
  if (num_row_blocks >= kHalvesSplitMinRowBlocks && longest > halves.tiles_per_split &&
      total >= kHalvesDenseMinTiles) {
    return halves;
  }
  return best_plan(row_tiles, {{4, &kDenseQuarters, kMinSplitTiles, false}});
}

// The choice depends only on the chunk geometry, which repeats for every layer
// of a step: a per-thread cache keeps the simulation (4-200 us on the host for
// a chunk, a few ms for a whole long prompt) off the launch path.  64 entries
// hold every chunk of a 131072-token prefill in chunks of 2048, so even a
// sequence of distinct chunks repeated layer by layer plans each chunk once.
struct PlanKey {
  int64_t num_row_blocks, query_start, seq_len, sparse_begin, sparse_end;
  bool operator==(const PlanKey& o) const {
    return num_row_blocks == o.num_row_blocks && query_start == o.query_start && seq_len == o.seq_len &&
           sparse_begin == o.sparse_begin && sparse_end == o.sparse_end;
  }
};

#ifdef TRIANGLEMIX_PLAN_OVERRIDE
// Diagnostic builds only (-DTRIANGLEMIX_PLAN_OVERRIDE): a plan that every
// call takes instead of the planner's, for the forced-plan sweeps the costs
// above are fitted to.  Not thread-safe; the product library is built without
// it.
int g_override_parts = 0, g_override_tiles = 0;
#endif

ChunkPlan cached_plan(const PlanKey& key) {
#ifdef TRIANGLEMIX_PLAN_OVERRIDE
  if (g_override_parts > 0) return ChunkPlan{g_override_parts, g_override_tiles};
#endif
  constexpr int kEntries = 64;
  thread_local PlanKey keys[kEntries];
  thread_local ChunkPlan values[kEntries];
  thread_local int used = 0, next = 0;
  for (int i = 0; i < used; ++i) {
    if (keys[i] == key) return values[i];
  }
  std::vector<int> row_tiles((size_t)key.num_row_blocks);
  for (int64_t o = 0; o < key.num_row_blocks; ++o) {
    row_tiles[(size_t)o] = tmx::row_block_splits((int)o, (int)key.num_row_blocks, (int)key.query_start,
                                                 (int)key.seq_len, (int)key.sparse_begin, (int)key.sparse_end, 1);
  }
  const ChunkPlan plan = choose_plan(row_tiles, key.sparse_begin != 0);  // 0 only for the dense companion
  keys[next] = key;
  values[next] = plan;
  next = (next + 1) % kEntries;
  used = used < kEntries ? used + 1 : used;
  return plan;
}

// Work items per KV head beyond which a launch is refused (its grid would
// exceed 2^30 workgroups).
constexpr int64_t kMaxItemsPerHead = int64_t(1) << 26;

struct Geometry {
  int sparse_begin, sparse_end, num_row_blocks, tiles_per_split, kv_parts;
  int64_t items_per_head;
  int split_row_blocks;  // row blocks in issue order up to the last split one (0: nothing splits)
  int64_t split_items;   // their items: the partial records per KV head
  int64_t workspace_bytes;
};

Geometry make_geometry(bool sparse, int64_t query_tokens, int64_t query_start, int64_t seq_len, int64_t prompt_len) {
  Geometry g{};
  g.sparse_begin = sparse ? tmx::kSparseBegin : 0;
  g.sparse_end = sparse ? (int)(prompt_len > tmx::kDenseTail ? prompt_len - tmx::kDenseTail : 0) : 0;
  g.num_row_blocks = (int)((query_tokens + tmx::kRowBlock - 1) / tmx::kRowBlock);
  const ChunkPlan plan = cached_plan(PlanKey{g.num_row_blocks, query_start, seq_len, g.sparse_begin, g.sparse_end});
  g.kv_parts = plan.kv_parts;
  g.tiles_per_split = plan.tiles_per_split;
  int64_t items = 0;
  for (int o = 0; o < g.num_row_blocks; ++o) {
    const int s = tmx::row_block_splits(o, g.num_row_blocks, (int)query_start, (int)seq_len, g.sparse_begin,
                                        g.sparse_end, g.tiles_per_split);
    items += s;
    if (s > 1) {
      g.split_row_blocks = o + 1;
      g.split_items = items;
    }
  }
  g.items_per_head = items;
  g.workspace_bytes = g.split_row_blocks > 0
                          ? tmx::kCounterBytes + int64_t(tmx::kKvHeads) * g.split_items * tmx::kPartialBytes
                          : 0;
  return g;
}

// Validates a call's attributes and plans it: the launch, the workspace-size
// queries and tm_chunk_plan share this, so a size query answers -1 for
// exactly the calls a launch would refuse for their attributes.
int plan_call(bool sparse, int64_t query_tokens, int64_t query_start, int64_t seq_len, int64_t prompt_len,
              Geometry* g) {
  const int st = check_attributes(query_tokens, query_start, seq_len, prompt_len, sparse);
  if (st != TM_OK) return st;
  *g = make_geometry(sparse, query_tokens, query_start, seq_len, prompt_len);
  // The planner keeps every plan within these bounds; they guard the kernel's
  // indexing should that ever change.
  if (g->split_row_blocks > tmx::kMaxSplitRowBlocks || g->split_items > tmx::kMaxSplitItems ||
      g->workspace_bytes > tmx::kMaxWorkspaceBytes) {
    return fail(TM_ERR_UNSUPPORTED, "chunk plan needs %lld bytes of workspace; the limit is %lld",
                (long long)g->workspace_bytes, (long long)tmx::kMaxWorkspaceBytes);
  }
  if (g->items_per_head > kMaxItemsPerHead) {
    return fail(TM_ERR_UNSUPPORTED, "chunk needs %lld work items per KV head; the limit is %lld",
                (long long)g->items_per_head, (long long)kMaxItemsPerHead);
  }
  return TM_OK;
}

// A fresh arrival tag: nonzero and below 2^48, different from every other tag
// this process hands out (and, by its seed, unlikely to meet another
// process's tags in a shared workspace).
unsigned long long next_epoch() {
  static std::atomic<unsigned long long> counter{[] {
    const unsigned long long t = (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count();
    return (t * 0x9E3779B97F4A7C15ull) ^ ((unsigned long long)getpid() << 24);
  }()};
  for (;;) {
    const unsigned long long e = counter.fetch_add(1, std::memory_order_relaxed) & tmx::kEpochMask;
    if (e != 0) return e;
  }
}

// Arrival tag of a launch on `workspace`: one per workspace address, kept
// across calls.  Every completed launch leaves its arrival words at (its
// tag, count 0), so the next launch on the same workspace -- which gets the
// same tag -- counts each arrival with one fetch-and-add; a word with any
// other content (another address's tag, a fresh or reused buffer, garbage)
// is foreign and takes the install.  Only completed launches write a word
// with this tag, and launches that overlap on one workspace race anyway, so
// a word carrying it always has count 0 when a launch starts.  A small
// direct-mapped table holds the tags; an evicted address gets a fresh tag
// on its next call (one install per word, then fast again).
unsigned long long workspace_epoch(const void* workspace) {
  constexpr int kSlots = 64;
  struct Slot {
    const void* workspace;
    unsigned long long epoch;
  };
  static Slot slots[kSlots] = {};
  static std::mutex mutex;
  const uintptr_t a = (uintptr_t)workspace;
  Slot& s = slots[(a >> 8 ^ a >> 16 ^ a >> 24) % kSlots];
  std::lock_guard<std::mutex> lock(mutex);
  if (s.workspace != workspace || s.epoch == 0) s = Slot{workspace, next_epoch()};
  return s.epoch;
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

  Geometry g;
  st = plan_call(sparse, query_tokens, query_start, seq_len, prompt_len, &g);
  if (st != TM_OK) return st;
  if (workspace_bytes < g.workspace_bytes) {
    return fail(TM_ERR_WORKSPACE, "workspace of %lld bytes is smaller than the %lld bytes this call needs",
                (long long)workspace_bytes, (long long)g.workspace_bytes);
  }
  if (g.workspace_bytes > 0) {
    // 64-bit atomics on the arrival words and 16-byte partial stores
    if (((uintptr_t)workspace & 15) != 0) return fail(TM_ERR_WORKSPACE, "workspace must be 16-byte aligned");
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
  const bool split = g.split_row_blocks > 0;
  p.counters = split ? static_cast<unsigned long long*>(workspace) : nullptr;
  p.partials = split ? reinterpret_cast<float*>(static_cast<char*>(workspace) + tmx::kCounterBytes) : nullptr;
  p.epoch = split ? workspace_epoch(workspace) : 0;
  p.num_pages = (int)num_pages;
  p.query_start = (int)query_start;
  p.seq_len = (int)seq_len;
  p.sparse_begin = g.sparse_begin;
  p.sparse_end = g.sparse_end;
  p.num_row_blocks = g.num_row_blocks;
  p.tiles_per_split = g.tiles_per_split;
  p.items_per_head = (int)g.items_per_head;
  p.split_row_blocks = g.split_row_blocks;
  p.split_items = (int)g.split_items;
  p.scale_log2 = scale * 1.4426950408889634f;
  const hipError_t err =
      tmx::launch_triangle_paged_attention(p, sparse, g.kv_parts, static_cast<hipStream_t>(stream));
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
  Geometry g;
  if (plan_call(true, query_tokens, query_start, seq_len, prompt_len, &g) != TM_OK) return -1;
  return g.workspace_bytes;
}

int tm_triangle_paged_sparse_attention_noalloc(const void* query, const void* key_cache, const void* value_cache,
                                               const int32_t* block_table, void* out, int64_t query_tokens,
                                               int64_t num_pages, int64_t block_table_cols, int64_t query_start,
                                               int64_t seq_len, int64_t prompt_len, float scale, void* stream) {
  g_last_error[0] = '\0';
  // Attributes first (same errors as the workspace entry point), then the
  // scratch this geometry needs against what the per-GPU array holds (the
  // array is as large as any plan's workspace, so this guards a change of
  // either bound).
  Geometry g;
  const int st = plan_call(true, query_tokens, query_start, seq_len, prompt_len, &g);
  if (st != TM_OK) return st;
  const int64_t need = g.workspace_bytes;
  if (need > tmx::kNoAllocScratchBytes) {
    return fail(TM_ERR_WORKSPACE,
                "chunk needs %lld bytes of split-KV scratch; the no-allocation entry point holds %lld per GPU",
                (long long)need, (long long)tmx::kNoAllocScratchBytes);
  }
  void* scratch = nullptr;
  if (need > 0) {
    const hipError_t err = tmx::noalloc_scratch(&scratch);
    if (err != hipSuccess) return fail(TM_ERR_LAUNCH, "no-allocation scratch lookup failed: %s", hipGetErrorString(err));
  }
  return launch(true, query, key_cache, value_cache, block_table, out, query_tokens, num_pages, block_table_cols,
                query_start, seq_len, prompt_len, scale, scratch, need > 0 ? tmx::kNoAllocScratchBytes : 0, stream);
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
  Geometry g;
  if (plan_call(false, query_tokens, query_start, seq_len, seq_len, &g) != TM_OK) return -1;
  return g.workspace_bytes;
}

int tm_chunk_plan(int dense, int64_t query_tokens, int64_t query_start, int64_t seq_len, int64_t prompt_len,
                  int32_t* kv_parts, int32_t* tiles_per_split, int64_t* items_per_kv_head) {
  g_last_error[0] = '\0';
  if (kv_parts == nullptr || tiles_per_split == nullptr || items_per_kv_head == nullptr) {
    return fail(TM_ERR_INVALID_ARGUMENT, "tm_chunk_plan: null output pointer");
  }
  const bool sparse = dense == 0;
  const int64_t prompt = sparse ? prompt_len : seq_len;
  Geometry g;
  const int status = plan_call(sparse, query_tokens, query_start, seq_len, prompt, &g);
  if (status != TM_OK) return status;
  *kv_parts = g.kv_parts;
  *tiles_per_split = g.tiles_per_split;
  *items_per_kv_head = g.items_per_head;
  return TM_OK;
}

#ifdef TRIANGLEMIX_PLAN_OVERRIDE
// Diagnostic export: every later call takes (kv_parts, tiles_per_split) as
// its plan; kv_parts 0 returns to the planner.  Calls the planner would not
// make (a layout beyond the workspace bound) are still refused.
void tm_plan_override(int32_t kv_parts, int32_t tiles_per_split) {
  const bool valid = (kv_parts == 1 || kv_parts == 2 || kv_parts == 4) && tiles_per_split > 0;
  g_override_parts = valid ? kv_parts : 0;
  g_override_tiles = valid ? tiles_per_split : 0;
}
#endif

int tm_reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                         const int64_t* slot_mapping, int64_t num_tokens, int64_t key_stride, int64_t value_stride,
                         int64_t num_pages, void* stream) {
  g_last_error[0] = '\0';
  if (num_tokens < 0 || num_tokens > tmx::kMaxPositions) {
    return fail(TM_ERR_INVALID_ARGUMENT, "key and value must be [num_tokens, 8, 128] with 0 <= num_tokens <= %lld",
                (long long)tmx::kMaxPositions);
  }
  if (num_pages <= 0) {
    return fail(TM_ERR_INVALID_ARGUMENT, "key_cache must be [pages, 128, 8, 128] with pages > 0");
  }
  if (num_pages > tmx::kMaxPages) {
    return fail(TM_ERR_UNSUPPORTED, "key_cache has %lld pages; the limit is %lld", (long long)num_pages,
                (long long)tmx::kMaxPages);
  }
  if (num_tokens == 0) return TM_OK;  // nothing to write, nothing enqueued
  if (!key || !value || !key_cache || !value_cache || !slot_mapping) {
    return fail(TM_ERR_INVALID_ARGUMENT, "key, value, key_cache, value_cache and slot_mapping must be non-null");
  }
  constexpr int64_t kRowElems = int64_t(tmx::kKvHeads) * tmx::kHeadDim;
  if (key_stride < kRowElems || value_stride < kRowElems || key_stride % 8 != 0 || value_stride % 8 != 0) {
    return fail(TM_ERR_INVALID_ARGUMENT,
                "key and value rows must hold [8, 128] contiguous elements with a row stride >= 1024 that is a "
                "multiple of 8");
  }
  const uintptr_t misaligned = ((uintptr_t)key | (uintptr_t)value | (uintptr_t)key_cache | (uintptr_t)value_cache) & 15;
  if (misaligned) {
    return fail(TM_ERR_INVALID_ARGUMENT, "key, value and the caches must be 16-byte aligned");
  }
  // The caches are written: they must not overlap each other, the sources or the slot mapping.
  const Range r_k{(uintptr_t)key, (uintptr_t)key + uintptr_t(((num_tokens - 1) * key_stride + kRowElems) * 2)};
  const Range r_v{(uintptr_t)value, (uintptr_t)value + uintptr_t(((num_tokens - 1) * value_stride + kRowElems) * 2)};
  const Range r_kc{(uintptr_t)key_cache, (uintptr_t)key_cache + uintptr_t(num_pages * kPageBytes)};
  const Range r_vc{(uintptr_t)value_cache, (uintptr_t)value_cache + uintptr_t(num_pages * kPageBytes)};
  const Range r_s{(uintptr_t)slot_mapping, (uintptr_t)slot_mapping + uintptr_t(num_tokens * 8)};
  if (overlaps(r_kc, r_vc) || overlaps(r_kc, r_k) || overlaps(r_kc, r_v) || overlaps(r_kc, r_s) ||
      overlaps(r_vc, r_k) || overlaps(r_vc, r_v) || overlaps(r_vc, r_s)) {
    return fail(TM_ERR_INVALID_ARGUMENT,
                "key_cache and value_cache must not overlap each other, key, value or slot_mapping");
  }
  const hipError_t err = tmx::launch_paged_kv_write(key, value, key_cache, value_cache, slot_mapping, num_tokens,
                                                    key_stride, value_stride, num_pages,
                                                    static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    return fail(TM_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  }
  return TM_OK;
}

}  // extern "C"
