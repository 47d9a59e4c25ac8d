// TriangleMix paged sparse prefill attention for MI355X (gfx950).
//
// Work decomposition
// ------------------
// A work item is (row block of 32 query tokens, KV head, KV split).  A
// workgroup's wave64s are (query head hl) x (KV part kq), in one of three
// shapes (template parameter P, chosen per chunk by the host):
//  * P = 4, KV quarters (eight waves): each item runs as two workgroups, one
//    per pair of the KV head's four GQA query heads; wave w owns the 32 rows
//    {32 tokens} x {head 4*kvh + 2*hp + hl} and processes every fourth 32-key
//    tile of the item (tiles kq, kq+4, ...).  A 512-token chunk fills the 256
//    CUs.
//  * P = 2, KV halves (eight waves): one workgroup holds all four heads of the
//    group and every wave every second tile; each K/V tile then serves four
//    heads, so a workgroup issues half the DMA per MFMA -- for chunks with
//    enough row blocks (or split items) to fill the CUs anyway.
//  * P = 1, KV whole (four waves): one wave per head of the group, every tile
//    of the item; two workgroups share a CU, so a 2048-token chunk's 512
//    workgroups run in one round, and there is no KV-part merge.
// Each K/V tile staged in LDS is read by the waves of its part, and the parts
// merge through LDS at the end.  Two waves per SIMD (of one workgroup, or one
// of each of two KV-whole workgroups) let one wave's softmax run while the
// other's MFMAs occupy the matrix core.
// The KV tiles of a row block are cut into splits of at most
// `tiles_per_split` tiles (host-chosen for load balance: at least 768 keys,
// no upper bound -- an item of any length runs in one workgroup), so only
// long dense rows split.  A row block with one
// split writes its output directly; otherwise every split writes an fp32
// partial (O, row max, row sum) to the workspace and counts its arrival, and
// the workgroup that arrives last merges all partials in split order
// (deterministic) and writes the output -- every chunk is one launch.
// The output leaves through an LDS stage as whole rows of the workgroup's
// heads, written through L2 (sc1), so the kernel's end has no dirty output
// lines to write back.
// Items are numbered per KV head, heaviest row blocks first; KV head =
// blockIdx % 8 keeps every workgroup of one KV head on one XCD (workgroups
// are dispatched round-robin over the 8 XCDs), so both head pairs of a row
// block (KV quarters), neighbouring row blocks' overlapping local windows and
// a row block's partials share one L2.
//
// Tiles, memory path and pipeline
// -------------------------------
// K/V tiles are 32 logical keys aligned to 32, so a tile never straddles a
// 128-token page: one block-table lookup per tile.  Tiles go from HBM straight
// into LDS with buffer_load_dwordx4 ... lds (no register staging).  Each wave
// runs a software pipeline over its tiles: in iteration i it issues the QK^T
// MFMAs of its tile of iteration i+1 interleaved with the exponentials of its
// tile of iteration i, then the PV MFMAs of tile i interleaved with the mask
// and row max of tile i+1 (the interleave is fixed in program order with
// scheduling barriers); the item's last iteration has no tile i+1 and runs
// only the exponentials and PV of its tile, after which each wave hands its
// share of the KV-part merge to LDS slots that iteration no longer reads
// without waiting for the others.  LDS holds two K slots and two V slots, each with the
// P tiles (one per part) of one iteration, plus the workgroup's Q (DMA'd
// once, read into registers in the prologue); the DMA of K for iteration
// i+2 (waves 0-3) and of V for iteration i+1 (waves 4-7) is spread over the
// MFMA steps of iteration i.  The four slots are
// distinct LDS objects and the loop is unrolled by two so every access names
// its slot statically: the compiler then sees that the prefetch never aliases
// the tiles being read and does not wait for it.  Each wave waits for its own
// DMA (vmcnt 0) before the barrier that opens the next iteration; iteration 0
// alone publishes its V tiles later, at a barrier before their first read, so
// that the prologue's DMA serves Q and K first.  Each tile
// is addressed through a buffer resource whose range stops at seq_len, so key
// rows past seq_len read as zeros.  LDS rows are 256 B (one key x 128 dims)
// with the 16-byte chunks XOR-swizzled so both read patterns are bank-conflict
// free:
//   K: chunk c of key row r sits in slot c ^ (r % 16)
//   V: chunk c of key row r sits in slot c ^ (4 * (r % 4))
//
// Contractions (per wave, v_mfma_f32_32x32x16_bf16)
// ---------------------------------------------------
//   S^T (32 keys x 32 rows) = K Q^T   A = K rows from LDS, B = Q in registers
//   O^T (128 x 32 rows)    += V^T P^T  A = V via ds_read_b64_tr_b16, B = P
// In the 32x32 accumulator layout lane l owns column l % 32, i.e. one query
// row: accumulator element v is key 8(v/4) + 4(l/32) + v%4 of the tile.  Row
// max / row sum are lane-local plus one exchange between the two 32-lane
// halves (v_permlane32_swap), and the fp32 scores convert in registers into
// the bf16 B operand of PV.  ds_read_b64_tr_b16 transposes within 16-lane
// groups: when the 4 source lanes 4j..4j+3 of a group point at 4 consecutive
// dims of key row j, destination lane t of the group receives dim t of keys
// 0..3 -- exactly the A-operand slice (one dim, four consecutive keys) of V^T.
//
// Mask
// ----
// Only tiles holding at least one attended (row, key) pair are visited (see
// row_block_tiles).  The exact per-element rule
//   attended(q, k) = k <= q && (dense(q) || k < 8 || q - k <= 512)
// is applied as two one-sided tests, each only on the tiles that need it
// (wave-uniform branches): the causal bound on tiles reaching past the block's
// first row, the window bound (with the sink exception on tile 0) on tiles
// starting below the block's last window start.  Interior tiles run unmasked.
//
// Numerics follow the reference order (operator/op_kernel/vendor/cann_9_0_1/
// block_sparse_attention/attn_infra/epilogue/block/
// block_epilogue_online_softmax.hpp:1002-1086 and
// block_epilogue_rescale_o.hpp:153-344): s*scale -> mask -> row max -> p = exp(s - m) in
// fp32 -> P to bf16 (round to nearest even) for PV, row sum from the fp32 p
// -> O = O*exp(m_old - m_new) + P V -> O / l -> bf16 round to nearest even.
// Exponentials are exp2 of log2(e)-prescaled scores; the KV parts and the
// split partials merge with the same rescale rule.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "trianglemix_kernel.h"

namespace tmx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

#define TM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

constexpr int kMaxWaves = 8;  // waves of the largest workgroup shape

// Phase clocks (diagnostic builds only, -DTRIANGLEMIX_PHASE_CLOCKS): lane 0 of
// every wave stores the 100 MHz s_memrealtime clock at the TM_PHASE(slot)
// points below, one 64-bit slot per (workgroup, wave, phase),
// for grids of up to kPhaseClockWorkgroups workgroups.  The product library
// is built without them.
#ifdef TRIANGLEMIX_PHASE_CLOCKS
constexpr int kPhaseClockWorkgroups = 4096;
constexpr int kPhaseClockSlots = 32;
__device__ unsigned long long phase_clocks[kPhaseClockWorkgroups * kMaxWaves * kPhaseClockSlots];
#define TM_PHASE(slot)                                                                                   \
  do {                                                                                                   \
    const unsigned long long tm_clock_ = __builtin_amdgcn_s_memrealtime();                               \
    if ((threadIdx.x & 63) == 0 && blockIdx.x < kPhaseClockWorkgroups)                                   \
      phase_clocks[(blockIdx.x * kMaxWaves + (threadIdx.x >> 6)) * kPhaseClockSlots + (slot)] = tm_clock_; \
  } while (0)
#else
#define TM_PHASE(slot) \
  do {                 \
  } while (0)
#endif
constexpr int kRowBytes = kHeadDim * 2;          // 256 B: one key row
constexpr int kTileBytes = kKvTile * kRowBytes;  // 8 KB: K or V of one tile
constexpr int kDmaPerTile = kTileBytes / 1024;   // 1 KB (4 key rows) per DMA instruction

// Workgroup shape: the waves are kParts KV parts x kHeads query heads.
// P = 4 (two heads, KV quarters) puts a 512-token chunk's 16 row blocks on
// 256 workgroups; P = 2 (all four heads of the GQA group, KV halves) loads
// each K/V tile once for four heads and cuts an aligned sparse row block's 18
// tiles into 9 + 9, for chunks with enough row blocks to fill the CUs.
// P = 1 (KV whole: four waves, one per head of the group, every tile of the
// item) has no KV-part merge and needs 64 KB of LDS, so two workgroups share
// a CU (one wave of each per SIMD): a chunk of 64 row blocks runs its 512
// workgroups in one round instead of two rounds of KV halves.
template <int P>
struct Shape {
  static constexpr int kParts = P;                      // KV parts: tiles kq, kq + P, ...
  static constexpr int kWaves = P == 1 ? 4 : 8;         // waves per workgroup
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kHeads = kWaves / P;             // query heads per workgroup
  static constexpr int kWgPerKvHead = kGroup / kHeads;  // workgroups per (row block, KV head)
  static constexpr int kSlotBytes = P * kTileBytes;     // the tiles of all parts of one iteration
  static constexpr int kDmaPerWave = 2 * P * kDmaPerTile / kWaves;  // DMA instructions per wave and iteration
  static constexpr int kWavesPerTile = kDmaPerTile / kDmaPerWave;   // waves sharing one tile's DMA
  static constexpr int kOwned = (kHeadDim / 32) / P;    // 32-wide d-blocks a wave keeps in the merge
  static constexpr int kQBlocksPerWave = 8 * kHeads / kWaves;  // 1 KB blocks of Q each wave DMAs
  static_assert((P == 4 || P == 2 || P == 1) && kHeads * P == kWaves && kHeads <= kGroup,
                "supported shapes: 4 x 2, 2 x 4 and 1 x 4");
};
// Buffer-resource word 3 for raw (unformatted, stride 0) dword loads on gfx9.
constexpr int kBufferFlags = 0x00020000;
// A buffer offset past every range used here: such a load returns 0.
constexpr unsigned kOutOfRange = 0x40000000u;

static_assert(kKvTile == 32 && kPageSize % kKvTile == 0, "a tile must stay inside one page");
static_assert(kRowBlock == 32, "one MFMA column per query token");
static_assert(kDmaPerTile == 8, "a tile is eight 1 KB DMA instructions, one per MFMA step at most");

// Wait until every LDS DMA (and other vector-memory load) this wave issued has
// landed: s_waitcnt vmcnt(0), expcnt / lgkmcnt unconstrained.  Each wave runs
// it before a barrier that publishes DMA'd tiles to the other waves -- the
// barrier alone does not order the DMA's LDS writes.
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// All but the last N (< 64) vector-memory operations of this wave have landed
// (vmcnt bits 3:0 and 15:14 of the gfx9 s_waitcnt immediate).
template <int N>
__device__ __forceinline__ void wait_dma_but() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ int k_slot(int row, int chunk) { return chunk ^ (row & 15); }
__device__ __forceinline__ int v_slot(int row, int chunk) { return chunk ^ ((row & 3) << 2); }

// The launch fields the prologue needs before its first memory round trip.
// They are the kernel's leading scalar arguments, which the command processor
// preloads into SGPRs (the library is built with
// -amdgpu-kernarg-preload-count): the block-table loads and the Q DMA issue
// without waiting for a kernarg load first (measured 0.3-0.4 us per launch).
// KernelParams, an aggregate passed by reference and never preloaded, carries
// the rest, which is first needed after that round trip.
struct PrologueArgs {
  const int32_t* block_table;
  const __bf16* query;
  int query_start;
  int seq_len;
  int num_row_blocks;
  int sparse_begin;
  int sparse_end;
  int split_items;
  int split_row_blocks;
  int tiles_per_split;
};

// Work item -> (row-block order index, split index, split count), computed
// by every wave from the split counts of the first p.split_row_blocks row
// blocks in issue order (lane i: row block base + i), which hold items
// 0 .. p.split_items - 1.
// The exclusive prefix sum over the lanes needs no cross-lane data move: bit
// by bit, it adds 2^b times the number of lower lanes whose count has bit b
// set (v_mbcnt of a ballot).  That is a few VALU and SALU instructions per
// bit -- six bits cover 63 splits, and a non-negative int has at most 31 --
// instead of a chain of dependent ds_bpermute round trips.
__device__ __forceinline__ void decode_item(const PrologueArgs& p, int sparse_begin, int sparse_end, int item,
                                            int lane, int& order, int& split, int& nsplit) {
  int acc = 0;
  order = 0;
  split = 0;
  nsplit = 1;
  for (int base = 0; base < p.split_row_blocks; base += 64) {
    const int o = base + lane;
    const int cnt = o < p.split_row_blocks ? row_block_splits(o, p.num_row_blocks, p.query_start, p.seq_len,
                                                            sparse_begin, sparse_end, p.tiles_per_split)
                                         : 0;
    int excl = 0;   // items of the row blocks on lower lanes
    int total = 0;  // items of the 64 row blocks
    for (int b = 0; __ballot((cnt >> b) != 0) != 0; ++b) {
      const unsigned long long bit = __ballot(((cnt >> b) & 1) != 0);
      excl += (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bit >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bit, 0u)) << b;
      total += __popcll(bit) << b;
    }
    if (item < acc + total) {
      const bool mine = cnt > 0 && item >= acc + excl && item < acc + excl + cnt;
      const int src = __ffsll((unsigned long long)__ballot(mine)) - 1;
      order = base + src;
      split = item - acc - __builtin_amdgcn_readlane(excl, src);
      nsplit = __builtin_amdgcn_readlane(cnt, src);
      return;
    }
    acc += total;
  }
}

// Rescale the running O / row sum only when some row's max grew by more than
// 2^kLazyRescale (log2 units); otherwise keep the stale max as the exponent
// shift, so p <= 2^kLazyRescale -- exact in fp32 and bf16 range -- and the
// 64 multiplies of the O rescale are skipped on most tiles.
constexpr float kLazyRescale = 8.0f;

// max / sum of x over the lane pair (i, i ^ 32), in every lane: v_permlane32_swap
// hands each lane both halves, so no lane select is needed.
__device__ __forceinline__ float half_max(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Key offset inside the tile of accumulator element v, for lanes of the
// first 32-lane half (the second half adds 4).
__device__ __forceinline__ constexpr int elem_key(int v) { return 8 * (v >> 2) + (v & 3); }

// MFMA step c of S^T = K Q^T (dims 16c .. 16c+15): the K operand from LDS.
__device__ __forceinline__ bf16x8_t k_operand(const char* kt, const int* k_off, int c) {
  return *reinterpret_cast<const bf16x8_t*>(kt + k_off[c]);
}

// MFMA step k of O^T += V^T P^T (k = 0..7: d-block m = k % 4, k-group j = k / 4
// of 16 keys): the V^T operand, two transposed reads.  k-slot e of half h in
// k-group j is key 16j + 8(e/4) + 4h + e%4 -- the keys of P's bf16 lane
// vector pb[j].
__device__ __forceinline__ bf16x8_t v_operand(const char* vt, const int* v_off, int k) {
  const char* a0 = vt + 16 * (k >> 2) * kRowBytes + v_off[k & 3];
  const i16x4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(a0));
  const i16x4_t hi4 =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(a0 + 8 * kRowBytes));
  const i16x4_t lohi[2] = {lo4, hi4};
  bf16x8_t a;
  __builtin_memcpy(&a, lohi, sizeof(a));
  return a;
}

// The i-th exponential a full iteration adds to the row sum: block 1 step k
// adds element k and, on even k, 8 + k/2; block 2 adds 12-15.
__device__ __forceinline__ constexpr int sum_order(int i) {
  return i < 12 ? (i % 3 == 1 ? 8 + i / 3 : i - (i + 1) / 3) : i;
}
static_assert(sum_order(0) == 0 && sum_order(1) == 8 && sum_order(2) == 1 && sum_order(4) == 9 &&
                  sum_order(10) == 11 && sum_order(11) == 7 && sum_order(12) == 12,
              "block 1 adds 0, 8, 1, 2, 9, 3, ..., 7");

// How many MFMA steps ahead of their use the LDS operand reads are issued.
constexpr int kReadAhead = 3;

// Causal bound: keep elements whose key offset is <= thr (per lane).
__device__ __forceinline__ void mask_causal(f32x16_t& s, int thr) {
#pragma unroll
  for (int v = 0; v < 16; ++v) s[v] = elem_key(v) <= thr ? s[v] : -INFINITY;
}

// Window bound: keep elements whose key offset is >= thr; the elements that
// can hold sink keys (v < 4 on tile 0) compare against thr_sink instead.
__device__ __forceinline__ void mask_window(f32x16_t& s, int thr, int thr_sink) {
#pragma unroll
  for (int v = 0; v < 16; ++v) s[v] = elem_key(v) >= (v < 4 ? thr_sink : thr) ? s[v] : -INFINITY;
}

// Online softmax of one tile in the log2 domain (max commutes with the
// positive scale), state update: the tile's row max m_tile (already scaled to
// log2 units) updates the row state and rescales O when needed.  Returns the
// exponent shift of the tile's exponentials.
__device__ __forceinline__ float softmax_update(float m_tile, float& m_run, float& l_run, f32x16_t* o_acc) {
  // Wave-uniform branch, taken when some row's max grows past the lazy bound
  // (or a row meets its first attended keys after an all-masked first tile).
  if (__any(m_tile > m_run + kLazyRescale)) {
    const float m_new = fmaxf(m_run, m_tile);
    // exp2(-inf - x) = 0 rescales an empty state; a row still without keys keeps m = -inf.
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) o_acc[m] *= alpha;
    m_run = m_new;
  }
  // Rows with no attended key yet keep m = -inf; shift by 0 then so that
  // exp2(-inf - 0) = 0 and no NaN is formed.
  return m_run == -INFINITY ? 0.0f : m_run;
}

// At least two waves per SIMD: the eight-wave shapes hold two by themselves,
// and two KV-whole workgroups share a CU only within that register budget.
template <bool kSparse, int P>
__global__ void __launch_bounds__(Shape<P>::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
triangle_paged_attention_kernel(const int32_t* block_table, const __bf16* query, int query_start, int seq_len,
                                int num_row_blocks, int sparse_begin_arg, int sparse_end_arg, int split_items,
                                int split_row_blocks, int tiles_per_split, KernelParams p) {
  const PrologueArgs pa{block_table,    query,          query_start, seq_len,          num_row_blocks,
                        sparse_begin_arg, sparse_end_arg, split_items, split_row_blocks, tiles_per_split};
  using S = Shape<P>;
  constexpr int H = S::kHeads;
  // K slots 0/1 and V slots 0/1: the P tiles of iteration i live in slot i % 2.
  __shared__ __attribute__((aligned(1024))) char k_lds0[S::kSlotBytes];
  __shared__ __attribute__((aligned(1024))) char k_lds1[S::kSlotBytes];
  __shared__ __attribute__((aligned(1024))) char v_lds0[S::kSlotBytes];
  __shared__ __attribute__((aligned(1024))) char v_lds1[S::kSlotBytes];
  // Q of the workgroup's heads: [head][row][16-byte slot], K's swizzle.
  __shared__ __attribute__((aligned(1024))) char q_lds[H * kRowBlock * kRowBytes];
  __shared__ int s_last;  // this workgroup completed its row block's splits

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, kept scalar
  const int hl = wave % H;   // query head inside the workgroup's heads
  const int kq = wave / H;   // KV part: tiles kq, kq+P, ... of the item
  const int lane = tid & 63;
  const int n = lane & 31;  // MFMA column = query token of this lane
  const int half = lane >> 5;

  const int sparse_begin = kSparse ? pa.sparse_begin : 0;
  const int sparse_end = kSparse ? pa.sparse_end : 0;
  TM_PHASE(0);

  const int kvh = blockIdx.x % kKvHeads;
  const int hp = (blockIdx.x / kKvHeads) % S::kWgPerKvHead;
  const int item = blockIdx.x / (kKvHeads * S::kWgPerKvHead);
  int order, split, nsplit;
  if (item < pa.split_items) {
    decode_item(pa, sparse_begin, sparse_end, item, lane, order, split, nsplit);
    // The decoded item is wave-uniform; say so, so that all tile arithmetic,
    // block-table loads and buffer resources stay scalar.
    order = __builtin_amdgcn_readfirstlane(order);
    split = __builtin_amdgcn_readfirstlane(split);
    nsplit = __builtin_amdgcn_readfirstlane(nsplit);
  } else {
    order = pa.split_row_blocks + (item - pa.split_items);
    split = 0;
    nsplit = 1;
  }
  const int rb = pa.num_row_blocks - 1 - order;
  const int tb = pa.query_start + rb * kRowBlock;
  const int te = min(tb + kRowBlock, pa.seq_len);
  const int hq = H * hp + hl;  // query head inside the GQA group
  const int q = tb + n;

  const TileRuns runs = row_block_tiles(tb, te, sparse_begin, sparse_end);
  const int all_tiles = runs.count();
  // Split s of n takes tiles [s*b + min(s, r), ...) with b = all / n and
  // r = all % n: the first r splits get b + 1 tiles, the rest b.
  int t_lo = 0;
  int num_tiles = all_tiles;
  if (nsplit > 1) {
    const int base = all_tiles / nsplit;
    const int rem = all_tiles - base * nsplit;
    t_lo = split * base + min(split, rem);
    num_tiles = base + (split < rem ? 1 : 0);
  }
  const int num_iters = (num_tiles + P - 1) / P;

  // ---- DMA: per iteration the 2P tiles (K and V of every part) ----
  // A tile is eight wave-instructions of 1 KB (4 key rows).  With P = 4 wave w
  // loads one whole tile (waves 0-3 the K tile of quarter w, waves 4-7 the V
  // tile of quarter w - 4); with P = 2 and P = 1 two waves share a tile, four
  // instructions each (P = 1: waves 0-1 load K, 2-3 V).  Lane i of instruction j writes LDS slot (row 4j + i/16,
  // slot i%16), so it loads the global chunk the swizzle puts in that slot.
  const int dma_tile = wave / S::kWavesPerTile;
  const int dma_t = dma_tile / P;  // 0 = K, 1 = V
  const int dma_u = dma_tile % P;  // part
  const int dma_j0 = (wave % S::kWavesPerTile) * S::kDmaPerWave;  // this wave's first instruction of the tile
  unsigned dma_voff[kDmaPerTile];  // the first kDmaPerWave are used (fixed size: see kept below)
  static_assert(S::kDmaPerWave <= kDmaPerTile, "dma_voff holds one tile's instructions");
#pragma unroll
  for (int j = 0; j < S::kDmaPerWave; ++j) {
    const int row = 4 * (dma_j0 + j) + (lane >> 4);
    const int slot = dma_t == 0 ? k_slot(row, lane & 15) : v_slot(row, lane & 15);
    dma_voff[j] = (unsigned)(row * kKvHeads * kRowBytes + 16 * slot);
  }
  // DMA source of the item's tiles, 64 at a time: table block b (tiles 64b ..
  // 64b + 63) lives in row_lo when b is even and in row_hi when b is odd,
  // tile 64b + i in lane i.  The prologue fills blocks 0 and 1; an item of
  // more than 128 tiles refills a register in the loop once its block has
  // been issued (see refill below).  The value is the
  // cache row index of the tile's first key row of this KV head (its byte
  // offset / 256, below 2^32 as the host caps the cache at kMaxPages pages);
  // bytes_lo / bytes_hi hold the tile's valid byte count (rows cut at seq_len,
  // 0 past the item's end).  The loop reads them with v_readlane -- it never
  // waits on a scalar memory load (whose counter it shares with the LDS reads)
  // and builds a buffer resource in a few scalar instructions.  The
  // block-table loads go through a buffer resource whose range ends at the
  // data: an offset past it reads 0, so no load sits in a divergent branch
  // (the compiler waits for a load before such a branch joins).  Order: block
  // table, then Q, then the tile DMA -- loads complete in issue order, so the
  // DMA (which needs the page numbers) does not wait for Q, and Q's latency
  // hides behind the block-table round trip.
  const int logical_pages = (pa.seq_len + kPageSize - 1) / kPageSize;
  const __amdgpu_buffer_rsrc_t bt_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pa.block_table, (short)0, logical_pages * 4, kBufferFlags);
  auto lane_k0 = [&](int ti) { return ti < num_tiles ? runs.tile(t_lo + ti) * kKvTile : 0; };
  auto lane_page = [&](int ti) {
    const unsigned off = ti < num_tiles ? (unsigned)(lane_k0(ti) / kPageSize) * 4u : kOutOfRange;
    return __builtin_amdgcn_raw_buffer_load_b32(bt_rsrc, off, 0, 0);
  };
  const int phys_lo = lane_page(lane);
  const int phys_hi = lane_page(kTableTiles + lane);
  // Table block 2, for an item of more than 128 tiles (for a shorter one the
  // offset is out of range: the load returns 0 and touches no memory); the
  // loop turns it into rows when block 0 is used up (refill below).
  int refill_phys = lane_page(2 * kTableTiles + lane);
  // ---- Q: the workgroup's H heads x 32 rows (8 KB per head), DMA'd once into LDS ----
  // (each of the P part waves of a head needs all of it; loading it per wave
  // would multiply the start-up traffic through the CU).  Wave w loads the B =
  // 8 H / waves 1 KB blocks g = B w .. B w + B - 1: head g / 8, rows 4 (g % 8)
  // .. + 3; lane i writes slot i % 16 of row 4 (g % 8) + i / 16, i.e. global
  // chunk k_slot(row, i % 16).  The range ends at the block's last row: rows
  // past seq_len read 0.  Issued before the wait on the block table (no
  // dependency).
  {
    const __amdgpu_buffer_rsrc_t q_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(pa.query + ((size_t)(tb - pa.query_start) * kQueryHeads + kvh * kGroup + H * hp) * kHeadDim),
        (short)0, (te - tb - 1) * kQueryHeads * kRowBytes + H * kRowBytes, kBufferFlags);
#pragma unroll
    for (int j = 0; j < S::kQBlocksPerWave; ++j) {
      const int g = S::kQBlocksPerWave * wave + j;
      const int row = 4 * (g & 7) + (lane >> 4);
      const unsigned off = (unsigned)(row * kQueryHeads * kRowBytes + (g >> 3) * kRowBytes + 16 * k_slot(row, lane & 15));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(q_rsrc, TM_LDS(q_lds + g * 1024), 16, off, 0, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the Q DMA ahead of the K/V DMA (the prologue waits count on it)

  auto lane_row = [&](int ti, int phys) {
    phys = min(max(phys, 0), p.num_pages - 1);
    return ((unsigned)phys * kPageSize + (unsigned)(lane_k0(ti) % kPageSize)) * kKvHeads + kvh;
  };
  auto lane_bytes = [&](int ti) {
    const int valid_rows = ti < num_tiles ? min(kKvTile, pa.seq_len - lane_k0(ti)) : 0;
    return valid_rows > 0 ? (valid_rows - 1) * kKvHeads * kRowBytes + kRowBytes : 0;
  };
  unsigned row_lo = lane_row(lane, phys_lo);
  unsigned row_hi = lane_row(kTableTiles + lane, phys_hi);
  int bytes_lo = lane_bytes(lane);
  int bytes_hi = lane_bytes(kTableTiles + lane);
  // The tile tables are complete here, before any tile DMA: left to itself the
  // compiler sinks the part it needs only for tiles 64-127 into the loop's
  // preheader, and the wait for its block-table load there would also wait
  // for the V DMA of iteration 0, which must stay in flight until block 1 of
  // iteration 0 (below).
  asm volatile("" ::"v"(row_lo), "v"(row_hi), "v"(bytes_lo), "v"(bytes_hi));
  TM_PHASE(1);
  // Buffer resource of tensor t (0 = K, 1 = V) of tile ti: the tile's key rows
  // of this KV head, range cut at seq_len; a tile past the item's end gets an
  // empty range (its loads return zeros).
  auto tile_rsrc = [&](int ti, int t) {
    const unsigned u = (unsigned)ti;  // ti >= 0
    const bool odd = ((u / kTableTiles) & 1) != 0;
    const unsigned row = __builtin_amdgcn_readlane(odd ? row_hi : row_lo, u % kTableTiles);
    const int bytes = ti < num_tiles ? __builtin_amdgcn_readlane(odd ? bytes_hi : bytes_lo, u % kTableTiles) : 0;
    const char* cache = reinterpret_cast<const char*>(t == 0 ? p.key_cache : p.value_cache);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(cache + (size_t)row * kRowBytes), (short)0, bytes, kBufferFlags);
  };
  // DMA instruction j of this wave's share of a tile.
  auto dma = [&](__amdgpu_buffer_rsrc_t rsrc, char* lds_tile, int j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TM_LDS(lds_tile + (dma_j0 + j) * 1024), 16, dma_voff[j], 0, 0,
                                             0);
  };
  auto issue_tile = [&](int ti, int t, char* lds_tile) {
    const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(ti, t);
#pragma unroll
    for (int j = 0; j < S::kDmaPerWave; ++j) dma(rsrc, lds_tile, j);
  };

  // Prologue DMA: K of iterations 0 and 1.  V of iteration 0 follows the
  // first barrier: before iteration 0 a CU streams Q, two K rounds and a V
  // round at the CU's DMA rate, and V is needed last (block 1 of iteration 0
  // reads it from step 8 - kReadAhead on), so Q and K take the bandwidth
  // first.  Iteration 0 then starts once K of iteration 1 has landed
  // (measured 3 % faster per config-2 chunk than loading V with the K of
  // iteration 0).
  if (dma_t == 0) {
    issue_tile(dma_u, 0, k_lds0 + dma_u * kTileBytes);
    __builtin_amdgcn_sched_barrier(0);  // K of iteration 1 goes last: the prologue wait leaves it in flight
    issue_tile(P + dma_u, 0, k_lds1 + dma_u * kTileBytes);
  }

  // ---- mask geometry ----
  // Row q attends [lo, q] plus, when sparse, the sink [0, 8).  lo_max is the
  // largest window start over the block's rows: tiles at or above it need no
  // window test.
  const bool sparse_row = kSparse && q >= sparse_begin && q < sparse_end;
  const int lo = sparse_row ? q - kLocalWindow : 0;
  int lo_max = 0;
  if (kSparse) {
    const int last_sparse = min(te, sparse_end) - 1;
    if (last_sparse >= max(tb, sparse_begin)) lo_max = last_sparse - kLocalWindow;
  }
  const int q_rel = q - 4 * half;  // row position minus this lane half's key offset
  const int lo_rel = lo - 4 * half;

  float m_run = -INFINITY;
  float l_run = 0.0f;  // partial row sum over this lane's keys
  f32x16_t o_acc[kHeadDim / 32];
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) o_acc[m] = f32x16_t{};

  // Per-lane LDS read offsets inside a slot (loop invariant): this wave's
  // tile plus the lane's position in it, so that a read address is the slot's
  // constant base plus one of these (no per-iteration address arithmetic).
  const int tile_off = kq * kTileBytes;
  // K (A operand of QK): row n, chunk 2c + half.
  int k_off[kHeadDim / 16];
#pragma unroll
  for (int c = 0; c < kHeadDim / 16; ++c) k_off[c] = tile_off + n * kRowBytes + 16 * k_slot(n, 2 * c + half);
  // V (A operand of PV, transposed read): 16-lane group g = lane/16 reads key
  // quad 4*(g/2) + (lane%16)/4 at dims 32m + 16*(g%2) + 4*(lane%4); the key
  // offsets 16j and +8 are multiples of 4, so they do not change the swizzle.
  const int tr_key = 4 * (lane >> 5) + ((lane & 15) >> 2);
  int v_off[kHeadDim / 32];
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) {
    const int d = 32 * m + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    v_off[m] = tile_off + tr_key * kRowBytes + 16 * v_slot(tr_key, d >> 3) + 2 * (d & 7);
  }
  const float c2 = p.scale_log2;
  const int dma_off = dma_u * kTileBytes;  // the tile this wave loads

  // Mask of tile ti of the item (in place, before its row max), applied only
  // where some (row, key) pair of the tile is outside the row's keys.
  auto mask_tile = [&](f32x16_t& s, int ti) {
    const int k0 = runs.tile(t_lo + min(ti, num_tiles - 1)) * kKvTile;
    if (k0 + kKvTile - 1 > tb) mask_causal(s, q_rel - k0);
    if (kSparse && k0 < lo_max) {
      const int thr = lo_rel - k0;
      mask_window(s, thr, (k0 == 0 && sparse_row) ? -kKvTile : thr);
    }
  };

  // Q and K of iteration 0 landed; the K waves' share of K of iteration 1 may
  // still be in flight (it is not read before the barrier that opens
  // iteration 0).  Only DMA data is published here, so a bare barrier (no
  // fence: the fence of __syncthreads would wait for every outstanding load)
  // suffices.  Then the V waves issue V of iteration 0 into its slot, which
  // nothing has touched yet.
  if (dma_t == 0) {
    wait_dma_but<S::kDmaPerWave>();
  } else {
    wait_dma();
  }
  __builtin_amdgcn_s_barrier();
  if (dma_t == 1) issue_tile(dma_u, 1, v_lds0 + dma_u * kTileBytes);
  TM_PHASE(2);
  // Q^T operand: lane (token n, half) holds Q[q][head][16c + 8*half .. +8].
  // Read in one asm block that waits for its own reads: the compiler cannot
  // tell q_lds from the slots the K and V DMA still write, and would
  // otherwise wait for that DMA here.  The waits above cover the Q DMA (issued
  // before all K/V DMA).
  bf16x8_t qreg[kHeadDim / 16];
  {
    // k_off includes the K tile offset; Q has no tiles, so take it back out.
    const unsigned qb = (unsigned)(size_t)TM_LDS(q_lds + hl * kRowBlock * kRowBytes) - (unsigned)tile_off;
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %9\n\t"
        "ds_read_b128 %2, %10\n\t"
        "ds_read_b128 %3, %11\n\t"
        "ds_read_b128 %4, %12\n\t"
        "ds_read_b128 %5, %13\n\t"
        "ds_read_b128 %6, %14\n\t"
        "ds_read_b128 %7, %15\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(qreg[0]), "=&v"(qreg[1]), "=&v"(qreg[2]), "=&v"(qreg[3]), "=&v"(qreg[4]), "=&v"(qreg[5]),
          "=&v"(qreg[6]), "=&v"(qreg[7])
        : "v"(qb + k_off[0]), "v"(qb + k_off[1]), "v"(qb + k_off[2]), "v"(qb + k_off[3]), "v"(qb + k_off[4]),
          "v"(qb + k_off[5]), "v"(qb + k_off[6]), "v"(qb + k_off[7])
        : "memory");
  }
  f32x16_t s_a, s_b;
  float m_tile = -INFINITY;  // row max of the tile the next iteration exponentiates (log2 units)
  if (kq < num_tiles) {
    // All eight K operands are read before the MFMA chain starts.
    bf16x8_t k0f[kHeadDim / 16];
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) k0f[c] = k_operand(k_lds0, k_off, c);
    __builtin_amdgcn_sched_barrier(0);
    s_a = f32x16_t{};
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) s_a = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k0f[c], qreg[c], s_a, 0, 0, 0);
    mask_tile(s_a, kq);
    float tmax = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) tmax = fmaxf(tmax, s_a[v]);
    m_tile = half_max(tmax) * c2;
  }
  // O and the row sum are still zero: the first tile's max becomes the state
  // directly (the first update then rescales nothing).
  m_run = m_tile;
  TM_PHASE(3);

  // Table refill for items of more than 128 tiles.  Table block nb >= 2
  // takes the register of block nb - 2.  The DMA of iteration it reaches
  // tile P (it + 2) + P - 1 (K) and P (it + 1) + P - 1 (V), so block nb - 2
  // is read for the last time in iteration 64 (nb - 1) / P - 2 and block nb
  // first in iteration 64 nb / P - 2.  Right after the barrier that opens
  // iteration 64 (nb - 1) / P - 1, before that iteration's DMA, block nb's
  // pages (loaded 64 / P iterations earlier, in the prologue for block 2,
  // and waited for by every iteration's wait for the wave's DMA since)
  // become rows and byte counts, and block nb + 1's page loads are issued.
  // One scalar compare per iteration; the refill itself is out of line.
  int refill_it = num_tiles > 2 * kTableTiles ? kTableTiles / P - 1 : __INT_MAX__;
  int refill_block = 2;
  auto refill = [&](int it) {
    if (__builtin_expect(it == refill_it, 0)) {
      const int ti = kTableTiles * refill_block + lane;
      const unsigned row = lane_row(ti, refill_phys);
      const int bytes = lane_bytes(ti);
      if (refill_block & 1) {
        row_hi = row;
        bytes_hi = bytes;
      } else {
        row_lo = row;
        bytes_lo = bytes;
      }
      ++refill_block;
      refill_phys = lane_page(kTableTiles * refill_block + lane);
      refill_it += kTableTiles / P;
    }
  };

  // Iteration it (this wave's tile ti = 4*it + kq): state update with tile
  // ti's row max, then [QK^T of tile ti+4 (K slot kr) || exponentials of tile
  // ti], then [PV of tile ti (V slot vr) || mask and row max of tile ti+4];
  // the prefetch of K for iteration it+2 into kw and V for it+1 into vw (one
  // tile per wave) is spread over the first block.  Iteration 0 runs only when
  // the item has more than P tiles, so every part has a tile in it and all
  // waves take its two extra barriers.
  auto iteration = [&](int it, f32x16_t& s_cur, f32x16_t& s_nxt, const char* kr, const char* vr, char* kw,
                       char* vw) {
    if (it == 0) {
      // K of iteration 1 landed (the K waves' only load in flight); V of
      // iteration 0 may still be landing: it is published before its first
      // read in block 1.  The bare barrier does not wait for it.
      if (dma_t == 0) wait_dma();
      __builtin_amdgcn_s_barrier();
    } else {
      wait_dma();
      __syncthreads();  // DMA issued one iteration ago landed; slots kw / vw are no longer read
      refill(it);
    }
    if (it < 8) TM_PHASE(4 + it);
    // The two waves of a SIMD (waves w and w + 4) leave the barrier
    // together and the older one issues first, so the younger one ends every
    // iteration ~0.25 us late while the older waits at the next barrier.
    // With KV halves the younger waves take priority for block 1 and give it
    // back for block 2, so both reach the barrier at about the same time
    // (1-2 % faster per chunk; with KV quarters it measured neutral to 1 %
    // slower, so that shape keeps equal priorities).
    if (P == 2 && wave >= S::kWaves / 2) __builtin_amdgcn_s_setprio(1);
    const int ti = P * it + kq;
    // Ragged last iteration: the parts without a tile idle; nothing is
    // left to prefetch in the last iteration.
    if (ti >= num_tiles) return;
    // This wave's prefetch: K of iteration it+2 (waves 0-3) or V of it+1
    // (waves 4-7).  Past the item's last iteration the resource is empty:
    // those loads return zeros into a slot nobody reads, which keeps the steps
    // below free of branches.
    const int pf_it = dma_t == 0 ? it + 2 : it + 1;
    const __amdgpu_buffer_rsrc_t pf_rsrc =
        tile_rsrc(pf_it < num_iters ? P * pf_it + dma_u : num_tiles, dma_t);
    char* pf_lds = (dma_t == 0 ? kw : vw) + dma_off;
    const float shift = softmax_update(m_tile, m_run, l_run, o_acc);
    // Block 1: the QK^T MFMAs of the next tile (run unconditionally: past the
    // last tile they read a stale slot and the result is unused) interleaved,
    // in program order, with the exponentials of this tile and one prefetch
    // DMA instruction per step.  Step k exponentiates element k and, on even
    // steps, element 8 + k/2 (twelve of the sixteen); block 2 does the last
    // four before the PV steps that need them, so the VALU work is spread
    // over both blocks' MFMAs.  K operands are read kReadAhead steps ahead of
    // their MFMA; the last steps also start the V reads of block 2.
    bf16x8_t kf[8], va[8];
#pragma unroll
    for (int k = 0; k < kReadAhead; ++k) kf[k] = k_operand(kr, k_off, k);
    float px[16];
    float rsum = 0.0f;
    auto expo = [&](int e) {
      px[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[e], c2, -shift));
      rsum += px[e];
    };
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k == 8 - kReadAhead && it == 0) {
        // The first V read of iteration 0 follows: each V wave waits for its
        // V of iteration 0 (older than this iteration's prefetch, of which
        // ceil(k / step) instructions are issued), then the barrier publishes it.
        constexpr int kStep = 8 / S::kDmaPerWave;
        if (dma_t == 1) wait_dma_but<(8 - kReadAhead + kStep - 1) / kStep>();
        __builtin_amdgcn_s_barrier();
      }
      // one DMA instruction every 8 / kDmaPerWave steps
      if (k % (8 / S::kDmaPerWave) == 0) dma(pf_rsrc, pf_lds, k / (8 / S::kDmaPerWave));
      if (k + kReadAhead < 8) {
        kf[k + kReadAhead] = k_operand(kr, k_off, k + kReadAhead);
      } else {
        va[k + kReadAhead - 8] = v_operand(vr, v_off, k + kReadAhead - 8);
      }
      s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[k], qreg[k], k == 0 ? f32x16_t{} : s_nxt, 0, 0, 0);
      expo(k);
      if ((k & 1) == 0) expo(8 + (k >> 1));
      __builtin_amdgcn_sched_barrier(0);
    }
    bf16x8_t pb[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[0][e] = (__bf16)px[e];
    // An empty statement that consumes these values here keeps the
    // exponentials in block 1 (otherwise they sink past the mask branches
    // below, next to their use).
    asm volatile("" ::"v"(pb[0]), "v"(px[8]), "v"(px[9]), "v"(px[10]), "v"(px[11]), "v"(rsum));
    if (P == 2) __builtin_amdgcn_s_setprio(0);
    // Block 2: the PV MFMAs of this tile interleaved with the last four
    // exponentials (steps 0-3, before pb[1] is first used at step 4) and the
    // row max of the next tile (masked first; its state update opens the next
    // iteration).
    mask_tile(s_nxt, ti + P);
    float tmax = -INFINITY;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k + kReadAhead < 8) va[k + kReadAhead] = v_operand(vr, v_off, k + kReadAhead);
      if (k < 4) {
        expo(12 + k);
        if (k == 3) {
#pragma unroll
          for (int e = 8; e < 16; ++e) pb[1][e - 8] = (__bf16)px[e];
        }
      }
      o_acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[k], pb[k >> 2], o_acc[k & 3], 0, 0, 0);
      tmax = fmaxf(fmaxf(tmax, s_nxt[2 * k]), s_nxt[2 * k + 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += rsum;
    m_tile = half_max(tmax) * c2;
  };
  // The item's last iteration: no tile follows, so there is no QK^T, no
  // prefetch and no row max of a next tile -- only this tile's exponentials
  // and its PV.  Exponentials 0-7 (pb[0]) run before the PV steps, 8-15 two
  // per step in steps 0-3 (pb[1] is first used at step 4), and the row sum
  // adds them in steps 4-7 in the order the full iteration adds them, so both
  // kinds of iteration sum a tile alike.
  auto last_iteration = [&](int it, const f32x16_t& s_cur, const char* vr) {
    wait_dma();
    __syncthreads();  // V of this iteration landed
    if (it < 8) TM_PHASE(4 + it);
    const int ti = P * it + kq;
    if (ti >= num_tiles) return;
    const float shift = softmax_update(m_tile, m_run, l_run, o_acc);
    bf16x8_t va[8];
#pragma unroll
    for (int k = 0; k < kReadAhead; ++k) va[k] = v_operand(vr, v_off, k);
    float px[16];
    auto expo = [&](int e) { px[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[e], c2, -shift)); };
#pragma unroll
    for (int e = 0; e < 8; ++e) expo(e);
    bf16x8_t pb[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[0][e] = (__bf16)px[e];
    __builtin_amdgcn_sched_barrier(0);
    float rsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k + kReadAhead < 8) va[k + kReadAhead] = v_operand(vr, v_off, k + kReadAhead);
      if (k < 4) {
        expo(8 + 2 * k);
        expo(9 + 2 * k);
        if (k == 3) {
#pragma unroll
          for (int e = 8; e < 16; ++e) pb[1][e - 8] = (__bf16)px[e];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) rsum += px[sum_order(4 * (k - 4) + j)];
      }
      o_acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[k], pb[k >> 2], o_acc[k & 3], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += rsum;
  };
  // Pairs of full iterations (slots alternate, so the loop is unrolled by
  // two), at most one more full iteration, then the last.  The last iteration
  // has one call site (its slots chosen by parity): with one per parity the
  // compiler copies the O accumulators between the two paths.
  int it = 0;
  for (; it + 2 < num_iters; it += 2) {
    iteration(it, s_a, s_b, k_lds1, v_lds0, k_lds0, v_lds1);
    iteration(it + 1, s_b, s_a, k_lds0, v_lds1, k_lds1, v_lds0);
  }
  if (it + 1 < num_iters) {
    iteration(it, s_a, s_b, k_lds1, v_lds0, k_lds0, v_lds1);
    ++it;
  }
  if (it < num_iters) {
    const bool odd = (it & 1) != 0;
    last_iteration(it, odd ? s_b : s_a, odd ? v_lds1 : v_lds0);
  }

  TM_PHASE(12);
  // ---- merge the P KV parts through LDS ----
  // Part kq keeps the O = 4 / P d-blocks kq * O .. kq * O + O - 1 and hands
  // its other 4 - O d-blocks to their owners.  The given-block index gi (0 ..
  // 3 - O among the blocks a part gives away) and the giving wave w = hl * P +
  // part select a 4 KB stretch xo(gi, w) = [v/4][lane][4] (16-byte accesses,
  // one 1 KB stretch per instruction).  The item's last iteration reads only
  // its V slot: the K slots, the other V slot (v_free) and q_lds are idle from
  // the barrier that opens it (no DMA is in flight after that barrier), so each
  // wave writes its blocks as soon as its own last PV is done, with no barrier
  // in between.  For P = 4 the stretches of gi = 0, 1, 2 fill k_lds0, k_lds1,
  // v_free and xm / xl [hl][part][lane] live in q_lds; for P = 2 gi = 0 fills
  // q_lds, gi = 1 fills k_lds0 (waves 0-3) and k_lds1 (waves 4-7), and xm / xl
  // live in v_free.  kq is wave-uniform, so the per-block branches are scalar;
  // the barrier stays outside them.  With P = 1 there is nothing to merge.
  if (num_iters == 0) {  // no iteration ran: the prologue DMA may still be landing
    wait_dma();
    __syncthreads();
  }
  char* v_free = (num_iters & 1) ? v_lds1 : v_lds0;  // the last iteration read v_lds((num_iters - 1) % 2)
  constexpr int O = S::kOwned;
  // The merged (unnormalised) d-blocks kq * O + o.  Local arrays keep a fixed
  // size (the largest shape's): hipcc's host pass drops a kernel template
  // whose local arrays have a size that depends on the template parameters.
  f32x16_t kept[kHeadDim / 32];
  static_assert(O <= kHeadDim / 32 && P <= 4, "kept, mq and lq hold the largest shape's blocks");
  if constexpr (P == 1) {
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) kept[m] = o_acc[m];
  } else {
  static_assert(P != 4 || H * P * 4 * 64 * 16 == S::kSlotBytes, "P = 4: one given block of all waves fills a slot");
  static_assert(P != 4 || 2 * H * P * 64 * 4 <= H * kRowBlock * kRowBytes, "P = 4: xm / xl fit in q_lds");
  static_assert(P != 2 || (H * P * 4 * 64 * 16 == H * kRowBlock * kRowBytes && 4 * 4 * 64 * 16 == S::kSlotBytes),
                "P = 2: one given block of all waves fills q_lds, half of one fills a slot");
  static_assert(P != 2 || 2 * H * P * 64 * 4 <= S::kSlotBytes, "P = 2: xm / xl fit in a slot");
  auto xo = [&](int gi, int w) -> f32x4_t* {
    if constexpr (P == 4) {
      return reinterpret_cast<f32x4_t*>(gi == 0 ? k_lds0 : (gi == 1 ? k_lds1 : v_free)) + w * 4 * 64;
    } else {
      if (gi == 0) return reinterpret_cast<f32x4_t*>(q_lds) + w * 4 * 64;
      return reinterpret_cast<f32x4_t*>(w < 4 ? k_lds0 : k_lds1) + (w & 3) * 4 * 64;
    }
  };
  float* xm = reinterpret_cast<float*>(P == 4 ? q_lds : v_free);
  float* xl = xm + H * P * 64;
  const int self = hl * P + kq;
  // Index of d-block m among the blocks part r gives away (m is not r's).
  auto given_index = [](int m, int r) { return m < r * O ? m : m - O; };
  // Every o_acc / kept index below is a compile-time constant and each d-block
  // takes its own uniform branch: arms that differ only in which accumulator
  // they touch would be merged by the compiler into one arm addressing o_acc
  // through a pointer, which forces o_acc out of registers for the whole loop.
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) {
    if (m / O == kq) continue;
    f32x4_t* dst = xo(given_index(m, kq), self) + lane;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      dst[g * 64] = f32x4_t{o_acc[m][4 * g], o_acc[m][4 * g + 1], o_acc[m][4 * g + 2], o_acc[m][4 * g + 3]};
    }
  }
  xm[self * 64 + lane] = m_run;
  xl[self * 64 + lane] = l_run;
  __syncthreads();
  {
    float mq[4], lq[4];  // the first P are used
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < P; ++r) {
      mq[r] = xm[(hl * P + r) * 64 + lane];
      lq[r] = xl[(hl * P + r) * 64 + lane];
      mt = fmaxf(mt, mq[r]);
    }
    const float mu = mt == -INFINITY ? 0.0f : mt;
    float lt = 0.0f;
#pragma unroll
    for (int r = 0; r < P; ++r) lt += lq[r] * __builtin_amdgcn_exp2f(mq[r] - mu);
    const float self_scale = __builtin_amdgcn_exp2f(m_run - mu);
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) {
      if (m / O != kq) continue;
      f32x16_t acc = o_acc[m] * self_scale;
#pragma unroll
      for (int r = 0; r < P; ++r) {
        if (r == kq) continue;
        const float a = __builtin_amdgcn_exp2f(mq[r] - mu);
        const f32x4_t* src = xo(given_index(m, r), hl * P + r) + lane;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4_t x = src[g * 64];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[4 * g + e] += x[e] * a;
        }
      }
      kept[m % O] = acc;
    }
    l_run = lt;
    m_run = mt;
  }
  }  // P > 1

  // The sc1 cache policy (agent scope): stores are written through to, and
  // loads served from, the level where every L2 of the GPU is coherent.  The
  // split partials need it to be seen across XCDs inside the launch; the
  // output rows use it so that no dirty output line is left in an L2 for the
  // end of the kernel to write back.
  constexpr int kCpolAgent = 16;  // sc1
  // Normalise the O merged d-blocks (row sum: the two 32-lane halves hold
  // one row), round them to bf16 (nearest even) and store the workgroup's
  // output as whole rows.  A lane holds 8-byte pieces of one row, so the
  // pieces are first gathered in LDS: row r of the stage holds the H heads'
  // 256-byte rows in output order (16-byte chunk c at position c ^ (r % 16),
  // which spreads the 32 rows' writes over the banks), and then each
  // instruction stores 64 x 16 B of whole output rows (the H heads of a
  // token are adjacent in the output), written through L2.  The same number
  // of bytes as piecewise stores, but in whole cache lines: measured 4-7 %
  // faster per chunk, most of it from the write-through.  stage is an LDS
  // region of kRowBlock * H * 256 bytes that no wave still reads.
  constexpr int kStageRow = H * kRowBytes;
  constexpr int kChunksPerRow = kStageRow / 16;     // 32 (H = 2) or 64 (H = 4)
  constexpr int kRowsPerStore = 64 / kChunksPerRow;  // rows per store instruction: 2 or 1
  constexpr int kStores = kRowBlock / (kRowsPerStore * S::kWaves);
  static_assert(kRowsPerStore * kChunksPerRow == 64 && kStores * kRowsPerStore * S::kWaves == kRowBlock,
                "the stores cover the row block");
  auto store_rows = [&](const f32x16_t* blocks, float l_lane, char* stage) {
    const float l_tot = half_sum(l_lane);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
#pragma unroll
    for (int o = 0; o < O; ++o) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4_t o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(blocks[o][4 * g + e] * inv);
        const int chunk = (hl * (kRowBytes / 16) + 4 * (kq * O + o) + g) ^ (n & 15);
        *reinterpret_cast<bf16x4_t*>(stage + n * kStageRow + 16 * chunk + 8 * half) = o4;
      }
    }
    __syncthreads();
    // Rows past seq_len fall outside the buffer's range: their stores are dropped.
    const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.out + ((size_t)(tb - pa.query_start) * kQueryHeads + kvh * kGroup + H * hp) * kHeadDim), (short)0,
        (te - tb - 1) * kQueryHeads * kRowBytes + kStageRow, kBufferFlags);
    const int c = lane % kChunksPerRow;
#pragma unroll
    for (int j = 0; j < kStores; ++j) {
      const int r = (wave * kStores + j) * kRowsPerStore + lane / kChunksPerRow;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stage + r * kStageRow + 16 * (c ^ (r & 15)));
      __builtin_amdgcn_raw_buffer_store_b128(v, out_rsrc, (unsigned)(r * kQueryHeads * kRowBytes + 16 * c), 0,
                                             kCpolAgent);
    }
  };
  // Stage: KV quarters use the last iteration's V slot (its reads ended
  // before the merge barrier; 16 KB of its 32 KB); KV halves need 32 KB and
  // use q_lds, whose merge reads must end first; KV whole uses q_lds too,
  // whose only reads (the Q operand, before the first iteration) every wave
  // finished before a barrier all waves have passed since.
  static_assert(kRowBlock * kStageRow <= (P == 4 ? S::kSlotBytes : H * kRowBlock * kRowBytes), "stage fits");
  char* const stage = P == 4 ? ((num_iters & 1) ? v_lds0 : v_lds1) : q_lds;
  TM_PHASE(13);
  if (nsplit == 1) {
    if constexpr (P == 2) __syncthreads();  // every wave has read its merge blocks from q_lds
    store_rows(kept, l_run, stage);
    TM_PHASE(14);
    return;
  }

  // ---- split-KV, merged in this launch ----
  // Every split publishes its partial; the workgroup whose arrival completes
  // the row block (per workgroup position hp) merges all partials in split
  // order -- the same sums whichever split arrives last, so the result is
  // deterministic -- and writes the output.  Record per (KV head, item):
  // O [hq][d-block][v/4][lane][v%4] (unnormalised), then row max [hq][lane] and the
  // lane's partial row sum [hq][lane]; workgroups of one item write disjoint
  // heads, the parts disjoint d-blocks.  The records are written and read
  // with the sc1 cache policy (agent scope: stores written through to the
  // level where every L2 of the GPU is coherent, loads served from it), and
  // the arrival word is updated by agent-scope atomics, so no fence (a
  // whole-L2 writeback and invalidate) is needed.  Each wave waits for its
  // own stores before the workgroup's arrival is counted; the workgroup that
  // counts last has seen every other split arrive after their stores
  // completed.
  constexpr int kStatM = kGroup * 64 * 64;     // row maxima [hq][lane]
  constexpr int kStatL = kGroup * 64 * 65;     // partial row sums [hq][lane]
  const int first = item - split;
  // Buffer over the row block's records (offsets stay 32-bit for any chunk).
  const __amdgpu_buffer_rsrc_t rec = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.partials + ((size_t)kvh * pa.split_items + first) * kPartialFloats), (short)0,
      nsplit * (int)kPartialBytes, kBufferFlags);
  // 16-byte piece g of d-block o: each instruction moves 64 lanes x 16 B = 1 KB contiguous.
  auto blk_off = [&](int s, int o, int g) {
    return (unsigned)(s * (int)kPartialBytes + ((((hq * 4 + kq * O + o) * 4 + g) * 64 + lane) * 4) * 4);
  };
  {
#pragma unroll
    for (int o = 0; o < O; ++o) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4_t x = {kept[o][4 * g], kept[o][4 * g + 1], kept[o][4 * g + 2], kept[o][4 * g + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, x), rec, blk_off(split, o, g), 0,
                                               kCpolAgent);
      }
    }
    if (kq == 0) {  // every part holds the same merged row max and row sum
      const unsigned so = (unsigned)(split * (int)kPartialBytes + (hq * 64 + lane) * 4);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_run), rec, so + kStatM * 4, 0, kCpolAgent);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_run), rec, so + kStatL * 4, 0, kCpolAgent);
    }
  }
  wait_dma();  // this wave's partial stores completed (vmcnt also counts stores)
  TM_PHASE(16);
  __syncthreads();
  // Arrival word of (KV head, row block, workgroup position): this launch's
  // epoch above the count of splits arrived under it.  A word that carries
  // another epoch (another workspace's launches, a fresh buffer, or whatever
  // the workspace held) counts as zero.  Each arrival adds one: when the word
  // already carries this launch's epoch that is its count (one round trip:
  // every arrival on a word a previous launch of this workspace left clean,
  // and every arrival after the first otherwise).  An arrival that finds
  // another epoch has added to a void word; it then installs this launch's
  // epoch with a count of one, or -- if another arrival installed it first
  // -- adds itself under it, by compare-and-swap from the value last seen.
  // Either way each arrival is counted exactly once under the epoch.
  unsigned long long* ctr = p.counters + ((size_t)kvh * pa.split_row_blocks + order) * S::kWgPerKvHead + hp;
  if (tid == 0) {
    const unsigned long long old = __hip_atomic_fetch_add(ctr, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long mine = old + 1;
    if ((old >> kEpochShift) != p.epoch) {
      unsigned long long seen = old + 1;  // the word if nobody else changed it since
      do {
        mine = (seen >> kEpochShift) == p.epoch ? seen + 1 : (p.epoch << kEpochShift) + 1;
      } while (!__hip_atomic_compare_exchange_strong(ctr, &seen, mine, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
    }
    s_last = (int)((mine & ((1ull << kEpochShift) - 1)) == (unsigned long long)nsplit);
  }
  __syncthreads();
  TM_PHASE(17);
  if (!s_last) return;
  // Every split has arrived: leave the word at this launch's epoch with a
  // count of zero.  The next launch on this workspace carries the same epoch
  // (the host keeps one per workspace, and a HIP graph replays its captured
  // one), so each of its arrivals is counted by its fetch-and-add alone,
  // without the install a foreign word takes.
  if (tid == 0) __hip_atomic_store(ctr, p.epoch << kEpochShift, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // One pass over the splits, kMergeBatch at a time with all of a batch's
  // loads in flight: a batch that raises the running max rescales what is
  // already summed (the online-softmax rule).  Slots past the last split
  // take this workgroup's own values again (registers, no load), weighted 0.
  // A KV-whole wave holds all four d-blocks, so it takes one split at a time
  // (four would hold 256 more VGPRs).
  constexpr int kMergeBatch = P == 1 ? 1 : 4;
  f32x16_t acc[kHeadDim / 32];
#pragma unroll
  for (int o = 0; o < O; ++o) acc[o] = f32x16_t{};
  float mt = -INFINITY, lt = 0.0f;
  for (int s0 = 0; s0 < nsplit; s0 += kMergeBatch) {
    float ms[4], ls[4];  // fixed sizes (see kept); the first kMergeBatch are used
    f32x4_t xs[4][kHeadDim / 32][4];
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) {
      const int sb = s0 + b;
      if (sb == split || sb >= nsplit) {
        // This workgroup's own partial: the values it stored are still in
        // registers, so it is not loaded back (the same sums in the same
        // order; measured 0.45 us less on the config-2 last chunk).
        ms[b] = m_run;
        ls[b] = l_run;
#pragma unroll
        for (int o = 0; o < O; ++o) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            xs[b][o][g] = f32x4_t{kept[o][4 * g], kept[o][4 * g + 1], kept[o][4 * g + 2], kept[o][4 * g + 3]};
          }
        }
        continue;
      }
      const unsigned so = (unsigned)(sb * (int)kPartialBytes + (hq * 64 + lane) * 4);
      ms[b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rec, so + kStatM * 4, 0, kCpolAgent));
      ls[b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rec, so + kStatL * 4, 0, kCpolAgent));
#pragma unroll
      for (int o = 0; o < O; ++o) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          xs[b][o][g] =
              __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rec, blk_off(sb, o, g), 0, kCpolAgent));
        }
      }
    }
    float mb = mt;
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) mb = s0 + b < nsplit ? fmaxf(mb, ms[b]) : mb;
    const float mu = mb == -INFINITY ? 0.0f : mb;  // no keys in any split so far: nothing summed yet
    const float keep = mt == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mt - mu);
    lt *= keep;
#pragma unroll
    for (int o = 0; o < O; ++o) acc[o] *= keep;
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) {
      const float w = s0 + b < nsplit ? __builtin_amdgcn_exp2f(ms[b] - mu) : 0.0f;
      lt += ls[b] * w;
#pragma unroll
      for (int o = 0; o < O; ++o) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[o][4 * g + e] += xs[b][o][g][e] * w;
        }
      }
    }
    mt = mb;
    if (s0 == 0) TM_PHASE(18);
  }
  TM_PHASE(19);
  // The stage is free: for KV halves, q_lds was last read before the barrier
  // ahead of the arrival count.
  store_rows(acc, lt, stage);
  TM_PHASE(15);
}

template <bool kSparse, int P>
hipError_t launch(const KernelParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((triangle_paged_attention_kernel<kSparse, P>),
                     dim3((unsigned)(p.items_per_head * Shape<P>::kWgPerKvHead * kKvHeads)),
                     dim3(Shape<P>::kThreads), 0,
                     stream, p.block_table, p.query, p.query_start, p.seq_len, p.num_row_blocks, p.sparse_begin,
                     p.sparse_end, p.split_items, p.split_row_blocks, p.tiles_per_split, p);
  return hipGetLastError();
}

hipError_t launch_triangle_paged_attention(const KernelParams& p, bool sparse, int kv_parts, hipStream_t stream) {
  if (kv_parts == 1) return sparse ? launch<true, 1>(p, stream) : launch<false, 1>(p, stream);
  if (kv_parts == 2) return sparse ? launch<true, 2>(p, stream) : launch<false, 2>(p, stream);
  return sparse ? launch<true, 4>(p, stream) : launch<false, 4>(p, stream);
}

// Split-KV scratch of the no-allocation entry point: one array per GPU for
// the life of the process.  Zero at load; every completed launch leaves its
// arrival counters zero again.  In host code `scratch` is only a stand-in
// for the symbol: its device address comes from hipGetSymbolAddress, once
// per device, and only that address is ever handed to a kernel.
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

hipError_t noalloc_scratch(void** ptr) {
  constexpr int kMaxDevices = 64;
  static void* addresses[kMaxDevices] = {};
  static std::mutex mutex;
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mutex);
  if (addresses[device] == nullptr) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));  // with `device` current
    if (err != hipSuccess) return err;
    addresses[device] = address;
  }
  *ptr = addresses[device];
  return hipSuccess;
}

#ifdef TRIANGLEMIX_PHASE_CLOCKS
// Diagnostic exports of the phase-clock build: copy the clock slots to the
// host, or clear them (before the launch to be read).
extern "C" int tm_phase_clocks_read(void* host, int64_t bytes) {
  if (bytes < 0 || bytes > (int64_t)sizeof(phase_clocks)) return (int)hipErrorInvalidValue;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(phase_clocks), (size_t)bytes, 0, hipMemcpyDeviceToHost);
}

extern "C" int tm_phase_clocks_clear(void) {
  void* address = nullptr;
  hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(phase_clocks));
  if (err != hipSuccess) return (int)err;
  err = hipMemset(address, 0, sizeof(phase_clocks));
  if (err != hipSuccess) return (int)err;
  return (int)hipDeviceSynchronize();
}
#endif

}  // namespace tmx
