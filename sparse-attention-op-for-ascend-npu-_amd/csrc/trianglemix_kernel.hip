// TriangleMix paged sparse prefill attention for MI355X (gfx950).
//
// Work decomposition
// ------------------
// A work item is (row block of 32 query tokens, KV head, KV split); each item
// runs as two workgroups, one per pair of the KV head's four GQA query heads.
// A workgroup has four wave64s, one per SIMD: (query head hl of the pair) x
// (KV half kh).  Wave w owns the 32 rows {32 tokens} x {head 4*kvh + 2*hp +
// hl} and processes every other tile of the item (even tiles for kh = 0, odd
// for kh = 1); each K/V tile staged in LDS is read by the two waves of its
// half, and the two halves merge through LDS at the end.  Splitting the GQA
// group over two workgroups puts 256 workgroups on the 256 CUs for a
// 512-token chunk.
// The KV tiles of a row block are cut into splits of at most
// `tiles_per_split` tiles (host-chosen, never below 16 tiles = 1024 keys, so
// only long dense rows split).  A row block with one split writes its output
// directly; otherwise every split writes an fp32 partial (O, row max, row
// sum) to the workspace and a small combine kernel, enqueued right after on
// the same stream, merges the partials in split order (deterministic) and
// writes the output.  Chunks without long rows -- every sparse middle chunk --
// are one launch.
// Items are numbered per KV head, heaviest row blocks first; KV head =
// blockIdx % 8 keeps every workgroup of one KV head on one XCD (workgroups
// are dispatched round-robin over the 8 XCDs), so both head pairs of a row
// block, neighbouring row blocks' overlapping local windows and a row block's
// partials share one L2.
//
// Tiles, memory path and pipeline
// -------------------------------
// K/V tiles are 64 logical keys aligned to 64, so a tile never straddles a
// 128-token page: one block-table lookup per tile.  Tiles go from HBM straight
// into LDS with buffer_load_dwordx4 ... lds (no register staging).  Each wave
// runs a software pipeline over its tiles: in iteration i it issues the
// QK^T MFMAs of tile i+1 interleaved with the exponentials of tile i, then the
// PV MFMAs of tile i interleaved with the mask and row max of tile i+1, so the
// SIMD's matrix core and VALU work at the same time (one wave per SIMD, the
// interleave is fixed in program order with scheduling barriers).  LDS holds
// two K slots and two V slots, each with the tiles of both halves; the DMA of
// K for iteration i+2 and of V for iteration i+1 is issued right after the
// barrier that opens iteration i.  The four slots are distinct LDS objects
// and the loop is unrolled by two so every access names its slot statically:
// the compiler then sees that the prefetch never aliases the tiles being
// read and does not wait for it.  Each tile is addressed through a buffer
// resource whose range stops at seq_len, so key rows past seq_len read as
// zeros.  LDS rows are 256 B (one key x 128 dims) with the 16-byte chunks
// XOR-swizzled so both read patterns are bank-conflict free:
//   K: chunk c of key row r sits in slot c ^ (r % 16)
//   V: chunk c of key row r sits in slot c ^ (4 * (r % 4))
//
// Contractions (per wave, v_mfma_f32_32x32x16_bf16)
// ---------------------------------------------------
//   S^T (64 keys x 32 rows) = K Q^T   A = K rows from LDS, B = Q in registers
//   O^T (128 x 32 rows)    += V^T P^T  A = V via ds_read_b64_tr_b16, B = P
// In the 32x32 accumulator layout lane l owns column l % 32, i.e. one query
// row: accumulator element v of key block b is key 32b + 8(v/4) + 4(l/32) +
// v%4.  Row max / row sum are lane-local plus one exchange between the two
// 32-lane halves, and the fp32 scores convert in registers into the bf16 B
// operand of PV.  ds_read_b64_tr_b16 transposes within 16-lane groups: when
// the 4 source lanes 4j..4j+3 of a group point at 4 consecutive dims of key
// row j, destination lane t of the group receives dim t of keys 0..3 --
// exactly the A-operand slice (one dim, four consecutive keys) of V^T.
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
// Exponentials are exp2 of log2(e)-prescaled scores; split partials merge
// with the same rescale rule.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "trianglemix_kernel.h"

namespace tmx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#define TM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

constexpr int kWaves = 4;                        // 2 query heads x 2 KV halves
constexpr int kThreads = kWaves * 64;
constexpr int kHeadsPerGroup = 2;                // query heads per workgroup
constexpr int kGroupsPerKvHead = kGroup / kHeadsPerGroup;
constexpr int kRowBytes = kHeadDim * 2;          // 256 B: one key row
constexpr int kTileBytes = kKvTile * kRowBytes;  // 16 KB: K or V of one tile
constexpr int kSlotBytes = 2 * kTileBytes;       // the tiles of both KV halves of one iteration
// Buffer-resource word 3 for raw (unformatted, stride 0) dword loads on gfx9.
constexpr int kBufferFlags = 0x00020000;

static_assert(kKvTile == 64 && kPageSize % kKvTile == 0, "a tile must stay inside one page");
static_assert(kRowBlock == 32, "one MFMA column per query token");
static_assert(kWaves * 16 == kKvTile, "each wave loads 16 key rows of every tile");

// Wait until every LDS DMA (and other vector-memory load) this wave issued has
// landed: s_waitcnt vmcnt(0), expcnt / lgkmcnt unconstrained.  Each wave runs
// it before a barrier that publishes DMA'd tiles to the other waves -- the
// barrier alone does not order the DMA's LDS writes.
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ int k_slot(int row, int chunk) { return chunk ^ (row & 15); }
__device__ __forceinline__ int v_slot(int row, int chunk) { return chunk ^ ((row & 3) << 2); }

// Work item -> (row-block order index, split index, split count), computed
// by every wave with a wave-wide prefix sum over the row blocks' split counts.
__device__ __forceinline__ void decode_item(const KernelParams& p, int sparse_begin, int sparse_end, int item,
                                            int lane, int& order, int& split, int& nsplit) {
  int acc = 0;
  order = 0;
  split = 0;
  nsplit = 1;
  for (int base = 0; base < p.num_row_blocks; base += 64) {
    const int o = base + lane;
    const int cnt = o < p.num_row_blocks ? row_block_splits(o, p.num_row_blocks, p.query_start, p.seq_len,
                                                            sparse_begin, sparse_end, p.tiles_per_split)
                                         : 0;
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d);
      if (lane >= d) incl += t;
    }
    const int total = __shfl(incl, 63);
    if (item < acc + total) {
      const bool mine = cnt > 0 && item >= acc + incl - cnt && item < acc + incl;
      const unsigned long long m = __ballot(mine);
      const int src = __ffsll(m) - 1;
      order = __shfl(o, src);
      split = item - (acc + __shfl(incl - cnt, src));
      nsplit = __shfl(cnt, src);
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

// The value held by the lane 32 positions away (v_permlane32_swap: a VALU
// exchange of the two 32-lane halves, no LDS round trip).
__device__ __forceinline__ float other_half(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  // r[0]: lanes 0-31 keep x, lanes 32-63 get x of lanes 0-31; r[1]: lanes
  // 0-31 get x of lanes 32-63, lanes 32-63 keep x.
  return __uint_as_float(__lane_id() < 32 ? r[1] : r[0]);
}

// Key offset inside the tile of accumulator element v of key block b, for
// lanes of the first 32-lane half (the second half adds 4).
__device__ __forceinline__ constexpr int elem_key(int b, int v) { return 32 * b + 8 * (v >> 2) + (v & 3); }

// MFMA step k of S^T = K Q^T (k = 0..15: key block b = k % 2, dims
// 16c .. 16c+15 with c = k / 2): the K operand read from LDS.
__device__ __forceinline__ bf16x8_t k_operand(const char* kt, const int* k_off, int k) {
  return *reinterpret_cast<const bf16x8_t*>(kt + 32 * (k & 1) * kRowBytes + k_off[k >> 1]);
}

// S^T = K Q^T for one 64-key tile (raw scores, two 32-key blocks).
__device__ __forceinline__ void qk_tile(const char* kt, const int* k_off, const bf16x8_t* qreg, f32x16_t* s) {
  bf16x8_t kf[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) kf[k] = k_operand(kt, k_off, k);
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int b = k & 1, c = k >> 1;
    s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[k], qreg[c], c == 0 ? f32x16_t{} : s[b], 0, 0, 0);
  }
}

// Causal bound: keep elements whose key offset is <= thr (per lane).
__device__ __forceinline__ void mask_causal(f32x16_t* s, int thr) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int v = 0; v < 16; ++v) s[b][v] = elem_key(b, v) <= thr ? s[b][v] : -INFINITY;
  }
}

// Window bound: keep elements whose key offset is >= thr; the elements that
// can hold sink keys (b = 0, v < 4) compare against thr_sink instead.
__device__ __forceinline__ void mask_window(f32x16_t* s, int thr, int thr_sink) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int t = (b == 0 && v < 4) ? thr_sink : thr;
      s[b][v] = elem_key(b, v) >= t ? s[b][v] : -INFINITY;
    }
  }
}

// Online softmax of one tile in the log2 domain (max commutes with the
// positive scale), state update: the tile's row max m_tile (already scaled to
// log2 units) updates the row state and rescales O when needed.  Returns the
// exponent shift of the tile's exponentials.
__device__ __forceinline__ float softmax_update(float m_tile, float& m_run, float& l_run, f32x16_t* o_acc) {
  if (__any(m_tile > m_run + kLazyRescale)) {  // wave-uniform branch; always taken on a row's first keys
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

// MFMA step k of O^T += V^T P^T (k = 0..15: d-block m = k % 4, k-group
// bj = k / 4 = 2b + j of 16 keys): the V^T operand, two transposed reads.
// k-slot e of half h in k-group (b, j) is key 32b + 16j + 8(e/4) + 4h + e%4.
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

// How many MFMA steps ahead of their use the LDS operand reads are issued.
constexpr int kReadAhead = 4;

template <bool kSparse>
__global__ void __launch_bounds__(kThreads)
triangle_paged_attention_kernel(KernelParams p) {
  // K slots 0/1 and V slots 0/1: tiles of iteration i live in slot i % 2.
  __shared__ __attribute__((aligned(1024))) char k_lds0[kSlotBytes];
  __shared__ __attribute__((aligned(1024))) char k_lds1[kSlotBytes];
  __shared__ __attribute__((aligned(1024))) char v_lds0[kSlotBytes];
  __shared__ __attribute__((aligned(1024))) char v_lds1[kSlotBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, kept scalar
  const int hl = wave & 1;   // query head inside the workgroup's pair
  const int kh = wave >> 1;  // KV half: even (0) or odd (1) tiles of the item
  const int lane = tid & 63;
  const int n = lane & 31;  // MFMA column = query token of this lane
  const int half = lane >> 5;

  const int sparse_begin = kSparse ? p.sparse_begin : 0;
  const int sparse_end = kSparse ? p.sparse_end : 0;

  const int kvh = blockIdx.x % kKvHeads;
  const int hp = (blockIdx.x / kKvHeads) % kGroupsPerKvHead;
  const int item = blockIdx.x / (kKvHeads * kGroupsPerKvHead);
  int order, split, nsplit;
  if (p.any_split) {
    decode_item(p, sparse_begin, sparse_end, item, lane, order, split, nsplit);
    // The decoded item is wave-uniform; say so, so that all tile arithmetic,
    // block-table loads and buffer resources stay scalar.
    order = __builtin_amdgcn_readfirstlane(order);
    split = __builtin_amdgcn_readfirstlane(split);
    nsplit = __builtin_amdgcn_readfirstlane(nsplit);
  } else {
    order = item;
    split = 0;
    nsplit = 1;
  }
  const int rb = p.num_row_blocks - 1 - order;
  const int tb = p.query_start + rb * kRowBlock;
  const int te = min(tb + kRowBlock, p.seq_len);
  const int hq = kHeadsPerGroup * hp + hl;  // query head inside the GQA group
  const int head = kvh * kGroup + hq;
  const int q = tb + n;
  const bool row_active = q < te;

  const TileRuns runs = row_block_tiles(tb, te, sparse_begin, sparse_end);
  const int all_tiles = runs.count();
  const int t_lo = (int)((long long)split * all_tiles / nsplit);
  const int t_hi = (int)((long long)(split + 1) * all_tiles / nsplit);
  const int num_tiles = t_hi - t_lo;
  const int num_iters = (num_tiles + 1) >> 1;

  // ---- DMA: wave w loads key rows 16w .. 16w+15 of every tile ----
  // Four wave-instructions of 1 KB (4 key rows) per tile and tensor.  Lane i
  // writes LDS slot (row 16w + 4j + i/16, slot i%16), so it loads the global
  // chunk the swizzle puts in that slot.
  const int dma_slot = lane & 15;
  unsigned dma_voff[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * wave + 4 * j + (lane >> 4);
    dma_voff[0][j] = (unsigned)(row * kKvHeads * kRowBytes + 16 * k_slot(row, dma_slot));
    dma_voff[1][j] = (unsigned)(row * kKvHeads * kRowBytes + 16 * v_slot(row, dma_slot));
  }
  // Physical page of every tile of the item (at most kMaxItemTiles = 128):
  // lane i of page_lo / page_hi holds tile i / 64 + i (one vector load each,
  // issued with the Q loads); the loop reads them with v_readlane, so it never
  // waits on a scalar memory load (whose counter it shares with the LDS reads).
  auto lane_page = [&](int ti) {
    int phys = 0;
    if (ti < num_tiles) phys = p.block_table[runs.tile(t_lo + ti) * kKvTile / kPageSize];
    return min(max(phys, 0), p.num_pages - 1);
  };
  const int page_lo = lane_page(lane);
  const int page_hi = lane_page(64 + lane);
  auto tile_page = [&](int ti) {
    return __builtin_amdgcn_readlane(ti < 64 ? page_lo : page_hi, ti & 63);
  };
  // Buffer resource of tensor t (0 = K, 1 = V) of tile ti: the tile's 64 key
  // rows of this KV head, range cut at seq_len; a tile past the item's end
  // gets an empty range (its loads return zeros).
  auto tile_rsrc = [&](int ti, int t) {
    const bool live = ti < num_tiles;
    const int phys = tile_page(ti);
    const int k0 = live ? runs.tile(t_lo + ti) * kKvTile : 0;
    const size_t first_row = (((size_t)phys * kPageSize + (k0 % kPageSize)) * kKvHeads + kvh) * kHeadDim;
    const int valid_rows = live ? min(kKvTile, p.seq_len - k0) : 0;
    const int bytes = valid_rows > 0 ? (valid_rows - 1) * kKvHeads * kRowBytes + kRowBytes : 0;
    const __bf16* cache = t == 0 ? p.key_cache : p.value_cache;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(cache + first_row), (short)0, bytes, kBufferFlags);
  };
  // DMA instruction j (0..3) of this wave for one tile: 4 key rows.
  auto dma = [&](__amdgpu_buffer_rsrc_t rsrc, int t, char* lds_tile, int j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TM_LDS(lds_tile + (4 * wave + j) * 1024), 16, dma_voff[t][j], 0, 0,
                                             0);
  };
  auto issue_tile = [&](int ti, int t, char* lds_tile) {
    const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(ti, t);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma(rsrc, t, lds_tile, j);
  };

  // Prologue DMA: K and V of iteration 0, K of iteration 1.
  if (num_iters > 0) {
    issue_tile(0, 0, k_lds0);
    issue_tile(1, 0, k_lds0 + kTileBytes);
    issue_tile(0, 1, v_lds0);
    issue_tile(1, 1, v_lds0 + kTileBytes);
  }
  if (num_iters > 1) {
    issue_tile(2, 0, k_lds1);
    issue_tile(3, 0, k_lds1 + kTileBytes);
  }

  // ---- Q^T operand: lane (token n, half) holds Q[q][head][16c + 8*half .. +8] ----
  bf16x8_t qreg[kHeadDim / 16];
  {
    const __bf16* qrow = p.query + ((size_t)(q - p.query_start) * kQueryHeads + head) * kHeadDim + 8 * half;
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) {
      qreg[c] = row_active ? *reinterpret_cast<const bf16x8_t*>(qrow + 16 * c) : bf16x8_t{};
    }
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

  // Per-lane LDS read offsets inside a 16 KB tile (loop invariant).
  // K (A operand of QK): row 32b + n, chunk 2c + half; the swizzle depends on
  // row % 16 = n % 16 only, so b adds the constant 32 rows.
  int k_off[kHeadDim / 16];
#pragma unroll
  for (int c = 0; c < kHeadDim / 16; ++c) k_off[c] = n * kRowBytes + 16 * k_slot(n, 2 * c + half);
  // V (A operand of PV, transposed read): 16-lane group g = lane/16 reads key
  // quad 4*(g/2) + (lane%16)/4 at dims 32m + 16*(g%2) + 4*(lane%4); the key
  // offsets kb and +8 are multiples of 4, so they do not change the swizzle.
  const int tr_key = 4 * (lane >> 5) + ((lane & 15) >> 2);
  int v_off[kHeadDim / 32];
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) {
    const int d = 32 * m + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    v_off[m] = tr_key * kRowBytes + 16 * v_slot(tr_key, d >> 3) + 2 * (d & 7);
  }
  const float c2 = p.scale_log2;
  const int tile_off = kh * kTileBytes;  // this wave's tile inside a slot

  wait_dma();
  __syncthreads();  // prologue DMA of every wave landed
  // Mask of tile ti of this wave (in place, before its row max), applied only
  // where some (row, key) pair of the tile is outside the row's keys.
  auto mask_tile = [&](f32x16_t* s, int ti) {
    const int k0 = runs.tile(t_lo + min(ti, num_tiles - 1)) * kKvTile;
    if (k0 + kKvTile - 1 > tb) mask_causal(s, q_rel - k0);
    if (kSparse && k0 < lo_max) {
      const int thr = lo_rel - k0;
      mask_window(s, thr, (k0 == 0 && sparse_row) ? -kKvTile : thr);
    }
  };

  f32x16_t s_a[2], s_b[2];
  float m_tile = -INFINITY;  // row max of the tile the next iteration exponentiates (log2 units)
  if (kh < num_tiles) {
    qk_tile(k_lds0 + tile_off, k_off, qreg, s_a);
    mask_tile(s_a, kh);
    float tmax = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; ++v) tmax = fmaxf(tmax, s_a[b][v]);
    }
    m_tile = fmaxf(tmax, other_half(tmax)) * c2;
  }

  // Iteration it (this wave's tile ti = 2*it + kh): state update with tile
  // ti's row max, then [QK^T of tile ti+2 (K slot kr) || exponentials of tile
  // ti], then [PV of tile ti (V slot vr) || mask and row max of tile ti+2];
  // the prefetch of K for iteration it+2 into kw and V for it+1 into vw is
  // spread over the first block.
  auto iteration = [&](int it, f32x16_t* s_cur, f32x16_t* s_nxt, const char* kr, const char* vr, char* kw,
                       char* vw) {
    wait_dma();
    __syncthreads();  // DMA issued one iteration ago landed; slots kw / vw are no longer read
    const int ti = 2 * it + kh;
    // Odd tile count: half 1 idles in the last iteration, which prefetches nothing.
    if (ti >= num_tiles) return;
    // This iteration's prefetch -- K of iteration it+2 into kw, V of it+1 into
    // vw -- goes out one DMA instruction per MFMA step below, so its issue
    // overlaps the MFMAs instead of stalling the wave in one burst.
    // Past the item's last iteration the resources are empty: those loads
    // return zeros into a slot nobody reads, which keeps the steps below
    // free of branches (a branch would let the compiler move the softmax work
    // out of the MFMA steps).
    __amdgpu_buffer_rsrc_t dma_rsrc[2][2];  // [tensor][tile of the pair]
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      dma_rsrc[0][u] = tile_rsrc(it + 2 < num_iters ? 2 * (it + 2) + u : num_tiles, 0);
      dma_rsrc[1][u] = tile_rsrc(it + 1 < num_iters ? 2 * (it + 1) + u : num_tiles, 1);
    }
    const float shift = softmax_update(m_tile, m_run, l_run, o_acc);
    // Block 1: the QK^T MFMAs of the next tile (run unconditionally: past the
    // last tile they read a stale slot and the result is unused) interleaved,
    // in program order, with the exponentials of this tile -- one MFMA, then
    // two elements' exp / row-sum / bf16 work -- and one prefetch DMA
    // instruction per step.  K operands are read kReadAhead steps ahead of
    // their MFMA; the last steps also start the V reads of block 2.
    const char* kt = kr + tile_off;
    const char* vt = vr + tile_off;
    bf16x8_t kf[16], va[16];
#pragma unroll
    for (int k = 0; k < kReadAhead; ++k) kf[k] = k_operand(kt, k_off, k);
    bf16x8_t pb[2][2];
    float rsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      dma(dma_rsrc[k >> 3][(k >> 2) & 1], k >> 3, ((k >> 3) == 0 ? kw : vw) + ((k >> 2) & 1) * kTileBytes, k & 3);
      if (k + kReadAhead < 16) {
        kf[k + kReadAhead] = k_operand(kt, k_off, k + kReadAhead);
      } else {
        va[k + kReadAhead - 16] = v_operand(vt, v_off, k + kReadAhead - 16);
      }
      const int b = k & 1, c = k >> 1;
      s_nxt[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[k], qreg[c], c == 0 ? f32x16_t{} : s_nxt[b], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int e = 2 * k + t, eb = e >> 4, ev = e & 15;
        const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[eb][ev], c2, -shift));
        rsum += x;
        pb[eb][ev >> 3][ev & 7] = (__bf16)x;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += rsum;
    // An empty statement that consumes P here keeps the exponentials in block
    // 1 (otherwise they sink past the mask branches below, next to their use).
    asm volatile("" ::"v"(pb[0][0]), "v"(pb[0][1]), "v"(pb[1][0]), "v"(pb[1][1]), "v"(l_run));
    // Block 2: the PV MFMAs of this tile interleaved with the row max of the
    // next one (masked first; its state update opens the next iteration).
    mask_tile(s_nxt, ti + 2);
    float tmax = -INFINITY;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k + kReadAhead < 16) va[k + kReadAhead] = v_operand(vt, v_off, k + kReadAhead);
      const int bj = k >> 2;
      o_acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[k], pb[bj >> 1][bj & 1], o_acc[k & 3], 0, 0, 0);
      tmax = fmaxf(tmax, fmaxf(s_nxt[k >> 3][(2 * k) & 15], s_nxt[k >> 3][(2 * k + 1) & 15]));
      __builtin_amdgcn_sched_barrier(0);
    }
    m_tile = fmaxf(tmax, other_half(tmax)) * c2;
  };
  for (int it = 0; it < num_iters; it += 2) {
    iteration(it, s_a, s_b, k_lds1, v_lds0, k_lds0, v_lds1);
    if (it + 1 < num_iters) iteration(it + 1, s_b, s_a, k_lds0, v_lds1, k_lds1, v_lds0);
  }

  // ---- merge the two KV halves through LDS ----
  // Half kh keeps d-blocks 2*kh, 2*kh+1 and hands the other two to its partner.
  wait_dma();
  __syncthreads();  // all compute and every (empty) prefetch done; the slots are free
  float* xo = reinterpret_cast<float*>(k_lds0);  // [kh][hl][2 blocks][v][lane]
  static_assert(2 * kHeadsPerGroup * 2 * 16 * 64 * 4 == kSlotBytes, "exchanged O fills one slot");
  float* xm = reinterpret_cast<float*>(v_lds0);  // [kh][hl][lane]
  float* xl = xm + 2 * kHeadsPerGroup * 64;
  const int keep = 2 * kh;
  f32x16_t kept[2], given[2];
  if (kh == 0) {
    kept[0] = o_acc[0]; kept[1] = o_acc[1]; given[0] = o_acc[2]; given[1] = o_acc[3];
  } else {
    kept[0] = o_acc[2]; kept[1] = o_acc[3]; given[0] = o_acc[0]; given[1] = o_acc[1];
  }
  const int self = kh * kHeadsPerGroup + hl;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
    for (int v = 0; v < 16; ++v) xo[((self * 2 + mm) * 16 + v) * 64 + lane] = given[mm][v];
  }
  xm[self * 64 + lane] = m_run;
  xl[self * 64 + lane] = l_run;
  __syncthreads();
  const int other = (kh ^ 1) * kHeadsPerGroup + hl;
  {
    const float m1 = xm[other * 64 + lane];
    const float l1 = xl[other * 64 + lane];
    const float mt = fmaxf(m_run, m1);
    const float mu = mt == -INFINITY ? 0.0f : mt;
    const float a0 = __builtin_amdgcn_exp2f(m_run - mu);
    const float a1 = __builtin_amdgcn_exp2f(m1 - mu);
    l_run = l_run * a0 + l1 * a1;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
      for (int v = 0; v < 16; ++v) kept[mm][v] = kept[mm][v] * a0 + xo[((other * 2 + mm) * 16 + v) * 64 + lane] * a1;
    }
    m_run = mt;
  }

  if (nsplit == 1) {
    const float l_tot = l_run + other_half(l_run);  // the two 32-lane halves hold one row
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (!row_active) return;
    __bf16* orow = p.out + ((size_t)(q - p.query_start) * kQueryHeads + head) * kHeadDim;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4_t o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(kept[mm][4 * g + e] * inv);
        *reinterpret_cast<bf16x4_t*>(orow + 32 * (keep + mm) + 8 * g + 4 * half) = o4;
      }
    }
    return;
  }

  // ---- split-KV: publish this split's partial; the combine kernel merges ----
  // Layout per (KV head, item): O [hq][m][v/4][lane][v%4], then row max
  // [hq][lane], then the lane's partial row sum [hq][lane] -- every access is
  // a lane-contiguous 16- or 4-byte vector.  The two head-pair workgroups
  // write disjoint heads.
  float* part = p.partials + ((size_t)kvh * p.items_per_head + item) * kPartialFloats;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4_t o4 = {kept[mm][4 * g], kept[mm][4 * g + 1], kept[mm][4 * g + 2], kept[mm][4 * g + 3]};
      *reinterpret_cast<f32x4_t*>(part + (((hq * 4 + keep + mm) * 4 + g) * 64 + lane) * 4) = o4;
    }
  }
  if (kh == 0) {  // both halves hold the same merged row max and row sum
    part[kGroup * 64 * 64 + hq * 64 + lane] = m_run;
    part[kGroup * 64 * 65 + hq * 64 + lane] = l_run;
  }
}

// Merge the split-KV partials of every split row block with the online-
// softmax rescale rule, then normalise and write bf16.  One workgroup per
// (row block, KV head) with one wave per query head of the group; unsplit
// row blocks exit.  The partials' row maxima are read first, so the O loads
// of all splits are independent of each other and stay in flight together;
// the weighted sums run in split order (deterministic).
constexpr int kCombineThreads = kGroup * 64;

// Occupancy is not the limit here (one small workgroup per split row block):
// let the compiler keep every load of a split in flight.
template <bool kSparse>
__global__ void __launch_bounds__(kCombineThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
triangle_paged_attention_combine_kernel(KernelParams p) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int kvh = blockIdx.x % kKvHeads;
  const int order = blockIdx.x / kKvHeads;
  const int sparse_begin = kSparse ? p.sparse_begin : 0;
  const int sparse_end = kSparse ? p.sparse_end : 0;

  // First item of this row block = sum of the split counts of the row blocks
  // issued before it (wave-wide prefix sum, as in decode_item).
  int first_item = 0, nsplit = 1;
  for (int base = 0; base <= order; base += 64) {
    const int o = base + lane;
    const int cnt = o <= order ? row_block_splits(o, p.num_row_blocks, p.query_start, p.seq_len, sparse_begin,
                                                  sparse_end, p.tiles_per_split)
                               : 0;
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d);
      if (lane >= d) incl += t;
    }
    if (order < base + 64) {
      const int src = order - base;
      nsplit = __shfl(cnt, src);
      first_item += __shfl(incl - cnt, src);
    } else {
      first_item += __shfl(incl, 63);
    }
  }
  if (nsplit == 1) return;

  const int rb = p.num_row_blocks - 1 - order;
  const int q = p.query_start + rb * kRowBlock + n;
  const bool row_active = q < p.seq_len;
  const int head = kvh * kGroup + wave;
  const float* base = p.partials + ((size_t)kvh * p.items_per_head + first_item) * kPartialFloats;

  float mt = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) mt = fmaxf(mt, base[s * kPartialFloats + kGroup * 64 * 64 + wave * 64 + lane]);
  const float mu = mt == -INFINITY ? 0.0f : mt;

  float lt = 0.0f;
  f32x4_t ot[kHeadDim / 8];  // [m][v/4], 4 consecutive v each
#pragma unroll
  for (int i = 0; i < kHeadDim / 8; ++i) ot[i] = f32x4_t{};
  for (int s = 0; s < nsplit; ++s) {
    const float* part = base + s * kPartialFloats;
    // All 16 vector loads of the split first, then the arithmetic.
    f32x4_t os[kHeadDim / 8];
#pragma unroll
    for (int i = 0; i < kHeadDim / 8; ++i) {
      os[i] = *reinterpret_cast<const f32x4_t*>(part + ((wave * 16 + i) * 64 + lane) * 4);
    }
    const float w = __builtin_amdgcn_exp2f(part[kGroup * 64 * 64 + wave * 64 + lane] - mu);
    lt += part[kGroup * 64 * 65 + wave * 64 + lane] * w;
#pragma unroll
    for (int i = 0; i < kHeadDim / 8; ++i) ot[i] += os[i] * w;
  }
  const float l_tot = lt + other_half(lt);  // the two 32-lane halves hold one row
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (!row_active) return;
  __bf16* orow = p.out + ((size_t)(q - p.query_start) * kQueryHeads + head) * kHeadDim;
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4_t o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(ot[4 * m + g][e] * inv);
      *reinterpret_cast<bf16x4_t*>(orow + 32 * m + 8 * g + 4 * half) = o4;
    }
  }
}

template <bool kSparse>
hipError_t launch(const KernelParams& p, bool any_split, hipStream_t stream) {
  hipLaunchKernelGGL(triangle_paged_attention_kernel<kSparse>,
                     dim3((unsigned)(p.items_per_head * kGroupsPerKvHead * kKvHeads)), dim3(kThreads), 0, stream,
                     p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !any_split) return err;
  hipLaunchKernelGGL(triangle_paged_attention_combine_kernel<kSparse>, dim3((unsigned)(p.num_row_blocks * kKvHeads)),
                     dim3(kCombineThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_triangle_paged_attention(const KernelParams& p, bool sparse, bool any_split, hipStream_t stream) {
  return sparse ? launch<true>(p, any_split, stream) : launch<false>(p, any_split, stream);
}

}  // namespace tmx
