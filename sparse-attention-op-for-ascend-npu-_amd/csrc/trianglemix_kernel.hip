// TriangleMix paged sparse prefill attention for MI355X (gfx950).
//
// Work decomposition
// ------------------
// A work item is (row block of 32 query tokens, KV head, KV split).  Its
// workgroup has eight wave64s: (query head hq = wave % 4 of the KV head's GQA
// group) x (KV half kh = wave / 4).  Wave w owns the 32 rows {32 tokens} x
// {head 4*kvh + hq} and processes every other tile of the item (even tiles
// for kh = 0, odd for kh = 1); each K/V tile staged in LDS is read by the four
// waves of its half (4x reuse, 128 query rows per tile), two waves share each
// SIMD so one's softmax overlaps the other's MFMAs, and the two halves merge
// through LDS at the end.
// The KV tiles of a row block are cut into splits of at most
// `tiles_per_split` tiles (host-chosen so the grid covers the 256 CUs, and
// never below 16 tiles = 1024 keys per split, so only long dense rows split).
// A row block with one split writes its output directly; otherwise every
// split writes an fp32 partial (O, row max, row sum) to the workspace and a
// small combine kernel, enqueued right after on the same stream, merges the
// partials in split order (deterministic) and writes the output.  Chunks
// without long rows -- every sparse middle chunk -- are one launch.
// Items are numbered per KV head, heaviest row blocks first; KV head =
// blockIdx % 8 keeps every item of one KV head on one XCD (workgroups are
// dispatched round-robin over the 8 XCDs), so neighbouring row blocks'
// overlapping local windows and a row block's partials share one L2.
//
// Tiles and memory path
// ---------------------
// K/V tiles are 64 logical keys aligned to 64, so a tile never straddles a
// 128-token page: one block-table lookup per tile.  Tiles go from HBM
// straight into LDS with buffer_load_dwordx4 ... lds (no register staging),
// two tiles (one per half) per iteration, double buffered: the DMA of
// iteration i+1 is issued right after the barrier that opens iteration i and
// overlaps its compute.  Each tile is addressed through a
// buffer resource whose range stops at seq_len, so key rows past seq_len read
// as zeros.  LDS rows are 256 B (one key x 128 dims) with the 16-byte chunks
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
// row_block_tiles).  Tiles that cross the causal diagonal or a window edge
// apply the exact per-element rule
//   attended(q, k) = k <= q && (dense(q) || k < 8 || q - k <= 512)
// branch-free; interior tiles run unmasked.
//
// Numerics follow the reference order (online_softmax.hpp:1002-1086,
// rescale_o.hpp:153-344): s*scale -> mask -> row max -> p = exp(s - m) in
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

#define TM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

constexpr int kThreads = 512;                    // 8 waves = 4 query heads x 2 KV halves
constexpr int kRowBytes = kHeadDim * 2;          // 256 B: one key row
constexpr int kTileBytes = kKvTile * kRowBytes;  // 16 KB: K or V of one tile
constexpr int kStages = 2;
constexpr int kStageBytes = 2 * 2 * kTileBytes;  // K + V of the two tiles of an iteration
constexpr int kLdsBytes = kStages * kStageBytes; // 128 KB
// Buffer-resource word 3 for raw (unformatted, stride 0) dword loads on gfx9.
constexpr int kBufferFlags = 0x00020000;

static_assert(kKvTile == 64 && kPageSize % kKvTile == 0, "a tile must stay inside one page");
static_assert(kRowBlock == 32, "one MFMA column per query token");

__device__ __forceinline__ int k_slot(int row, int chunk) { return chunk ^ (row & 15); }
__device__ __forceinline__ int v_slot(int row, int chunk) { return chunk ^ ((row & 3) << 2); }

// Work item -> (row-block order index, split index, split count), computed
// by every wave with a wave-wide prefix sum over the row blocks' split counts.
__device__ __forceinline__ void decode_item(const KernelParams& p, int item, int lane, int& order, int& split,
                                            int& nsplit) {
  int acc = 0;
  order = 0;
  split = 0;
  nsplit = 1;
  for (int base = 0; base < p.num_row_blocks; base += 64) {
    const int o = base + lane;
    const int cnt = o < p.num_row_blocks
                        ? row_block_splits(o, p.num_row_blocks, p.query_start, p.seq_len, p.sparse_begin,
                                           p.sparse_end, p.tiles_per_split)
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

// Per-lane row geometry of the mask: key k is attended iff (k - lo) <= span
// (unsigned, i.e. lo <= k <= q) or k < sink_end.
struct RowMask {
  int lo;
  unsigned span;
  int sink_end;
};

// Rescale the running O / row sum only when some row's max grew by more than
// 2^kLazyRescale (log2 units); otherwise keep the stale max as the exponent
// shift, so p <= 2^kLazyRescale -- exact in fp32 and bf16 range -- and the
// 64 multiplies of the O rescale are skipped on most tiles.
constexpr float kLazyRescale = 8.0f;

// One 64-key tile for one wave: S^T = K Q^T, mask, online softmax, O^T += V^T P^T.
// kMode 0: no mask; 1: causal / window mask; 2: mask with the sink (tile 0).
template <int kMode>
__device__ __forceinline__ void tile_step(const char* kt, const char* vt, int k0, int half, const int* k_off,
                                          const int* v_off, const bf16x8_t* qreg, const RowMask& rm, float c2,
                                          float& m_run, float& l_run, f32x16_t* o_acc) {
  // ---- S^T = K Q^T (raw scores) ----
  f32x16_t s[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    bf16x8_t kf[kHeadDim / 16];
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) {
      kf[c] = *reinterpret_cast<const bf16x8_t*>(kt + 32 * b * kRowBytes + k_off[c]);
    }
    s[b] = f32x16_t{};
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) {
      s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[c], qreg[c], s[b], 0, 0, 0);
    }
  }

  // ---- mask; accumulator element v of block b is key k0 + 32b + 8(v/4) + 4*half + v%4 ----
  if (kMode != 0) {
    const unsigned rel = (unsigned)(k0 + 4 * half - rm.lo);
    const int key0 = k0 + 4 * half;  // key of element (b = 0, v = 0)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int koff = 32 * b + 8 * (v >> 2) + (v & 3);
        bool ok = rel + (unsigned)koff <= rm.span;
        // Sink keys [0, 8) can only be elements b = 0, v < 4 of the tile at k0 = 0.
        if (kMode == 2 && b == 0 && v < 4) ok = ok | (key0 + koff < rm.sink_end);
        s[b][v] = ok ? s[b][v] : -INFINITY;
      }
    }
  }

  // ---- online softmax in the log2 domain (max commutes with the positive scale) ----
  float tmax = -INFINITY;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int v = 0; v < 16; ++v) tmax = fmaxf(tmax, s[b][v]);
  }
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
  const float m_tile = tmax * c2;
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
  const float m_use = m_run == -INFINITY ? 0.0f : m_run;
  float rsum = 0.0f;
  bf16x8_t pb[2][2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][v], c2, -m_use));
      rsum += e;
      pb[b][v >> 3][v & 7] = (__bf16)e;
    }
  }
  l_run += rsum;

  // ---- O^T += V^T P^T; k-slot e of half h in k-group (b, j) is key 32b + 16j + 8(e/4) + 4h + e%4 ----
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = 32 * b + 16 * j;
#pragma unroll
      for (int m = 0; m < kHeadDim / 32; ++m) {
        const char* a0 = vt + kb * kRowBytes + v_off[m];
        const i16x4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(a0));
        const i16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(a0 + 8 * kRowBytes));
        const i16x4_t lohi[2] = {lo4, hi4};
        bf16x8_t a;
        __builtin_memcpy(&a, lohi, sizeof(a));
        o_acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[b][j], o_acc[m], 0, 0, 0);
      }
    }
  }
}

// LDS block of (stage, tile u of the iteration, tensor t: 0 = K, 1 = V).
__device__ __forceinline__ int lds_block(int stage, int u, int t) { return ((stage * 2 + u) * 2 + t) * kTileBytes; }

__global__ void __launch_bounds__(kThreads)
triangle_paged_attention_kernel(KernelParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, kept scalar
  const int hq = wave & 3;   // query head inside the GQA group
  const int kh = wave >> 2;  // KV half: even (0) or odd (1) tiles of the item
  const int lane = tid & 63;
  const int n = lane & 31;  // MFMA column = query token of this lane
  const int half = lane >> 5;

  const int kvh = blockIdx.x % kKvHeads;
  const int item = blockIdx.x / kKvHeads;
  int order, split, nsplit;
  if (p.any_split) {
    decode_item(p, item, lane, order, split, nsplit);
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
  const int head = kvh * kGroup + hq;
  const int q = tb + n;
  const bool row_active = q < te;

  const TileRuns runs = row_block_tiles(tb, te, p.sparse_begin, p.sparse_end);
  const int all_tiles = runs.count();
  const int t_lo = (int)((long long)split * all_tiles / nsplit);
  const int t_hi = (int)((long long)(split + 1) * all_tiles / nsplit);
  const int num_tiles = t_hi - t_lo;
  const int num_iters = (num_tiles + 1) >> 1;

  // ---- DMA of iteration `it`'s tiles (K and V) into stage `stage` ----
  // 64 wave-instructions of 1 KB (4 key rows) per iteration: the waves of
  // half kh load tile u = kh of the pair, both tensors, row quads
  // rq = 4*hq .. 4*hq+3.  Lane i writes LDS slot (row 4rq + i/16, slot i%16),
  // so it loads the global chunk the swizzle puts in that slot.
  const int dma_slot = lane & 15;
  unsigned dma_voff[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * hq + 4 * j + (lane >> 4);
    dma_voff[0][j] = (unsigned)(row * kKvHeads * kRowBytes + 16 * k_slot(row, dma_slot));
    dma_voff[1][j] = (unsigned)(row * kKvHeads * kRowBytes + 16 * v_slot(row, dma_slot));
  }
  // Physical page of this wave's tile in iteration `it`.  The block table is
  // read-only for the whole launch, so it is read through the constant
  // address space: a scalar load that never waits on the vector-memory
  // counter (which also tracks the in-flight K/V DMA).
  const __attribute__((address_space(4))) int32_t* table =
      (const __attribute__((address_space(4))) int32_t*)p.block_table;
  auto page_of = [&](int it) {
    const int ti = 2 * it + kh;
    if (ti >= num_tiles) return 0;
    const int k0 = runs.tile(t_lo + ti) * kKvTile;
    const int phys = table[k0 / kPageSize];
    return min(max(phys, 0), p.num_pages - 1);
  };
  auto issue_iter = [&](int it, int stage, int phys) {
    const int ti = 2 * it + kh;
    if (ti >= num_tiles) return;  // uniform per wave
    const int k0 = runs.tile(t_lo + ti) * kKvTile;
    const size_t first_row = (((size_t)phys * kPageSize + (k0 % kPageSize)) * kKvHeads + kvh) * kHeadDim;
    const int valid_rows = min(kKvTile, p.seq_len - k0);
    const int bytes = (valid_rows - 1) * kKvHeads * kRowBytes + kRowBytes;
#pragma unroll
    for (int t = 0; t < 2; ++t) {  // 0 = K, 1 = V
      const __bf16* cache = t == 0 ? p.key_cache : p.value_cache;
      const __amdgpu_buffer_rsrc_t rsrc =
          __builtin_amdgcn_make_buffer_rsrc((void*)(cache + first_row), (short)0, bytes, kBufferFlags);
      char* lds_tile = smem + lds_block(stage, kh, t);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TM_LDS(lds_tile + (4 * hq + j) * 1024), 16, dma_voff[t][j],
                                                 0, 0, 0);
      }
    }
  };

  if (num_iters > 0) issue_iter(0, 0, page_of(0));
  // Block-table entry for the next DMA, loaded one iteration ahead.
  int next_phys = page_of(1);

  // ---- Q^T operand: lane (token n, half) holds Q[q][head][16c + 8*half .. +8] ----
  bf16x8_t qreg[kHeadDim / 16];
  {
    const __bf16* qrow = p.query + ((size_t)(q - p.query_start) * kQueryHeads + head) * kHeadDim + 8 * half;
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) {
      qreg[c] = row_active ? *reinterpret_cast<const bf16x8_t*>(qrow + 16 * c) : bf16x8_t{};
    }
  }

  const bool sparse_row = q >= p.sparse_begin && q < p.sparse_end;
  RowMask rm;
  rm.lo = sparse_row ? q - kLocalWindow : 0;
  rm.span = (unsigned)(q - rm.lo);
  rm.sink_end = sparse_row ? kSinkTokens : 0;

  float m_run = -INFINITY;
  float l_run = 0.0f;  // partial row sum over this lane's keys
  f32x16_t o_acc[kHeadDim / 32];
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) o_acc[m] = f32x16_t{};

  // Per-lane LDS read offsets inside a 16 KB tile block (loop invariant).
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

  for (int it = 0; it < num_iters; ++it) {
    __syncthreads();  // own DMA of this iteration landed + every wave done with the other stage
    if (it + 1 < num_iters) {
      issue_iter(it + 1, (it + 1) & 1, next_phys);
      next_phys = page_of(it + 2);
    }
    const int ti = 2 * it + kh;
    if (ti >= num_tiles) continue;  // odd tile count: half 1 idles in the last iteration
    const int k0 = runs.tile(t_lo + ti) * kKvTile;
    const char* kt = smem + lds_block(it & 1, kh, 0);
    const char* vt = smem + lds_block(it & 1, kh, 1);

    // One instantiation for every tile: a branch between masked and unmasked
    // variants of the tile body raises register pressure past 256 VGPRs.
    tile_step<2>(kt, vt, k0, half, k_off, v_off, qreg, rm, c2, m_run, l_run, o_acc);
  }

  // ---- merge the two KV halves through LDS ----
  // Half kh keeps d-blocks 2*kh, 2*kh+1 and hands the other two to its partner.
  __syncthreads();  // all compute done; the stage buffers are free
  float* xo = reinterpret_cast<float*>(smem);  // [kh][hq][2 blocks][v][lane]
  float* xm = xo + 2 * kGroup * 2 * 16 * 64;   // [kh][hq][lane]
  float* xl = xm + 2 * kGroup * 64;
  const int keep = 2 * kh;
  f32x16_t kept[2], given[2];
  if (kh == 0) {
    kept[0] = o_acc[0]; kept[1] = o_acc[1]; given[0] = o_acc[2]; given[1] = o_acc[3];
  } else {
    kept[0] = o_acc[2]; kept[1] = o_acc[3]; given[0] = o_acc[0]; given[1] = o_acc[1];
  }
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
    for (int v = 0; v < 16; ++v) xo[(((kh * kGroup + hq) * 2 + mm) * 16 + v) * 64 + lane] = given[mm][v];
  }
  xm[(kh * kGroup + hq) * 64 + lane] = m_run;
  xl[(kh * kGroup + hq) * 64 + lane] = l_run;
  __syncthreads();
  const int other = (kh ^ 1) * kGroup + hq;
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
    const float l_tot = l_run + __shfl_xor(l_run, 32);  // the two 32-lane halves hold one row
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
  // Layout per item: O [hq][m][v][lane], then row max [hq][lane], then the
  // lane's partial row sum [hq][lane] -- every access is lane-contiguous.
  float* part = p.partials + ((size_t)kvh * p.items_per_head + item) * kPartialFloats;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
    for (int v = 0; v < 16; ++v) part[((hq * 4 + keep + mm) * 16 + v) * 64 + lane] = kept[mm][v];
  }
  if (kh == 0) {  // both halves hold the same merged row max and row sum
    part[kGroup * 64 * 64 + hq * 64 + lane] = m_run;
    part[kGroup * 64 * 65 + hq * 64 + lane] = l_run;
  }
}

// Merge the split-KV partials of every split row block, in split order
// (deterministic), with the online-softmax rescale rule, then normalise and
// write bf16.  One workgroup per (row block, KV head); unsplit row blocks exit.
constexpr int kCombineThreads = 256;  // 4 waves = 4 query heads

__global__ void __launch_bounds__(kCombineThreads)
triangle_paged_attention_combine_kernel(KernelParams p) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int kvh = blockIdx.x % kKvHeads;
  const int order = blockIdx.x / kKvHeads;

  // First item of this row block = sum of the split counts of the row blocks
  // issued before it (wave-wide prefix sum, as in decode_item).
  int first_item = 0, nsplit = 1;
  for (int base = 0; base <= order; base += 64) {
    const int o = base + lane;
    const int cnt = o <= order ? row_block_splits(o, p.num_row_blocks, p.query_start, p.seq_len, p.sparse_begin,
                                                  p.sparse_end, p.tiles_per_split)
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

  float mt = -INFINITY, lt = 0.0f;
  f32x16_t ot[kHeadDim / 32];
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) ot[m] = f32x16_t{};
  for (int s = 0; s < nsplit; ++s) {
    const float* part = p.partials + ((size_t)kvh * p.items_per_head + first_item + s) * kPartialFloats;
    const float ms = part[kGroup * 64 * 64 + wave * 64 + lane];
    const float ls = part[kGroup * 64 * 65 + wave * 64 + lane];
    f32x16_t os[kHeadDim / 32];
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) {
#pragma unroll
      for (int v = 0; v < 16; ++v) os[m][v] = part[((wave * 4 + m) * 16 + v) * 64 + lane];
    }
    const float mn = fmaxf(mt, ms);
    const float mu = mn == -INFINITY ? 0.0f : mn;
    const float a = __builtin_amdgcn_exp2f(mt - mu);
    const float b = __builtin_amdgcn_exp2f(ms - mu);
    lt = lt * a + ls * b;
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) ot[m] = ot[m] * a + os[m] * b;
    mt = mn;
  }
  const float l_tot = lt + __shfl_xor(lt, 32);  // the two 32-lane halves hold one row
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (!row_active) return;
  __bf16* orow = p.out + ((size_t)(q - p.query_start) * kQueryHeads + head) * kHeadDim;
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4_t o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(ot[m][4 * g + e] * inv);
      *reinterpret_cast<bf16x4_t*>(orow + 32 * m + 8 * g + 4 * half) = o4;
    }
  }
}

hipError_t launch_triangle_paged_attention(const KernelParams& p, bool any_split, hipStream_t stream) {
  hipLaunchKernelGGL(triangle_paged_attention_kernel, dim3((unsigned)(p.items_per_head * kKvHeads)),
                     dim3(kThreads), 0, stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !any_split) return err;
  hipLaunchKernelGGL(triangle_paged_attention_combine_kernel, dim3((unsigned)(p.num_row_blocks * kKvHeads)),
                     dim3(kCombineThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace tmx
