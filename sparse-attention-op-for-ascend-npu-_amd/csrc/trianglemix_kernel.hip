// TriangleMix paged sparse prefill attention for MI355X (gfx950).
//
// One workgroup = one (row block of 32 query tokens, KV head) pair.  Its four
// wave64s are the four query heads of that KV head's GQA group: every K/V
// tile staged in LDS is read by all four waves (4x reuse), and all four waves
// share one tile schedule and one mask, because they own the same tokens.
//
// Per wave the contraction is done transposed, S^T = K Q^T and O^T = V^T P^T,
// with v_mfma_f32_32x32x16_bf16.  In the accumulator layout of a 32x32 MFMA
// lane l owns column l%32, so each lane owns one query row: the row max and
// row sum of the online softmax are lane-local plus one exchange between the
// two 32-lane halves, and the fp32 scores convert in registers into the bf16
// B operand of the PV MFMA (no LDS round trip for P).
//
// K/V tiles are 64 logical keys, aligned to 64, so a tile never straddles a
// 128-token page: one block-table lookup per tile.  Only tiles that hold at
// least one attended (row, key) pair are visited: for a row block whose rows
// are all sparse that is the sink tile plus the tiles of [q_first-512,
// q_last]; otherwise [0, q_last].  Tiles that cross the causal diagonal or a
// window edge get the exact per-element rule
//   attended(q, k) = k <= q && (dense(q) || k < 8 || q - k <= 512),
// interior tiles run unmasked.
//
// Numerics follow the reference order (online_softmax.hpp:1002-1086,
// rescale_o.hpp:153-344): s*scale -> mask -> row max -> p = exp(s - m) in
// fp32 -> P to bf16 (round to nearest even) for PV, row sum from the fp32 p
// -> O = O*exp(m_old - m_new) + P V -> O / l -> bf16 round to nearest even.
// The exponentials are computed as exp2 of log2(e)-prescaled scores.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "trianglemix_kernel.h"

namespace tmx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;           // 4 waves = 4 query heads of one GQA group
constexpr int kKeyStride = kHeadDim + 8; // padded K row in LDS (bf16 elements): 272 B
constexpr int kVtStride = kKvTile + 4;   // padded V^T row in LDS (bf16 elements): 136 B
constexpr int kKLdsElems = kKvTile * kKeyStride;
constexpr int kVtLdsElems = kHeadDim * kVtStride;

__device__ __forceinline__ bool attended(int q, int k, int sparse_begin, int sparse_end) {
  const bool sparse_row = q >= sparse_begin && q < sparse_end;
  return k <= q && (!sparse_row || k < kSinkTokens || q - k <= kLocalWindow);
}

// Tile schedule of one row block, uniform across the workgroup.
struct TileRange {
  int first0, count0;  // first run of 64-key tiles
  int first1, count1;  // second run (sparse blocks: the local band), may be empty
};

__device__ __forceinline__ TileRange row_block_tiles(int tb, int te, int sparse_begin, int sparse_end) {
  TileRange r;
  const int last_tile = (te - 1) / kKvTile;  // tile holding key te-1
  const bool all_sparse = tb >= sparse_begin && te <= sparse_end;
  if (!all_sparse) {
    r.first0 = 0; r.count0 = last_tile + 1;
    r.first1 = 0; r.count1 = 0;
    return r;
  }
  const int local_first = (tb - kLocalWindow) / kKvTile;  // tb >= 521 so tb-512 >= 9
  if (local_first <= 0) {
    r.first0 = 0; r.count0 = last_tile + 1;
    r.first1 = 0; r.count1 = 0;
  } else {
    r.first0 = 0; r.count0 = 1;  // sink tile [0, 64)
    r.first1 = local_first; r.count1 = last_tile - local_first + 1;
  }
  return r;
}

__device__ __forceinline__ uint32_t lo_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);  // {a.lo16, b.lo16}
}
__device__ __forceinline__ uint32_t hi_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);  // {a.hi16, b.hi16}
}

__device__ __forceinline__ float wave_half_max(float x) {
  return fmaxf(x, __shfl_xor(x, 32));
}

__global__ void __launch_bounds__(kThreads)
triangle_paged_attention_kernel(KernelParams p) {
  __shared__ __attribute__((aligned(16))) __bf16 k_lds[kKLdsElems];
  __shared__ __attribute__((aligned(16))) __bf16 vt_lds[kVtLdsElems];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 31;   // query row of this lane inside the row block
  const int half = lane >> 5;

  // blockIdx -> (row block, KV head).  KV head = blockIdx % 8 keeps every
  // workgroup of one KV head on one XCD (dispatch is round-robin over the 8
  // XCDs), so overlapping local windows of neighbouring row blocks hit the
  // same L2.  Row blocks are issued last-first: later rows attend more keys.
  const int kvh = blockIdx.x % kKvHeads;
  const int rb = p.num_row_blocks - 1 - (int)(blockIdx.x / kKvHeads);
  const int tb = p.query_start + rb * kQueryTile;
  const int te = min(tb + kQueryTile, p.seq_len);
  const int qh = kvh * kGroup + wave;
  const int q = tb + n;
  const bool row_active = q < te;

  // ---- Q^T operand: lane (row n, half) holds Q[q][qh][16c + 8*half .. +8] ----
  bf16x8_t qreg[kHeadDim / 16];
  {
    const __bf16* qrow = p.query + ((size_t)(q - p.query_start) * kQueryHeads + qh) * kHeadDim + 8 * half;
#pragma unroll
    for (int c = 0; c < kHeadDim / 16; ++c) {
      if (row_active) {
        qreg[c] = *reinterpret_cast<const bf16x8_t*>(qrow + 16 * c);
      } else {
        qreg[c] = bf16x8_t{};
      }
    }
  }

  const TileRange tiles = row_block_tiles(tb, te, p.sparse_begin, p.sparse_end);
  const int num_tiles = tiles.count0 + tiles.count1;
  const bool block_has_sparse = tb < p.sparse_end && te > p.sparse_begin && p.sparse_begin < p.sparse_end;
  const int last_sparse_row = min(te, p.sparse_end) - 1;

  // Global -> register staging of one tile (issued one tile ahead).
  // K: thread t copies 16-byte chunk (t & 15) of key rows (t >> 4) + 16 i.
  // V: thread t copies chunk (t & 15) of the 4 keys 4*(t >> 4) .. +3, then
  //    writes them transposed (4 keys x 8 dims) into V^T.
  const int kchunk = tid & 15;
  const int krow0 = tid >> 4;
  uint4 kst[4], vst[4];

  auto tile_id = [&](int i) { return i < tiles.count0 ? tiles.first0 + i : tiles.first1 + (i - tiles.count0); };

  auto load_tile = [&](int i) {
    const int k0 = tile_id(i) * kKvTile;
    int phys = p.block_table[k0 / kPageSize];
    phys = min(max(phys, 0), p.num_pages - 1);
    const size_t page_base = ((size_t)phys * kPageSize + (k0 % kPageSize)) * kKvHeads + kvh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kr = krow0 + 16 * j;
      const size_t off = (page_base + (size_t)kr * kKvHeads) * kHeadDim + 8 * kchunk;
      kst[j] = (k0 + kr < p.seq_len) ? *reinterpret_cast<const uint4*>(p.key_cache + off) : make_uint4(0, 0, 0, 0);
      const int vr = 4 * krow0 + j;
      const size_t voff = (page_base + (size_t)vr * kKvHeads) * kHeadDim + 8 * kchunk;
      vst[j] = (k0 + vr < p.seq_len) ? *reinterpret_cast<const uint4*>(p.value_cache + voff) : make_uint4(0, 0, 0, 0);
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<uint4*>(&k_lds[(krow0 + 16 * j) * kKeyStride + 8 * kchunk]) = kst[j];
    }
    // vst[j] = 8 dims (8*kchunk ..) of key 4*krow0 + j; word w holds dims 2w, 2w+1.
    const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&vst[0]);
    const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&vst[1]);
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&vst[2]);
    const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&vst[3]);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int d = 8 * kchunk + 2 * w;
      uint2 even, odd;
      even.x = lo_halves(w0[w], w1[w]);
      even.y = lo_halves(w2[w], w3[w]);
      odd.x = hi_halves(w0[w], w1[w]);
      odd.y = hi_halves(w2[w], w3[w]);
      *reinterpret_cast<uint2*>(&vt_lds[d * kVtStride + 4 * krow0]) = even;
      *reinterpret_cast<uint2*>(&vt_lds[(d + 1) * kVtStride + 4 * krow0]) = odd;
    }
  };

  // Online-softmax state of this lane's row (log2 domain) and O^T accumulators.
  float m_run = -INFINITY;
  float l_run = 0.0f;  // partial row sum over this lane's keys
  f32x16_t o_acc[kHeadDim / 32];
#pragma unroll
  for (int m = 0; m < kHeadDim / 32; ++m) o_acc[m] = f32x16_t{};

  if (num_tiles > 0) load_tile(0);

  for (int i = 0; i < num_tiles; ++i) {
    __syncthreads();  // every wave finished reading the previous tile
    store_tile();
    __syncthreads();
    const int k0 = tile_id(i) * kKvTile;
    if (i + 1 < num_tiles) load_tile(i + 1);

    // ---- S^T (64 keys x 32 rows) = K Q^T ----
    f32x16_t s[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      s[b] = f32x16_t{};
      const __bf16* krow = &k_lds[(32 * b + n) * kKeyStride + 8 * half];
#pragma unroll
      for (int c = 0; c < kHeadDim / 16; ++c) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(krow + 16 * c);
        s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[c], s[b], 0, 0, 0);
      }
    }

    // Accumulator element v of block b is key k0 + 32b + 8(v/4) + 4*half + v%4.
    const bool need_mask = (k0 + kKvTile - 1 > tb) ||
                           (block_has_sparse && max(k0, kSinkTokens) < last_sparse_row - kLocalWindow);
    float tile_max = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float x = s[b][v] * p.scale_log2;
        if (need_mask) {
          const int k = k0 + 32 * b + 8 * (v >> 2) + 4 * half + (v & 3);
          x = attended(q, k, p.sparse_begin, p.sparse_end) ? x : -INFINITY;
        }
        s[b][v] = x;
        tile_max = fmaxf(tile_max, x);
      }
    }
    tile_max = wave_half_max(tile_max);
    const float m_new = fmaxf(m_run, tile_max);
    // A row with no attended key yet keeps m = -inf; use 0 as the shift so
    // exp2(-inf - 0) = 0 and no NaN is formed.
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;

    float row_sum = 0.0f;
    bf16x8_t pb[2][2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float e = __builtin_amdgcn_exp2f(s[b][v] - m_use);
        row_sum += e;
        pb[b][v >> 3][v & 7] = (__bf16)e;
      }
    }
    l_run = l_run * alpha + row_sum;
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) o_acc[m] *= alpha;

    // ---- O^T (128 dims x 32 rows) += V^T P^T ----
    // MFMA k-slot e of half h in k-group (b, j) is key 32b + 16j + 8(e/4) + 4h + e%4,
    // both in P (accumulator elements 8j..8j+7) and in V^T (two 4-key reads).
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) {
      const __bf16* vrow = &vt_lds[(32 * m + n) * kVtStride + 4 * half];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int kb = 32 * b + 16 * j;
          const bf16x4_t lo = *reinterpret_cast<const bf16x4_t*>(vrow + kb);
          const bf16x4_t hi = *reinterpret_cast<const bf16x4_t*>(vrow + kb + 8);
          const bf16x8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          o_acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[b][j], o_acc[m], 0, 0, 0);
        }
      }
    }
  }

  // ---- finalize: O / l, bf16, write out[q][qh][d] ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (row_active) {
    __bf16* orow = p.out + ((size_t)(q - p.query_start) * kQueryHeads + qh) * kHeadDim;
#pragma unroll
    for (int m = 0; m < kHeadDim / 32; ++m) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4_t o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(o_acc[m][4 * g + e] * inv);
        *reinterpret_cast<bf16x4_t*>(orow + 32 * m + 8 * g + 4 * half) = o4;
      }
    }
  }
}

hipError_t launch_triangle_paged_attention(const KernelParams& p, hipStream_t stream) {
  const dim3 grid((unsigned)(p.num_row_blocks * kKvHeads));
  hipLaunchKernelGGL(triangle_paged_attention_kernel, grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace tmx
