// Paged KV write for gfx950: scatter one chunk's fresh K/V rows into their
// cache slots, upstream of the attention kernel (the chunked-prefill step that
// fills pages before they are attended).
//
// Semantics follow vLLM's reshape_and_cache on the BSND page layout the
// attention kernel reads: token i's K row [8, 128] goes to
// key_cache[slot / 128][slot % 128], V likewise, with slot = slot_mapping[i].
// A negative slot is padding and is skipped; a slot past the cache is skipped
// too, so a bad mapping can never write outside the caches.  The reference
// fills pages by the same page / offset rule
// (operator/tests/npu_v2_correctness.py:385-398, physical_location).
//
// HBM-bound scatter: each token moves 2 KB of K and 2 KB of V in and out.
// One thread per 16-byte chunk of a token's row (128 chunks per token), a
// wave covering half a token: every load and store is a coalesced 1 KB
// stretch.  The stores are written through L2 (sc1): nothing the attention
// launches after it will read stays dirty in an L2, and the writes stream out
// during the kernel instead of at its end (measured: 8192 tokens in 8.5 us
// instead of 11.4, one 512-token chunk 2.66 us instead of 2.85).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "trianglemix_kernel.h"

namespace tmx {
namespace {

constexpr int kCacheThreads = 256;
constexpr int kChunksPerRow = kKvHeads * kHeadDim * 2 / 16;  // 16-byte chunks per token row (128)
static_assert(kCacheThreads % kChunksPerRow == 0 && kChunksPerRow % 64 == 0, "a wave stays inside one token");
constexpr int kRawBufferFlags = 0x00020000;  // buffer resource word 3 for raw byte-addressed access
constexpr int kCpolWriteThrough = 16;        // sc1

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kCacheThreads)
paged_kv_write_kernel(const uint4* __restrict__ key, const uint4* __restrict__ value, uint4* __restrict__ key_cache,
                      uint4* __restrict__ value_cache, const int64_t* __restrict__ slot_mapping, int64_t num_tokens,
                      int64_t key_stride_chunks, int64_t value_stride_chunks, int64_t num_slots) {
  const int64_t g = (int64_t)blockIdx.x * kCacheThreads + threadIdx.x;
  const int64_t token = g / kChunksPerRow;
  const int chunk = (int)(g % kChunksPerRow);
  if (token >= num_tokens) return;
  // The K / V loads do not depend on the slot: issued together with the slot
  // load, the two memory round trips overlap instead of following each other
  // (the compiler cannot hoist loads above the slot test by itself).
  const uint4 k = key[token * key_stride_chunks + chunk];
  const uint4 v = value[token * value_stride_chunks + chunk];
  // A wave covers one token, so its slot is wave-uniform: say so, and the
  // buffer resources below stay scalar.
  const int64_t lane_slot = slot_mapping[token];
  const int64_t slot = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(lane_slot >> 32)) << 32) |
                                 (uint32_t)__builtin_amdgcn_readfirstlane((int)lane_slot));
  if (slot < 0 || slot >= num_slots) return;
  const __amdgpu_buffer_rsrc_t k_row = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(key_cache + slot * kChunksPerRow), (short)0, kChunksPerRow * 16, kRawBufferFlags);
  const __amdgpu_buffer_rsrc_t v_row = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(value_cache + slot * kChunksPerRow), (short)0, kChunksPerRow * 16, kRawBufferFlags);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, k), k_row, (unsigned)(chunk * 16), 0,
                                         kCpolWriteThrough);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), v_row, (unsigned)(chunk * 16), 0,
                                         kCpolWriteThrough);
}

}  // namespace

hipError_t launch_paged_kv_write(const void* key, const void* value, void* key_cache, void* value_cache,
                                 const int64_t* slot_mapping, int64_t num_tokens, int64_t key_stride,
                                 int64_t value_stride, int64_t num_pages, hipStream_t stream) {
  const int64_t threads = num_tokens * kChunksPerRow;
  const int64_t blocks = (threads + kCacheThreads - 1) / kCacheThreads;
  // Strides arrive in bf16 elements; the kernel indexes 16-byte chunks.
  hipLaunchKernelGGL(paged_kv_write_kernel, dim3((unsigned)blocks), dim3(kCacheThreads), 0, stream,
                     static_cast<const uint4*>(key), static_cast<const uint4*>(value), static_cast<uint4*>(key_cache),
                     static_cast<uint4*>(value_cache), slot_mapping, num_tokens, key_stride / 8, value_stride / 8,
                     num_pages * kPageSize);
  return hipGetLastError();
}

}  // namespace tmx
