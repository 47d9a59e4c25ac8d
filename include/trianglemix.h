/*
 * trianglemix.h -- C ABI of the MI355X (gfx950) TriangleMix paged sparse
 * prefill attention library (libtrianglemix.so).
 *
 * Geometry is fixed to the reference operator's compiled ABI
 * (operator/schema/triangle_paged_sparse_attention.json:38-89,
 * operator/op_host/triangle_paged_sparse_attention.cpp:26-37):
 *   query        [query_tokens, 32, 128]        bf16, contiguous
 *   key_cache    [num_pages, 128, 8, 128]       bf16, contiguous (BSND pages)
 *   value_cache  [num_pages, 128, 8, 128]       bf16, contiguous
 *   block_table  [1, block_table_cols]          int32, logical page -> physical page
 *   out          [query_tokens, 32, 128]        bf16, contiguous, written in place
 * GQA 4:1 (query head h reads KV head h/4), page 128, sink 8, local window
 * 512, dense tail 128, q_tile 32.
 *
 * All pointers are device pointers; `stream` is a hipStream_t (NULL = the
 * null stream).  Every call is asynchronous: it validates its arguments on
 * the host, enqueues ONE kernel on `stream` and returns.  No call allocates
 * device memory, synchronises, or reads device memory on the host.
 * Arguments are validated before any HIP call, so a rejected call touches
 * no device state.
 */
#ifndef TRIANGLEMIX_H
#define TRIANGLEMIX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TM_ABI_VERSION 3

/* Status codes. */
#define TM_OK 0
#define TM_ERR_INVALID_ARGUMENT 1 /* shape / attribute / pointer contract breach */
#define TM_ERR_UNSUPPORTED 2      /* outside the fixed compiled geometry or limits */
#define TM_ERR_WORKSPACE 3        /* workspace too small for this call */
#define TM_ERR_LAUNCH 4           /* the HIP launch itself failed */

/* A non-empty workspace starts with this many bytes of arrival words, one
 * per split row block, KV head and workgroup position; the split-KV partials
 * follow.  A workspace's contents before a call do not matter (as the
 * reference's workspace, it is scratch): each word carries the arrival tag
 * the library keeps for that workspace address, and a word with any other
 * tag counts as zero.  One workspace serves any sequence of calls on one
 * stream; calls that overlap in time on one workspace race. */
#define TM_WORKSPACE_COUNTER_BYTES 65536

/* No call needs more workspace than this (64 MiB): the planner keeps every
 * chunk's split-KV partials within it, and a chunk whose rows need no split
 * needs none.  A caller may allocate this once per stream and pass it to
 * every call. */
#define TM_MAX_WORKSPACE_BYTES 67108864

/* ABI version of the loaded library (TM_ABI_VERSION it was built with). */
int tm_abi_version(void);

/* Static name of a status code. */
const char* tm_status_string(int status);

/* Human-readable detail of the last failing call on the calling thread
 * (empty string if none).  The text mirrors the reference's TORCH_CHECK /
 * tiling messages. */
const char* tm_last_error(void);

/*
 * TriangleMix sparse prefill over one scheduler chunk: rows
 * [query_start, seq_len) of a prompt of final length prompt_len.
 * Rows q with 521 <= q < prompt_len-128 attend keys [0,8) U [q-512, q];
 * all other rows attend [0, q].  One softmax per row over all its keys;
 * fp32 accumulation; bf16 output rounded to nearest even.
 *
 * Replaces trianglemix::triangle_paged_sparse_attention.out
 * (operator/torch_adapter/triangle_paged_attention_torch.cpp:140-178, schema
 * :290-297) and the aclnnTrianglePagedSparseAttention launch it wraps
 * (:161-176); validation follows check_inputs/check_output (:29-97) and
 * TilingFunc (operator/op_host/triangle_paged_sparse_attention.cpp:122-237).
 *
 * Any chunk the attributes allow is accepted: a row of any length runs in
 * one workgroup, and rows are split across workgroups only to balance the
 * GPU, within TM_MAX_WORKSPACE_BYTES of workspace.
 *
 * workspace / workspace_bytes: device scratch of at least
 * tm_triangle_paged_sparse_attention_workspace_size(...) bytes (may be NULL
 * when that size is 0; never more than TM_MAX_WORKSPACE_BYTES), with any
 * contents.  Its first TM_WORKSPACE_COUNTER_BYTES hold the arrival words of
 * row blocks whose keys are split across workgroups (long dense rows); the
 * rest receives their fp32 partials, which the last workgroup of each such
 * row block merges within the same kernel.  Launches that may overlap in
 * time need distinct workspaces.  It must not overlap any input or out.
 */
int tm_triangle_paged_sparse_attention(
    const void* query, const void* key_cache, const void* value_cache,
    const int32_t* block_table, void* out,
    int64_t query_tokens, int64_t num_pages, int64_t block_table_cols,
    int64_t query_start, int64_t seq_len, int64_t prompt_len, float scale,
    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Device scratch bytes the call above needs for these arguments (0 when the
 * whole chunk runs without split-KV partials, at most TM_MAX_WORKSPACE_BYTES),
 * or -1, with the reason in tm_last_error, for exactly the attributes the
 * call above refuses.
 * Replaces trianglemix_reference::triangle_paged_sparse_attention_workspace_size
 * (operator/torch_adapter/triangle_paged_attention_torch.cpp:180-261).
 */
int64_t tm_triangle_paged_sparse_attention_workspace_size(
    int64_t query_tokens, int64_t query_start, int64_t seq_len,
    int64_t prompt_len);

/*
 * The same TriangleMix call for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * has no counterpart in the reference.  No call allocates: the split-KV
 * scratch (arrival words + partials) is a static array of
 * TM_MAX_WORKSPACE_BYTES (64 MiB) per GPU where the library's code loads,
 * held until the process ends -- as large as any chunk's workspace, so every
 * chunk the workspace entry point accepts is accepted here.  The device
 * address of the array is looked up once per device, with that device
 * current -- call with the stream's device current, as for any launch.  All
 * calls in one process on one GPU share the array: calls that may overlap in
 * time on that GPU (on different streams, or graphs replayed on different
 * streams) race and must not be made.  Other arguments, results and errors
 * as tm_triangle_paged_sparse_attention.
 */
int tm_triangle_paged_sparse_attention_noalloc(
    const void* query, const void* key_cache, const void* value_cache,
    const int32_t* block_table, void* out,
    int64_t query_tokens, int64_t num_pages, int64_t block_table_cols,
    int64_t query_start, int64_t seq_len, int64_t prompt_len, float scale,
    void* stream);

/*
 * Dense paged causal prefill (row q attends [0, q]) built from the same
 * tiles; serves unselected layers and fallbacks.  Replaces the dense CANN
 * FIA call the reference falls back to
 * (operator/tests/npu_v2_crossover.py:156-188,
 * harness/npu_harness_common.py:278-316: TND layout, page 128,
 * sparse_mode=3, next_tokens=0).
 */
int tm_dense_paged_causal_attention(
    const void* query, const void* key_cache, const void* value_cache,
    const int32_t* block_table, void* out,
    int64_t query_tokens, int64_t num_pages, int64_t block_table_cols,
    int64_t query_start, int64_t seq_len, float scale,
    void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes for tm_dense_paged_causal_attention, or -1 if invalid. */
int64_t tm_dense_paged_causal_attention_workspace_size(
    int64_t query_tokens, int64_t query_start, int64_t seq_len);

/*
 * The launch plan the entry points above use for one chunk geometry: the
 * workgroup shape (*kv_parts: 4 = two query heads over KV quarters, 2 = the
 * four heads of a GQA group over KV halves, 1 = the four heads over the whole
 * KV range, two workgroups per CU), the most tiles of 32 keys one
 * work item takes (*tiles_per_split) and the work items per KV head
 * (*items_per_kv_head).  dense != 0 plans the dense companion (prompt_len is
 * then ignored).  Returns TM_OK, or TM_ERR_INVALID_ARGUMENT for attributes the
 * entry points would refuse.  No counterpart in the reference: a diagnostic
 * for tests and tooling (planner regression pins, bench reports).
 */
int tm_chunk_plan(int dense, int64_t query_tokens, int64_t query_start, int64_t seq_len, int64_t prompt_len,
                  int32_t* kv_parts, int32_t* tiles_per_split, int64_t* items_per_kv_head);

/*
 * Paged KV write, upstream of the attention: scatters one chunk's fresh K and
 * V rows into their cache slots.  key / value: [num_tokens, 8, 128] bf16 with
 * the [8, 128] part contiguous and a row stride of key_stride / value_stride
 * elements (>= 1024, multiples of 8; a slice of a fused QKV buffer works).
 * slot_mapping: int64 [num_tokens]; token i goes to page slot_mapping[i] / 128,
 * offset slot_mapping[i] % 128 of both caches.  A negative slot is padding and
 * is skipped, as is a slot >= num_pages * 128.  Pointers 16-byte aligned; the
 * caches must not overlap each other or the sources.  num_tokens == 0 enqueues
 * nothing.
 *
 * Replaces vLLM's reshape_and_cache on this page layout (the step that fills
 * a chunk's pages before they are attended; the reference leaves it to the
 * engine, planning.py:79-83, and fills pages in its harness by the same page
 * / offset rule, operator/tests/npu_v2_correctness.py:385-398).
 */
int tm_reshape_and_cache(
    const void* key, const void* value, void* key_cache, void* value_cache,
    const int64_t* slot_mapping, int64_t num_tokens, int64_t key_stride,
    int64_t value_stride, int64_t num_pages, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIANGLEMIX_H */
