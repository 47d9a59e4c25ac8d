"""ctypes binding of the C ABI in ``include/trianglemix.h``.

For callers that do not go through ``torch.ops`` (and for the parity tests,
which exercise the C boundary directly).  Tensors are only used for their
device pointers; the launch goes on the given stream (default: torch's
current stream of the query's device).
"""

from __future__ import annotations

import ctypes

from .native import load_hip_library

TM_OK = 0
TM_ERR_INVALID_ARGUMENT = 1
TM_ERR_UNSUPPORTED = 2
TM_ERR_WORKSPACE = 3
TM_ERR_LAUNCH = 4


class TriangleMixError(RuntimeError):
    def __init__(self, status: int, message: str) -> None:
        super().__init__(f"{message} (status {status})")
        self.status = status


def _check(status: int) -> None:
    if status != TM_OK:
        lib = load_hip_library()
        raise TriangleMixError(status, lib.tm_last_error().decode() or lib.tm_status_string(status).decode())


def _stream(query, stream):
    if stream is not None:
        return int(stream)
    import torch

    return torch.cuda.current_stream(query.device).cuda_stream


def workspace_size(query_tokens: int, query_start: int, seq_len: int, prompt_len: int | None) -> int:
    lib = load_hip_library()
    if prompt_len is None:
        n = lib.tm_dense_paged_causal_attention_workspace_size(query_tokens, query_start, seq_len)
    else:
        n = lib.tm_triangle_paged_sparse_attention_workspace_size(query_tokens, query_start, seq_len, prompt_len)
    if n < 0:
        raise TriangleMixError(TM_ERR_INVALID_ARGUMENT, lib.tm_last_error().decode())
    return int(n)


def chunk_plan(query_tokens: int, query_start: int, seq_len: int, prompt_len: int | None) -> tuple[int, int, int]:
    """(KV parts, tiles per work item, work items per KV head) the launch uses for this chunk geometry;
    ``prompt_len`` None plans the dense companion."""
    lib = load_hip_library()
    parts, tiles, items = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    dense = prompt_len is None
    status = lib.tm_chunk_plan(int(dense), query_tokens, query_start, seq_len, 0 if dense else prompt_len,
                               ctypes.byref(parts), ctypes.byref(tiles), ctypes.byref(items))
    _check(status)
    return parts.value, tiles.value, items.value


# Split-KV workspace per (device, stream), at most MAX_WORKSPACE_BYTES.  Its
# contents before a call do not matter (the library tags every arrival word
# for its workspace), so a buffer is never cleared.  One buffer is kept per
# (device, stream), allocated on that stream; a call that needs more replaces
# it, and PyTorch's caching allocator hands the old buffer's memory out again
# only in that stream's order, after the work queued on it.
WORKSPACE_COUNTER_BYTES = 65536
MAX_WORKSPACE_BYTES = 64 << 20
_WORKSPACES: dict = {}


def _workspace(query, query_start, seq_len, prompt_len, workspace, stream):
    need = workspace_size(query.shape[0], query_start, seq_len, prompt_len)
    if need == 0:
        return None, 0
    if workspace is None:
        import torch

        key = (query.device.index, int(stream))
        held = _WORKSPACES.get(key)
        if held is None or held.numel() < need:
            _WORKSPACES.pop(key, None)
            with torch.cuda.stream(torch.cuda.ExternalStream(int(stream), device=query.device)):
                held = _WORKSPACES[key] = torch.empty(need, dtype=torch.uint8, device=query.device)
        workspace = held
    return workspace.data_ptr(), workspace.numel() * workspace.element_size()


def triangle_paged_sparse_attention(query, key_cache, value_cache, block_table, out, *, query_start: int,
                                    seq_len: int, prompt_len: int, scale: float, stream=None,
                                    workspace=None) -> None:
    lib = load_hip_library()
    st = _stream(query, stream)
    ws_ptr, ws_bytes = _workspace(query, query_start, seq_len, prompt_len, workspace, st)
    _check(lib.tm_triangle_paged_sparse_attention(
        query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(), out.data_ptr(),
        query.shape[0], key_cache.shape[0], block_table.shape[-1], query_start, seq_len, prompt_len,
        float(scale), ws_ptr, ws_bytes, st))


def triangle_paged_sparse_attention_noalloc(query, key_cache, value_cache, block_table, out, *, query_start: int,
                                            seq_len: int, prompt_len: int, scale: float, stream=None) -> None:
    """The no-allocation entry point: split-KV scratch from the library's static per-GPU array."""
    lib = load_hip_library()
    st = _stream(query, stream)
    _check(lib.tm_triangle_paged_sparse_attention_noalloc(
        query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(), out.data_ptr(),
        query.shape[0], key_cache.shape[0], block_table.shape[-1], query_start, seq_len, prompt_len,
        float(scale), st))


def dense_paged_causal_attention(query, key_cache, value_cache, block_table, out, *, query_start: int,
                                 seq_len: int, scale: float, stream=None, workspace=None) -> None:
    lib = load_hip_library()
    st = _stream(query, stream)
    ws_ptr, ws_bytes = _workspace(query, query_start, seq_len, None, workspace, st)
    _check(lib.tm_dense_paged_causal_attention(
        query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(), out.data_ptr(),
        query.shape[0], key_cache.shape[0], block_table.shape[-1], query_start, seq_len,
        float(scale), ws_ptr, ws_bytes, st))


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, *, stream=None) -> None:
    """Scatter key / value rows ``[T, 8, 128]`` (row-strided views allowed) into cache slots.

    Token ``i`` goes to page ``slot_mapping[i] // 128``, offset ``slot_mapping[i] % 128``
    (int64); negative slots are padding and are skipped.
    """
    lib = load_hip_library()
    st = _stream(key, stream)
    _check(lib.tm_reshape_and_cache(
        key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.data_ptr(),
        key.shape[0], key.stride(0), value.stride(0), key_cache.shape[0], st))
