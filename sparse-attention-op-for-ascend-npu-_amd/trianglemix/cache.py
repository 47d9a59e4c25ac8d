"""Paged KV write: fill a chunk's cache pages before they are attended.

``reshape_and_cache`` is ``torch.ops.trianglemix.reshape_and_cache`` (vLLM's
argument order, bf16 caches in the ``[pages, 128, 8, 128]`` layout the
attention reads); ``chunk_slot_mapping`` builds the slot of every token of one
chunk from its block table on the device, the mapping an engine passes for a
single request (slot = block_table[t // 128] * 128 + t % 128, the page /
offset rule of the reference's harness, operator/tests/npu_v2_correctness.py:385-398).
"""

from __future__ import annotations

PAGE_SIZE = 128


def chunk_slot_mapping(block_table, query_start: int, num_tokens: int):
    """int64 slots of logical tokens ``query_start .. query_start + num_tokens - 1`` (device of the table)."""
    import torch

    if block_table.dim() != 2 or block_table.size(0) != 1:
        raise ValueError("block_table must be [1, max_pages]")
    if query_start < 0 or num_tokens < 0:
        raise ValueError("query_start and num_tokens must be non-negative")
    last = query_start + num_tokens
    if num_tokens and (last - 1) // PAGE_SIZE >= block_table.size(1):
        raise ValueError("block_table lacks logical pages required by the chunk")
    t = torch.arange(query_start, last, dtype=torch.int64, device=block_table.device)
    return block_table[0].to(torch.int64)[t // PAGE_SIZE] * PAGE_SIZE + t % PAGE_SIZE


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping) -> None:
    """Write ``key[i]`` / ``value[i]`` (``[8, 128]`` bf16) to cache slot ``slot_mapping[i]`` (-1 = padding)."""
    import torch

    from .native import require_adapter

    require_adapter()  # no CPU fallback: fails loudly without the native library
    torch.ops.trianglemix.reshape_and_cache(key, value, key_cache, value_cache, slot_mapping)


def write_chunk_kv(key, value, key_cache, value_cache, block_table, query_start: int) -> None:
    """Fill the pages of logical tokens ``query_start .. query_start + len(key) - 1``."""
    reshape_and_cache(key, value, key_cache, value_cache,
                      chunk_slot_mapping(block_table, query_start, key.shape[0]))
