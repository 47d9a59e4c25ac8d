"""CPU restatement of the paged KV write (the chunked-prefill step upstream of the attention).

TEST INFRASTRUCTURE ONLY: see the package header.  Nothing in the product path
imports this module.

Semantics: vLLM's reshape_and_cache on the BSND page layout the attention
reads.  Token i's K row ``[8, 128]`` goes to ``key_cache[slot // 128, slot % 128]``
and its V row to the same place of ``value_cache``, with
``slot = slot_mapping[i]``; a negative slot is padding and is skipped, and so is
a slot past the cache.  For one chunk of a prompt, the slot of logical token
``t`` is ``block_table[t // 128] * 128 + t % 128`` -- the page / offset rule of
``physical_location`` (triangle_v2_reference.py:255-270), by which the
reference's harness fills pages (operator/tests/npu_v2_correctness.py:385-398).

Pinned by (tests/test_oracle_cache.py):

* ``chunk_slots``: the reference's address known answer (token 139, table
  [7, 2, 19], KV head 3 -> element 273,792) and, for every token of several
  tables, agreement with ``geometry.bsnd_element_offset``;
* ``reshape_and_cache``: agreement with an independent formulation (one fancy
  assignment into the flattened ``[pages * 128, 8, 128]`` view), padding and
  out-of-range slots left untouched, and a planted mistake (page and offset
  swapped) that the checks must catch.
"""

from __future__ import annotations

import numpy as np

PAGE_SIZE = 128


def chunk_slots(block_table, query_start: int, num_tokens: int) -> np.ndarray:
    """int64 slot of logical tokens ``query_start .. query_start + num_tokens - 1``."""
    table = np.asarray(block_table, dtype=np.int64).reshape(-1)
    t = np.arange(query_start, query_start + num_tokens, dtype=np.int64)
    return table[t // PAGE_SIZE] * PAGE_SIZE + t % PAGE_SIZE


def reshape_and_cache(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                      slot_mapping) -> None:
    """Write ``key[i]`` / ``value[i]`` (``[8, 128]``) to cache slot ``slot_mapping[i]``, in place."""
    num_slots = key_cache.shape[0] * PAGE_SIZE
    for i, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64).reshape(-1)):
        if slot < 0 or slot >= num_slots:
            continue
        page, offset = divmod(int(slot), PAGE_SIZE)
        key_cache[page, offset] = key[i]
        value_cache[page, offset] = value[i]
