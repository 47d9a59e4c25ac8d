"""Seeded synthetic chunks and closed-form work accounting.

Input generation follows the reference's harness
(operator/tests/npu_v2_correctness.py:219-274): a CPU ``torch.Generator``
seeds a random permutation of ``logical + 7`` physical pages (a
non-consecutive transition is forced), then Q, K and V are drawn
``randn * std`` and rounded to bf16.  Everything is generated on the CPU so
every consumer (GPU kernel, CPU oracle) sees bit-identical tensors.

Work accounting (per chunk, per launch):

* attended pairs per head  P = sum over rows of |selected keys(row)|
* algorithmic FLOPs        4 * D * Hq * P    (2 for QK^T + 2 for PV)
* algorithmic bytes        unique K/V tokens * 8 * 128 * 2 B * 2 + Q + O bytes
"""

from __future__ import annotations

import math
from dataclasses import dataclass

HQ, HKV, D, PAGE = 32, 8, 128, 128
SINK, WINDOW, TAIL = 8, 512, 128
SPARSE_BEGIN = SINK + WINDOW + 1
SCALE = D ** -0.5


@dataclass(frozen=True)
class Chunk:
    """Rows [query_start, seq_len) of a prompt of length prompt_len."""

    query_start: int
    seq_len: int
    prompt_len: int

    @property
    def query_tokens(self) -> int:
        return self.seq_len - self.query_start


def prompt_chunks(prompt_len: int, chunk: int) -> list[Chunk]:
    """The scheduler chunks of a chunked prefill, in order."""
    return [Chunk(q0, min(prompt_len, q0 + chunk), prompt_len) for q0 in range(0, prompt_len, chunk)]


def _sparse_range(q0: int, q1: int, prompt_len: int) -> tuple[int, int]:
    s0 = max(q0, SPARSE_BEGIN)
    s1 = min(q1, max(0, prompt_len - TAIL))
    return s0, max(s0, s1)


def attended_pairs(c: Chunk, *, dense: bool = False) -> int:
    """Attended (q, k) pairs per head, closed form."""
    q0, q1 = c.query_start, c.seq_len
    causal = (q1 - q0) * (q0 + q1 + 1) // 2  # sum of (q + 1)
    if dense:
        return causal
    s0, s1 = _sparse_range(q0, q1, c.prompt_len)
    sparse_rows = s1 - s0
    sparse_causal = sparse_rows * (s0 + s1 + 1) // 2
    return causal - sparse_causal + sparse_rows * (SINK + WINDOW + 1)


def chunk_flops(c: Chunk, *, dense: bool = False) -> int:
    return 4 * D * HQ * attended_pairs(c, dense=dense)


def unique_kv_tokens(c: Chunk, *, dense: bool = False) -> int:
    q0, q1 = c.query_start, c.seq_len
    if dense:
        return q1
    s0, s1 = _sparse_range(q0, q1, c.prompt_len)
    if s1 <= s0:  # no sparse rows: every row is causal-dense
        return q1
    dense_rows_max = -1
    if q0 < s0:
        dense_rows_max = s0 - 1
    if s1 < q1:
        dense_rows_max = q1 - 1
    lo, hi = s0 - WINDOW, s1  # local band of the sparse rows
    if dense_rows_max >= 0:
        n = dense_rows_max + 1
        return max(n, hi) if lo <= n else n + (hi - lo)
    return SINK + (hi - lo)


def chunk_bytes(c: Chunk, *, dense: bool = False) -> int:
    kv = unique_kv_tokens(c, dense=dense) * HKV * D * 2 * 2
    qo = c.query_tokens * HQ * D * 2 * 2
    return kv + qo


def kv_bytes(c: Chunk, *, dense: bool = False) -> int:
    return unique_kv_tokens(c, dense=dense) * HKV * D * 2 * 2


KV_TILE = 32   # keys per kernel tile
ROW_BLOCK = 32  # query tokens per work item


def executed_tiles(c: Chunk, *, dense: bool = False) -> int:
    """KV tiles the kernel visits per KV head (mirror of its tile schedule)."""
    sb = 0 if dense else SPARSE_BEGIN
    se = 0 if dense else max(0, c.prompt_len - TAIL)
    total = 0
    for tb in range(c.query_start, c.seq_len, ROW_BLOCK):
        te = min(tb + ROW_BLOCK, c.seq_len)
        last = (te - 1) // KV_TILE
        if tb >= sb and te <= se and sb < se:
            first = (tb - WINDOW) // KV_TILE
            total += (last + 1) if first <= 0 else 1 + (last - first + 1)
        else:
            total += last + 1
    return total


def executed_flops(c: Chunk, *, dense: bool = False) -> int:
    """MFMA FLOPs actually issued (masked lanes of edge tiles included)."""
    return executed_tiles(c, dense=dense) * HKV * (4 * D * KV_TILE * ROW_BLOCK * (HQ // HKV))


def noncontiguous_block_table(logical_pages: int, physical_pages: int, generator):
    import torch

    perm = torch.randperm(physical_pages, generator=generator, dtype=torch.int64)
    table = perm[:logical_pages].clone()
    if logical_pages > 1 and bool(torch.all(table[1:] == table[:-1] + 1)):
        table[0], table[-1] = table[-1].clone(), table[0].clone()
    return table.to(torch.int32).view(1, -1).contiguous()


def make_cache(seq_len: int, seed: int, *, std: float = 0.5, extra_pages: int = 7, outlier_frac: float = 0.0,
               outlier_value: float = 8.0):
    """(key_cache, value_cache, block_table) covering logical tokens [0, seq_len)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    logical = math.ceil(seq_len / PAGE)
    physical = logical + extra_pages
    table = noncontiguous_block_table(logical, physical, g)
    shape = (physical, PAGE, HKV, D)
    key = torch.randn(shape, generator=g).mul_(std)
    if outlier_frac > 0.0:
        mask = torch.rand(shape, generator=g) < outlier_frac
        signs = torch.where(torch.rand(shape, generator=g) < 0.5, -1.0, 1.0)
        key = torch.where(mask, signs * outlier_value, key)
    value = torch.randn(shape, generator=g).mul_(std)
    return key.to(torch.bfloat16), value.to(torch.bfloat16), table


def make_query(rows: int, seed: int, *, std: float = 0.5):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, HQ, D, generator=g).mul_(std).to(torch.bfloat16)


def make_inputs(query_start: int, query_tokens: int, seq_len: int, seed: int, *, std: float = 0.5,
                outlier_frac: float = 0.0):
    """(query, key_cache, value_cache, block_table) for one chunk, CPU bf16.

    Same draw order as the reference harness: table, query, key, value from
    one generator.
    """
    import torch

    if query_start + query_tokens > seq_len:
        raise ValueError("query extends beyond seq_len")
    g = torch.Generator().manual_seed(seed)
    logical = math.ceil(seq_len / PAGE)
    physical = logical + 7
    table = noncontiguous_block_table(logical, physical, g)
    query = torch.randn(query_tokens, HQ, D, generator=g).mul_(std).to(torch.bfloat16)
    shape = (physical, PAGE, HKV, D)
    key = torch.randn(shape, generator=g).mul_(std)
    if outlier_frac > 0.0:
        mask = torch.rand(shape, generator=g) < outlier_frac
        signs = torch.where(torch.rand(shape, generator=g) < 0.5, -1.0, 1.0)
        key = torch.where(mask, signs * 8.0, key)
    value = torch.randn(shape, generator=g).mul_(std)
    return query, key.to(torch.bfloat16), value.to(torch.bfloat16), table
