"""Integer restatement of the TriangleMix mask / schedule / address rules.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference (``/root/reference``) sources restated here:

* per-row key intervals ........ operator/tests/triangle_v2_reference.py:193-232
* dense tail start ............. operator/tests/triangle_v2_reference.py:185-190
* query-span split ............. operator/tests/triangle_v2_reference.py:95-149,
                                 operator/op_kernel/triangle_schedule.h:74-99
* span KV intervals ............ operator/tests/triangle_v2_reference.py:152-182,
                                 operator/op_kernel/triangle_schedule.h:101-142
* logical -> physical page ..... operator/tests/triangle_v2_reference.py:255-270
* BSND element offset .......... operator/op_kernel/fia_paged_kv_address.h:36-53
* saved-QK / span closed forms . package/src/vllm_ascend_trianglemix/kernel.py:185-237

How each function is pinned (tests/test_oracle_geometry.py):

* ``selected_intervals``: the reference's KATs (q=520/521/522/895/896,
  prompt 1024 tail), and brute force against the set-builder rule
  ``{k <= q and (dense(q) or k < 8 or q - k <= 512)}`` over every row of
  several prompts.
* ``split_query_spans``: the reference's exact span tuples and the coverage
  invariants of test_query_span_contract.py.
* ``span_intervals``: the reference's schedule KATs (test_project_contract.py)
  plus "span intervals + per-row boundary mask == row intervals" brute force.
* ``bsnd_element_offset``: the reference's KAT (273,792).
* ``saved_qk_bruteforce`` / ``attended_pairs``: direct counting, checked
  against the reference's closed-form KATs 70,500 and 1,300,078.
"""

from __future__ import annotations

from dataclasses import dataclass

QUERY_HEADS = 32
KV_HEADS = 8
HEAD_DIM = 128
PAGE_SIZE = 128
GROUP = QUERY_HEADS // KV_HEADS
SINK = 8
WINDOW = 512
DENSE_TAIL = 128
Q_TILE = 32
SPARSE_BEGIN = SINK + WINDOW + 1  # 521: first row with a real sink/local gap

Interval = tuple[int, int]


def dense_tail_start(prompt_len: int) -> int:
    """First query row of the final dense tail (triangle_v2_reference.py:185-190)."""
    if prompt_len < 0:
        raise ValueError("prompt_len must be non-negative")
    return max(0, prompt_len - DENSE_TAIL)


def row_is_sparse(q: int, prompt_len: int) -> bool:
    """Row ``q`` uses sink+window iff 521 <= q < prompt_len - 128."""
    return SPARSE_BEGIN <= q < dense_tail_start(prompt_len)


def selected_intervals(q: int, seq_len: int, prompt_len: int) -> tuple[Interval, ...]:
    """Half-open logical key intervals attended by query row ``q``.

    Restates triangle_v2_reference.py:193-232: a dense row attends
    ``[0, min(q+1, seq_len))``; a sparse row attends the sink ``[0, 8)`` and
    the local band ``[q-512, q+1)``, merged into one interval when they touch.
    """
    if q < 0 or seq_len < 0 or prompt_len < 0:
        raise ValueError("positions must be non-negative")
    end = min(q + 1, seq_len)
    if end <= 0:
        return ()
    if not row_is_sparse(q, prompt_len):
        return ((0, end),)
    sink_end = min(SINK, end)
    local_begin = min(max(0, q - WINDOW), end)
    if local_begin <= sink_end:
        return ((0, end),)
    out: list[Interval] = []
    if sink_end:
        out.append((0, sink_end))
    if local_begin < end:
        out.append((local_begin, end))
    return tuple(out)


def selected_keys(q: int, seq_len: int, prompt_len: int) -> list[int]:
    return [k for b, e in selected_intervals(q, seq_len, prompt_len) for k in range(b, e)]


def attended(q: int, k: int, seq_len: int, prompt_len: int) -> bool:
    """Set-builder form of the mask, used as the brute-force cross-check."""
    if k < 0 or k > q or k >= seq_len:
        return False
    if not row_is_sparse(q, prompt_len):
        return True
    return k < SINK or q - k <= WINDOW


@dataclass(frozen=True)
class Span:
    begin: int
    end: int
    sparse: bool


def split_query_spans(query_start: int, query_tokens: int, sparse_begin: int,
                      sparse_end: int, q_tile: int = Q_TILE) -> tuple[Span, ...]:
    """Cut each q-tile at sparse_begin / sparse_end into homogeneous spans.

    Restates triangle_v2_reference.py:95-149 (same result as
    triangle_schedule.h:74-99 for every input the op accepts).
    """
    if query_start < 0 or query_tokens <= 0:
        raise ValueError("bad query range")
    spans: list[Span] = []
    for r0 in range(0, query_tokens, q_tile):
        lo = query_start + r0
        hi = query_start + min(query_tokens, r0 + q_tile)
        cuts = sorted({lo, hi} | {c for c in (sparse_begin, sparse_end) if lo < c < hi})
        tile: list[Span] = []
        for b, e in zip(cuts, cuts[1:]):
            sp = sparse_begin <= b < sparse_end
            if tile and tile[-1].sparse == sp and tile[-1].end == b:
                b = tile.pop().begin
            tile.append(Span(b, e, sp))
        spans.extend(tile)
    return tuple(spans)


def span_intervals(q_begin: int, q_end: int, kv_len: int, sparse_begin: int,
                   sparse_end: int) -> tuple[bool, tuple[Interval, ...]]:
    """(is_dense, KV intervals) submitted for one span.

    Restates triangle_schedule.h:101-142: a span that is not wholly sparse
    submits ``[0, q_end)``; a sparse span submits the sink and the union
    local band ``[q_begin-512, q_end)``, merged when they touch.
    """
    q_end = min(q_end, kv_len)
    if not (q_begin >= sparse_begin and q_end <= sparse_end):
        return True, (() if q_end == 0 else ((0, q_end),))
    sink_end = min(SINK, kv_len)
    local_begin = min(max(0, q_begin - WINDOW), q_end)
    if local_begin <= sink_end:
        return False, (() if q_end == 0 else ((0, q_end),))
    out: list[Interval] = []
    if sink_end:
        out.append((0, sink_end))
    if local_begin < q_end:
        out.append((local_begin, q_end))
    return False, tuple(out)


def physical_location(token: int, block_table: list[int]) -> tuple[int, int]:
    """(physical page, offset in page) of a logical token (triangle_v2_reference.py:255-270)."""
    if token < 0:
        raise ValueError("token must be non-negative")
    lp, off = divmod(token, PAGE_SIZE)
    if lp >= len(block_table):
        raise ValueError("block_table does not cover token")
    pp = int(block_table[lp])
    if pp < 0:
        raise ValueError("negative physical page")
    return pp, off


def bsnd_element_offset(token: int, kv_head: int, block_table: list[int]) -> int:
    """Element offset of K/V[token, kv_head, 0] in a [pages,128,8,128] cache."""
    pp, off = physical_location(token, block_table)
    return ((pp * PAGE_SIZE + off) * KV_HEADS + kv_head) * HEAD_DIM


def attended_pairs(q0: int, q1: int, seq_len: int, prompt_len: int) -> int:
    """Number of attended (q, k) pairs per head over rows [q0, q1), by counting."""
    return sum(e - b for q in range(q0, q1) for b, e in selected_intervals(q, seq_len, prompt_len))


def saved_qk_bruteforce(q0: int, q1: int, prompt_len: int) -> int:
    """Causal QK pairs skipped by the sparse rows of [q0, q1), by counting."""
    return sum((q + 1) - len(selected_keys(q, q + 1, prompt_len))
               for q in range(q0, q1) if row_is_sparse(q, prompt_len))


def unique_kv_tokens(q0: int, q1: int, seq_len: int, prompt_len: int) -> int:
    """Distinct logical tokens read by rows [q0, q1) (for byte accounting)."""
    toks: set[int] = set()
    for q in range(q0, q1):
        for b, e in selected_intervals(q, seq_len, prompt_len):
            toks.update(range(b, e))
    return len(toks)
