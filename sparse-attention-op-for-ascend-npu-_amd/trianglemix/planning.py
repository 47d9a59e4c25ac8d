"""Per-scheduler-step routing plan: one immutable plan reused by every layer.

Contract shared with the reference (package/src/vllm_ascend_trianglemix/
planning.py): the 24 ``FallbackReason`` values (:14-38) -- they are the
counter keys of ``stats.py`` -- the plan records (:41-75), the request gates
and their order (:86-116) and the batch gates (:119-207).  Golden plan records
of the reference pin the behaviour (tests/test_policy_golden.py).
"""

from __future__ import annotations

import functools
import itertools
import time
from dataclasses import dataclass
from enum import Enum
from typing import Sequence

from .kernel import TriangleMixConfig, TriangleSparseSpan, triangle_sparse_span


class FallbackReason(str, Enum):
    NONE = "none"
    STATE_UNSUPPORTED = "state_unsupported"
    MIXED_DECODE = "mixed_decode"
    BATCH_UNSUPPORTED = "batch_unsupported"
    MISSING_METADATA = "missing_metadata"
    INVALID_LENGTHS = "invalid_lengths"
    NO_SPARSE_MIDDLE = "no_sparse_middle"
    BELOW_MIN_SEQ_LEN = "below_min_seq_len"
    BELOW_MIN_SPARSE_ROWS = "below_min_sparse_rows"
    BELOW_MIN_SAVED_QK = "below_min_saved_qk"
    BELOW_SPLIT_MIN_SPARSE_ROWS = "below_split_min_sparse_rows"
    BELOW_SPLIT_MIN_SAVED_QK = "below_split_min_saved_qk"
    GEOMETRY_UNSUPPORTED = "geometry_unsupported"
    ADAPTER_UNAVAILABLE = "adapter_unavailable"
    DIRECT_LAUNCH_ERROR = "direct_launch_error"
    STATIC_CAPABILITY = "static_capability"
    GRAPH_CAPTURE = "graph_capture"
    CONTEXT_PARALLEL = "context_parallel"
    TENSOR_PARALLEL = "tensor_parallel"
    NON_CAUSAL = "non_causal"
    MODEL_UNSUPPORTED = "model_unsupported"
    QUERY_UNSUPPORTED = "query_unsupported"
    KV_CACHE_UNSUPPORTED = "kv_cache_unsupported"
    BLOCK_TABLE_UNSUPPORTED = "block_table_unsupported"


@dataclass(frozen=True)
class TriangleRequestPlan:
    request_index: int
    q_begin: int
    q_end: int
    seq_len: int
    prompt_len: int
    span: TriangleSparseSpan | None
    eligible: bool
    reason: FallbackReason

    @property
    def query_len(self) -> int:
        return self.q_end - self.q_begin

    @functools.cached_property
    def saved_qk(self) -> int:
        # cached: the routing layer reads it on every direct layer call of the plan
        return 0 if self.span is None else self.span.saved_qk


@dataclass(frozen=True)
class TriangleBatchPlan:
    plan_id: int
    state_name: str
    batch_size: int
    requests: tuple[TriangleRequestPlan, ...]
    direct: bool
    routing_ns: int

    @property
    def primary_reason(self) -> FallbackReason:
        for request in self.requests:
            if request.reason is not FallbackReason.NONE:
                return request.reason
        return FallbackReason.NONE


_PLAN_IDS = itertools.count(1)
PREFILL_STATES = frozenset({"PrefillNoCache", "PrefillCacheHit", "ChunkedPrefill"})


def _request_reason(*, query_len: int, seq_len: int, prompt_len: int,
                    config: TriangleMixConfig) -> tuple[TriangleSparseSpan | None, FallbackReason]:
    if query_len <= 0 or seq_len < query_len or prompt_len < seq_len:
        return None, FallbackReason.INVALID_LENGTHS
    span = triangle_sparse_span(query_len=query_len, seq_len=seq_len, prompt_len=prompt_len, config=config)
    gates = (
        (not config.has_supported_geometry, FallbackReason.GEOMETRY_UNSUPPORTED),
        (not span.has_sparse_middle, FallbackReason.NO_SPARSE_MIDDLE),
        (seq_len < config.direct_min_seq_len, FallbackReason.BELOW_MIN_SEQ_LEN),
        (span.sparse_rows < config.direct_min_sparse_rows, FallbackReason.BELOW_MIN_SPARSE_ROWS),
        (span.saved_qk < config.direct_min_saved_qk, FallbackReason.BELOW_MIN_SAVED_QK),
        (span.is_split and span.sparse_rows < config.direct_split_min_sparse_rows,
         FallbackReason.BELOW_SPLIT_MIN_SPARSE_ROWS),
        (span.is_split and span.saved_qk < config.direct_split_min_saved_qk,
         FallbackReason.BELOW_SPLIT_MIN_SAVED_QK),
    )
    for failed, reason in gates:
        if failed:
            return span, reason
    return span, FallbackReason.NONE


def _batch_reason(state_name: str, ends: tuple[int, ...], seqs: tuple[int, ...], prompts: tuple[int, ...],
                  num_decodes: int, num_prefills: int) -> FallbackReason:
    """The first batch-level gate the step fails, in gate order (NONE when it passes all)."""
    batch = len(seqs)
    complete = bool(ends and seqs and prompts) and len(ends) == len(prompts) == num_prefills == batch
    gates = (
        (lambda: state_name not in PREFILL_STATES, FallbackReason.STATE_UNSUPPORTED),
        (lambda: num_decodes != 0, FallbackReason.MIXED_DECODE),
        (lambda: not complete, FallbackReason.MISSING_METADATA),
        (lambda: batch != 1, FallbackReason.BATCH_UNSUPPORTED),
    )
    return next((reason for failed, reason in gates if failed()), FallbackReason.NONE)


def _request_lengths(ends: tuple[int, ...], seqs: tuple[int, ...],
                     prompts: tuple[int, ...]) -> list[tuple[int, int, int]]:
    """(query_len, seq_len, prompt_len) per request.

    ``ends`` are cumulative query ends.  Metadata shorter than ``seqs`` is
    completed so that every request still gets a record: a missing end
    repeats the previous one (query length 0) and a missing prompt length is
    the request's sequence length.
    """
    last = ends[-1] if ends else 0
    padded = list(ends[:len(seqs)]) + [last] * max(0, len(seqs) - len(ends))
    starts = [0] + padded[:-1]
    return [(end - start, seq, prompts[i] if i < len(prompts) else seq)
            for i, (start, end, seq) in enumerate(zip(starts, padded, seqs))]


def build_batch_plan(*, state_name: str, cumulative_query_ends: Sequence[int] | None,
                     seq_lens: Sequence[int] | None, prompt_lens: Sequence[int] | None,
                     num_decodes: int, num_prefills: int, config: TriangleMixConfig) -> TriangleBatchPlan:
    """Build the step's immutable plan, reused by every selected layer.

    A batch-level reason, when there is one, overrides every request's own.
    A step without any request still yields one placeholder request so the
    plan carries its reason; ``batch_size`` stays 0, so stats never count it.
    """
    started = time.perf_counter_ns()
    ends, seqs, prompts = (tuple(int(v) for v in (x or ())) for x in (cumulative_query_ends, seq_lens, prompt_lens))
    batch_reason = _batch_reason(state_name, ends, seqs, prompts, num_decodes, num_prefills)
    requests = []
    for index, (query_len, seq_len, prompt_len) in enumerate(_request_lengths(ends, seqs, prompts)):
        span, own_reason = _request_reason(query_len=query_len, seq_len=seq_len, prompt_len=prompt_len,
                                           config=config)
        reason = own_reason if batch_reason is FallbackReason.NONE else batch_reason
        requests.append(TriangleRequestPlan(request_index=index, q_begin=seq_len - query_len, q_end=seq_len,
                                            seq_len=seq_len, prompt_len=prompt_len, span=span,
                                            eligible=reason is FallbackReason.NONE, reason=reason))
    if not requests:
        placeholder = FallbackReason.MISSING_METADATA if batch_reason is FallbackReason.NONE else batch_reason
        requests.append(TriangleRequestPlan(request_index=0, q_begin=0, q_end=0, seq_len=0, prompt_len=0,
                                            span=None, eligible=False, reason=placeholder))
    return TriangleBatchPlan(plan_id=next(_PLAN_IDS), state_name=state_name, batch_size=len(seqs),
                             requests=tuple(requests), direct=len(requests) == 1 and requests[0].eligible,
                             routing_ns=time.perf_counter_ns() - started)
