"""Per-scheduler-step routing plan: one immutable plan reused by every layer.

Mirror of package/src/vllm_ascend_trianglemix/planning.py: the same 24
``FallbackReason`` values (:14-38), plan records (:41-75), request gates in
the same order (:86-116) and batch gates (:119-207).  The string values are
the counter keys of ``stats.py`` and must not change.
"""

from __future__ import annotations

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

    @property
    def saved_qk(self) -> int:
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


def build_batch_plan(*, state_name: str, cumulative_query_ends: Sequence[int] | None,
                     seq_lens: Sequence[int] | None, prompt_lens: Sequence[int] | None,
                     num_decodes: int, num_prefills: int, config: TriangleMixConfig) -> TriangleBatchPlan:
    """Build the step's immutable plan, reused by every selected layer."""
    started = time.perf_counter_ns()
    ends = tuple(int(v) for v in (cumulative_query_ends or ()))
    seqs = tuple(int(v) for v in (seq_lens or ()))
    prompts = tuple(int(v) for v in (prompt_lens or ()))
    batch = len(seqs)

    if state_name not in PREFILL_STATES:
        global_reason = FallbackReason.STATE_UNSUPPORTED
    elif num_decodes:
        global_reason = FallbackReason.MIXED_DECODE
    elif (not ends or not seqs or not prompts or len(ends) != batch or len(prompts) != batch
          or num_prefills != batch):
        global_reason = FallbackReason.MISSING_METADATA
    elif batch != 1:
        global_reason = FallbackReason.BATCH_UNSUPPORTED
    else:
        global_reason = FallbackReason.NONE

    requests: list[TriangleRequestPlan] = []
    prev_end = 0
    for i in range(batch):
        end = ends[i] if i < len(ends) else prev_end
        qlen = end - prev_end
        seq = seqs[i]
        prompt = prompts[i] if i < len(prompts) else seq
        span, local = _request_reason(query_len=qlen, seq_len=seq, prompt_len=prompt, config=config)
        reason = global_reason if global_reason is not FallbackReason.NONE else local
        requests.append(TriangleRequestPlan(
            request_index=i, q_begin=seq - qlen, q_end=seq, seq_len=seq, prompt_len=prompt,
            span=span, eligible=reason is FallbackReason.NONE, reason=reason))
        prev_end = end

    if not requests:
        # A placeholder keeps the reason when metadata is absent; stats never
        # count it as a user request (batch_size stays 0).
        requests.append(TriangleRequestPlan(
            request_index=0, q_begin=0, q_end=0, seq_len=0, prompt_len=0, span=None, eligible=False,
            reason=global_reason if global_reason is not FallbackReason.NONE else FallbackReason.MISSING_METADATA))

    return TriangleBatchPlan(
        plan_id=next(_PLAN_IDS), state_name=state_name, batch_size=batch, requests=tuple(requests),
        direct=len(requests) == 1 and requests[0].eligible, routing_ns=time.perf_counter_ns() - started)
