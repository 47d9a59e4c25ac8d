"""Thread-safe process counters for TriangleMix routing and launches.

The observable contract is the reference's (package/src/vllm_ascend_trianglemix/
stats.py): the counter names, the ``snapshot()`` layout and the structured-log
payload of ``structured_log_if_due()`` (:373-486), so dashboards and log
aggregators built for the reference read these unchanged.  Golden outputs
of the reference for a fixed scenario pin it (tests/test_policy_golden.py).

Counter families:

* planner, once per plan: ``request_total``, ``request_planner_eligible``,
  ``request_planner_ineligible``, ``routing_ns``, ``fallback_reasons``
* per layer execution: ``layer_direct``, ``single_launch``,
  ``estimated_saved_qk``, ``host_enqueue_ns``, ``host_enqueue_ns_max``,
  ``layer_fia`` and ``layer_fia_reason:<reason>`` (the dense companion kernel
  plays the role of the reference's official FIA fallback)
* failures: ``runtime_error``, ``runtime_error_stage:<stage>``
* retention drops: ``recent_layer_events_dropped``,
  ``structured_log_deltas_dropped``

Design: one lock guards three parts that each own one concern --

* ``_Tallies``: the flat counter maps;
* ``_PlanTrace``: a bounded, oldest-first record per plan (the planner's view,
  an execution tally for the plan and for each request slot, and the plan's
  layer events up to a cap);
* ``_LogCadence``: the structured-log schedule -- buffered deltas, the
  request boundary they flush at, and the plans a boundary left open, whose
  late layer events flush on their own before the next boundary.

Plans are recognised by ``plan_id`` in a bounded first-seen window, so a plan
replayed by every selected layer is counted once.
"""

from __future__ import annotations

import os
import threading
from collections import Counter, OrderedDict, deque
from typing import Any, Iterable, NamedTuple

from .planning import FallbackReason, TriangleBatchPlan

EVENTS_PER_PLAN = 256     # layer events kept per traced plan (later ones are counted as dropped)
LOG_BUFFER = 8192         # structured-log deltas buffered between flushes (oldest dropped first)
SEEN_PLAN_WINDOW = 8192   # plan ids remembered for counting each plan once
_HOST_SCOPE = "host_enqueue_not_device_latency"


class _LayerEvent(NamedTuple):
    layer_index: int | None
    route: str            # "direct" or "fia"
    reason: str
    slots: tuple[int, ...]
    launches: int
    saved_qk: int
    enqueue_ns: int

    def as_dict(self) -> dict[str, Any]:
        return {"layer_index": self.layer_index, "route": self.route, "reason": self.reason,
                "request_slots": list(self.slots), "single_launch": self.launches,
                "estimated_saved_qk": self.saved_qk, "host_enqueue_ns": self.enqueue_ns,
                "timing_scope": _HOST_SCOPE}

    def order(self) -> tuple:
        return (-1 if self.layer_index is None else self.layer_index, self.route, self.reason, self.slots,
                self.enqueue_ns)


class _Execution:
    """What the layers of one plan (or of one request slot of it) did."""

    __slots__ = ("direct", "dense", "reasons", "launches", "saved_qk", "enqueue_ns", "enqueue_max", "dropped")

    def __init__(self) -> None:
        self.direct = self.dense = self.launches = self.saved_qk = self.enqueue_ns = self.enqueue_max = 0
        self.dropped = 0
        self.reasons: dict[str, int] = {}

    def add(self, ev: _LayerEvent) -> None:
        if ev.route == "direct":
            self.direct += 1
        else:
            self.dense += 1
            self.reasons[ev.reason] = self.reasons.get(ev.reason, 0) + 1
        self.launches += ev.launches
        self.saved_qk += ev.saved_qk
        self.enqueue_ns += ev.enqueue_ns
        if ev.enqueue_ns > self.enqueue_max:  # (not max(): this runs for every direct layer call)
            self.enqueue_max = ev.enqueue_ns

    def as_dict(self) -> dict[str, Any]:
        seen = self.direct + self.dense
        route = {(False, False): "unobserved", (True, False): "all_direct", (False, True): "all_fia",
                 (True, True): "mixed"}[(self.direct > 0, self.dense > 0)]
        return {"observed_route": route, "layer_direct": self.direct, "layer_fia": self.dense,
                "layer_hit_rate": self.direct / seen if seen else 0.0, "fallback_reasons": dict(self.reasons),
                "single_launch": self.launches, "estimated_saved_qk": self.saved_qk,
                "host_enqueue_ns_total": self.enqueue_ns, "host_enqueue_ns_max": self.enqueue_max,
                "timing_scope": _HOST_SCOPE, "layer_events_dropped": self.dropped}


def _plan_route(plan: TriangleBatchPlan) -> str:
    return "planner_eligible" if plan.direct else "planner_ineligible"


class _PlanRecord:
    """One traced plan: its header, request summaries and execution tallies."""

    def __init__(self, plan: TriangleBatchPlan, requests: Iterable) -> None:
        self.header = {"plan_id": plan.plan_id, "state": plan.state_name, "batch_size": plan.batch_size,
                       "route": _plan_route(plan), "reason": plan.primary_reason.value}
        self.execution = _Execution()
        self.events: list[_LayerEvent] = []
        self.requests: list[tuple[dict[str, Any], _Execution]] = []
        self.by_slot: dict[int, _Execution] = {}
        for r in requests:
            summary = {"slot": r.request_index, "q_begin": r.q_begin, "q_end": r.q_end, "seq_len": r.seq_len,
                       "prompt_len": r.prompt_len, "saved_qk": r.saved_qk, "eligible": r.eligible,
                       "reason": r.reason.value}
            tally = _Execution()
            self.requests.append((summary, tally))
            self.by_slot[r.request_index] = tally

    def record(self, ev: _LayerEvent) -> bool:
        """Tally ``ev``; returns False when the event list is full and the event itself is not kept."""
        kept = len(self.events) < EVENTS_PER_PLAN
        if kept:
            self.events.append(ev)
        else:
            self.execution.dropped += 1
        self.execution.add(ev)
        for slot in ev.slots:
            tally = self.by_slot.get(slot)
            if tally is None:
                continue
            if not kept:
                tally.dropped += 1
            tally.add(ev)
        return kept

    def as_dict(self) -> dict[str, Any]:
        return {**self.header, "execution": self.execution.as_dict(),
                "layer_events": [ev.as_dict() for ev in sorted(self.events, key=_LayerEvent.order)],
                "requests": [{**summary, "execution": tally.as_dict()} for summary, tally in self.requests]}


class _PlanTrace:
    """The most recent ``capacity`` plans, oldest evicted first."""

    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.records: OrderedDict[int, _PlanRecord] = OrderedDict()

    def resize(self, capacity: int) -> None:
        self.capacity = capacity
        self._evict()

    def add(self, plan: TriangleBatchPlan, requests: Iterable) -> None:
        if self.capacity:
            self.records[plan.plan_id] = _PlanRecord(plan, requests)
            self._evict()

    def _evict(self) -> None:
        while len(self.records) > self.capacity:
            self.records.popitem(last=False)

    def clear(self) -> None:
        self.records.clear()


class _LogCadence:
    """When the structured log flushes, and what it has buffered.

    A flush is due once the request total reaches the next multiple of the
    interval.  Plans counted at or past a boundary stay "open" after it: a
    buffer holding only their (late) layer events flushes on the next poll
    without waiting for the next boundary, reported under the last boundary.
    """

    def __init__(self) -> None:
        self.interval = 0
        self.next_boundary = 0
        self.last_boundary = 0
        self.buffer: deque[dict[str, Any]] = deque()
        self.closing: set[int] = set()   # plans counted at or past the coming boundary
        self.open: set[int] = set()      # plans the last boundary closed over

    def restart(self, interval: int, request_total: int) -> None:
        self.interval = interval
        self.buffer.clear()
        self.closing.clear()
        self.open.clear()
        self.last_boundary = 0
        self.next_boundary = (request_total // interval + 1) * interval if interval else 0

    def reset(self) -> None:
        self.buffer.clear()
        self.closing.clear()
        self.open.clear()
        self.next_boundary = self.interval
        self.last_boundary = 0

    def push(self, delta: dict[str, Any]) -> bool:
        """Buffer ``delta``; returns True when the oldest buffered delta had to be dropped for it."""
        dropped = len(self.buffer) >= LOG_BUFFER
        if dropped:
            self.buffer.popleft()
        self.buffer.append(delta)
        return dropped

    def plan_counted(self, plan_id: int, request_total: int) -> None:
        if self.next_boundary and request_total >= self.next_boundary:
            self.closing.add(plan_id)

    def take(self, request_total: int) -> tuple[int, list[dict[str, Any]]] | None:
        """(boundary, buffered deltas) when a flush is due or a supplemental flush applies, else None."""
        if not self.interval or not self.buffer:
            return None
        if request_total >= self.next_boundary:
            boundary = request_total - request_total % self.interval
            self.next_boundary = boundary + self.interval
            self.last_boundary = boundary
            self.open, self.closing = self.closing, set()
        elif self.open and all(int(d["plan_id"]) in self.open for d in self.buffer):
            boundary = self.last_boundary
        else:
            return None
        deltas = list(self.buffer)
        self.buffer.clear()
        return boundary, deltas


# layer index -> its counter key, str(layer index) (the routing layer records one per call)
_LAYER_KEYS: dict = {}
_NONE_REASON = FallbackReason.NONE.value


class _Tallies:
    def __init__(self) -> None:
        self.counters: Counter[str] = Counter()
        self.reasons: Counter[str] = Counter()
        self.direct_layers: Counter[str] = Counter()
        self.dense_layers: Counter[str] = Counter()

    def clear(self) -> None:
        for c in (self.counters, self.reasons, self.direct_layers, self.dense_layers):
            c.clear()

    def as_dict(self) -> dict[str, Any]:
        c = self.counters
        total, launches = c["request_total"], c["layer_direct"]
        return {
            "counters": dict(c),
            "fallback_reasons": dict(self.reasons),
            "layers": {"direct": dict(self.direct_layers), "fia": dict(self.dense_layers)},
            "performance": {
                "planner_eligibility_rate": c["request_planner_eligible"] / total if total else 0.0,
                "routing_us_per_request": c["routing_ns"] / total / 1_000 if total else 0.0,
                "host_enqueue_us_per_launch": c["host_enqueue_ns"] / launches / 1_000 if launches else 0.0,
                "host_enqueue_us_max": c["host_enqueue_ns_max"] / 1_000,
                "host_enqueue_timing_scope": "host_wall_time_not_device_latency",
            },
        }


class TriangleMixRuntimeStats:
    """Counters, a bounded per-plan trace and the structured-log cadence of one process."""

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._tallies = _Tallies()
        self._trace = _PlanTrace(256)
        self._log = _LogCadence()
        self._seen: OrderedDict[int, None] = OrderedDict()

    def configure(self, recent_capacity: int, log_interval: int = 0) -> None:
        """Set the plan-trace capacity and the structured-log interval (0 turns either off)."""
        if recent_capacity < 0 or log_interval < 0:
            raise ValueError("TriangleMix stats configuration must be non-negative")
        with self._lock:
            self._trace.resize(recent_capacity)
            if log_interval != self._log.interval:
                self._log.restart(log_interval, self._tallies.counters["request_total"])

    # ------------------------------------------------------------ recording
    def record_planner_decision(self, plan: TriangleBatchPlan) -> None:
        """Count a plan's planner result, once per plan id.

        Layer outcomes never feed these request counters, so they do not
        depend on the order the selected layers run in.  A plan built without
        request metadata carries one placeholder request for its reason; it is
        not a user request (``batch_size`` is 0) and is not counted.
        """
        with self._lock:
            self._count_plan_locked(plan)

    def _count_plan_locked(self, plan: TriangleBatchPlan) -> None:
        if plan.plan_id in self._seen:
            return
        self._seen[plan.plan_id] = None
        if len(self._seen) > SEEN_PLAN_WINDOW:
            self._seen.popitem(last=False)
        counted = plan.requests[:plan.batch_size]
        ineligible = [r for r in counted if not r.eligible]
        c = self._tallies.counters
        c["routing_ns"] += plan.routing_ns
        c["request_total"] += plan.batch_size
        c["request_planner_eligible"] += plan.batch_size - len(ineligible)
        c["request_planner_ineligible"] += len(ineligible)
        self._tallies.reasons.update(r.reason.value for r in ineligible)
        if self._log.interval:
            self._buffer_locked({
                "kind": "planner", "plan_id": plan.plan_id, "state": plan.state_name,
                "batch_size": plan.batch_size, "route": _plan_route(plan), "reason": plan.primary_reason.value,
                "requests": [{"slot": r.request_index, "eligible": r.eligible, "reason": r.reason.value}
                             for r in counted],
            })
            self._log.plan_counted(plan.plan_id, c["request_total"])
        self._trace.add(plan, counted)

    def record_layer_dispatch(self, *, plan_id: int, layer_index: int | None, saved_qk: int,
                              host_enqueue_ns: int, request_index: int = 0) -> None:
        """A selected layer ran the sparse kernel (one launch)."""
        with self._lock:
            self._dispatch_locked(plan_id, layer_index, saved_qk, host_enqueue_ns, request_index)

    def record_direct_launch(self, plan: TriangleBatchPlan, *, layer_index: int | None,
                             host_enqueue_ns: int) -> None:
        """``record_planner_decision(plan)`` then ``record_layer_dispatch`` of the plan's first request,
        under one lock: what the routing layer records for every direct layer call."""
        request = plan.requests[0]
        with self._lock:
            self._count_plan_locked(plan)
            self._dispatch_locked(plan.plan_id, layer_index, request.saved_qk, host_enqueue_ns,
                                  request.request_index)

    def _dispatch_locked(self, plan_id: int, layer_index: int | None, saved_qk: int, host_enqueue_ns: int,
                         request_index: int) -> None:
        c = self._tallies.counters
        c["layer_direct"] += 1
        c["single_launch"] += 1
        c["estimated_saved_qk"] += saved_qk
        c["host_enqueue_ns"] += host_enqueue_ns
        if host_enqueue_ns > c["host_enqueue_ns_max"]:
            c["host_enqueue_ns_max"] = host_enqueue_ns
        key = _LAYER_KEYS.get(layer_index)
        if key is None:
            key = str(layer_index)
            if len(_LAYER_KEYS) < 4096:
                _LAYER_KEYS[layer_index] = key
        self._tallies.direct_layers[key] += 1
        self._layer_event_locked(plan_id, _LayerEvent(layer_index, "direct", _NONE_REASON, (request_index,), 1,
                                                      saved_qk, host_enqueue_ns))

    def record_layer_fallback(self, *, plan_id: int | None = None, layer_index: int | None,
                              reason: FallbackReason, request_indices: tuple[int, ...] = ()) -> None:
        """A selected layer that ran the dense companion kernel instead."""
        with self._lock:
            c = self._tallies.counters
            c["layer_fia"] += 1
            c[f"layer_fia_reason:{reason.value}"] += 1
            self._tallies.dense_layers[str(layer_index)] += 1
            if plan_id is not None:
                self._layer_event_locked(plan_id, _LayerEvent(layer_index, "fia", reason.value,
                                                              tuple(sorted(set(request_indices))), 0, 0, 0))

    def record_runtime_error(self, *, stage: str) -> None:
        """Count a fail-open error (no exception text is kept)."""
        with self._lock:
            self._tallies.counters["runtime_error"] += 1
            self._tallies.counters[f"runtime_error_stage:{stage}"] += 1

    def _layer_event_locked(self, plan_id: int, ev: _LayerEvent) -> None:
        # The structured log gets every event of a plan it has counted, traced or not: production runs
        # often disable the trace, and a plan can leave the trace before its last layers run.
        if self._log.interval and plan_id in self._seen:
            self._buffer_locked({"kind": "layer_execution", "plan_id": plan_id, **ev.as_dict()})
        record = self._trace.records.get(plan_id)
        if record is not None and not record.record(ev):
            self._tallies.counters["recent_layer_events_dropped"] += 1

    def _buffer_locked(self, delta: dict[str, Any]) -> None:
        if self._log.push(delta):
            self._tallies.counters["structured_log_deltas_dropped"] += 1

    # ------------------------------------------------------------- reading
    def structured_log_if_due(self) -> dict[str, Any] | None:
        """This worker's counters plus the plan events buffered since the last flush, when a flush applies."""
        if not self._log.interval:  # logging off (the default): nothing is ever buffered or due
            return None
        with self._lock:
            taken = self._log.take(self._tallies.counters["request_total"])
            if taken is None:
                return None
            boundary, deltas = taken
            return {
                "event": "trianglemix_runtime_stats",
                "scope": "worker_local",
                "worker": {"pid": os.getpid(), "rank": os.getenv("RANK"), "local_rank": os.getenv("LOCAL_RANK")},
                "request_boundary": boundary,
                "delta_mode": "incremental_not_final_plan_snapshot",
                "recent_delta": deltas,
                "stats": self._tallies.as_dict(),
            }

    def snapshot(self, reset: bool = False) -> dict[str, Any]:
        """Counters, per-layer maps, derived rates and the plan trace; ``reset`` starts every part afresh."""
        with self._lock:
            result = self._tallies.as_dict()
            result["recent"] = [record.as_dict() for record in self._trace.records.values()]
            if reset:
                self._tallies.clear()
                self._trace.clear()
                self._seen.clear()
                self._log.reset()
            return result


_STATS = TriangleMixRuntimeStats()


def stats_snapshot(reset: bool = False) -> dict[str, Any]:
    return _STATS.snapshot(reset=reset)


def runtime_stats() -> TriangleMixRuntimeStats:
    return _STATS
