"""Thread-safe process counters for TriangleMix routing and launches.

Mirror of package/src/vllm_ascend_trianglemix/stats.py (:14-514): the same
counter names, snapshot layout, bounded "recent" plan trace and structured
JSON log deltas, so dashboards and log aggregators built for the reference
read these unchanged.

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
"""

from __future__ import annotations

import os
import threading
from collections import Counter, OrderedDict, deque
from copy import deepcopy
from typing import Any

from .planning import FallbackReason, TriangleBatchPlan

_HOST_SCOPE = "host_enqueue_not_device_latency"


def _route_of(plan: TriangleBatchPlan) -> str:
    return "planner_eligible" if plan.direct else "planner_ineligible"


def _empty_execution() -> dict[str, Any]:
    return {
        "observed_route": "unobserved",
        "layer_direct": 0,
        "layer_fia": 0,
        "layer_hit_rate": 0.0,
        "fallback_reasons": {},
        "single_launch": 0,
        "estimated_saved_qk": 0,
        "host_enqueue_ns_total": 0,
        "host_enqueue_ns_max": 0,
        "timing_scope": _HOST_SCOPE,
        "layer_events_dropped": 0,
    }


def _apply_event(execution: dict[str, Any], *, route: str, reason: FallbackReason, single_launch: int,
                 estimated_saved_qk: int, host_enqueue_ns: int) -> None:
    if route == "direct":
        execution["layer_direct"] += 1
    else:
        execution["layer_fia"] += 1
        reasons = execution["fallback_reasons"]
        reasons[reason.value] = reasons.get(reason.value, 0) + 1
    direct, fia = execution["layer_direct"], execution["layer_fia"]
    execution["layer_hit_rate"] = direct / (direct + fia) if direct + fia else 0.0
    if direct and fia:
        execution["observed_route"] = "mixed"
    elif direct:
        execution["observed_route"] = "all_direct"
    elif fia:
        execution["observed_route"] = "all_fia"
    execution["single_launch"] += single_launch
    execution["estimated_saved_qk"] += estimated_saved_qk
    execution["host_enqueue_ns_total"] += host_enqueue_ns
    execution["host_enqueue_ns_max"] = max(execution["host_enqueue_ns_max"], host_enqueue_ns)


def _event_sort_key(event: dict[str, Any]) -> tuple:
    layer = event["layer_index"]
    return (-1 if layer is None else layer, event["route"], event["reason"], tuple(event["request_slots"]),
            event["host_enqueue_ns"])


class TriangleMixRuntimeStats:
    _LAYER_EVENT_CAPACITY = 256
    _LOG_DELTA_CAPACITY = 8192
    _SEEN_PLAN_CAPACITY = 8192

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._counters: Counter[str] = Counter()
        self._fallback_reasons: Counter[str] = Counter()
        self._layer_direct: Counter[str] = Counter()
        self._layer_fia: Counter[str] = Counter()
        self._seen_plans: OrderedDict[int, None] = OrderedDict()
        self._recent: OrderedDict[int, dict[str, Any]] = OrderedDict()
        self._recent_capacity = 256
        self._log_deltas: deque[dict[str, Any]] = deque()
        self._due_log_plan_ids: set[int] = set()
        self._active_log_plan_ids: set[int] = set()
        self._log_interval = 0
        self._next_log_request = 0
        self._last_log_boundary = 0

    # ------------------------------------------------------------------ config
    def configure(self, recent_capacity: int, log_interval: int = 0) -> None:
        if recent_capacity < 0 or log_interval < 0:
            raise ValueError("TriangleMix stats configuration must be non-negative")
        with self._lock:
            self._recent_capacity = recent_capacity
            self._trim_recent_locked()
            if log_interval != self._log_interval:
                self._log_interval = log_interval
                self._log_deltas.clear()
                self._due_log_plan_ids.clear()
                self._active_log_plan_ids.clear()
                self._last_log_boundary = 0
                total = self._counters["request_total"]
                self._next_log_request = (total // log_interval + 1) * log_interval if log_interval else 0

    def _trim_recent_locked(self) -> None:
        while len(self._recent) > self._recent_capacity:
            self._recent.popitem(last=False)

    # ----------------------------------------------------------------- planner
    def _first_sight_locked(self, plan_id: int) -> bool:
        if plan_id in self._seen_plans:
            return False
        self._seen_plans[plan_id] = None
        if len(self._seen_plans) > self._SEEN_PLAN_CAPACITY:
            self._seen_plans.popitem(last=False)
        return True

    def record_planner_decision(self, plan: TriangleBatchPlan) -> None:
        """Count the deterministic planner result once per plan.

        Layer outcomes are kept out of the request counters, so the exported
        request totals do not depend on the order selected layers run in.
        """
        with self._lock:
            if not self._first_sight_locked(plan.plan_id):
                return
            c = self._counters
            c["routing_ns"] += plan.routing_ns
            # The placeholder request of a metadata-less plan is not a user request.
            requests = plan.requests[:plan.batch_size]
            eligible = sum(1 for r in requests if r.eligible)
            c["request_total"] += plan.batch_size
            c["request_planner_eligible"] += eligible
            c["request_planner_ineligible"] += plan.batch_size - eligible
            for r in requests:
                if not r.eligible:
                    self._fallback_reasons[r.reason.value] += 1
            if self._log_interval:
                self._append_delta_locked({
                    "kind": "planner",
                    "plan_id": plan.plan_id,
                    "state": plan.state_name,
                    "batch_size": plan.batch_size,
                    "route": _route_of(plan),
                    "reason": plan.primary_reason.value,
                    "requests": [{"slot": r.request_index, "eligible": r.eligible, "reason": r.reason.value}
                                 for r in requests],
                })
                if self._next_log_request and c["request_total"] >= self._next_log_request:
                    self._due_log_plan_ids.add(plan.plan_id)
            if self._recent_capacity:
                entries = [{
                    "slot": r.request_index,
                    "q_begin": r.q_begin,
                    "q_end": r.q_end,
                    "seq_len": r.seq_len,
                    "prompt_len": r.prompt_len,
                    "saved_qk": r.saved_qk,
                    "eligible": r.eligible,
                    "reason": r.reason.value,
                    "execution": _empty_execution(),
                } for r in requests]
                self._recent[plan.plan_id] = {
                    "plan_id": plan.plan_id,
                    "state": plan.state_name,
                    "batch_size": plan.batch_size,
                    "route": _route_of(plan),
                    "reason": plan.primary_reason.value,
                    "execution": _empty_execution(),
                    "layer_events": [],
                    "requests": entries,
                    "_request_positions": {e["slot"]: i for i, e in enumerate(entries)},
                }
                self._trim_recent_locked()

    def record_request_decision(self, plan: TriangleBatchPlan, *, direct: bool | None = None,
                                reason: FallbackReason | None = None) -> None:
        """Compatibility alias: runtime outcomes never override the planner."""
        del direct, reason
        self.record_planner_decision(plan)

    # ------------------------------------------------------------------ layers
    def record_layer_dispatch(self, *, plan_id: int, layer_index: int | None, saved_qk: int,
                              host_enqueue_ns: int, request_index: int = 0) -> None:
        with self._lock:
            c = self._counters
            c["layer_direct"] += 1
            c["single_launch"] += 1
            c["estimated_saved_qk"] += saved_qk
            c["host_enqueue_ns"] += host_enqueue_ns
            c["host_enqueue_ns_max"] = max(c["host_enqueue_ns_max"], host_enqueue_ns)
            self._layer_direct[str(layer_index)] += 1
            self._layer_event_locked(plan_id=plan_id, layer_index=layer_index, route="direct",
                                     reason=FallbackReason.NONE, request_indices=(request_index,),
                                     single_launch=1, estimated_saved_qk=saved_qk, host_enqueue_ns=host_enqueue_ns)

    def record_layer_fallback(self, *, plan_id: int | None = None, layer_index: int | None,
                              reason: FallbackReason, request_indices: tuple[int, ...] = ()) -> None:
        """A selected layer that ran the dense companion kernel instead."""
        with self._lock:
            self._counters["layer_fia"] += 1
            self._layer_fia[str(layer_index)] += 1
            self._counters[f"layer_fia_reason:{reason.value}"] += 1
            if plan_id is not None:
                self._layer_event_locked(plan_id=plan_id, layer_index=layer_index, route="fia", reason=reason,
                                         request_indices=request_indices, single_launch=0,
                                         estimated_saved_qk=0, host_enqueue_ns=0)

    def _layer_event_locked(self, *, plan_id: int, layer_index: int | None, route: str, reason: FallbackReason,
                            request_indices: tuple[int, ...], single_launch: int, estimated_saved_qk: int,
                            host_enqueue_ns: int) -> None:
        slots = sorted(set(request_indices))
        event = {
            "layer_index": layer_index,
            "route": route,
            "reason": reason.value,
            "request_slots": list(slots),
            "single_launch": single_launch,
            "estimated_saved_qk": estimated_saved_qk,
            "host_enqueue_ns": host_enqueue_ns,
            "timing_scope": _HOST_SCOPE,
        }
        # The structured log is fed even when the recent trace is disabled or
        # the plan was already evicted from it.
        if self._log_interval and plan_id in self._seen_plans:
            self._append_delta_locked({"kind": "layer_execution", "plan_id": plan_id, **event})
        entry = self._recent.get(plan_id)
        if entry is None:
            return
        dropped = len(entry["layer_events"]) >= self._LAYER_EVENT_CAPACITY
        if dropped:
            entry["execution"]["layer_events_dropped"] += 1
            self._counters["recent_layer_events_dropped"] += 1
        else:
            entry["layer_events"].append(event)
        kwargs = dict(route=route, reason=reason, single_launch=single_launch,
                      estimated_saved_qk=estimated_saved_qk, host_enqueue_ns=host_enqueue_ns)
        _apply_event(entry["execution"], **kwargs)
        for slot in slots:
            pos = entry["_request_positions"].get(slot)
            if pos is None:
                continue
            request = entry["requests"][pos]
            if dropped:
                request["execution"]["layer_events_dropped"] += 1
            _apply_event(request["execution"], **kwargs)

    def _append_delta_locked(self, delta: dict[str, Any]) -> None:
        if len(self._log_deltas) >= self._LOG_DELTA_CAPACITY:
            self._log_deltas.popleft()
            self._counters["structured_log_deltas_dropped"] += 1
        self._log_deltas.append(delta)

    def record_runtime_error(self, *, stage: str) -> None:
        """Count a fail-open error (no exception text is stored)."""
        with self._lock:
            self._counters["runtime_error"] += 1
            self._counters[f"runtime_error_stage:{stage}"] += 1

    # --------------------------------------------------------------- snapshot
    def _snapshot_locked(self, *, include_recent: bool) -> dict[str, Any]:
        c = self._counters
        total = c["request_total"]
        direct = c["layer_direct"]
        result: dict[str, Any] = {
            "counters": dict(c),
            "fallback_reasons": dict(self._fallback_reasons),
            "layers": {"direct": dict(self._layer_direct), "fia": dict(self._layer_fia)},
            "performance": {
                "planner_eligibility_rate": c["request_planner_eligible"] / total if total else 0.0,
                "routing_us_per_request": c["routing_ns"] / total / 1_000 if total else 0.0,
                "host_enqueue_us_per_launch": c["host_enqueue_ns"] / direct / 1_000 if direct else 0.0,
                "host_enqueue_us_max": c["host_enqueue_ns_max"] / 1_000,
                "host_enqueue_timing_scope": "host_wall_time_not_device_latency",
            },
        }
        if include_recent:
            recent = deepcopy(list(self._recent.values()))
            for entry in recent:
                entry.pop("_request_positions", None)
                entry["layer_events"].sort(key=_event_sort_key)
            result["recent"] = recent
        return result

    def structured_log_if_due(self) -> dict[str, Any] | None:
        """Worker-local counters plus incremental plan events, when due."""
        with self._lock:
            total = self._counters["request_total"]
            if not self._log_interval or not self._log_deltas:
                return None
            due = total >= self._next_log_request
            pending = {int(d["plan_id"]) for d in self._log_deltas}
            # Layer events of the plans that crossed the last boundary are
            # flushed between boundaries as supplemental deltas.
            supplemental = (not due and bool(self._active_log_plan_ids)
                            and pending.issubset(self._active_log_plan_ids))
            if not due and not supplemental:
                return None
            if due:
                boundary = (total // self._log_interval) * self._log_interval
                self._next_log_request = boundary + self._log_interval
                self._last_log_boundary = boundary
                self._active_log_plan_ids = set(self._due_log_plan_ids)
                self._due_log_plan_ids.clear()
            else:
                boundary = self._last_log_boundary
            deltas = deepcopy(list(self._log_deltas))
            self._log_deltas.clear()
            return {
                "event": "trianglemix_runtime_stats",
                "scope": "worker_local",
                "worker": {"pid": os.getpid(), "rank": os.getenv("RANK"), "local_rank": os.getenv("LOCAL_RANK")},
                "request_boundary": boundary,
                "delta_mode": "incremental_not_final_plan_snapshot",
                "recent_delta": deltas,
                "stats": self._snapshot_locked(include_recent=False),
            }

    def snapshot(self, reset: bool = False) -> dict[str, Any]:
        with self._lock:
            result = self._snapshot_locked(include_recent=True)
            if reset:
                for container in (self._counters, self._fallback_reasons, self._layer_direct, self._layer_fia,
                                   self._seen_plans, self._recent, self._log_deltas, self._due_log_plan_ids,
                                   self._active_log_plan_ids):
                    container.clear()
                self._next_log_request = self._log_interval
                self._last_log_boundary = 0
            return result


_STATS = TriangleMixRuntimeStats()


def stats_snapshot(reset: bool = False) -> dict[str, Any]:
    return _STATS.snapshot(reset=reset)


def runtime_stats() -> TriangleMixRuntimeStats:
    return _STATS
