"""Structured counter log: worker-local JSON events -> run totals.

Every worker process writes the payloads of
``TriangleMixRuntimeStats.structured_log_if_due()`` to its log, one compact
JSON object per line (``format_event``; the reference's
``_log_stats_if_due``, package/src/vllm_ascend_trianglemix/plugin.py:1344-1355).
Log handlers put prefixes in front of it and JSON log formatters wrap it in a
``message`` string, so the reader looks for every JSON object in a line whose
``event`` is ``trianglemix_runtime_stats``, also inside ``message`` strings.

The counters of a snapshot are cumulative per worker, so the run totals are
the sum over workers of each worker's last snapshot.  A worker is
``(log file, pid, rank, local_rank)``.  Next to the totals the report lists
what makes a log untrustworthy:

* schema errors: scope other than ``worker_local``, no integer pid, a request
  boundary that is not a non-negative integer, a missing snapshot or mapping,
  a counter that is not a finite number;
* counter regressions: a cumulative counter, or the request boundary, that
  goes back between two events of one worker;
* invariant errors, per snapshot and for the totals: negative counters,
  ``request_total = eligible + ineligible``, fallback reasons summing to the
  ineligible requests, ``layer_direct = single_launch``, the per-layer maps
  summing to ``layer_direct`` / ``layer_fia``, and the ``layer_fia_reason:*``
  counters summing to ``layer_fia``.

The report layout, error kinds and the PASS rule follow
release_validation/counters.py:17-448 so tools written for the reference's
report read this one.  Command line::

    python -m trianglemix.counters worker0.log worker1.log --output counters.json
"""

from __future__ import annotations

import argparse
import json
import math
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable, Iterator

EVENT_NAME = "trianglemix_runtime_stats"
SCHEMA_VERSION = 1
_MAPPINGS = ("counters", "fallback_reasons", "layers", "performance")
_ROUTES = ("direct", "fia")


def format_event(payload: dict[str, Any]) -> str:
    """One log line for a structured stats payload (ASCII, sorted keys, no spaces)."""
    return json.dumps(payload, ensure_ascii=True, sort_keys=True, separators=(",", ":"))


def log_if_due(stats, logger) -> dict[str, Any] | None:
    """Log the stats' structured payload when one is due; returns it (or None)."""
    payload = stats.structured_log_if_due()
    if payload is not None:
        logger.info("%s", format_event(payload))
    return payload


@dataclass(frozen=True)
class StatsEvent:
    """One structured stats object found in a log: where, and its value."""

    source: str
    line_number: int
    value: dict[str, Any]

    @property
    def worker_key(self) -> tuple[str, str, str, str]:
        worker = self.value.get("worker")
        if not isinstance(worker, dict):
            worker = {}
        return (self.source, str(worker.get("pid")), str(worker.get("rank")), str(worker.get("local_rank")))

    @property
    def snapshot(self) -> dict[str, Any]:
        stats = self.value.get("stats")
        return stats if isinstance(stats, dict) else {}

    @property
    def location(self) -> str:
        return f"{self.source}:{self.line_number}"

    def to_dict(self) -> dict[str, Any]:
        return {"source": self.source, "line_number": self.line_number, "worker_key": list(self.worker_key),
                "value": self.value}


# ------------------------------------------------------------------ reading
def _json_objects(text: str) -> Iterator[dict[str, Any]]:
    """Every JSON object that starts at some ``{`` of ``text``, and those inside their ``message`` strings."""
    decoder = json.JSONDecoder()
    start = text.find("{")
    while start >= 0:
        try:
            value, _ = decoder.raw_decode(text, start)
        except json.JSONDecodeError:
            value = None
        if isinstance(value, dict):
            yield value
            inner = value.get("message")
            if isinstance(inner, str) and inner != text:
                yield from _json_objects(inner)
        start = text.find("{", start + 1)


def scan_events(text: str, *, source: str = "<memory>") -> list[StatsEvent]:
    """Stats events of a log text in line order; an object repeated within one line counts once."""
    found: list[StatsEvent] = []
    for number, line in enumerate(text.splitlines(), start=1):
        seen: set[str] = set()
        for obj in _json_objects(line):
            if obj.get("event") != EVENT_NAME:
                continue
            key = json.dumps(obj, ensure_ascii=True, sort_keys=True, separators=(",", ":"))
            if key not in seen:
                seen.add(key)
                found.append(StatsEvent(source, number, obj))
    return found


def read_events(paths: Iterable[Path]) -> list[StatsEvent]:
    """Stats events of every file, files in the given order (source = resolved path)."""
    events: list[StatsEvent] = []
    for path in paths:
        path = Path(path)
        events += scan_events(path.read_text(encoding="utf-8", errors="replace"), source=str(path.resolve()))
    return events


# -------------------------------------------------------------- arithmetic
def _numbers(mapping: object) -> dict[str, int | float]:
    """The numeric entries of a mapping with string keys (anything else reads as absent)."""
    if not isinstance(mapping, dict):
        return {}
    return {k: v for k, v in mapping.items() if isinstance(k, str) and isinstance(v, (int, float))}


def _accumulate(total: dict[str, int | float], mapping: object) -> None:
    for k, v in _numbers(mapping).items():
        total[k] = total.get(k, 0) + v


def _layers(snapshot: dict[str, Any], route: str) -> object:
    layers = snapshot.get("layers")
    return layers.get(route) if isinstance(layers, dict) else None


# ---------------------------------------------------------------- checking
def invariant_errors(snapshot: dict[str, Any], *, location: str) -> list[dict[str, object]]:
    """Violations of the counter identities every cumulative snapshot satisfies."""
    counters = _numbers(snapshot.get("counters"))
    reasons = _numbers(snapshot.get("fallback_reasons"))
    direct = _numbers(_layers(snapshot, "direct"))
    fia = _numbers(_layers(snapshot, "fia"))
    c = lambda name: counters.get(name, 0)  # noqa: E731
    errors: list[dict[str, object]] = []
    for mapping, values in (("counters", counters), ("fallback_reasons", reasons), ("layers.direct", direct),
                            ("layers.fia", fia)):
        errors += [{"kind": "negative_counter", "location": location, "mapping": mapping, "counter": k, "value": v}
                   for k, v in values.items() if v < 0]
    planner = c("request_planner_eligible") + c("request_planner_ineligible")
    if c("request_total") != planner:
        errors.append({"kind": "request_total_invariant", "location": location, "request_total": c("request_total"),
                       "planner_sum": planner})
    if sum(reasons.values()) != c("request_planner_ineligible"):
        errors.append({"kind": "fallback_reason_invariant", "location": location,
                       "reason_sum": sum(reasons.values()),
                       "request_planner_ineligible": c("request_planner_ineligible")})
    if c("layer_direct") != c("single_launch"):
        errors.append({"kind": "single_launch_invariant", "location": location, "layer_direct": c("layer_direct"),
                       "single_launch": c("single_launch")})
    if sum(direct.values()) != c("layer_direct"):
        errors.append({"kind": "direct_layer_sum_invariant", "location": location})
    if sum(fia.values()) != c("layer_fia"):
        errors.append({"kind": "fia_layer_sum_invariant", "location": location})
    fia_reasons = sum(v for k, v in counters.items() if k.startswith("layer_fia_reason:"))
    if fia_reasons != c("layer_fia"):
        errors.append({"kind": "fia_reason_sum_invariant", "location": location, "reason_sum": fia_reasons,
                       "layer_fia": c("layer_fia")})
    return errors


def _is_count(value: object) -> bool:
    return (isinstance(value, (int, float)) and not isinstance(value, bool) and math.isfinite(float(value)))


def schema_errors(event: StatsEvent) -> list[dict[str, object]]:
    """Ways in which one event departs from the worker-local payload layout."""
    value, where = event.value, event.location
    errors: list[dict[str, object]] = []
    if value.get("scope") != "worker_local":
        errors.append({"kind": "invalid_scope", "location": where, "value": value.get("scope")})
    worker = value.get("worker")
    if not (isinstance(worker, dict) and isinstance(worker.get("pid"), int)):
        errors.append({"kind": "missing_worker_pid", "location": where})
    boundary = value.get("request_boundary")
    if not (isinstance(boundary, int) and not isinstance(boundary, bool) and boundary >= 0):
        errors.append({"kind": "invalid_request_boundary", "location": where})
    snapshot = value.get("stats")
    if not isinstance(snapshot, dict):
        errors.append({"kind": "missing_stats_snapshot", "location": where})
        return errors
    errors += [{"kind": "invalid_snapshot_mapping", "location": where, "mapping": name}
               for name in _MAPPINGS if not isinstance(snapshot.get(name), dict)]
    layers = snapshot.get("layers")
    if isinstance(layers, dict):
        errors += [{"kind": "invalid_layer_mapping", "location": where, "mapping": f"layers.{route}"}
                   for route in _ROUTES if not isinstance(layers.get(route), dict)]
    checked = {"counters": snapshot.get("counters"), "fallback_reasons": snapshot.get("fallback_reasons"),
               "layers.direct": _layers(snapshot, "direct"), "layers.fia": _layers(snapshot, "fia")}
    for name, mapping in checked.items():
        if not isinstance(mapping, dict):
            continue
        errors += [{"kind": "invalid_counter_value", "location": where, "mapping": name, "counter": str(k),
                    "value_type": type(v).__name__}
                   for k, v in mapping.items() if not (isinstance(k, str) and _is_count(v))]
    return errors


def counter_regressions(events: Iterable[StatsEvent]) -> list[dict[str, object]]:
    """Cumulative counters (and the request boundary) that decrease between events of one worker."""
    last_counters: dict[tuple, dict[str, int | float]] = {}
    last_boundary: dict[tuple, int] = {}
    found: list[dict[str, object]] = []
    for event in events:
        key = event.worker_key

        def regress(counter: str, before, now) -> None:
            found.append({"worker_key": list(key), "source": event.source, "line_number": event.line_number,
                          "counter": counter, "previous": before, "current": now})

        boundary = event.value.get("request_boundary")
        is_boundary = isinstance(boundary, int) and not isinstance(boundary, bool)
        if is_boundary and key in last_boundary and boundary < last_boundary[key]:
            regress("request_boundary", last_boundary[key], boundary)
        now = _numbers(event.snapshot.get("counters"))
        before = last_counters.get(key, {})
        for name in sorted(before.keys() | now.keys()):
            if now.get(name, 0) < before.get(name, 0):
                regress(name, before.get(name, 0), now.get(name, 0))
        last_counters[key] = now
        if is_boundary:
            last_boundary[key] = boundary
    return found


def _performance(counters: dict[str, int | float]) -> dict[str, float]:
    requests = float(counters.get("request_total", 0))
    direct = float(counters.get("layer_direct", 0))
    return {
        "planner_eligibility_rate": counters.get("request_planner_eligible", 0) / requests if requests else 0.0,
        "routing_us_per_request": counters.get("routing_ns", 0) / requests / 1_000 if requests else 0.0,
        "host_enqueue_us_per_launch": counters.get("host_enqueue_ns", 0) / direct / 1_000 if direct else 0.0,
    }


def aggregate(events: Iterable[StatsEvent]) -> dict[str, Any]:
    """Run report: totals over each worker's last snapshot, plus every schema / regression / invariant finding."""
    events = list(events)
    last: dict[tuple, StatsEvent] = {}
    for event in events:
        last[event.worker_key] = event
    totals = {"counters": {}, "fallback_reasons": {}, "direct": {}, "fia": {}}
    workers = []
    for key in sorted(last):
        event = last[key]
        snap = event.snapshot
        _accumulate(totals["counters"], snap.get("counters"))
        _accumulate(totals["fallback_reasons"], snap.get("fallback_reasons"))
        _accumulate(totals["direct"], _layers(snap, "direct"))
        _accumulate(totals["fia"], _layers(snap, "fia"))
        workers.append({"worker_key": list(key), "source": event.source, "line_number": event.line_number,
                        "worker": event.value.get("worker"), "request_boundary": event.value.get("request_boundary"),
                        "stats": snap})
    run = {
        "counters": totals["counters"],
        "fallback_reasons": totals["fallback_reasons"],
        "layers": {"direct": totals["direct"], "fia": totals["fia"]},
        "performance": _performance(totals["counters"]),
    }
    return {
        "schema_version": SCHEMA_VERSION,
        "event": EVENT_NAME,
        "scope": "sum_of_latest_worker_local_snapshots",
        "event_count": len(events),
        "worker_count": len(last),
        "schema_errors": [e for event in events for e in schema_errors(event)],
        "counter_regressions": counter_regressions(events),
        "snapshot_invariant_errors": [e for event in events
                                      for e in invariant_errors(event.snapshot, location=event.location)],
        "aggregate_invariant_errors": invariant_errors(run, location="<aggregate>"),
        "aggregate": run,
        "workers": workers,
    }


def report_status(report: dict[str, Any]) -> str:
    """PASS when at least one event was found and no check found anything."""
    clean = not any(report[k] for k in ("schema_errors", "counter_regressions", "snapshot_invariant_errors",
                                         "aggregate_invariant_errors"))
    return "PASS" if report["event_count"] and clean else "FAIL"


# Names used by the reference's parser module.
extract_stats_events = scan_events
read_stats_events = read_events
aggregate_worker_events = aggregate


def _write_json(path: Path, value: object) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(f".{path.name}.{os.getpid()}.tmp")
    tmp.write_text(json.dumps(value, ensure_ascii=False, indent=2, sort_keys=True) + "\n", encoding="utf-8")
    tmp.replace(path)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="Sum the TriangleMix worker-local stats events of one run's logs.")
    ap.add_argument("logs", nargs="+", type=Path)
    ap.add_argument("--output", type=Path, required=True)
    args = ap.parse_args(argv)
    report = aggregate(read_events(args.logs))
    report["sources"] = [str(p.resolve()) for p in args.logs]
    report["status"] = report_status(report)
    out = args.output.resolve()
    _write_json(out, report)
    print(json.dumps({"status": report["status"], "events": report["event_count"], "workers": report["worker_count"],
                      "output": str(out)}, sort_keys=True), flush=True)
    return 0 if report["status"] == "PASS" else 1


if __name__ == "__main__":
    raise SystemExit(main())
