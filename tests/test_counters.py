"""Structured counter log and its run aggregator (``trianglemix.counters``).

Mirrors the reference's counter-parser tests
(release_validation/tests/test_release_validation.py:85-137,
test_release_contracts.py:283-306, test_ttft_abba_hardening.py:30-52,
:181-199) and adds end-to-end checks against the stats module itself:

* the reference's mixed-log case: two snapshots of one worker behind log
  prefixes aggregate to the latest one (request_total 2, single_launch 5), and
  a counter that goes back is reported;
* a malformed snapshot yields every schema error kind the reference checks;
* events wrapped in a JSON log formatter's ``message`` string are found, a
  repeat of one object within one line counts once;
* workers are summed over their latest snapshots (two real processes, their
  own pids and log files);
* the router's own log lines, parsed back, sum to the stats snapshot, with
  every invariant satisfied; a planted counter error is caught by exactly the
  identity it breaks;
* the command line writes the report and exits 0 on PASS, 1 on FAIL (no
  events).
"""

from __future__ import annotations

import json
import logging
import multiprocessing as mp
from pathlib import Path

import torch

from trianglemix import counters as C
from trianglemix import kernel as K
from trianglemix.config import PluginConfig
from trianglemix.planning import build_batch_plan
from trianglemix.router import TriangleMixRouter
from trianglemix.stats import TriangleMixRuntimeStats


def _stats_line(*, pid=17, boundary, counters, reasons=None, direct=None, fia=None, prefix="INFO worker payload "):
    """A log line holding one worker-local payload (the layout the stats module emits)."""
    payload = {
        "event": C.EVENT_NAME,
        "scope": "worker_local",
        "worker": {"pid": pid, "rank": "0", "local_rank": "0"},
        "request_boundary": boundary,
        "stats": {"counters": counters, "fallback_reasons": reasons or {},
                  "layers": {"direct": direct or {}, "fia": fia or {}}, "performance": {}},
    }
    return prefix + json.dumps(payload, sort_keys=True)


def _consistent(request_total, single_launch):
    """Counters that satisfy every identity: all requests eligible, one direct layer per launch."""
    return {"request_total": request_total, "request_planner_eligible": request_total,
            "request_planner_ineligible": 0, "layer_direct": single_launch, "single_launch": single_launch,
            "layer_fia": 0}


def test_mixed_log_latest_snapshot_per_worker():
    text = "\n".join([
        "unrelated log",
        _stats_line(boundary=1, counters=_consistent(1, 2), direct={"selected": 2}),
        _stats_line(boundary=2, counters=_consistent(2, 5), direct={"selected": 5}),
    ])
    events = C.extract_stats_events(text, source="worker.log")
    assert [e.line_number for e in events] == [2, 3]
    report = C.aggregate_worker_events(events)
    assert report["worker_count"] == 1 and report["event_count"] == 2
    assert report["aggregate"]["counters"]["request_total"] == 2
    assert report["aggregate"]["counters"]["single_launch"] == 5
    assert report["counter_regressions"] == [] and report["snapshot_invariant_errors"] == []
    assert C.report_status(report) == "PASS"


def test_counter_and_boundary_regressions_are_reported():
    text = "\n".join([
        _stats_line(boundary=2, counters=_consistent(2, 0)),
        _stats_line(boundary=1, counters=_consistent(1, 0)),
    ])
    report = C.aggregate(C.scan_events(text, source="worker.log"))
    regressed = {r["counter"] for r in report["counter_regressions"]}
    assert {"request_total", "request_planner_eligible", "request_boundary"} <= regressed
    assert C.report_status(report) == "FAIL"
    # a different worker going lower is not a regression
    other = _stats_line(pid=18, boundary=1, counters=_consistent(1, 0))
    ok = C.aggregate(C.scan_events(_stats_line(boundary=2, counters=_consistent(2, 0)) + "\n" + other))
    assert ok["counter_regressions"] == [] and ok["worker_count"] == 2
    assert ok["aggregate"]["counters"]["request_total"] == 3


def test_malformed_worker_snapshot_is_rejected():
    malformed = {
        "event": C.EVENT_NAME, "scope": "global", "worker": {"pid": "not-an-integer"}, "request_boundary": -1,
        "stats": {"counters": {"request_total": "one", "routing_ns": float("inf"), "layer_fia": True},
                  "fallback_reasons": {}, "layers": {"direct": [], "fia": {}}, "performance": {}},
    }
    report = C.aggregate(C.scan_events(json.dumps(malformed), source="bad.log"))
    kinds = {e["kind"] for e in report["schema_errors"]}
    assert {"invalid_scope", "missing_worker_pid", "invalid_request_boundary", "invalid_counter_value",
            "invalid_layer_mapping"} <= kinds
    bad_values = {e["counter"] for e in report["schema_errors"] if e["kind"] == "invalid_counter_value"}
    assert bad_values == {"request_total", "routing_ns", "layer_fia"}
    missing = dict(malformed, scope="worker_local", worker={"pid": 3}, request_boundary=0)
    del missing["stats"]
    kinds2 = {e["kind"] for e in C.aggregate(C.scan_events(json.dumps(missing)))["schema_errors"]}
    assert kinds2 == {"missing_stats_snapshot"}


def test_wrapped_and_repeated_events():
    inner = _stats_line(boundary=1, counters=_consistent(1, 1), direct={"5": 1}, prefix="")
    record = json.dumps({"level": "INFO", "logger": "trianglemix.router", "message": inner})
    # the same object twice on one line counts once; on the next line it counts again
    text = record + " " + inner + "\n" + inner + "\n" + '{"event": "something_else"} {not json'
    events = C.scan_events(text, source="json.log")
    assert [e.line_number for e in events] == [1, 2]
    assert events[0].value == json.loads(inner)


def _plan(seq, qlen=512, prompt=8192):
    cfg = K.TriangleMixConfig(enabled=True, layer_indices=frozenset({5, 7}))
    return build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[qlen], seq_lens=[seq],
                            prompt_lens=[prompt], num_decodes=0, num_prefills=1, config=cfg)


class _ListHandler(logging.Handler):
    def __init__(self):
        super().__init__()
        self.lines = []

    def emit(self, record):
        self.lines.append(f"INFO {record.name} " + record.getMessage())


def _run_router_steps(log_interval, steps):
    """Drive the router (host side only: the kernels are stand-ins) through ``steps`` chunk plans of
    two selected and one unselected layer; return its log lines and the stats."""
    stats = TriangleMixRuntimeStats()
    out_fn = lambda **kw: kw["output"]  # noqa: E731
    kcfg = K.TriangleMixConfig(enabled=True, layer_indices=frozenset({5, 7}))
    router = TriangleMixRouter(PluginConfig(kernel=kcfg, stats_log_interval=log_interval), stats=stats,
                               direct_fn=out_fn, dense_fn=out_fn, native_ready=lambda: True)
    handler = _ListHandler()
    log = logging.getLogger("trianglemix.router")
    log.addHandler(handler)
    old_level = log.level
    log.setLevel(logging.INFO)
    try:
        k = torch.zeros(72, 128, 8, 128, dtype=torch.bfloat16)
        bt = torch.arange(72, dtype=torch.int32)[None]
        for step in range(steps):
            seq = 512 * (step + 1)
            plan = _plan(seq)
            q = torch.zeros(512, 32, 128, dtype=torch.bfloat16)
            out = torch.empty_like(q)
            for layer in (5, 6, 7):
                router.prefill_attention(layer_name=f"model.layers.{layer}.self_attn.attn", plan=plan, query=q,
                                         key_cache=k, value_cache=k, block_table=bt, output=out,
                                         softmax_scale=0.088)
    finally:
        log.removeHandler(handler)
        log.setLevel(old_level)
    return handler.lines, stats


def test_router_log_lines_sum_to_the_stats_snapshot():
    lines, stats = _run_router_steps(log_interval=1, steps=16)
    assert lines and all(C.EVENT_NAME in line for line in lines)
    report = C.aggregate(C.scan_events("\n".join(lines), source="worker0.log"))
    assert C.report_status(report) == "PASS", report
    snap = stats.snapshot()
    agg = report["aggregate"]
    assert agg["counters"] == snap["counters"]
    assert agg["fallback_reasons"] == snap["fallback_reasons"]
    assert agg["layers"] == snap["layers"]
    # the planner's verdicts on the 16 chunks (reference gates): layers 5 and 7 run direct on the eligible
    # ones and fall back with the planner's reason on the others; layer 6 is not selected (no counters)
    plans = [_plan(512 * (i + 1)) for i in range(16)]
    direct = sum(p.direct for p in plans)
    reasons = {}
    for p in plans:
        if not p.direct:
            reasons[p.primary_reason.value] = reasons.get(p.primary_reason.value, 0) + 1
    assert 0 < direct < 16 and "no_sparse_middle" in reasons
    assert agg["counters"]["request_total"] == 16 and agg["counters"]["single_launch"] == 2 * direct
    assert agg["fallback_reasons"] == reasons
    assert agg["layers"] == {"direct": {"5": direct, "7": direct}, "fia": {"5": 16 - direct, "7": 16 - direct}}
    assert agg["performance"]["planner_eligibility_rate"] == direct / 16
    for key in ("planner_eligibility_rate", "routing_us_per_request", "host_enqueue_us_per_launch"):
        assert abs(agg["performance"][key] - snap["performance"][key]) < 1e-9


def test_planted_counter_errors_break_their_identity():
    lines, _ = _run_router_steps(log_interval=4, steps=8)
    last = C.scan_events(lines[-1])[0].value
    plants = {
        "request_total_invariant": lambda c, s: c.__setitem__("request_planner_eligible",
                                                              c["request_planner_eligible"] - 1),
        "single_launch_invariant": lambda c, s: c.__setitem__("single_launch", c["single_launch"] + 1),
        "fia_reason_sum_invariant": lambda c, s: c.__setitem__("layer_fia_reason:no_sparse_middle", 0),
        "fallback_reason_invariant": lambda c, s: s["fallback_reasons"].clear(),
        "direct_layer_sum_invariant": lambda c, s: s["layers"]["direct"].pop("5"),
    }
    for kind, plant in plants.items():
        value = json.loads(json.dumps(last))
        plant(value["stats"]["counters"], value["stats"])
        report = C.aggregate(C.scan_events(json.dumps(value)))
        assert {e["kind"] for e in report["snapshot_invariant_errors"]} == {kind}, kind
        assert {e["kind"] for e in report["aggregate_invariant_errors"]} == {kind}, kind
    negative = json.loads(json.dumps(last))
    negative["stats"]["counters"]["routing_ns"] = -5
    kinds = {e["kind"] for e in C.aggregate(C.scan_events(json.dumps(negative)))["snapshot_invariant_errors"]}
    assert kinds == {"negative_counter"}


def _worker(log_path: str, steps: int) -> None:
    lines, _ = _run_router_steps(log_interval=2, steps=steps)
    Path(log_path).write_text("\n".join(lines) + "\n")


def test_two_worker_processes_are_summed(tmp_path):
    ctx = mp.get_context("spawn")
    paths = [tmp_path / "worker0.log", tmp_path / "worker1.log"]
    procs = [ctx.Process(target=_worker, args=(str(p), n)) for p, n in zip(paths, (4, 6))]
    for p in procs:
        p.start()
    for p in procs:
        p.join(120)
        assert p.exitcode == 0
    report = C.aggregate(C.read_events(paths))
    assert report["worker_count"] == 2 and C.report_status(report) == "PASS"
    pids = {tuple(w["worker_key"])[1] for w in report["workers"]}
    assert len(pids) == 2
    c = report["aggregate"]["counters"]
    direct = [sum(_plan(512 * (i + 1)).direct for i in range(n)) for n in (4, 6)]
    assert c["request_total"] == 4 + 6 and c["single_launch"] == 2 * sum(direct)


def test_command_line_pass_and_fail(tmp_path, capsys):
    lines, _ = _run_router_steps(log_interval=2, steps=4)
    log = tmp_path / "worker.log"
    log.write_text("startup noise\n" + "\n".join(lines) + "\n")
    out = tmp_path / "report" / "counters.json"
    assert C.main([str(log), "--output", str(out)]) == 0
    report = json.loads(out.read_text())
    assert report["status"] == "PASS" and report["sources"] == [str(log.resolve())]
    assert json.loads(capsys.readouterr().out.strip())["status"] == "PASS"
    empty = tmp_path / "empty.log"
    empty.write_text("no events here\n")
    assert C.main([str(empty), "--output", str(tmp_path / "empty.json")]) == 1
    assert json.loads((tmp_path / "empty.json").read_text())["status"] == "FAIL"
