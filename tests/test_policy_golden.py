"""The policy layer against golden outputs of the reference's own plugin layer.

``tests/golden/policy_snapshots.json`` holds what the reference's
``build_batch_plan`` (package/src/vllm_ascend_trianglemix/planning.py:119-207),
``TriangleMixRuntimeStats`` (stats.py:14-514, snapshot and structured-log
layout :373-486) and ``resolve_plugin_config`` (config.py:59-197) return for
the scenario in ``tests/golden/policy_ops.py``; the generator is
``tests/golden/make_policy_snapshots.py``.  This build's ``planning``,
``stats`` and ``config`` modules replay the same scenario and must reproduce
every plan record, snapshot, structured-log payload, counter map, error type
and error message exactly.
"""

from __future__ import annotations

import json
import sys
import types
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import policy_ops  # noqa: E402

from trianglemix import config, kernel, planning, stats  # noqa: E402

GOLDEN = json.loads((HERE / "golden" / "policy_snapshots.json").read_text())
MODS = types.SimpleNamespace(kernel=kernel, planning=planning, stats=stats, config=config)


def _roundtrip(x):
    return json.loads(json.dumps(x, sort_keys=True))


@pytest.mark.parametrize("index", range(len(policy_ops.PLAN_CASES)))
def test_plan_records_match_reference(index):
    plan = planning.build_batch_plan(**policy_ops._plan_inputs(MODS, policy_ops.PLAN_CASES[index]))
    assert _roundtrip(policy_ops.plan_record(plan)) == GOLDEN["planning"][index]


def test_plan_ids_are_fresh_and_routing_time_recorded():
    case = policy_ops._plan_inputs(MODS, policy_ops.PLAN_CASES[0])
    a, b = planning.build_batch_plan(**case), planning.build_batch_plan(**case)
    assert b.plan_id > a.plan_id and a.routing_ns >= 0 and b.routing_ns >= 0


def test_stats_scenario_matches_reference():
    got = _roundtrip(policy_ops.run_stats(MODS))
    want = GOLDEN["stats"]
    ops = policy_ops.stats_ops()
    assert len(got) == len(want) == len(ops)
    for i, (op, g, w) in enumerate(zip(ops, got, want)):
        assert g == w, f"stats op {i} {op} differs"


def test_config_cases_match_reference():
    got = _roundtrip(policy_ops.run_config(MODS))
    for case, g, w in zip(policy_ops.CONFIG_CASES, got, GOLDEN["config"]):
        assert g == w, case
    assert len(got) == len(GOLDEN["config"])


def test_golden_scenario_covers_every_stats_entry_point():
    kinds = {op["op"] for op in policy_ops.stats_ops()}
    assert {"configure", "configure_error", "planner", "planner_many", "dispatch", "dispatch_many", "fallback",
            "error", "log", "log_digest", "snapshot", "snapshot_digest", "counters"} <= kinds
    # the scenario reaches both bounded containers and both log flush kinds
    logs = [r for op, r in zip(policy_ops.stats_ops(), GOLDEN["stats"]) if op["op"] in ("log", "log_digest") and r]
    assert any(r["stats"]["counters"].get("structured_log_deltas_dropped") for r in logs)
    assert len({r["request_boundary"] for r in logs}) >= 2
    counters = [r for op, r in zip(policy_ops.stats_ops(), GOLDEN["stats"]) if op["op"] == "counters"]
    assert counters[-1]["request_total"] > counters[-2]["request_total"]  # an evicted plan id counts again
