"""Plan / fallback layer and counters (host logic, CPU only).

Mirrors the reference's package/tests/test_planning_stats.py: the same
configuration coercion rules, the plan-route known answers (held as data in
``tests/golden/reference_kats.json``) and the counter semantics of
``TriangleMixRuntimeStats`` (counted once per plan, planner result not
overridden by runtime outcomes, bounded recent trace, structured log deltas).
"""

from __future__ import annotations

import json
import os
import types
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from unittest.mock import patch

import pytest

from trianglemix.config import resolve_plugin_config
from trianglemix.kernel import TriangleMixConfig
from trianglemix.planning import FallbackReason, build_batch_plan
from trianglemix import stats as stats_module
from trianglemix.stats import TriangleMixRuntimeStats

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def config(**overrides) -> TriangleMixConfig:
    values = dict(enabled=True, layer_indices=frozenset({1, 3, 5}), sink_tokens=8, local_window=512, last_rows=128,
                  direct_min_seq_len=0, direct_min_sparse_rows=128, direct_min_saved_qk=913_152,
                  direct_split_min_sparse_rows=192, direct_split_min_saved_qk=1_299_264)
    values.update(overrides)
    return TriangleMixConfig(**values)


def plan4096(**kw):
    return build_batch_plan(state_name="PrefillNoCache", cumulative_query_ends=[4096], seq_lens=[4096],
                            prompt_lens=[4096], num_decodes=0, num_prefills=1, config=config(**kw))


# ----------------------------------------------------------------- config

def test_additional_config_string_false_is_false():
    holder = types.SimpleNamespace(additional_config={"trianglemix": {"enabled": "false", "strict": "off",
                                                                      "layers": "1,3-4"}})
    resolved = resolve_plugin_config(holder)
    assert not resolved.kernel.enabled and not resolved.strict
    assert resolved.kernel.layer_indices == frozenset({1, 3, 4})


def test_invalid_boolean_is_rejected():
    holder = types.SimpleNamespace(additional_config={"trianglemix": {"enabled": "sometimes", "layers": "1"}})
    with pytest.raises(ValueError, match="must be a boolean"):
        resolve_plugin_config(holder)


def test_environment_is_compatibility_fallback():
    env = {"VLLM_ASCEND_ENABLE_TRIANGLE_MIX": "yes", "VLLM_ASCEND_TRIANGLE_MIX_LAYERS": "2-3"}
    with patch.dict(os.environ, env, clear=True):
        resolved = resolve_plugin_config(None)
    assert resolved.enabled and resolved.kernel.layer_indices == frozenset({2, 3})


def test_config_rejects_negative_thresholds():
    with pytest.raises(ValueError):
        config(direct_min_saved_qk=-1)
    with pytest.raises(ValueError):
        config(sink_tokens=0)
    assert not config(local_window=1024).has_supported_geometry


# ---------------------------------------------------------------- planning

@pytest.mark.parametrize("kat", KATS["plan_routes"], ids=lambda k: f"{k['state']}-{k['query_ends']}-{k['seq_lens']}")
def test_plan_route_kats(kat):
    plan = build_batch_plan(state_name=kat["state"], cumulative_query_ends=kat["query_ends"],
                            seq_lens=kat["seq_lens"], prompt_lens=kat["prompt_lens"],
                            num_decodes=kat["num_decodes"], num_prefills=kat["num_prefills"], config=config())
    assert plan.direct == kat["direct"], kat["source"]
    if kat["reason"] == "batch_unsupported":
        assert all(r.reason is FallbackReason.BATCH_UNSUPPORTED for r in plan.requests)
        assert [r.query_len for r in plan.requests] == kat["query_lens"]
    else:
        assert plan.primary_reason.value == kat["reason"], kat["source"]
    if "saved_qk" in kat:
        assert plan.requests[0].saved_qk == kat["saved_qk"]
    if "q_begin" in kat:
        assert (plan.requests[0].q_begin, plan.requests[0].q_end) == (kat["q_begin"], kat["q_end"])


def test_non_abi_geometry_has_specific_fallback():
    plan = plan4096(local_window=1024)
    assert not plan.direct and plan.primary_reason is FallbackReason.GEOMETRY_UNSUPPORTED


def test_gates_fire_in_reference_order():
    # sparse rows < 128 -> BELOW_MIN_SPARSE_ROWS before the saved-QK gates
    p = build_batch_plan(state_name="PrefillNoCache", cumulative_query_ends=[600], seq_lens=[600],
                         prompt_lens=[8192], num_decodes=0, num_prefills=1, config=config())
    assert p.primary_reason is FallbackReason.BELOW_MIN_SPARSE_ROWS
    p = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[128], seq_lens=[8192],
                         prompt_lens=[8192], num_decodes=0, num_prefills=1, config=config())
    assert p.primary_reason is FallbackReason.NO_SPARSE_MIDDLE
    p = plan4096(direct_min_seq_len=5000)
    assert p.primary_reason is FallbackReason.BELOW_MIN_SEQ_LEN
    p = build_batch_plan(state_name="PrefillNoCache", cumulative_query_ends=[100], seq_lens=[50],
                         prompt_lens=[50], num_decodes=0, num_prefills=1, config=config())
    assert p.primary_reason is FallbackReason.INVALID_LENGTHS


def test_fallback_reason_values_are_the_reference_counter_keys():
    assert len(FallbackReason) == 24
    assert FallbackReason.NONE.value == "none" and FallbackReason("graph_capture") is FallbackReason.GRAPH_CAPTURE


def test_plans_are_immutable_and_ids_increase():
    a, b = plan4096(), plan4096()
    assert b.plan_id > a.plan_id
    with pytest.raises(Exception):
        a.direct = False  # frozen dataclass


# ------------------------------------------------------------------- stats

@pytest.fixture
def stats():
    s = TriangleMixRuntimeStats()
    s.configure(4)
    return s


def test_plan_is_counted_once_across_layers(stats):
    plan = plan4096()
    stats.record_planner_decision(plan)
    stats.record_planner_decision(plan)
    snap = stats.snapshot()
    assert snap["counters"]["request_total"] == 1 and snap["counters"]["request_planner_eligible"] == 1
    assert snap["performance"]["planner_eligibility_rate"] == 1.0


def test_runtime_outcome_cannot_override_planner_result(stats):
    plan = plan4096()
    stats.record_planner_decision(plan)
    stats.record_layer_fallback(plan_id=plan.plan_id, layer_index=3, reason=FallbackReason.STATIC_CAPABILITY,
                                request_indices=(0,))
    snap = stats.snapshot()
    assert snap["counters"]["request_planner_eligible"] == 1 and snap["fallback_reasons"] == {}
    request = snap["recent"][0]["requests"][0]
    assert request["reason"] == "none" and request["execution"]["observed_route"] == "all_fia"
    assert snap["counters"]["layer_fia_reason:static_capability"] == 1


def test_layer_and_host_enqueue_performance_counters(stats):
    stats.record_layer_dispatch(plan_id=1, layer_index=7, saved_qk=2_000_000, host_enqueue_ns=31_000)
    stats.record_layer_dispatch(plan_id=1, layer_index=7, saved_qk=2_000_000, host_enqueue_ns=41_000)
    stats.record_layer_fallback(layer_index=9, reason=FallbackReason.GRAPH_CAPTURE)
    snap = stats.snapshot()
    assert snap["counters"]["single_launch"] == 2
    assert snap["layers"]["direct"]["7"] == 2 and snap["layers"]["fia"]["9"] == 1
    perf = snap["performance"]
    assert perf["host_enqueue_us_per_launch"] == 36.0 and perf["host_enqueue_us_max"] == 41.0
    assert perf["host_enqueue_timing_scope"] == "host_wall_time_not_device_latency"


def test_recent_links_actual_layers_to_plan_and_request(stats):
    plan = plan4096()
    stats.record_planner_decision(plan)
    stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=3, request_index=0, saved_qk=2_000_000,
                                host_enqueue_ns=31_000)
    stats.record_layer_fallback(plan_id=plan.plan_id, layer_index=5, reason=FallbackReason.ADAPTER_UNAVAILABLE,
                                request_indices=(0,))
    recent = stats.snapshot()["recent"][0]
    ex = recent["execution"]
    assert ex["observed_route"] == "mixed" and ex["layer_direct"] == 1 and ex["layer_fia"] == 1
    assert ex["layer_hit_rate"] == 0.5 and ex["fallback_reasons"] == {"adapter_unavailable": 1}
    assert ex["single_launch"] == 1 and ex["estimated_saved_qk"] == 2_000_000
    assert ex["host_enqueue_ns_total"] == 31_000 and ex["timing_scope"] == "host_enqueue_not_device_latency"
    assert recent["requests"][0]["execution"] == ex
    assert [(e["layer_index"], e["route"], e["reason"], e["request_slots"]) for e in recent["layer_events"]] == [
        (3, "direct", "none", [0]), (5, "fia", "adapter_unavailable", [0])]


def test_recent_updates_are_thread_safe(stats):
    plan = plan4096()
    stats.record_planner_decision(plan)

    def record(i):
        if i % 2 == 0:
            stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=i % 4, request_index=0, saved_qk=100,
                                        host_enqueue_ns=i + 1)
        else:
            stats.record_layer_fallback(plan_id=plan.plan_id, layer_index=i % 4,
                                        reason=FallbackReason.STATIC_CAPABILITY, request_indices=(0,))

    with ThreadPoolExecutor(max_workers=8) as ex:
        list(ex.map(record, range(64)))
    snap = stats.snapshot()
    e = snap["recent"][0]["execution"]
    assert snap["counters"]["layer_direct"] == 32 and snap["counters"]["layer_fia"] == 32
    assert (e["layer_direct"], e["layer_fia"], e["single_launch"]) == (32, 32, 32)
    assert e["estimated_saved_qk"] == 3_200 and e["host_enqueue_ns_total"] == 1_024
    assert e["fallback_reasons"] == {"static_capability": 32}
    assert len(snap["recent"][0]["layer_events"]) == 64


def test_recent_capacity_eviction_and_snapshot_isolation(stats):
    stats.configure(2)
    plans = []
    for _ in range(3):
        p = plan4096()
        plans.append(p)
        stats.record_planner_decision(p)
        stats.record_layer_dispatch(plan_id=p.plan_id, layer_index=3, request_index=0, saved_qk=100,
                                    host_enqueue_ns=10)
    snap = stats.snapshot()
    assert [e["plan_id"] for e in snap["recent"]] == [plans[1].plan_id, plans[2].plan_id]
    snap["recent"][0]["execution"]["layer_direct"] = 999
    assert stats.snapshot()["recent"][0]["execution"]["layer_direct"] == 1
    stats.record_layer_fallback(plan_id=plans[0].plan_id, layer_index=5, reason=FallbackReason.STATIC_CAPABILITY,
                                request_indices=(0,))
    assert [e["plan_id"] for e in stats.snapshot()["recent"]] == [plans[1].plan_id, plans[2].plan_id]
    stats.configure(1)
    assert [e["plan_id"] for e in stats.snapshot()["recent"]] == [plans[2].plan_id]
    stats.configure(0)
    assert stats.snapshot()["recent"] == []


def test_per_plan_layer_event_sample_is_bounded(stats):
    plan = plan4096()
    stats.record_planner_decision(plan)
    for layer in range(300):
        stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=layer, request_index=0, saved_qk=100,
                                    host_enqueue_ns=10)
    snap = stats.snapshot()
    recent = snap["recent"][0]
    assert len(recent["layer_events"]) == stats_module.EVENTS_PER_PLAN == 256
    assert recent["execution"]["layer_direct"] == 300
    assert recent["execution"]["layer_events_dropped"] == 44
    assert recent["requests"][0]["execution"]["layer_events_dropped"] == 44
    assert snap["counters"]["recent_layer_events_dropped"] == 44


def test_reset_clears_every_counter_family(stats):
    plan = plan4096()
    stats.record_planner_decision(plan)
    stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=3, saved_qk=100, host_enqueue_ns=10)
    stats.record_runtime_error(stage="dispatch")
    snap = stats.snapshot(reset=True)
    assert snap["counters"]["runtime_error"] == 1 and len(snap["recent"]) == 1
    after = stats.snapshot()
    assert after["counters"] == {} and after["fallback_reasons"] == {}
    assert after["layers"] == {"direct": {}, "fia": {}} and after["recent"] == []


def test_missing_batch_metadata_is_not_a_phantom_request(stats):
    plan = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=None, seq_lens=None,
                            prompt_lens=None, num_decodes=0, num_prefills=0, config=config())
    stats.record_planner_decision(plan)
    snap = stats.snapshot()
    assert snap["counters"]["request_total"] == 0
    assert snap["counters"].get("request_planner_ineligible", 0) == 0
    assert snap["fallback_reasons"] == {} and snap["recent"][0]["requests"] == []


def test_structured_log_interval_is_compact_and_worker_local(stats):
    stats.configure(4, log_interval=2)
    payload = None
    for _ in range(2):
        stats.record_planner_decision(plan4096())
        candidate = stats.structured_log_if_due()
        if candidate is not None:
            payload = candidate
    assert payload is not None
    assert payload["event"] == "trianglemix_runtime_stats" and payload["scope"] == "worker_local"
    assert payload["request_boundary"] == 2 and payload["stats"]["counters"]["request_total"] == 2
    assert "recent" not in payload["stats"]
    assert stats.structured_log_if_due() is None


def test_structured_log_is_independent_of_recent_retention(stats):
    stats.configure(0, log_interval=1)
    plan = plan4096()
    stats.record_planner_decision(plan)
    stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=3, request_index=0, saved_qk=2_000_000,
                                host_enqueue_ns=31_000)
    payload = stats.structured_log_if_due()
    assert [d["kind"] for d in payload["recent_delta"]] == ["planner", "layer_execution"]
    assert payload["recent_delta"][1]["request_slots"] == [0]
    assert stats.snapshot()["recent"] == []
    text = repr(payload["recent_delta"])
    for forbidden in ("prompt_len", "seq_len", "q_begin", "q_end", "token_id", "token_ids"):
        assert forbidden not in text


def test_boundary_plan_layers_emit_supplemental_deltas(stats):
    stats.configure(4, log_interval=1)
    plan = plan4096()
    stats.record_planner_decision(plan)
    boundary = stats.structured_log_if_due()
    assert boundary["request_boundary"] == 1 and [d["kind"] for d in boundary["recent_delta"]] == ["planner"]
    stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=3, request_index=0, saved_qk=2_000_000,
                                host_enqueue_ns=31_000)
    direct = stats.structured_log_if_due()
    assert direct["request_boundary"] == 1 and [d["kind"] for d in direct["recent_delta"]] == ["layer_execution"]
    assert direct["recent_delta"][0]["route"] == "direct"
    stats.record_layer_fallback(plan_id=plan.plan_id, layer_index=5, reason=FallbackReason.ADAPTER_UNAVAILABLE,
                                request_indices=(0,))
    fallback = stats.structured_log_if_due()
    assert fallback["request_boundary"] == 1 and fallback["recent_delta"][0]["reason"] == "adapter_unavailable"
    assert fallback["delta_mode"] == "incremental_not_final_plan_snapshot"


def test_structured_delta_capacity_and_reset(stats):
    stats.configure(0, log_interval=1)
    plan = plan4096()
    with patch.object(stats_module, "LOG_BUFFER", 2):
        stats.record_planner_decision(plan)
        stats.record_layer_dispatch(plan_id=plan.plan_id, layer_index=3, request_index=0, saved_qk=2_000_000,
                                    host_enqueue_ns=31_000)
        stats.record_layer_fallback(plan_id=plan.plan_id, layer_index=5,
                                    reason=FallbackReason.ADAPTER_UNAVAILABLE, request_indices=(0,))
        payload = stats.structured_log_if_due()
    assert len(payload["recent_delta"]) == 2
    assert all(d["kind"] == "layer_execution" for d in payload["recent_delta"])
    assert payload["stats"]["counters"]["structured_log_deltas_dropped"] == 1
    stats.record_planner_decision(plan4096())
    assert stats.snapshot(reset=True)["counters"]["request_total"] == 2
    assert stats.structured_log_if_due() is None
    assert stats.snapshot()["counters"] == {}
