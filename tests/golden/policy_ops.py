"""Replayable scenario for the TriangleMix policy layer (planning, stats, config).

One interpreter drives a fixed list of operations against a ``planning`` /
``stats`` / ``config`` module triple and returns every observable result in
JSON form.  ``make_policy_snapshots.py`` runs it against the reference
package (package/src/vllm_ascend_trianglemix/) to write
``policy_snapshots.json``; ``tests/test_policy_golden.py`` runs it against
this build's modules and compares.  Only the scenario (inputs) lives here;
the expected outputs live in the JSON.

Non-deterministic fields are pinned or normalised: plans get fixed
``plan_id`` / ``routing_ns`` (``dataclasses.replace``), and the structured
log's worker ``pid`` is replaced by a marker.
"""

from __future__ import annotations

import dataclasses
import os
from contextlib import contextmanager
from typing import Any

# --------------------------------------------------------------------- planning
# build_batch_plan inputs (keyword form); the config is the default kernel
# config with every layer selected unless a case overrides fields.
PLAN_CASES: list[dict[str, Any]] = [
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [8192]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [512], "prompt_lens": [8192]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [8192], "prompt_lens": [8192]},
    {"state_name": "PrefillNoCache", "cumulative_query_ends": [2869], "seq_lens": [2869], "prompt_lens": [2869]},
    {"state_name": "PrefillCacheHit", "cumulative_query_ends": [512], "seq_lens": [2869], "prompt_lens": [2869]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [2048], "seq_lens": [8320], "prompt_lens": [8320]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [64], "seq_lens": [1100], "prompt_lens": [4096]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [300], "seq_lens": [900], "prompt_lens": [1000]},
    {"state_name": "DecodeOnly", "cumulative_query_ends": [1], "seq_lens": [4096], "prompt_lens": [4000]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [8192],
     "num_decodes": 1},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [100, 300], "seq_lens": [1000, 2000],
     "prompt_lens": [1000, 2000], "num_prefills": 2},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [100], "seq_lens": [1000, 2000],
     "prompt_lens": [1000], "num_prefills": 2},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": None, "seq_lens": [4096], "prompt_lens": None},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [], "seq_lens": [], "prompt_lens": [],
     "num_prefills": 0},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [4000]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [0], "seq_lens": [4608], "prompt_lens": [8192]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [600], "seq_lens": [500], "prompt_lens": [8192]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [8192],
     "config": {"sink_tokens": 4}},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [8192],
     "config": {"direct_min_seq_len": 5000}},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [8192],
     "config": {"direct_min_sparse_rows": 600}},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [2048], "seq_lens": [8320], "prompt_lens": [8320],
     "config": {"direct_split_min_sparse_rows": 4096}},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [2048], "seq_lens": [8320], "prompt_lens": [8320],
     "config": {"direct_split_min_saved_qk": 10**12}},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [700], "seq_lens": [1300], "prompt_lens": [1400]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [100, 200], "seq_lens": [1000], "prompt_lens": [1000]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [512], "seq_lens": [4608], "prompt_lens": [8192],
     "num_prefills": 2},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [100], "seq_lens": [1000],
     "prompt_lens": [1000, 2000]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [-5], "seq_lens": [1000], "prompt_lens": [1000]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": [300, 100, 250], "seq_lens": [900, 800, 700],
     "prompt_lens": [900, 800], "num_prefills": 3},
    {"state_name": "PrefillNoCache", "cumulative_query_ends": [8192], "seq_lens": [8192], "prompt_lens": [8192]},
    {"state_name": "ChunkedPrefill", "cumulative_query_ends": ["512"], "seq_lens": [4608.0], "prompt_lens": [8192]},
]


def _kernel_config(mods, overrides: dict[str, Any] | None):
    fields = {"enabled": True, "layer_indices": frozenset(range(64))}
    fields.update(overrides or {})
    return mods.kernel.TriangleMixConfig(**fields)


def _plan_inputs(mods, case: dict[str, Any]) -> dict[str, Any]:
    args = {k: v for k, v in case.items() if k != "config"}
    args.setdefault("num_decodes", 0)
    args.setdefault("num_prefills", 1)
    args["config"] = _kernel_config(mods, case.get("config"))
    return args


def plan_record(plan) -> dict[str, Any]:
    """A plan in JSON form (plan_id and routing_ns left out: they are per run)."""
    return {
        "state_name": plan.state_name,
        "batch_size": plan.batch_size,
        "direct": plan.direct,
        "primary_reason": plan.primary_reason.value,
        "requests": [{
            "request_index": r.request_index, "q_begin": r.q_begin, "q_end": r.q_end, "seq_len": r.seq_len,
            "prompt_len": r.prompt_len, "eligible": r.eligible, "reason": r.reason.value,
            "query_len": r.query_len, "saved_qk": r.saved_qk,
            "span": None if r.span is None else dataclasses.asdict(r.span),
        } for r in plan.requests],
    }


def run_planning(mods) -> list[dict[str, Any]]:
    return [plan_record(mods.planning.build_batch_plan(**_plan_inputs(mods, case))) for case in PLAN_CASES]


# ------------------------------------------------------------------------ stats
# Named plans for the stats scenario: (PLAN_CASES index, plan_id, routing_ns).
STATS_PLANS = {
    "direct": (0, 101, 1500),
    "first_chunk": (1, 102, 900),
    "last_chunk": (2, 103, 1100),
    "batch2": (10, 104, 2000),
    "decode": (8, 105, 700),
    "mixed": (9, 106, 800),
    "no_metadata": (12, 107, 600),
    "empty": (13, 108, 500),
    "short": (6, 109, 400),
}


def stats_ops() -> list[dict[str, Any]]:
    """The stats scenario: every public entry point, the log cadence, every bounded container."""
    R = "reason"
    ops: list[dict[str, Any]] = [
        {"op": "configure", "recent_capacity": 3, "log_interval": 2},
        {"op": "planner", "plan": "direct"},
        {"op": "dispatch", "plan": "direct", "layer_index": 5, "saved_qk": 1000, "host_enqueue_ns": 1200},
        {"op": "dispatch", "plan": "direct", "layer_index": 7, "saved_qk": 1000, "host_enqueue_ns": 3400},
        {"op": "fallback", "plan": "direct", "layer_index": 10, R: "direct_launch_error", "request_indices": [0]},
        {"op": "log"},
        {"op": "planner", "plan": "first_chunk"},
        {"op": "fallback", "plan": "first_chunk", "layer_index": 5, R: "no_sparse_middle", "request_indices": [0]},
        {"op": "log"},
        {"op": "dispatch", "plan": "direct", "layer_index": 15, "saved_qk": 1000, "host_enqueue_ns": 800},
        {"op": "log"},
        {"op": "fallback", "plan": "first_chunk", "layer_index": 7, R: "no_sparse_middle", "request_indices": [0]},
        {"op": "log"},
        {"op": "planner", "plan": "direct"},
        {"op": "planner", "plan": "batch2"},
        {"op": "fallback", "plan": "batch2", "layer_index": 5, R: "batch_unsupported", "request_indices": [1, 0, 1]},
        {"op": "fallback", "plan": "batch2", "layer_index": 7, R: "batch_unsupported", "request_indices": [3]},
        {"op": "log"},
        {"op": "log"},
        {"op": "error", "stage": "launch"},
        {"op": "error", "stage": "launch"},
        {"op": "error", "stage": "plan"},
        {"op": "snapshot", "reset": False},
        {"op": "configure", "recent_capacity": 1, "log_interval": 2},
        {"op": "snapshot", "reset": False},
        {"op": "planner", "plan": "decode"},
        {"op": "planner", "plan": "mixed"},
        {"op": "planner", "plan": "no_metadata"},
        {"op": "planner", "plan": "empty"},
        {"op": "fallback", "plan": "empty", "layer_index": None, R: "missing_metadata", "request_indices": []},
        {"op": "fallback", "plan": None, "layer_index": None, R: "graph_capture", "request_indices": [0]},
        {"op": "fallback", "plan": None, "layer_index": 12, R: "adapter_unavailable"},
        {"op": "log"},
        {"op": "planner", "plan": "last_chunk"},
        {"op": "dispatch_many", "plan": "last_chunk", "count": 260, "saved_qk": 7, "host_enqueue_ns": 10},
        {"op": "fallback", "plan": "last_chunk", "layer_index": 3, R: "static_capability", "request_indices": [0]},
        {"op": "log_digest"},
        {"op": "snapshot_digest", "reset": False},
        {"op": "configure", "recent_capacity": 4, "log_interval": 5},
        {"op": "planner", "plan": "short"},
        {"op": "dispatch", "plan": "short", "layer_index": None, "saved_qk": 0, "host_enqueue_ns": 50,
         "request_index": 2},
        {"op": "log"},
        {"op": "snapshot_digest", "reset": True},
        {"op": "snapshot", "reset": False},
        {"op": "log"},
        {"op": "planner", "plan": "direct"},
        {"op": "log"},
        {"op": "configure", "recent_capacity": 0, "log_interval": 0},
        {"op": "planner", "plan": "first_chunk"},
        {"op": "dispatch", "plan": "first_chunk", "layer_index": 9, "saved_qk": 5, "host_enqueue_ns": 5},
        {"op": "log"},
        {"op": "snapshot", "reset": False},
        {"op": "configure_error", "recent_capacity": -1, "log_interval": 0},
        {"op": "configure_error", "recent_capacity": 0, "log_interval": -3},
        # bounded containers: the delta buffer (8192) and the seen-plan set (8192)
        {"op": "configure", "recent_capacity": 2, "log_interval": 2},
        {"op": "planner", "plan": "last_chunk"},
        {"op": "dispatch_many", "plan": "last_chunk", "count": 8200, "saved_qk": 1, "host_enqueue_ns": 1},
        {"op": "planner", "plan": "decode"},
        {"op": "log_digest"},
        {"op": "counters"},
        {"op": "snapshot_digest", "reset": True},
        {"op": "configure", "recent_capacity": 2, "log_interval": 0},
        {"op": "planner_many", "plan": "direct", "first_id": 20000, "count": 8193},
        {"op": "counters"},
        {"op": "planner", "plan": "direct", "plan_id": 20000},
        {"op": "planner", "plan": "direct", "plan_id": 28192},
        {"op": "counters"},
    ]
    return ops


@contextmanager
def _clean_worker_env():
    saved = {k: os.environ.pop(k) for k in ("RANK", "LOCAL_RANK") if k in os.environ}
    try:
        yield
    finally:
        os.environ.update(saved)


def _normalise_log(payload):
    if payload is not None and isinstance(payload.get("worker"), dict) and "pid" in payload["worker"]:
        payload["worker"]["pid"] = "<pid>"
    return payload


def run_stats(mods) -> list[Any]:
    """Results of every op of ``stats_ops()`` in order (None for ops that return nothing)."""
    plans = {}
    for name, (case, plan_id, routing_ns) in STATS_PLANS.items():
        plan = mods.planning.build_batch_plan(**_plan_inputs(mods, PLAN_CASES[case]))
        plans[name] = dataclasses.replace(plan, plan_id=plan_id, routing_ns=routing_ns)
    reason = mods.planning.FallbackReason
    stats = mods.stats.TriangleMixRuntimeStats()
    out: list[Any] = []
    with _clean_worker_env():
        for op in stats_ops():
            kind = op["op"]
            result: Any = None
            if kind == "configure":
                stats.configure(op["recent_capacity"], op["log_interval"])
            elif kind == "configure_error":
                try:
                    stats.configure(op["recent_capacity"], op["log_interval"])
                    result = "no error"
                except ValueError as exc:
                    result = f"ValueError: {exc}"
            elif kind == "planner":
                plan = plans[op["plan"]]
                if "plan_id" in op:
                    plan = dataclasses.replace(plan, plan_id=op["plan_id"])
                stats.record_planner_decision(plan)
            elif kind == "planner_many":
                for i in range(op["count"]):
                    stats.record_planner_decision(dataclasses.replace(plans[op["plan"]], plan_id=op["first_id"] + i))
            elif kind == "dispatch":
                stats.record_layer_dispatch(plan_id=plans[op["plan"]].plan_id, layer_index=op["layer_index"],
                                            saved_qk=op["saved_qk"], host_enqueue_ns=op["host_enqueue_ns"],
                                            request_index=op.get("request_index", 0))
            elif kind == "dispatch_many":
                for i in range(op["count"]):
                    stats.record_layer_dispatch(plan_id=plans[op["plan"]].plan_id, layer_index=i % 40,
                                                saved_qk=op["saved_qk"], host_enqueue_ns=op["host_enqueue_ns"] + i)
            elif kind == "fallback":
                kwargs = {"layer_index": op["layer_index"], "reason": reason(op["reason"])}
                if op["plan"] is not None:
                    kwargs["plan_id"] = plans[op["plan"]].plan_id
                if "request_indices" in op:
                    kwargs["request_indices"] = tuple(op["request_indices"])
                stats.record_layer_fallback(**kwargs)
            elif kind == "error":
                stats.record_runtime_error(stage=op["stage"])
            elif kind == "log":
                result = _normalise_log(stats.structured_log_if_due())
            elif kind == "log_digest":
                payload = _normalise_log(stats.structured_log_if_due())
                if payload is not None:
                    deltas = payload.pop("recent_delta")
                    payload["recent_delta_len"] = len(deltas)
                    payload["recent_delta_first"] = deltas[:2]
                    payload["recent_delta_last"] = deltas[-2:]
                result = payload
            elif kind == "snapshot":
                result = stats.snapshot(reset=op["reset"])
            elif kind == "snapshot_digest":
                # a snapshot whose long per-plan event lists keep their length, first and last three
                result = stats.snapshot(reset=op["reset"])
                for entry in result.get("recent", []):
                    events = entry["layer_events"]
                    entry["layer_events"] = {"len": len(events), "first": events[:3], "last": events[-3:]}
            elif kind == "counters":
                result = stats.snapshot(reset=False)["counters"]
            else:
                raise ValueError(f"unknown op {kind}")
            out.append(result)
    return out


# ----------------------------------------------------------------------- config
_ENV_KEYS = (
    "VLLM_ASCEND_ENABLE_TRIANGLE_MIX", "VLLM_ASCEND_TRIANGLE_MIX_LAYERS", "VLLM_ASCEND_TRIANGLE_MIX_SINK_TOKENS",
    "VLLM_ASCEND_TRIANGLE_MIX_LOCAL_WINDOW", "VLLM_ASCEND_TRIANGLE_MIX_LAST_ROWS",
    "VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SEQ_LEN", "VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SPARSE_ROWS",
    "VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SAVED_QK", "VLLM_ASCEND_TRIANGLE_MIX_DIRECT_SPLIT_MIN_SPARSE_ROWS",
    "VLLM_ASCEND_TRIANGLE_MIX_DIRECT_SPLIT_MIN_SAVED_QK", "VLLM_ASCEND_TRIANGLE_MIX_STATS_RECENT_CAPACITY",
    "VLLM_ASCEND_TRIANGLE_MIX_STATS_LOG_INTERVAL", "VLLM_ASCEND_TRIANGLE_MIX_STRICT",
    "VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE",
)

CONFIG_CASES: list[dict[str, Any]] = [
    {"additional_config": None, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": True, "layers": "5,7,10,15-35"}}, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": "yes", "layers": [3, 1, 2]}}, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": 1, "layers": (4,), "strict": "off"}}, "env": {}},
    {"additional_config": {"enabled": "true", "layers": "0-3"}, "env": {}},
    {"additional_config": {"trianglemix": "not a mapping"}, "env": {"VLLM_ASCEND_ENABLE_TRIANGLE_MIX": "1"}},
    {"additional_config": None, "env": {"VLLM_ASCEND_ENABLE_TRIANGLE_MIX": " On ",
                                        "VLLM_ASCEND_TRIANGLE_MIX_LAYERS": "1,2",
                                        "VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SAVED_QK": "77",
                                        "VLLM_ASCEND_TRIANGLE_MIX_STATS_LOG_INTERVAL": "16",
                                        "VLLM_ASCEND_TRIANGLE_MIX_STRICT": "no"}},
    {"additional_config": {"trianglemix": {"enabled": True, "layers": "2", "min_saved_qk": 5}},
     "env": {"VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SAVED_QK": "77"}},
    {"additional_config": {"trianglemix": {"enabled": True, "layers": "2", "sink_tokens": "16",
                                           "local_window": 256.0, "last_rows": 64, "min_seq_len": 100,
                                           "min_sparse_rows": 1, "split_min_sparse_rows": 2,
                                           "split_min_saved_qk": 3, "stats_recent_capacity": 0}}, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": "maybe"}}, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": 2}}, "env": {}},
    {"additional_config": None, "env": {"VLLM_ASCEND_ENABLE_TRIANGLE_MIX": "sometimes"}},
    {"additional_config": {"trianglemix": {"strict": None}}, "env": {}},
    {"additional_config": {"trianglemix": {"stats_log_interval": -1}}, "env": {}},
    {"additional_config": None, "env": {"VLLM_ASCEND_TRIANGLE_MIX_STATS_RECENT_CAPACITY": "-5"}},
    {"additional_config": None, "env": {"VLLM_ASCEND_TRIANGLE_MIX_SINK_TOKENS": "eight"}},
    {"additional_config": {"trianglemix": {"sink_tokens": 0}}, "env": {}},
    {"additional_config": {"trianglemix": {"layers": "1-"}}, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": "maybe", "layers": "x"}}, "env": {}},
    {"additional_config": {"trianglemix": {"enabled": True, "layers": ""}}, "env": {}},
]


@contextmanager
def _env(values: dict[str, str]):
    saved = {k: os.environ.pop(k) for k in _ENV_KEYS if k in os.environ}
    os.environ.update(values)
    try:
        yield
    finally:
        for k in _ENV_KEYS:
            os.environ.pop(k, None)
        os.environ.update(saved)


def config_record(cfg) -> dict[str, Any]:
    kernel = dataclasses.asdict(cfg.kernel)
    kernel["layer_indices"] = sorted(kernel["layer_indices"])
    return {"kernel": kernel, "strict": cfg.strict, "stats_recent_capacity": cfg.stats_recent_capacity,
            "stats_log_interval": cfg.stats_log_interval, "enabled": cfg.enabled}


class _VllmConfig:
    def __init__(self, additional):
        self.additional_config = additional


def run_config(mods) -> list[dict[str, Any]]:
    results = []
    for case in CONFIG_CASES:
        with _env(case["env"]):
            try:
                results.append(config_record(mods.config.resolve_plugin_config(_VllmConfig(case["additional_config"]))))
            except Exception as exc:  # the error type and message are the contract
                results.append({"error": f"{type(exc).__name__}: {exc}"})
    return results
