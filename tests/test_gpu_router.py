"""The routing layer on the GPU, and its structured counter log.

A four-layer stack (layers 1 and 3 selected) runs the eight 512-token chunks
of a 4096-token prompt through ``TriangleMixRouter`` with the real gfx950
ops.  Checks:

* each layer's output is bit-identical to the op the planner chose for it
  (the sparse op for a selected layer on a direct plan, the dense companion
  otherwise), called directly on the same inputs, and the sparse outputs match
  the fp32 oracle on one middle chunk;
* the counters agree with the plans (one launch per selected layer and direct
  plan, the planner's reasons for the rest);
* the router's structured log lines, parsed back by ``trianglemix.counters``,
  aggregate to exactly the stats snapshot with no schema, regression or
  invariant finding.
"""

from __future__ import annotations

import logging

import pytest
import torch

from oracle import attention as OA
from trianglemix import counters as C
from trianglemix.config import resolve_plugin_config
from trianglemix.planning import build_batch_plan
from trianglemix.router import TriangleMixRouter
from trianglemix.stats import TriangleMixRuntimeStats
from trianglemix.workload import SCALE, make_cache, make_query, prompt_chunks

pytestmark = pytest.mark.gpu

L, CHUNK, LAYERS, SELECTED = 4096, 512, 4, (1, 3)


class _Lines(logging.Handler):
    def __init__(self):
        super().__init__()
        self.lines = []

    def emit(self, record):
        self.lines.append("INFO trianglemix.router " + record.getMessage())


class _Vllm:
    additional_config = {"trianglemix": {"enabled": True, "layers": ",".join(map(str, SELECTED)),
                                         "stats_log_interval": 2}}


def test_router_stack_outputs_and_log(gpu):
    cfg = resolve_plugin_config(_Vllm())
    caches = [make_cache(L, 40 + i, std=1.0) for i in range(LAYERS)]
    queries = [make_query(L, 60 + i, std=1.0) for i in range(LAYERS)]
    dev_caches = [(k.to(gpu), v.to(gpu), bt.to(gpu)) for k, v, bt in caches]
    dev_q = [q.to(gpu) for q in queries]
    outs = [torch.full_like(q, float("nan")) for q in dev_q]
    stats = TriangleMixRuntimeStats()
    router = TriangleMixRouter(cfg, stats=stats)
    handler = _Lines()
    log = logging.getLogger("trianglemix.router")
    log.addHandler(handler)
    old = log.level
    log.setLevel(logging.INFO)
    plans = []
    try:
        for c in prompt_chunks(L, CHUNK):
            plan = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[c.query_tokens],
                                    seq_lens=[c.seq_len], prompt_lens=[L], num_decodes=0, num_prefills=1,
                                    config=cfg.kernel)
            plans.append((c, plan))
            for i in range(LAYERS):
                k, v, bt = dev_caches[i]
                router.prefill_attention(layer_name=f"model.layers.{i}.self_attn.attn", plan=plan,
                                         query=dev_q[i][c.query_start:c.seq_len], key_cache=k, value_cache=v,
                                         block_table=bt, output=outs[i][c.query_start:c.seq_len],
                                         softmax_scale=SCALE)
        torch.cuda.synchronize()
    finally:
        log.removeHandler(handler)
        log.setLevel(old)

    direct_plans = 0
    for c, plan in plans:
        direct_plans += plan.direct
        for i in range(LAYERS):
            k, v, bt = dev_caches[i]
            q = dev_q[i][c.query_start:c.seq_len]
            want = torch.full_like(q, float("nan"))
            if i in SELECTED and plan.direct:
                torch.ops.trianglemix.triangle_paged_sparse_attention.out(
                    q, k, v, bt, c.query_start, c.seq_len, L, SCALE, out=want)
            else:
                torch.ops.trianglemix.dense_paged_causal_attention.out(
                    q, k, v, bt, c.query_start, c.seq_len, SCALE, out=want)
            torch.cuda.synchronize()
            got = outs[i][c.query_start:c.seq_len]
            assert torch.equal(got, want), (c.query_start, i)
    assert 0 < direct_plans < len(plans)

    # one middle chunk of a selected layer against the fp32 oracle
    c, plan = next((c, p) for c, p in plans if p.direct)
    k, v, bt = caches[SELECTED[0]]
    q = queries[SELECTED[0]][c.query_start:c.seq_len]
    expected = OA.attention_torch(q, k, v, bt, c.query_start, c.seq_len, L, SCALE)
    m = OA.error_metrics(outs[SELECTED[0]][c.query_start:c.seq_len].float().cpu().numpy(), expected.float().numpy())
    assert m["max_abs"] <= 2e-2 and m["mean_abs"] <= 2e-3, m

    snap = stats.snapshot()
    counters = snap["counters"]
    assert counters["single_launch"] == len(SELECTED) * direct_plans
    assert counters["layer_fia"] == len(SELECTED) * (len(plans) - direct_plans)
    assert counters["request_total"] == len(plans)

    report = C.aggregate(C.scan_events("\n".join(handler.lines), source="worker0.log"))
    print({k: report[k] for k in ("event_count", "worker_count")}, flush=True)
    assert C.report_status(report) == "PASS", report
    assert report["aggregate"]["counters"] == counters
    assert report["aggregate"]["fallback_reasons"] == snap["fallback_reasons"]
    assert report["aggregate"]["layers"] == snap["layers"]
