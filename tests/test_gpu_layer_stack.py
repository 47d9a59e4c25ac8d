"""BASELINE config 5 on the GPU: the 36-layer layer-selective prefill stack.

36 attention layers at Qwen3-8B geometry, each with its own random Q / K / V
(N(0,1) bf16, its own random page table), one 8192-token request in chunks of
512, through ``TriangleMixRouter`` with the reference's default gates and the
layer list ``5,7,10,15-35`` (24 selected layers).  The reference gates its
engine runs on the same counters (release_validation/model_smoke.py:582-1148)
and pins the chunk routes of a prompt by known answers
(package/tests/test_planning_stats.py:122-151).  Checks:

* every layer's output of every chunk is bit-identical to the op its route
  names (the sparse op for a selected layer on a direct plan, the dense
  companion otherwise), called directly on the same inputs;
* the counters agree with the plans: ``single_launch`` = 24 x direct plans,
  ``layer_fia`` and the ``layer_fia_reason:*`` counters = 24 x each fallback
  plan's reason, per-layer maps exact;
* one chunk of a selected layer on the sparse route and one chunk of an
  unselected layer (dense companion) match the fp32 oracle;
* the router's structured log aggregates to exactly the stats snapshot.
"""

from __future__ import annotations

import logging
from collections import Counter

import pytest
import torch

from oracle import attention as OA
from trianglemix import counters as C
from trianglemix.config import resolve_plugin_config
from trianglemix.kernel import parse_layer_indices
from trianglemix.planning import build_batch_plan
from trianglemix.router import TriangleMixRouter
from trianglemix.stats import TriangleMixRuntimeStats
from trianglemix.workload import SCALE, noncontiguous_block_table, prompt_chunks

pytestmark = pytest.mark.gpu

L, CHUNK, LAYERS, LAYER_SPEC = 8192, 512, 36, "5,7,10,15-35"
SELECTED = parse_layer_indices(LAYER_SPEC)


class _Lines(logging.Handler):
    def __init__(self):
        super().__init__()
        self.lines = []

    def emit(self, record):
        self.lines.append("INFO trianglemix.router " + record.getMessage())


class _Vllm:
    additional_config = {"trianglemix": {"enabled": True, "layers": LAYER_SPEC, "stats_log_interval": 16}}


def _layer_inputs(gpu, i):
    """Q [L, 32, 128] and a paged K/V cache with a random page table for layer i (seeded)."""
    g = torch.Generator(device=gpu).manual_seed(1000 + i)
    pages = L // 128
    bt = noncontiguous_block_table(pages, pages + 7, torch.Generator().manual_seed(2000 + i))
    k = torch.randn((pages + 7, 128, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn((pages + 7, 128, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn((L, 32, 128), generator=g, device=gpu).to(torch.bfloat16)
    return q, k, v, bt.to(gpu)


def test_config5_layer_stack(gpu):
    assert len(SELECTED) == 24
    cfg = resolve_plugin_config(_Vllm())
    inputs = [_layer_inputs(gpu, i) for i in range(LAYERS)]
    outs = [torch.full_like(q, float("nan")) for q, _, _, _ in inputs]
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
            for i, (q, k, v, bt) in enumerate(inputs):
                router.prefill_attention(layer_name=f"model.layers.{i}.self_attn.attn", plan=plan,
                                         query=q[c.query_start:c.seq_len], key_cache=k, value_cache=v,
                                         block_table=bt, output=outs[i][c.query_start:c.seq_len],
                                         softmax_scale=SCALE)
        torch.cuda.synchronize()
    finally:
        log.removeHandler(handler)
        log.setLevel(old)

    direct = [c for c, plan in plans if plan.direct]
    fallback = Counter(plan.primary_reason.value for _, plan in plans if not plan.direct)
    print(f"{len(direct)} direct chunk plans, fallbacks {dict(fallback)}", flush=True)
    assert 0 < len(direct) < len(plans)

    # every output is the op its route names, bit for bit
    for c, plan in plans:
        for i, (q, k, v, bt) in enumerate(inputs):
            qc = q[c.query_start:c.seq_len]
            want = torch.full_like(qc, float("nan"))
            if i in SELECTED and plan.direct:
                torch.ops.trianglemix.triangle_paged_sparse_attention.out(
                    qc, k, v, bt, c.query_start, c.seq_len, L, SCALE, out=want)
            else:
                torch.ops.trianglemix.dense_paged_causal_attention.out(
                    qc, k, v, bt, c.query_start, c.seq_len, SCALE, out=want)
            torch.cuda.synchronize()
            assert torch.equal(outs[i][c.query_start:c.seq_len], want), (c.query_start, i)

    # counters against the plans
    snap = stats.snapshot()
    counters = snap["counters"]
    assert counters["single_launch"] == len(SELECTED) * len(direct)
    assert counters["layer_direct"] == counters["single_launch"]
    assert counters["layer_fia"] == len(SELECTED) * (len(plans) - len(direct))
    for reason, n in fallback.items():
        assert counters[f"layer_fia_reason:{reason}"] == len(SELECTED) * n, reason
    assert sum(v for k, v in counters.items() if k.startswith("layer_fia_reason:")) == counters["layer_fia"]
    assert counters["request_total"] == len(plans)
    for i in SELECTED:
        assert snap["layers"]["direct"].get(str(i), 0) == len(direct)
    assert all(int(i) in SELECTED for i in snap["layers"]["direct"])

    # one sparse-route chunk and one dense-companion chunk against the fp32 oracle
    c = direct[len(direct) // 2]
    for i, dense in ((min(SELECTED), False), (0, True)):
        q, k, v, bt = inputs[i]
        qc = q[c.query_start:c.seq_len].cpu()
        expected = OA.attention_torch(qc, k.cpu(), v.cpu(), bt.cpu(), c.query_start, c.seq_len, L, SCALE,
                                      dense=dense)
        m = OA.error_metrics(outs[i][c.query_start:c.seq_len].float().cpu().numpy(), expected.float().numpy())
        print(f"layer {i} chunk {c.query_start} dense={dense}: {m}", flush=True)
        assert m["max_abs"] <= 2e-2 and m["mean_abs"] <= 2e-3 and m["relative_l2"] <= 2e-2, (i, m)

    # the structured counter log adds up to the snapshot
    report = C.aggregate(C.scan_events("\n".join(handler.lines), source="worker0.log"))
    assert C.report_status(report) == "PASS", report
    assert report["aggregate"]["counters"] == counters
    assert report["aggregate"]["fallback_reasons"] == snap["fallback_reasons"]
