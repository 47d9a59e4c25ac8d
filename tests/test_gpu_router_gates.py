"""The router's gates on GPU tensors: the fast paths equal the generic predicates.

``router.dispatch_reason`` checks torch tensors whose query is on a GPU in
one native call (the adapter's ``tensor_gate``; ``_tensor_reason`` is the
same gates in Python, for an adapter without that module) and everything
else through ``_query_reason`` / ``_kv_reason`` /
``_block_table_reason`` (the restatement of the reference's
``_validate_query`` / ``_validate_static_kv`` / ``_validate_block_table``,
plugin.py:1106-1192).  For a well-formed call and for one broken property at
a time -- dtype, shape, row count, contiguity, device, block-table length --
all three must name the same reason.
"""

from __future__ import annotations

import pytest
import torch

from trianglemix import router as R
from trianglemix.config import PluginConfig
from trianglemix.kernel import TriangleMixConfig
from trianglemix.planning import FallbackReason, build_batch_plan

pytestmark = pytest.mark.gpu


def _generic(features, plan, query, output, key_cache, value_cache, block_table):
    for reason in (R._query_reason(features, query, output, plan), R._kv_reason(key_cache, value_cache, query)):
        if reason is not FallbackReason.NONE:
            return reason
    return R._block_table_reason(block_table, query, plan.requests[0].seq_len)


def _variants(dev):
    tq, seq, prompt = 512, 4608, 8192
    pages = 40
    base = dict(query=torch.zeros(tq, 32, 128, dtype=torch.bfloat16, device=dev),
                output=torch.zeros(tq + 16, 32, 128, dtype=torch.bfloat16, device=dev),
                key_cache=torch.zeros(pages, 128, 8, 128, dtype=torch.bfloat16, device=dev),
                value_cache=torch.zeros(pages, 128, 8, 128, dtype=torch.bfloat16, device=dev),
                block_table=torch.zeros(1, 36, dtype=torch.int32, device=dev))
    cases = [("ok", {})]
    cases += [
        ("query fp16", {"query": base["query"].half()}),
        ("query rows", {"query": torch.zeros(tq - 1, 32, 128, dtype=torch.bfloat16, device=dev)}),
        ("query heads", {"query": torch.zeros(tq, 16, 128, dtype=torch.bfloat16, device=dev)}),
        ("query 2-d", {"query": torch.zeros(tq, 32 * 128, dtype=torch.bfloat16, device=dev)}),
        ("query strided", {"query": torch.zeros(tq, 32, 256, dtype=torch.bfloat16, device=dev)[:, :, :128]}),
        ("output short", {"output": torch.zeros(tq - 1, 32, 128, dtype=torch.bfloat16, device=dev)}),
        ("output fp32", {"output": torch.zeros(tq, 32, 128, dtype=torch.float32, device=dev)}),
        ("output cpu", {"output": torch.zeros(tq, 32, 128, dtype=torch.bfloat16)}),
        ("output strided", {"output": torch.zeros(tq, 64, 128, dtype=torch.bfloat16, device=dev)[:, ::2]}),
        ("output 0-d", {"output": torch.zeros((), dtype=torch.bfloat16, device=dev)}),
        ("kv page size", {"key_cache": torch.zeros(pages, 64, 8, 128, dtype=torch.bfloat16, device=dev)}),
        ("kv mismatch", {"value_cache": torch.zeros(pages + 1, 128, 8, 128, dtype=torch.bfloat16, device=dev)}),
        ("kv fp16", {"value_cache": base["value_cache"].half()}),
        ("kv cpu", {"key_cache": base["key_cache"].cpu(), "value_cache": base["value_cache"].cpu()}),
        ("v cpu", {"value_cache": base["value_cache"].cpu()}),
        ("kv strided", {"key_cache": torch.zeros(pages, 128, 16, 128, dtype=torch.bfloat16, device=dev)[:, :, ::2]}),
        ("kv 5-d", {"key_cache": base["key_cache"][None], "value_cache": base["value_cache"][None]}),
        ("table short", {"block_table": torch.zeros(1, 35, dtype=torch.int32, device=dev)}),
        ("table int64", {"block_table": torch.zeros(1, 36, dtype=torch.int64, device=dev)}),
        ("table batch 2", {"block_table": torch.zeros(2, 36, dtype=torch.int32, device=dev)}),
        ("table cpu", {"block_table": torch.zeros(1, 36, dtype=torch.int32)}),
        ("table strided", {"block_table": torch.zeros(1, 72, dtype=torch.int32, device=dev)[:, ::2]}),
    ]
    return base, cases, (tq, seq, prompt)


def test_fast_gates_equal_generic_gates(gpu):
    base, cases, (tq, seq, prompt) = _variants(gpu)
    kcfg = TriangleMixConfig(enabled=True, layer_indices=frozenset({5}))
    config = PluginConfig(kernel=kcfg)
    plan = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[tq], seq_lens=[seq],
                            prompt_lens=[prompt], num_decodes=0, num_prefills=1, config=kcfg)
    assert plan.direct
    features = R.LayerFeatures()
    seen = set()
    from trianglemix.native import routed_fast_path

    fast = routed_fast_path()
    assert fast is not None  # the adapter's routed-call module (dispatch_reason's gate on GPU tensors)
    for name, change in cases:
        t = {**base, **change}
        want = _generic(features, plan, **t)
        got = R.dispatch_reason(config=config, plan=plan, features=features, capturing=False, native_ready=True,
                                **t)
        assert got is want, (name, got, want)
        # the Python restatement of the same gates agrees with the native one
        py = R._tensor_reason(features, t["query"], t["output"], t["key_cache"], t["value_cache"],
                              t["block_table"], tq, seq)
        native = R._GATE_CODES[fast.tensor_gate(t["query"], t["output"], t["key_cache"], t["value_cache"],
                                                t["block_table"], tq, seq)]
        assert py is native is want, (name, py, native, want)
        seen.add(want)
    # the cases reach every tensor reason and the well-formed call passes
    assert seen == {FallbackReason.NONE, FallbackReason.QUERY_UNSUPPORTED, FallbackReason.KV_CACHE_UNSUPPORTED,
                    FallbackReason.BLOCK_TABLE_UNSUPPORTED}
    # the layer's head counts are checked with the query, on both paths
    bad = R.LayerFeatures(num_heads=16)
    assert R.dispatch_reason(config=config, plan=plan, features=bad, capturing=False, native_ready=True,
                             **base) is _generic(bad, plan, **base) is FallbackReason.QUERY_UNSUPPORTED


def test_gfx950_takes_the_mi355x_gate_profile_by_default(gpu):
    """On gfx950 the seam's and the router helper's configuration carry the MI355X gates (all 0: every chunk
    with a sparse middle goes direct), while ``resolve_plugin_config`` alone keeps the reference's."""
    from trianglemix.config import device_gate_profile, load_gate_profile, resolve_plugin_config
    from trianglemix.router import device_plugin_config

    class _V:
        additional_config = {"trianglemix": {"enabled": True, "layers": "5"}}

    assert device_gate_profile() == "mi355x"
    cfg = device_plugin_config(_V()).kernel
    for field, value in load_gate_profile("mi355x").items():
        assert getattr(cfg, field) == value
    assert resolve_plugin_config(_V()).kernel.direct_min_saved_qk == 913_152


def test_router_native_paths(gpu):
    """The routing layer's native paths with the real ops: a routed direct call (gates and launch in one native
    call) is bit-identical to the op called directly, writes only the query's rows of a padded output, and
    counts one launch; a call that fails a tensor gate there (a strided block table) counts that reason and
    runs the engine's fallback; a call with an engine hook between the gates and the launch (before_direct)
    takes the two-step path, runs the hook once, and gives the same bits."""
    from trianglemix.router import TriangleMixRouter
    from trianglemix.stats import TriangleMixRuntimeStats
    from trianglemix.workload import SCALE, make_cache, make_query

    tq, seq, prompt = 512, 4608, 8192
    k, v, bt = make_cache(seq, 21, std=1.0)
    qd, kd, vd, btd = make_query(tq, 22, std=1.0).to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    kcfg = TriangleMixConfig(enabled=True, layer_indices=frozenset({5}))
    plan = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[tq], seq_lens=[seq],
                            prompt_lens=[prompt], num_decodes=0, num_prefills=1, config=kcfg)
    stats = TriangleMixRuntimeStats()
    router = TriangleMixRouter(PluginConfig(kernel=kcfg), stats=stats)
    want = torch.empty_like(qd)
    torch.ops.trianglemix.triangle_paged_sparse_attention.out(qd, kd, vd, btd, seq - tq, seq, prompt, SCALE, out=want)
    layer = "model.layers.5.self_attn.attn"
    print("router native paths: routed direct call", flush=True)
    padded = torch.full((tq + 8, 32, 128), float("nan"), dtype=torch.bfloat16, device=gpu)
    router.prefill_attention(layer_name=layer, plan=plan, query=qd, key_cache=kd, value_cache=vd, block_table=btd,
                             output=padded, softmax_scale=SCALE)
    torch.cuda.synchronize()
    assert torch.equal(padded[:tq], want) and torch.isnan(padded[tq:].float()).all()
    strided = torch.zeros(1, 2 * btd.shape[1], dtype=torch.int32, device=gpu)
    strided[:, ::2] = btd
    fell_back = []
    router.prefill_attention(layer_name=layer, plan=plan, query=qd, key_cache=kd, value_cache=vd,
                             block_table=strided[:, ::2], output=torch.empty_like(qd), softmax_scale=SCALE,
                             fallback=lambda: fell_back.append(1))
    hooked = torch.full_like(qd, float("nan"))
    calls = []
    router.prefill_attention(layer_name=layer, plan=plan, query=qd, key_cache=kd, value_cache=vd, block_table=btd,
                             output=hooked, softmax_scale=SCALE, before_direct=lambda: calls.append(1))
    torch.cuda.synchronize()
    assert fell_back == [1] and calls == [1] and torch.equal(hooked, want)
    counters = stats.snapshot()["counters"]
    assert counters["layer_direct"] == 2 and counters["layer_fia_reason:block_table_unsupported"] == 1
    assert counters.get("runtime_error", 0) == 0
