"""Host-side op layer, router and work accounting (CPU only).

* ``trianglemix.kernel``: span closed forms against the reference's
  known answers and the oracle's brute-force counts, eligibility gates,
  layer-name parsing, the Python pre-check, ``estimate_tile_counts``
  against a tile-by-tile enumeration;
* ``trianglemix.workload``: the closed-form FLOP / byte accounting bench.py
  reports, against brute-force counting in the oracle;
* ``trianglemix.router``: every gate of the dispatch decision, fail-open and
  strict failure handling, with the launch functions replaced by fakes so
  no kernel runs (package/tests/test_plugin.py covers the same decisions for
  the reference's patched forward).
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from oracle import geometry as G
from trianglemix import kernel as K
from trianglemix import workload as W
from trianglemix.config import PluginConfig
from trianglemix.planning import FallbackReason, build_batch_plan
from trianglemix.router import LayerFeatures, TriangleMixRouter, dispatch_reason
from trianglemix.stats import TriangleMixRuntimeStats

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
CFG = K.TriangleMixConfig(enabled=True, layer_indices=frozenset({5, 7}))


# ----------------------------------------------------------------- spans

@pytest.mark.parametrize("kat", KATS["chunk_spans"], ids=lambda k: f"{k['query_start']}_{k['query_tokens']}")
def test_chunk_span_kats(kat):
    seq = kat["query_start"] + kat["query_tokens"]
    span = K.triangle_sparse_span(query_len=kat["query_tokens"], seq_len=seq, prompt_len=kat["prompt_len"],
                                  config=CFG)
    if "s0" in kat:
        assert (span.s0, span.s1) == (kat["s0"], kat["s1"])
    if "has_sparse_middle" in kat:
        assert span.has_sparse_middle == kat["has_sparse_middle"]
    if "saved_qk" in kat:
        assert span.saved_qk == kat["saved_qk"]
        # closed form == brute-force count of skipped causal pairs
        assert span.saved_qk == G.saved_qk_bruteforce(kat["query_start"], seq, kat["prompt_len"])


@pytest.mark.parametrize("q0,q1,prompt", [(0, 512, 8192), (512, 1024, 8192), (2357, 2869, 2869), (7680, 8192, 8192),
                                          (500, 900, 1024), (0, 650, 650), (6272, 8320, 8320)])
def test_saved_qk_closed_form_matches_counting(q0, q1, prompt):
    span = K.triangle_sparse_span(query_len=q1 - q0, seq_len=q1, prompt_len=prompt, config=CFG)
    assert span.saved_qk == G.saved_qk_bruteforce(q0, q1, prompt)
    assert span.sparse_rows == sum(G.row_is_sparse(q, prompt) for q in range(q0, q1))


def test_span_rejects_bad_lengths():
    with pytest.raises(ValueError):
        K.triangle_sparse_span(query_len=10, seq_len=5, prompt_len=5, config=CFG)
    with pytest.raises(ValueError):
        K.triangle_sparse_span(query_len=5, seq_len=10, prompt_len=9, config=CFG)


def test_direct_eligible_matches_planner_crossover():
    assert not K.triangle_direct_eligible(query_len=2260, seq_len=2260, prompt_len=2260, config=CFG)
    assert K.triangle_direct_eligible(query_len=2261, seq_len=2261, prompt_len=2261, config=CFG)
    assert K.triangle_direct_eligible(query_len=512, seq_len=4608, prompt_len=8192, config=CFG)  # config 2 middle


def test_layer_name_parsing():
    assert K.extract_layer_index("model.layers.7.self_attn.attn") == 7
    assert K.extract_layer_index("layers.12") == 12
    assert K.extract_layer_index("model.embed_tokens") is None
    assert K.parse_layer_indices("5,7,10,15-35") == frozenset({5, 7, 10, *range(15, 36)})
    for bad in ("3-1", "-2"):
        with pytest.raises(ValueError):
            K.parse_layer_indices(bad)
    assert CFG.uses_layer("model.layers.7.attn") and not CFG.uses_layer("model.layers.8.attn")


def _enumerate_tile_counts(seq_len, cfg, bm, bn):
    """Tile-by-tile enumeration of the 512-key tiles each submitted interval touches."""
    tri = dense = 0
    start = cfg.sink_tokens + cfg.local_window + 1
    for q_lo in range(0, seq_len, bm):
        q_hi = min(seq_len, q_lo + bm)
        causal = {t for t in range(0, seq_len, bn) if t < q_hi}
        dense += len(causal)
        if q_hi <= start:
            tri += len(causal)
            continue
        local_lo = max(cfg.sink_tokens, q_lo - cfg.local_window)
        for lo, hi in ((0, cfg.sink_tokens), (local_lo, q_hi)):
            tri += sum(1 for t in range(0, q_hi + bn, bn) if t < hi and t + bn > lo)
    return tri, dense


@pytest.mark.parametrize("seq_len", [0, 1, 521, 522, 1000, 2869, 8192])
def test_estimate_tile_counts_against_enumeration(seq_len):
    assert K.estimate_tile_counts(seq_len, CFG) == _enumerate_tile_counts(seq_len, CFG, 32, 512)
    assert K.estimate_tile_counts(seq_len, CFG, 64, 128) == _enumerate_tile_counts(seq_len, CFG, 64, 128)
    with pytest.raises(ValueError):
        K.estimate_tile_counts(-1, CFG)


def _tensors(tq=4, pages=2):
    q = torch.zeros(tq, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(pages, 128, 8, 128, dtype=torch.bfloat16)
    return q, k, k.clone(), torch.zeros(1, pages, dtype=torch.int32), torch.empty_like(q)


@pytest.mark.parametrize("mutate,msg", [
    (lambda t: t.update(query=t["query"].float()), "BF16"),
    (lambda t: t.update(query=t["query"][:, :16]), r"\[Tq, 32, 128\]"),
    (lambda t: t.update(output=t["output"][:2]), "output must match"),
    (lambda t: t.update(key_cache=t["key_cache"][:, :64]), r"\[pages, 128, 8, 128\]"),
    (lambda t: t.update(block_table=t["block_table"].long()), "INT32"),
    (lambda t: t.update(key_cache=t["key_cache"].transpose(0, 1).contiguous().transpose(0, 1)), "contiguous"),
    (lambda t: t.update(block_table=t["block_table"][:, :1]), "too short"),
])
def test_python_precheck_raises_value_error(mutate, msg):
    q, k, v, bt, out = _tensors()
    t = dict(query=q, key_cache=k, value_cache=v, block_table=bt, output=out)
    mutate(t)
    with pytest.raises(ValueError, match=msg):
        K._validate_direct_tensors(seq_len=200, **t)


def test_direct_path_rejects_chunk_without_sparse_middle():
    q, k, v, bt, out = _tensors()
    with pytest.raises(ValueError, match="sparse middle"):
        K.triangle_direct_paged_attention(query=q, key_cache=k, value_cache=v, block_table=bt, seq_len=4,
                                          prompt_len=1024, output=out, softmax_scale=W.SCALE, config=CFG)


# --------------------------------------------------------------- workload

CONFIG2 = W.prompt_chunks(8192, 512)


@pytest.mark.parametrize("c", [CONFIG2[0], CONFIG2[1], CONFIG2[8], CONFIG2[15], W.Chunk(2357, 2869, 2869),
                               W.Chunk(500, 900, 1024), W.Chunk(0, 650, 650)], ids=str)
def test_workload_closed_forms_match_oracle_counting(c):
    assert W.attended_pairs(c) == G.attended_pairs(c.query_start, c.seq_len, c.seq_len, c.prompt_len)
    assert W.attended_pairs(c, dense=True) == sum(q + 1 for q in range(c.query_start, c.seq_len))
    assert W.unique_kv_tokens(c) == G.unique_kv_tokens(c.query_start, c.seq_len, c.seq_len, c.prompt_len)


def test_config_figures():
    # 4 * D * Hq * pairs; the per-config GFLOP figures of the work model
    assert round(W.chunk_flops(W.Chunk(2357, 2869, 2869)) / 1e9, 3) == 9.161
    assert [round(W.chunk_flops(c) / 1e9, 3) for c in (CONFIG2[0], CONFIG2[1], CONFIG2[15])] == [2.152, 4.370, 20.325]
    assert round(sum(W.chunk_flops(c) for c in CONFIG2) / 1e9, 2) == 83.66
    assert round(sum(W.chunk_flops(c, dense=True) for c in CONFIG2) / 1e9, 2) == 549.82
    assert len(W.prompt_chunks(8320, 2048)) == 5 and W.prompt_chunks(8320, 2048)[-1].query_tokens == 128


def test_executed_tiles_cover_attended_keys():
    for c in CONFIG2 + [W.Chunk(2357, 2869, 2869)]:
        executed = W.executed_tiles(c) * W.KV_TILE * W.ROW_BLOCK
        assert executed >= W.attended_pairs(c)
    assert W.executed_tiles(CONFIG2[0], dense=True) == W.executed_tiles(CONFIG2[0])


def test_noncontiguous_block_table_is_a_permutation_prefix():
    g = torch.Generator().manual_seed(3)
    t = W.noncontiguous_block_table(64, 71, g).view(-1)
    assert t.dtype == torch.int32 and len(set(t.tolist())) == 64 and int(t.max()) < 71
    assert not bool(torch.all(t[1:] == t[:-1] + 1))


# ----------------------------------------------------------------- router

class Fakes:
    def __init__(self, fail=False):
        self.calls = []
        self.fail = fail

    def direct(self, **kw):
        self.calls.append(("direct", kw))
        if self.fail:
            raise RuntimeError("launch failed")
        return kw["output"]

    def dense(self, **kw):
        self.calls.append(("dense", kw))
        return kw["output"]


def _plan(seq=4608, qlen=512, prompt=8192, state="ChunkedPrefill"):
    return build_batch_plan(state_name=state, cumulative_query_ends=[qlen], seq_lens=[seq], prompt_lens=[prompt],
                            num_decodes=0, num_prefills=1, config=CFG)


def _router(fakes, *, strict=False, ready=True, enabled=True):
    kcfg = K.TriangleMixConfig(enabled=enabled, layer_indices=frozenset({5, 7}))
    stats = TriangleMixRuntimeStats()
    r = TriangleMixRouter(PluginConfig(kernel=kcfg, strict=strict), stats=stats, direct_fn=fakes.direct,
                          dense_fn=fakes.dense, native_ready=lambda: ready)
    return r, stats


def _call(router, plan, layer="model.layers.7.self_attn.attn", features=LayerFeatures(), capturing=False,
          **over):
    q, k, v, _, out = _tensors(tq=plan.requests[0].query_len if plan else 4, pages=40)
    bt = torch.zeros(1, 40, dtype=torch.int32)
    args = dict(query=q, key_cache=k, value_cache=v, block_table=bt, output=out)
    args.update(over)
    return router.prefill_attention(layer_name=layer, plan=plan, softmax_scale=W.SCALE, features=features,
                                    capturing=capturing, **args)


def test_router_direct_path_counts_launch():
    f = Fakes()
    r, stats = _router(f)
    plan = _plan()
    _call(r, plan)
    assert [c[0] for c in f.calls] == ["direct"]
    kw = f.calls[0][1]
    assert kw["seq_len"] == 4608 and kw["prompt_len"] == 8192 and kw["softmax_scale"] == W.SCALE
    snap = stats.snapshot()
    assert snap["counters"]["layer_direct"] == 1 and snap["counters"]["single_launch"] == 1
    assert snap["counters"]["estimated_saved_qk"] == plan.requests[0].saved_qk
    assert snap["layers"]["direct"] == {"7": 1}


def test_router_unselected_layer_and_disabled_go_dense_without_counters():
    f = Fakes()
    r, stats = _router(f)
    _call(r, _plan(), layer="model.layers.8.self_attn.attn")
    r2, stats2 = _router(f, enabled=False)
    _call(r2, _plan())
    assert [c[0] for c in f.calls] == ["dense", "dense"]
    assert f.calls[0][1]["seq_len"] == 4608
    assert stats.snapshot()["counters"] == {} and stats2.snapshot()["counters"] == {}


@pytest.mark.parametrize("kwargs,reason", [
    (dict(capturing=True), FallbackReason.GRAPH_CAPTURE),
    (dict(features=LayerFeatures(tensor_parallel_size=2)), FallbackReason.TENSOR_PARALLEL),
    (dict(features=LayerFeatures(context_parallel=True)), FallbackReason.CONTEXT_PARALLEL),
    (dict(features=LayerFeatures(causal=False)), FallbackReason.NON_CAUSAL),
    (dict(features=LayerFeatures(sliding_window=4096)), FallbackReason.MODEL_UNSUPPORTED),
    (dict(features=LayerFeatures(num_kv_heads=4)), FallbackReason.QUERY_UNSUPPORTED),
    (dict(key_cache=None), FallbackReason.KV_CACHE_UNSUPPORTED),
    (dict(block_table=torch.zeros(1, 3, dtype=torch.int32)), FallbackReason.BLOCK_TABLE_UNSUPPORTED),
    (dict(block_table=torch.zeros(1, 40, dtype=torch.int64)), FallbackReason.BLOCK_TABLE_UNSUPPORTED),
])
def test_router_gates_fall_back_with_reason(kwargs, reason):
    f = Fakes()
    r, stats = _router(f)
    _call(r, _plan(), **kwargs)
    assert [c[0] for c in f.calls] == ["dense"]
    snap = stats.snapshot()
    assert snap["counters"]["layer_fia"] == 1 and snap["counters"][f"layer_fia_reason:{reason.value}"] == 1
    # graph-capture metadata is not a scheduled request
    assert snap["counters"].get("request_total", 0) == (0 if reason is FallbackReason.GRAPH_CAPTURE else 1)


def test_router_planner_reason_and_adapter_unavailable():
    f = Fakes()
    r, stats = _router(f)
    _call(r, _plan(seq=512, qlen=512))  # first chunk: no sparse middle
    r2, stats2 = _router(f, ready=False)
    _call(r2, _plan())
    assert [c[0] for c in f.calls] == ["dense", "dense"]
    assert stats.snapshot()["fallback_reasons"] == {"no_sparse_middle": 1}
    assert stats2.snapshot()["counters"]["layer_fia_reason:adapter_unavailable"] == 1


def test_router_fail_open_and_strict():
    f = Fakes(fail=True)
    r, stats = _router(f)
    _call(r, _plan())
    assert [c[0] for c in f.calls] == ["direct", "dense"]
    c = stats.snapshot()["counters"]
    assert c["runtime_error_stage:direct_launch"] == 1 and c["layer_fia_reason:direct_launch_error"] == 1
    f2 = Fakes(fail=True)
    r2, _ = _router(f2, strict=True)
    with pytest.raises(RuntimeError, match="launch failed"):
        _call(r2, _plan())
    assert [c[0] for c in f2.calls] == ["direct"]


def test_dispatch_reason_order():
    plan = _plan()
    q, k, v, _, out = _tensors(tq=512, pages=40)
    bt = torch.zeros(1, 40, dtype=torch.int32)
    cfg = PluginConfig(kernel=CFG)
    common = dict(config=cfg, plan=plan, query=q, output=out, key_cache=k, value_cache=v, block_table=bt)
    assert dispatch_reason(features=LayerFeatures(), capturing=False, native_ready=True, **common) \
        is FallbackReason.NONE
    # capture wins over everything, then the planner, then the adapter
    assert dispatch_reason(features=LayerFeatures(causal=False), capturing=True, native_ready=False, **common) \
        is FallbackReason.GRAPH_CAPTURE
    assert dispatch_reason(features=LayerFeatures(causal=False), capturing=False, native_ready=False, **common) \
        is FallbackReason.ADAPTER_UNAVAILABLE


def test_whole_long_prompt_routes_direct():
    """A whole-prompt PrefillNoCache step of 40960 tokens (planning.py:79-83 routes such steps direct) is planned
    direct and launched on the direct path -- the op accepts a chunk of any length -- with no fallback."""
    f = Fakes()
    r, stats = _router(f)
    L = 40960
    plan = _plan(seq=L, qlen=L, prompt=L, state="PrefillNoCache")
    assert plan.direct and plan.requests[0].query_len == L
    q = torch.zeros(L, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(L // 128 + 1, 128, 8, 128, dtype=torch.bfloat16)
    bt = torch.zeros(1, L // 128 + 1, dtype=torch.int32)
    r.prefill_attention(layer_name="model.layers.7.self_attn.attn", plan=plan, query=q, key_cache=k,
                        value_cache=k.clone(), block_table=bt, output=torch.empty_like(q), softmax_scale=W.SCALE)
    assert [c[0] for c in f.calls] == ["direct"]
    assert stats.snapshot()["counters"]["layer_direct"] == 1
    from trianglemix import cabi
    assert cabi.workspace_size(L, 0, L, L) >= 0 and cabi.workspace_size(L, 0, L, None) == 0
