"""The vLLM-ROCm seam end to end on the GPU, with the real gfx950 ops.

A fake vLLM Triton backend (the allowlisted signatures; its own forward
writes the chunk's K/V and runs the dense companion kernel, standing in for
vLLM's Triton path) is patched by ``trianglemix.vllm_rocm``.  A chunked
prefill of 8192 tokens in 16 chunks of 512 then runs through the fake model
runner, builder and two layers (layer 1 selected, layer 0 not), with fresh
K/V per chunk written into each layer's ``[2, pages, 128, 8, 128]`` cache.
Checks:

* both layers' caches end up holding every token's K/V at its page slot,
  bit-exact: on the direct path the seam writes them
  (``trianglemix::reshape_and_cache``), on every other path vLLM's forward;
* every chunk's output is bit-identical to the op its route names (sparse op
  on direct chunks of layer 1, dense companion elsewhere) run on the final
  cache, and one direct chunk matches the fp32 oracle;
* the counters: one launch per direct chunk of layer 1, the planner's
  fallback reasons for the others (reference gates), nothing for layer 0.
"""

from __future__ import annotations

import types

import pytest
import torch

from oracle import attention as OA
from trianglemix import vllm_rocm as V
from trianglemix.cache import chunk_slot_mapping
from trianglemix.stats import runtime_stats
from trianglemix.workload import SCALE, make_cache, make_query, prompt_chunks

pytestmark = pytest.mark.gpu

L, CHUNK = 8192, 512


class _Metadata:
    def __init__(self, common):
        self.num_actual_tokens = int(common.query_start_loc_cpu[-1])
        self.seq_len = int(common.seq_lens_cpu[0])
        self.block_table = common.block_table_tensor
        self.slot_mapping = common.slot_mapping
        self.causal = True
        self.use_cascade = False


def _fake_vllm():
    class TritonAttentionMetadataBuilder:
        def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
            self.vllm_config = vllm_config

        def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
            return _Metadata(common_attn_metadata)

        def build_for_cudagraph_capture(self, common_attn_metadata):
            return self.build(0, common_attn_metadata)

    class TritonAttentionImpl:
        def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes, sliding_window, kv_cache_dtype,
                     logits_soft_cap=None, attn_type="decoder", kv_sharing_target_layer_name=None, sinks=None):
            self.num_heads, self.head_size, self.scale, self.num_kv_heads = num_heads, head_size, scale, num_kv_heads
            self.alibi_slopes, self.sinks, self.logits_soft_cap = alibi_slopes, sinks, logits_soft_cap
            self.sliding_window = (-1, -1)
            self.kv_cache_dtype, self.attn_type = kv_cache_dtype, attn_type
            self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
            self.vllm_calls = 0

        def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                    output_block_scale=None):
            # stand-in for vLLM's Triton path: write this step's K/V, then attend
            self.vllm_calls += 1
            kc, vc = kv_cache.unbind(0)
            n, seq = attn_metadata.num_actual_tokens, attn_metadata.seq_len
            torch.ops.trianglemix.reshape_and_cache(key[:n], value[:n], kc, vc, attn_metadata.slot_mapping[:n])
            torch.ops.trianglemix.dense_paged_causal_attention.out(
                query[:n], kc, vc, attn_metadata.block_table, seq - n, seq, self.scale, out=output[:n])
            return output

    class GPUModelRunner:
        def __init__(self, builder):
            self.builder = builder
            self.input_batch = types.SimpleNamespace(num_reqs=1, num_prompt_tokens=[L])
            self.speculative_config = None

        def _prepare_inputs(self, scheduler_output):
            return {"layers": self.builder.build(0, scheduler_output)}, None

    backend = types.SimpleNamespace(TritonAttentionMetadataBuilder=TritonAttentionMetadataBuilder,
                                    TritonAttentionImpl=TritonAttentionImpl,
                                    get_tensor_model_parallel_world_size=lambda: 1)
    return backend, types.SimpleNamespace(GPUModelRunner=GPUModelRunner)


def test_chunked_prefill_through_the_patched_backend(gpu, monkeypatch):
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_STRICT", raising=False)
    monkeypatch.setattr(V, "OPS", V.SeamOps())  # the real ops
    runtime_stats().snapshot(reset=True)
    backend, runner_mod = _fake_vllm()
    assert V.patch_modules(backend, runner_mod)
    cfg = types.SimpleNamespace(additional_config={"trianglemix": {"enabled": True, "layers": "1"}})
    builder = backend.TritonAttentionMetadataBuilder(None, [], cfg, gpu)
    runner = runner_mod.GPUModelRunner(builder)
    impls = [backend.TritonAttentionImpl(32, 128, SCALE, 8, None, None, "auto") for _ in range(2)]

    # per layer: the prompt's K/V (as a paged cache: the source of the fresh chunk K/V) and Q
    sources = [make_cache(L, 70 + i, std=1.0) for i in range(2)]
    table = sources[0][2].to(gpu)  # both layers use one page table (as vLLM does)
    pages = sources[0][0].shape[0]
    kv = []   # fresh K/V per token, [L, 8, 128]
    for k, v, bt in sources:
        rows = torch.arange(L)
        slot = bt[0].long()[rows // 128] * 128 + rows % 128
        kv.append((k.reshape(-1, 8, 128)[slot].to(gpu), v.reshape(-1, 8, 128)[slot].to(gpu)))
    qs = [make_query(L, 90 + i, std=1.0).to(gpu) for i in range(2)]
    caches = [torch.full((2, pages, 128, 8, 128), float("nan"), dtype=torch.bfloat16, device=gpu) for _ in range(2)]
    outs = [torch.full_like(q, float("nan")) for q in qs]

    routes = []
    for c in prompt_chunks(L, CHUNK):
        n = c.seq_len - c.query_start
        common = types.SimpleNamespace(
            query_start_loc_cpu=torch.tensor([0, n], dtype=torch.int32),
            seq_lens_cpu=torch.tensor([c.seq_len], dtype=torch.int32), num_reqs=1, causal=True,
            block_table_tensor=table, slot_mapping=chunk_slot_mapping(table, c.query_start, n))
        md = runner._prepare_inputs(common)[0]["layers"]
        plan = md._trianglemix_rocm_plan.plan
        routes.append((c, plan))
        for i, impl in enumerate(impls):
            sl = slice(c.query_start, c.seq_len)
            impl.forward(types.SimpleNamespace(layer_name=f"model.layers.{i}.self_attn.attn"), qs[i][sl],
                         kv[i][0][sl], kv[i][1][sl], caches[i], md, outs[i][sl])
    torch.cuda.synchronize()

    # caches: every token's K/V at its page slot (the shared table), bit-exact
    rows = torch.arange(L)
    slots = table[0].long().cpu()[rows // 128] * 128 + rows % 128
    for i in range(2):
        got_k, got_v = caches[i][0].cpu().reshape(-1, 8, 128), caches[i][1].cpu().reshape(-1, 8, 128)
        assert torch.equal(got_k[slots], kv[i][0].cpu()) and torch.equal(got_v[slots], kv[i][1].cpu()), i

    direct = [c for c, p in routes if p.direct]
    assert 0 < len(direct) < len(routes)
    for c, plan in routes:
        for i in range(2):
            sl = slice(c.query_start, c.seq_len)
            kc, vc = caches[i].unbind(0)
            want = torch.full_like(qs[i][sl], float("nan"))
            if i == 1 and plan.direct:
                torch.ops.trianglemix.triangle_paged_sparse_attention.out(
                    qs[i][sl], kc, vc, table, c.query_start, c.seq_len, L, SCALE, out=want)
            else:
                torch.ops.trianglemix.dense_paged_causal_attention.out(
                    qs[i][sl], kc, vc, table, c.query_start, c.seq_len, SCALE, out=want)
            torch.cuda.synchronize()
            assert torch.equal(outs[i][sl], want), (c.query_start, i)

    c = direct[len(direct) // 2]
    q = qs[1][c.query_start:c.seq_len].cpu()
    expected = OA.attention_torch(q, caches[1][0].cpu(), caches[1][1].cpu(), table.cpu(), c.query_start, c.seq_len,
                                  L, SCALE)
    m = OA.error_metrics(outs[1][c.query_start:c.seq_len].float().cpu().numpy(), expected.float().numpy())
    print(f"seam chunk {c.query_start}: {m}", flush=True)
    assert m["max_abs"] <= 2e-2 and m["mean_abs"] <= 2e-3, m

    snap = runtime_stats().snapshot()
    counters = snap["counters"]
    assert counters["single_launch"] == len(direct) and counters["request_total"] == len(routes)
    assert impls[0].vllm_calls == len(routes) and impls[1].vllm_calls == len(routes) - len(direct)
    assert snap["layers"] == {"direct": {"1": len(direct)}, "fia": {"1": len(routes) - len(direct)}}
    reasons = {}
    for _, p in routes:
        if not p.direct:
            reasons[p.primary_reason.value] = reasons.get(p.primary_reason.value, 0) + 1
    assert snap["fallback_reasons"] == reasons
