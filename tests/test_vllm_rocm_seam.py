"""vLLM-ROCm integration seam (``trianglemix.vllm_rocm``) against fake vLLM classes.

vLLM is not installed here, so, as the reference's plugin tests do
(package/tests/test_plugin.py:30-357 fakes; cases :404-1700), the Triton
attention builder / impl and the GPU model runner are small classes with the
allowlisted signatures, and the device calls are stand-ins.  Covered:

* patching is all-or-nothing, idempotent, refuses a signature outside the
  allowlist (counted; raised in strict mode) and restores every attribute
  when it fails halfway;
* a chunked-prefill step: the runner publishes the final prompt length, the
  builder attaches one plan that every layer of the step shares, a selected
  layer writes the chunk's K/V and then launches the op once (on the chunk's
  own rows when vLLM pads), other layers and steps run vLLM's forward;
* every fallback (feature off, unselected layer, no prompt length, first
  chunk, decode, batch of two, graph capture, unsupported modes, tensor
  parallel, KV cache / block table checks, a failing launch or K/V write) runs
  vLLM's forward and is counted with the reference's reason;
* metadata classes that refuse new attributes still carry their plan.
"""

from __future__ import annotations

import types

import pytest
import torch

from trianglemix import vllm_rocm as V
from trianglemix.stats import runtime_stats

PAGES = 40


def _vllm_config(enabled=True, layers="3,7", strict=False, **extra):
    section = {"enabled": enabled, "layers": layers, "strict": strict, **extra}
    return types.SimpleNamespace(additional_config={"trianglemix": section})


class _Metadata:
    def __init__(self, common):
        self.num_actual_tokens = int(common.query_start_loc_cpu[-1])
        self.block_table = common.block_table_tensor
        self.slot_mapping = common.slot_mapping
        self.causal = common.causal
        self.use_cascade = False


def make_backend_module(*, tp=1, bad_forward=False, kv_layout="kv_first"):
    class TritonAttentionBackend:
        @staticmethod
        def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, cache_dtype_str="auto"):
            if kv_layout == "kv_first":
                return (2, num_blocks, block_size, num_kv_heads, head_size)
            return (num_blocks, 2, block_size, num_kv_heads, head_size)

    class TritonAttentionMetadataBuilder:
        def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
            self.vllm_config = vllm_config
            self.metadata_cls = _Metadata

        def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
            return self.metadata_cls(common_attn_metadata)

        def build_for_cudagraph_capture(self, common_attn_metadata):
            return self.build(0, common_attn_metadata)

    class TritonAttentionImpl:
        def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes, sliding_window, kv_cache_dtype,
                     logits_soft_cap=None, attn_type="decoder", kv_sharing_target_layer_name=None, sinks=None):
            self.num_heads, self.head_size, self.scale, self.num_kv_heads = num_heads, head_size, scale, num_kv_heads
            self.alibi_slopes = alibi_slopes
            self.sliding_window = (-1, -1) if sliding_window is None else (sliding_window - 1, 0)
            self.kv_cache_dtype = kv_cache_dtype
            self.logits_soft_cap = logits_soft_cap
            self.attn_type = attn_type
            self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
            self.sinks = sinks
            self.vllm_calls = []

        if bad_forward:
            def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None):
                return output
        else:
            def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                        output_block_scale=None):
                self.vllm_calls.append(layer.layer_name)
                return output

    module = types.SimpleNamespace(TritonAttentionMetadataBuilder=TritonAttentionMetadataBuilder,
                                   TritonAttentionImpl=TritonAttentionImpl,
                                   get_tensor_model_parallel_world_size=lambda: tp)
    if kv_layout is not None:
        module.TritonAttentionBackend = TritonAttentionBackend
    return module


def make_runner_module(builder):
    class GPUModelRunner:
        def __init__(self):
            self.input_batch = types.SimpleNamespace(num_reqs=1, num_prompt_tokens=[0])
            self.speculative_config = None

        def _prepare_inputs(self, scheduler_output):
            return {"model.layers.all": builder.build(0, scheduler_output.common)}, None

    return types.SimpleNamespace(GPUModelRunner=GPUModelRunner)


def _common(q0, qlen, seq, *, reqs=None, capture=False, prompt_field=None):
    """CommonAttentionMetadata of one step (``reqs`` = [(qlen, seq)] for several requests)."""
    reqs = reqs or [(qlen, seq)]
    starts = [0]
    for ql, _ in reqs:
        starts.append(starts[-1] + ql)
    slots = torch.arange(q0, q0 + starts[-1], dtype=torch.int64)
    ns = types.SimpleNamespace(
        query_start_loc_cpu=torch.tensor(starts, dtype=torch.int32),
        seq_lens_cpu=torch.tensor([s for _, s in reqs], dtype=torch.int32),
        num_reqs=len(reqs), causal=True, slot_mapping=slots,
        block_table_tensor=torch.arange(PAGES, dtype=torch.int32).repeat(len(reqs), 1))
    if prompt_field is not None:
        ns.num_prompt_tokens_cpu = torch.tensor(prompt_field, dtype=torch.int32)
    return ns


class _Ops:
    def __init__(self, fail_direct=False, fail_kv=False):
        self.calls = []
        self.fail_direct, self.fail_kv = fail_direct, fail_kv

    def direct(self, **kw):
        self.calls.append(("direct", kw))
        if self.fail_direct:
            raise RuntimeError("launch failed")
        return kw["output"]

    def kv_write(self, key, value, key_cache, value_cache, slots):
        self.calls.append(("kv_write", dict(key=key, value=value, key_cache=key_cache, slots=slots)))
        if self.fail_kv:
            raise RuntimeError("kv write failed")


@pytest.fixture
def env(monkeypatch):
    """Fresh fake vLLM classes patched by the seam, stand-in device calls, zeroed process counters."""
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_STRICT", raising=False)
    ops = _Ops()
    monkeypatch.setattr(V, "OPS", V.SeamOps(direct=ops.direct, kv_write=ops.kv_write, native_ready=lambda: True))
    runtime_stats().snapshot(reset=True)
    runtime_stats().configure(256, 0)
    backend = make_backend_module()
    assert V.patch_modules(backend)
    return types.SimpleNamespace(backend=backend, ops=ops, monkeypatch=monkeypatch)


def _builder(env, **cfg):
    return env.backend.TritonAttentionMetadataBuilder(None, [], _vllm_config(**cfg), "cuda:0")


def _impl(env, **kw):
    args = dict(num_heads=32, head_size=128, scale=0.088, num_kv_heads=8, alibi_slopes=None, sliding_window=None,
                kv_cache_dtype="auto")
    args.update(kw)
    return env.backend.TritonAttentionImpl(**args)


def _runner(env, builder, prompt, num_reqs=1):
    runner_mod = make_runner_module(builder)
    V.patch_modules(env.backend, runner_mod)
    runner = runner_mod.GPUModelRunner()
    runner.input_batch.num_reqs = num_reqs
    runner.input_batch.num_prompt_tokens = [prompt] * num_reqs
    return runner


def _step(runner, common):
    return runner._prepare_inputs(types.SimpleNamespace(common=common))[0]["model.layers.all"]


def _forward(impl, md, layer, *, rows, pad=0, kv_cache=None, **kw):
    q = torch.zeros(rows + pad, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(rows + pad, 8, 128, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    if kv_cache is None:
        kv_cache = torch.zeros(2, PAGES, 128, 8, 128, dtype=torch.bfloat16)
    return impl.forward(types.SimpleNamespace(layer_name=f"model.layers.{layer}.self_attn.attn"), q, k, k.clone(),
                        kv_cache, md, out, **kw), out


def _counters():
    return runtime_stats().snapshot()["counters"]


# ---------------------------------------------------------------- patching
def test_patch_is_idempotent_and_checks_signatures(env):
    impl_cls = env.backend.TritonAttentionImpl
    wrapped = impl_cls.forward
    assert wrapped.__wrapped__ is not wrapped
    assert V.patch_modules(env.backend) is False  # already patched: nothing rewrapped
    assert impl_cls.forward is wrapped
    bad = make_backend_module(bad_forward=True)
    original = bad.TritonAttentionImpl.forward
    with pytest.raises(V.UnsupportedFramework, match="impl.forward signature"):
        V.patch_modules(bad)
    assert bad.TritonAttentionImpl.forward is original
    assert not vars(bad.TritonAttentionMetadataBuilder).get(V._MARK, False)


def test_failed_patch_restores_every_attribute():
    backend = make_backend_module()
    build, forward = backend.TritonAttentionMetadataBuilder.build, backend.TritonAttentionImpl.forward

    class Refusing(type):
        def __setattr__(cls, name, value):
            if name == "_prepare_inputs":
                raise TypeError("read-only")
            super().__setattr__(name, value)

    class GPUModelRunner(metaclass=Refusing):
        def _prepare_inputs(self, scheduler_output):
            return None

    with pytest.raises(TypeError, match="read-only"):
        V.patch_modules(backend, types.SimpleNamespace(GPUModelRunner=GPUModelRunner))
    assert backend.TritonAttentionMetadataBuilder.build is build
    assert backend.TritonAttentionImpl.forward is forward
    for cls in (backend.TritonAttentionMetadataBuilder, backend.TritonAttentionImpl):
        assert V._MARK not in vars(cls)


def test_register_counts_an_unsupported_framework(monkeypatch):
    bad = make_backend_module(bad_forward=True)
    monkeypatch.setattr(V, "_REGISTERED", False)
    monkeypatch.setattr(V.importlib, "import_module", lambda name: bad if name == V.BACKEND_MODULE
                        else make_runner_module(None))
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_STRICT", raising=False)
    runtime_stats().snapshot(reset=True)
    V.register()
    assert _counters()["runtime_error_stage:unsupported_version"] == 1 and V._REGISTERED is False
    monkeypatch.setenv("VLLM_ASCEND_TRIANGLE_MIX_STRICT", "1")
    with pytest.raises(V.UnsupportedFramework):
        V.register()
    # a missing vLLM is a registration error, not a crash
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_STRICT")

    def no_vllm(name):
        raise ModuleNotFoundError("No module named 'vllm'")

    monkeypatch.setattr(V.importlib, "import_module", no_vllm)
    V.register()
    assert _counters()["runtime_error_stage:plugin_register"] == 1
    good = make_backend_module()
    monkeypatch.setattr(V.importlib, "import_module", lambda name: good if name == V.BACKEND_MODULE
                        else make_runner_module(None))
    V.register()
    assert V._REGISTERED is True and vars(good.TritonAttentionImpl)[V._MARK]


# ----------------------------------------------------------- direct path
def test_chunked_prefill_writes_kv_then_launches_once(env):
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    impl = _impl(env)
    result, out = _forward(impl, md, 7, rows=512)
    assert result is out and impl.vllm_calls == []
    assert [c[0] for c in env.ops.calls] == ["kv_write", "direct"]
    kv = env.ops.calls[0][1]
    assert kv["key"].shape == (512, 8, 128) and torch.equal(kv["slots"], torch.arange(4096, 4608))
    d = env.ops.calls[1][1]
    assert d["seq_len"] == 4608 and d["prompt_len"] == 8192 and d["softmax_scale"] == 0.088
    assert d["query"].shape == (512, 32, 128) and d["output"].data_ptr() == out.data_ptr()
    assert d["key_cache"].shape == (PAGES, 128, 8, 128) and d["block_table"].shape == (1, PAGES)
    c = _counters()
    assert c["layer_direct"] == 1 and c["single_launch"] == 1 and c["request_total"] == 1


def test_one_plan_per_step_shared_by_layers(env):
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    impl = _impl(env)
    plans = []
    for q0 in (4096, 4608):
        md = _step(runner, _common(q0, 512, q0 + 512))
        plans.append(md._trianglemix_rocm_plan.plan.plan_id)
        for layer in (3, 5, 7):
            _forward(impl, md, layer, rows=512)
    assert plans[0] != plans[1]
    c = _counters()
    assert c["request_total"] == 2 and c["single_launch"] == 4
    assert impl.vllm_calls == ["model.layers.5.self_attn.attn"] * 2  # layer 5 is not selected
    assert runtime_stats().snapshot()["layers"]["direct"] == {"3": 2, "7": 2}


def test_padded_tokens_launch_on_the_chunk_rows(env):
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    _forward(_impl(env), md, 3, rows=512, pad=16)
    d = env.ops.calls[-1][1]
    assert d["query"].shape[0] == 512 and d["output"].shape[0] == 512


# ------------------------------------------------------------- fallbacks
def test_feature_off_never_touches_the_native_runtime(env, monkeypatch):
    def boom():
        raise AssertionError("native runtime touched while disabled")

    monkeypatch.setattr(V, "OPS", V.SeamOps(direct=env.ops.direct, kv_write=env.ops.kv_write, native_ready=boom))
    builder = _builder(env, enabled=False)
    runner = _runner(env, builder, prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    impl = _impl(env)
    _forward(impl, md, 7, rows=512)
    assert impl.vllm_calls == ["model.layers.7.self_attn.attn"] and env.ops.calls == []
    assert _counters() == {}


@pytest.mark.parametrize("name,common,prompt,reqs,reason", [
    ("first chunk", (0, 512, 512), 8192, 1, "no_sparse_middle"),
    ("decode", (8192, 1, 8193), 8192, 1, "state_unsupported"),
    ("two requests", None, 8192, 2, "batch_unsupported"),
])
def test_planner_fallbacks_run_vllm(env, name, common, prompt, reqs, reason):
    builder = _builder(env)
    runner = _runner(env, builder, prompt=prompt, num_reqs=reqs)
    c = _common(4096, 0, 0, reqs=[(512, 4608), (512, 4608)]) if reqs == 2 else _common(*common)
    md = _step(runner, c)
    impl = _impl(env)
    _forward(impl, md, 7, rows=int(c.query_start_loc_cpu[-1]))
    assert impl.vllm_calls and env.ops.calls == []
    assert runtime_stats().snapshot()["fallback_reasons"] == {reason: reqs}
    assert _counters()[f"layer_fia_reason:{reason}"] == 1


def test_no_prompt_length_outside_the_runner(env):
    builder = _builder(env)
    md = builder.build(0, _common(4096, 512, 4608))  # no runner step around it
    impl = _impl(env)
    _forward(impl, md, 7, rows=512)
    assert impl.vllm_calls and env.ops.calls == []
    assert runtime_stats().snapshot()["fallback_reasons"] == {"missing_metadata": 1}
    # an official prompt field on the common metadata is enough
    md2 = builder.build(0, _common(4096, 512, 4608, prompt_field=[8192]))
    _forward(impl, md2, 7, rows=512)
    assert [c[0] for c in env.ops.calls] == ["kv_write", "direct"]


def test_runner_prompt_rules():
    batch = types.SimpleNamespace(num_reqs=1, num_prompt_tokens=[8320, 0])
    runner = types.SimpleNamespace(input_batch=batch, speculative_config=None)
    assert V.runner_prompt(runner) == (8320,)
    assert V.runner_prompt(types.SimpleNamespace(input_batch=types.SimpleNamespace(num_reqs=2,
                                                 num_prompt_tokens=[1, 2, 0]), speculative_config=None)) == (1, 2)
    assert V.runner_prompt(types.SimpleNamespace(input_batch=batch, speculative_config=object())) is None
    assert V.runner_prompt(types.SimpleNamespace(input_batch=types.SimpleNamespace(num_reqs=1,
                                                 num_prompt_tokens=[0]), speculative_config=None)) is None
    assert V.runner_prompt(types.SimpleNamespace()) is None


def test_graph_capture_metadata_always_runs_vllm(env):
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    with_prompt = _step(runner, _common(4096, 512, 4608))
    assert with_prompt._trianglemix_rocm_plan.plan.direct
    md = builder.build_for_cudagraph_capture(_common(4096, 512, 4608))
    impl = _impl(env)
    _forward(impl, md, 7, rows=512)
    assert impl.vllm_calls and env.ops.calls == []
    c = _counters()
    assert c["layer_fia_reason:graph_capture"] == 1 and c.get("request_total", 0) == 0


@pytest.mark.parametrize("impl_kw,fwd_kw,tp,reason", [
    (dict(sliding_window=4096), {}, 1, "model_unsupported"),
    (dict(kv_cache_dtype="fp8"), {}, 1, "model_unsupported"),
    (dict(kv_sharing_target_layer_name="model.layers.1.self_attn.attn"), {}, 1, "model_unsupported"),
    (dict(logits_soft_cap=30.0), {}, 1, "model_unsupported"),
    (dict(attn_type="encoder_only"), {}, 1, "model_unsupported"),
    ({}, dict(output_scale=torch.ones(1)), 1, "model_unsupported"),
    (dict(num_kv_heads=4), {}, 1, "query_unsupported"),
    ({}, {}, 2, "tensor_parallel"),
    ({}, dict(kv_cache=torch.zeros(2, PAGES, 64, 8, 128, dtype=torch.bfloat16)), 1, "kv_cache_unsupported"),
])
def test_unsupported_modes_run_vllm(env, impl_kw, fwd_kw, tp, reason):
    if tp != 1:
        backend = make_backend_module(tp=tp)
        V.patch_modules(backend)
        env.backend = backend
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    impl = _impl(env, **impl_kw)
    _forward(impl, md, 7, rows=512, **fwd_kw)
    assert impl.vllm_calls and env.ops.calls == []
    assert _counters()[f"layer_fia_reason:{reason}"] == 1


def test_block_table_and_non_causal_checks(env):
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    common = _common(4096, 512, 4608)
    common.block_table_tensor = common.block_table_tensor.to(torch.int64)
    impl = _impl(env)
    _forward(impl, _step(runner, common), 7, rows=512)
    common2 = _common(4096, 512, 4608)
    common2.causal = False
    _forward(impl, _step(runner, common2), 7, rows=512)
    c = _counters()
    assert c["layer_fia_reason:block_table_unsupported"] == 1 and c["layer_fia_reason:non_causal"] == 1
    assert env.ops.calls == [] and len(impl.vllm_calls) == 2


@pytest.mark.parametrize("fail", ["direct", "kv"])
def test_failures_are_fail_open_by_default_and_raise_in_strict_mode(env, monkeypatch, fail):
    ops = _Ops(fail_direct=fail == "direct", fail_kv=fail == "kv")
    monkeypatch.setattr(V, "OPS", V.SeamOps(direct=ops.direct, kv_write=ops.kv_write, native_ready=lambda: True))
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    impl = _impl(env)
    _forward(impl, _step(runner, _common(4096, 512, 4608)), 7, rows=512)
    assert impl.vllm_calls == ["model.layers.7.self_attn.attn"]
    c = _counters()
    assert c["runtime_error_stage:direct_launch"] == 1 and c["layer_fia_reason:direct_launch_error"] == 1
    strict = _builder(env, strict=True)
    strict_runner = _runner(env, strict, prompt=8192)
    with pytest.raises(RuntimeError, match="failed"):
        _forward(_impl(env), _step(strict_runner, _common(4608, 512, 5120)), 7, rows=512)


def test_native_bootstrap_failure_counts_and_falls_back(env, monkeypatch):
    monkeypatch.setattr(V, "OPS", V.SeamOps(direct=env.ops.direct, kv_write=env.ops.kv_write, native_ready=None))
    import trianglemix.native as N

    def unavailable(*, strict=False):
        raise N.NativeUnavailable("no HIP library in this test")

    monkeypatch.setattr(N, "ensure_native_loaded", unavailable)
    builder = _builder(env)
    runner = _runner(env, builder, prompt=8192)
    impl = _impl(env)
    _forward(impl, _step(runner, _common(4096, 512, 4608)), 7, rows=512)
    c = _counters()
    assert c["runtime_error_stage:native_bootstrap"] == 1 and c["layer_fia_reason:adapter_unavailable"] == 1
    assert impl.vllm_calls and env.ops.calls == []


def test_metadata_that_refuses_attributes_keeps_its_plan(env):
    class Slotted:
        __slots__ = ("num_actual_tokens", "block_table", "slot_mapping", "causal", "use_cascade", "__weakref__")

        def __init__(self, common):
            self.num_actual_tokens = int(common.query_start_loc_cpu[-1])
            self.block_table = common.block_table_tensor
            self.slot_mapping = common.slot_mapping
            self.causal = True
            self.use_cascade = False

    builder = _builder(env)
    builder.metadata_cls = Slotted
    runner = _runner(env, builder, prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    assert not hasattr(md, "_trianglemix_rocm_plan")
    _forward(_impl(env), md, 7, rows=512)
    assert [c[0] for c in env.ops.calls] == ["kv_write", "direct"]


def test_plan_from_common_states():
    from trianglemix.kernel import TriangleMixConfig

    cfg = TriangleMixConfig(enabled=True, layer_indices=frozenset({7}))
    whole = V.plan_from_common(_common(0, 4096, 4096), cfg, (4096,))
    assert whole.state_name == "PrefillNoCache" and whole.direct
    chunk = V.plan_from_common(_common(4096, 512, 4608), cfg, (8192,))
    assert chunk.state_name == "ChunkedPrefill" and chunk.requests[0].q_begin == 4096
    decode = V.plan_from_common(_common(8192, 1, 8193), cfg, (8192,))
    assert decode.state_name == "DecodeOnly" and not decode.direct
    empty = V.plan_from_common(types.SimpleNamespace(), cfg, None)
    assert empty.batch_size == 0 and empty.primary_reason.value == "missing_metadata"


# ------------------------------------------------------------ KV cache layout
def _layout_env(monkeypatch, kv_layout):
    ops = _Ops()
    monkeypatch.setattr(V, "OPS", V.SeamOps(direct=ops.direct, kv_write=ops.kv_write, native_ready=lambda: True))
    runtime_stats().snapshot(reset=True)
    runtime_stats().configure(256, 0)
    backend = make_backend_module(kv_layout=kv_layout)
    assert V.patch_modules(backend)
    return types.SimpleNamespace(backend=backend, ops=ops, monkeypatch=monkeypatch)


def test_kv_layout_comes_from_the_backend_shape_rule():
    assert V.kv_cache_layout(make_backend_module(kv_layout="kv_first")) == V.KV_FIRST
    assert V.kv_cache_layout(make_backend_module(kv_layout="blocks_first")) == V.BLOCKS_FIRST
    assert V.kv_cache_layout(make_backend_module(kv_layout=None)) is None
    odd = types.SimpleNamespace(TritonAttentionBackend=types.SimpleNamespace(get_kv_cache_shape=lambda *a: (3, 4)))
    assert V.kv_cache_layout(odd) is None


def _kv(layout, blocks):
    shape = (2, blocks, 128, 8, 128) if layout == "kv_first" else (blocks, 2, 128, 8, 128)
    kv = torch.zeros(shape, dtype=torch.bfloat16)
    (kv[0] if layout == "kv_first" else kv[:, 0]).fill_(1.0)  # K = 1, V = 0
    return kv


@pytest.mark.parametrize("blocks", [2, PAGES])
def test_kv_first_cache_splits_on_dim0_even_with_two_blocks(monkeypatch, blocks):
    env = _layout_env(monkeypatch, "kv_first")
    runner = _runner(env, _builder(env), prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    impl = _impl(env)
    _forward(impl, md, 7, rows=512, kv_cache=_kv("kv_first", blocks))
    direct = [c[1] for c in env.ops.calls if c[0] == "direct"]
    assert len(direct) == 1 and impl.vllm_calls == []
    kc, vc = direct[0]["key_cache"], direct[0]["value_cache"]
    assert kc.shape == (blocks, 128, 8, 128) and kc.is_contiguous() and torch.all(kc == 1) and torch.all(vc == 0)


@pytest.mark.parametrize("blocks", [2, PAGES])
def test_blocks_first_cache_falls_back_with_a_reason(monkeypatch, blocks):
    env = _layout_env(monkeypatch, "blocks_first")
    runner = _runner(env, _builder(env), prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    impl = _impl(env)
    _forward(impl, md, 7, rows=512, kv_cache=_kv("blocks_first", blocks))
    assert not [c for c in env.ops.calls if c[0] == "direct"] and impl.vllm_calls == ["model.layers.7.self_attn.attn"]
    assert _counters()["layer_fia_reason:kv_cache_unsupported"] == 1


def test_two_block_cache_without_a_shape_rule_is_refused(monkeypatch):
    assert V._split_kv(torch.zeros(2, 2, 128, 8, 128), None) == (None, None)
    k, v = V._split_kv(torch.zeros(2, 5, 128, 8, 128), None)
    assert k.shape == v.shape == (5, 128, 8, 128)
    env = _layout_env(monkeypatch, None)
    runner = _runner(env, _builder(env), prompt=8192)
    md = _step(runner, _common(4096, 512, 4608))
    impl = _impl(env)
    _forward(impl, md, 7, rows=512, kv_cache=torch.zeros(2, 2, 128, 8, 128, dtype=torch.bfloat16))
    assert _counters()["layer_fia_reason:kv_cache_unsupported"] == 1 and impl.vllm_calls
