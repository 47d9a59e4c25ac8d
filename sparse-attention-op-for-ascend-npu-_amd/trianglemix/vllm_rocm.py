"""vLLM-ROCm integration seam: eligible prefill chunks of selected layers run the gfx950 op.

Counterpart of the reference's vLLM-Ascend plugin
(package/src/vllm_ascend_trianglemix/plugin.py:1-16, :778-1587, :1705-1744),
written for vLLM v1's Triton attention backend, the ROCm backend whose paged
KV cache ``[2, blocks, 128, 8, 128]`` is exactly the op's page layout.  The
layout is read from the backend's ``get_kv_cache_shape``; a blocks-first
cache (``[blocks, 2, ...]``) is split on its second axis and, since its pages
are not contiguous per tensor, its layers fall back (``kv_cache_unsupported``).
Four methods are wrapped and nothing else is touched:

* ``GPUModelRunner._prepare_inputs`` publishes, for the builders that run
  inside it, the scheduler-owned final prompt lengths of the step's requests
  (``input_batch.num_prompt_tokens``).  The plan needs it: the current
  sequence length cannot tell an intermediate chunk from the one holding the
  prompt's dense tail (plugin.py:834-1024 does the same on Ascend);
* ``TritonAttentionMetadataBuilder.build`` builds the step's immutable plan
  once (from the CPU copies of the query starts and sequence lengths, no
  device sync) and attaches it to the metadata every layer receives
  (plugin.py:778-831);
* ``TritonAttentionMetadataBuilder.build_for_cudagraph_capture`` marks
  capture metadata, which always takes vLLM's own path;
* ``TritonAttentionImpl.forward``: for a selected layer whose plan is direct
  and whose tensors pass every gate, the chunk's K/V are written into the
  paged cache (``trianglemix::reshape_and_cache``) and the chunk runs through
  one launch of the sparse op; every other call, and any failure on the way
  (fail-open, counted; raised in strict mode), runs the original forward
  unchanged, which writes the K/V itself (plugin.py:1358-1587).

Routing and counting go through ``TriangleMixRouter`` and the process
``runtime_stats()``, so counters, fallback reasons and structured log lines
are the same as for any other caller.  Before patching, the wrapped methods'
signatures are compared with an allowlist; a mismatch leaves vLLM untouched
(``runtime_error_stage:unsupported_version``, raised in strict mode), and a
failure halfway restores every attribute it had set
(plugin.py:1590-1702).  No vLLM-ROCm build was available to pin version
strings against, so the signatures are the compatibility contract.

vLLM loads the seam through its ``vllm.general_plugins`` entry point::

    [project.entry-points."vllm.general_plugins"]
    trianglemix_rocm = "trianglemix.vllm_rocm:register"
"""

from __future__ import annotations

import functools
import importlib
import inspect
import itertools
import logging
import os
import threading
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from typing import Any, Callable

from .config import PluginConfig
from .kernel import TriangleMixConfig
from .planning import TriangleBatchPlan, build_batch_plan
from .router import LayerFeatures, TriangleMixRouter, device_plugin_config, leading_rows
from .stats import runtime_stats

logger = logging.getLogger("vllm.trianglemix.rocm")

BACKEND_MODULE = "vllm.v1.attention.backends.triton_attn"
RUNNER_MODULE = "vllm.v1.worker.gpu_model_runner"
BUILDER_CLASS = "TritonAttentionMetadataBuilder"
IMPL_CLASS = "TritonAttentionImpl"
RUNNER_CLASS = "GPUModelRunner"

_MARK = "_trianglemix_rocm_patched"
_CONFIG_ATTR = "_trianglemix_rocm_config"
_ROUTER_ATTR = "_trianglemix_rocm_router"
_PLAN_ATTR = "_trianglemix_rocm_plan"
_CAPTURE_ATTR = "_trianglemix_rocm_capture"
_KV_SPLIT_ATTR = "_trianglemix_rocm_kv_split"  # (kv_cache, key view, value view) of the layer's last call
_MISSING = object()
_REQUIRED = "required"

_PATCH_LOCK = threading.Lock()
_REGISTERED = False
_STEP_TOKENS = itertools.count(1)
_STEP = threading.local()


class UnsupportedFramework(RuntimeError):
    """The installed vLLM does not offer the methods this seam wraps, with the expected signatures."""


# --------------------------------------------------------------- signatures
def _p(name: str, default: object = _REQUIRED, kind: str = "POSITIONAL_OR_KEYWORD") -> tuple[str, str, str]:
    return name, kind, default if default is _REQUIRED else repr(default)


SIGNATURES: dict[str, tuple[tuple[str, str, str], ...]] = {
    "builder.build": (_p("self"), _p("common_prefix_len"), _p("common_attn_metadata"), _p("fast_build", False)),
    "builder.build_for_cudagraph_capture": (_p("self"), _p("common_attn_metadata")),
    "impl.forward": (_p("self"), _p("layer"), _p("query"), _p("key"), _p("value"), _p("kv_cache"),
                     _p("attn_metadata"), _p("output", None), _p("output_scale", None),
                     _p("output_block_scale", None)),
    "runner._prepare_inputs": (_p("self"), _p("scheduler_output")),
}


def signature_key(fn: object) -> tuple[tuple[str, str, str], ...]:
    """(name, kind, default) of each parameter; a default is compared by its repr."""
    try:
        sig = inspect.signature(fn)
    except (TypeError, ValueError) as exc:
        raise UnsupportedFramework(f"cannot inspect the signature of {fn!r}") from exc
    return tuple((p.name, p.kind.name, _REQUIRED if p.default is inspect.Parameter.empty else repr(p.default))
                 for p in sig.parameters.values())


def _check(name: str, fn: object) -> None:
    if not callable(fn):
        raise UnsupportedFramework(f"unsupported_version: {name} is missing")
    if signature_key(fn) != SIGNATURES[name]:
        raise UnsupportedFramework(f"unsupported_version: {name} signature is not allowlisted")


# -------------------------------------------------------------- step prompt
def _ints(value: object) -> list[int] | None:
    if value is None:
        return None
    if hasattr(value, "tolist"):
        value = value.tolist()
    try:
        return [int(v) for v in value]  # type: ignore[union-attr]
    except (TypeError, ValueError):
        return None


def runner_prompt(runner: object) -> tuple[int, ...] | None:
    """Final prompt lengths of the step's requests (batch order), or None.

    None under speculative decoding (draft tokens make the query lengths
    differ from the scheduled chunk) or when any length is missing; the
    planner itself turns batches above one into ``batch_unsupported``.
    """
    batch = getattr(runner, "input_batch", None)
    try:
        num_reqs = int(getattr(batch, "num_reqs"))
    except (TypeError, ValueError, AttributeError):
        return None
    if num_reqs <= 0 or getattr(runner, "speculative_config", None) is not None:
        return None
    values = _ints(getattr(batch, "num_prompt_tokens", None))
    if not values or len(values) < num_reqs or min(values[:num_reqs]) <= 0:
        return None
    return tuple(values[:num_reqs])


@dataclass(frozen=True)
class _StepPrompt:
    prompt_lens: tuple[int, ...] | None
    token: int


def _current_step() -> _StepPrompt | None:
    return getattr(_STEP, "value", None)


# ------------------------------------------------------------ plan per step
class _PlanStore:
    """Plans attached to metadata objects, with a bounded side table for classes that refuse new attributes."""

    def __init__(self, capacity: int = 256) -> None:
        self._lock = threading.Lock()
        self._side: OrderedDict[int, tuple[Any, object, object]] = OrderedDict()
        self._capacity = capacity

    def _ref(self, obj: object):
        try:
            return weakref.ref(obj), None
        except TypeError:
            return None, obj

    def _side_put(self, obj: object, attr: str, value: object) -> None:
        ref, strong = self._ref(obj)
        with self._lock:
            key = (id(obj), attr)
            self._side[key] = (ref, strong, value)
            self._side.move_to_end(key)
            while len(self._side) > self._capacity:
                self._side.popitem(last=False)

    def _side_get(self, obj: object, attr: str) -> object:
        with self._lock:
            entry = self._side.get((id(obj), attr))
            if entry is None:
                return None
            ref, strong, value = entry
            if (ref() if ref is not None else strong) is not obj:
                del self._side[(id(obj), attr)]
                return None
            return value

    def put(self, obj: object, attr: str, value: object) -> None:
        try:
            setattr(obj, attr, value)
        except (AttributeError, TypeError):
            self._side_put(obj, attr, value)

    def get(self, obj: object, attr: str) -> object:
        value = getattr(obj, attr, None)
        return value if value is not None else self._side_get(obj, attr)


_STORE = _PlanStore()


def plan_from_common(common: object, config: TriangleMixConfig,
                     prompt_lens: tuple[int, ...] | None) -> TriangleBatchPlan:
    """The step's plan from vLLM's ``CommonAttentionMetadata`` (CPU fields only).

    The state follows from the query lengths: all one-token queries are a
    decode step; one request whose query is its whole sequence is a cache-less
    prefill; anything else with a longer query is a chunked prefill (the
    planner then rejects decodes mixed in and batches above one).
    """
    starts = _ints(getattr(common, "query_start_loc_cpu", None))
    seqs = _ints(getattr(common, "seq_lens_cpu", None))
    num_reqs = int(getattr(common, "num_reqs", 0) or 0)
    if not starts or not seqs or num_reqs <= 0 or len(starts) < num_reqs + 1 or len(seqs) < num_reqs:
        return build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=None, seq_lens=None,
                                prompt_lens=None, num_decodes=0, num_prefills=0, config=config)
    qlens = [starts[i + 1] - starts[i] for i in range(num_reqs)]
    decodes = sum(1 for q in qlens if q <= 1)
    if decodes == num_reqs:
        state = "DecodeOnly"
    elif num_reqs == 1 and qlens[0] == seqs[0]:
        state = "PrefillNoCache"
    else:
        state = "ChunkedPrefill"
    if prompt_lens is None:
        for name in ("num_prompt_tokens_cpu", "prompt_lens_cpu", "prompt_lens"):
            found = _ints(getattr(common, name, None))
            if found:
                prompt_lens = tuple(found[:num_reqs])
                break
    ends = [s - starts[0] for s in starts[1:num_reqs + 1]]
    return build_batch_plan(state_name=state, cumulative_query_ends=ends, seq_lens=seqs[:num_reqs],
                            prompt_lens=prompt_lens, num_decodes=decodes, num_prefills=num_reqs - decodes,
                            config=config)


# ----------------------------------------------------------------- config
def _strict_env() -> bool:
    return os.getenv("VLLM_ASCEND_TRIANGLE_MIX_STRICT", "false").strip().lower() in {"1", "true", "yes", "on"}


def _current_vllm_config() -> object | None:
    try:
        from vllm.config import get_current_vllm_config

        return get_current_vllm_config()
    except Exception:
        return None


def config_of(owner: object) -> PluginConfig:
    """Plugin config of a builder / impl (its ``vllm_config`` or vLLM's current one), resolved once per owner.

    An invalid configuration counts ``runtime_error_stage:config`` and turns
    the feature off (raised in strict mode).
    """
    cached = getattr(owner, _CONFIG_ATTR, None)
    if isinstance(cached, PluginConfig):
        return cached
    vllm_config = getattr(owner, "vllm_config", None) or _current_vllm_config()
    try:
        config = device_plugin_config(vllm_config)
    except Exception:
        runtime_stats().record_runtime_error(stage="config")
        if _strict_env():
            raise
        logger.exception("TriangleMix configuration is invalid; vLLM's attention stays in use")
        config = PluginConfig(kernel=TriangleMixConfig(enabled=False, layer_indices=frozenset()))
    try:
        setattr(owner, _CONFIG_ATTR, config)
    except (AttributeError, TypeError):
        pass
    return config


# ----------------------------------------------------------------- wrappers
@dataclass
class SeamOps:
    """The device calls of the direct path (tests substitute them on the CPU)."""

    direct: Callable[..., Any] | None = None      # default: the router's (kernel.triangle_direct_after_gates)
    kv_write: Callable[..., Any] | None = None    # default: cache.reshape_and_cache
    native_ready: Callable[[], bool] | None = None


OPS = SeamOps()


def _native_ready(config: PluginConfig) -> bool:
    if OPS.native_ready is not None:
        return OPS.native_ready()
    try:
        from .native import ensure_native_loaded

        status = ensure_native_loaded(strict=config.strict)
        if status.ready:
            return True
        reason = status.reason
    except Exception as exc:
        if config.strict:
            runtime_stats().record_runtime_error(stage="native_bootstrap")
            raise
        reason = f"{type(exc).__name__}: {exc}"
    runtime_stats().record_runtime_error(stage="native_bootstrap")
    logger.warning("TriangleMix native runtime is unavailable (%s); vLLM's attention stays in use", reason)
    return False


def _router_of(impl: object, config: PluginConfig) -> TriangleMixRouter:
    router = getattr(impl, _ROUTER_ATTR, None)
    if isinstance(router, TriangleMixRouter) and router.config is config:
        return router
    kwargs: dict[str, Any] = {}
    if OPS.direct is not None:
        kwargs["direct_fn"] = OPS.direct
    ready = _native_ready(config)
    router = TriangleMixRouter(config, stats=runtime_stats(), native_ready=lambda: ready, **kwargs)
    setattr(impl, _ROUTER_ATTR, router)
    return router


def _tp_world_size(module: object) -> int | None:
    getter = getattr(module, "get_tensor_model_parallel_world_size", None)
    if not callable(getter):
        try:
            from vllm.distributed import get_tensor_model_parallel_world_size as getter
        except Exception:
            return None
    try:
        return int(getter())
    except Exception:
        return None


def _sliding_window(impl: object) -> object:
    window = getattr(impl, "sliding_window", None)
    # The Triton backend stores "no window" as (-1, -1).
    if window is None or (isinstance(window, (tuple, list)) and tuple(window) == (-1, -1)):
        return None
    return window


def _unsupported_mode(impl: object, output_scale: object, output_block_scale: object, metadata: object) -> bool:
    """Quantised output, a quantised KV cache, shared KV, soft-capped logits or cascade attention."""
    soft_cap = getattr(impl, "logits_soft_cap", None)
    return (output_scale is not None or output_block_scale is not None
            or str(getattr(impl, "kv_cache_dtype", "auto")) != "auto"
            or getattr(impl, "kv_sharing_target_layer_name", None) is not None
            or bool(soft_cap) or bool(getattr(metadata, "use_cascade", False)))


def _heads(t: object, heads: int, size: int) -> object:
    """``[tokens, heads, size]`` view of a ``[tokens, heads * size]`` tensor (3-D tensors as they are)."""
    shape = tuple(getattr(t, "shape", ()))
    if len(shape) == 2 and shape[1] == heads * size:
        return t.view(shape[0], heads, size)
    return t


@dataclass(frozen=True)
class _Routing:
    """What the builder attaches to one step's metadata: the plan and the config it was made under."""

    plan: TriangleBatchPlan
    config: PluginConfig


def _missing_plan(config: TriangleMixConfig) -> TriangleBatchPlan:
    return build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=None, seq_lens=None,
                            prompt_lens=None, num_decodes=0, num_prefills=0, config=config)


KV_FIRST = "kv_first"          # [2, blocks, 128, 8, 128]: K and V are contiguous page arrays
BLOCKS_FIRST = "blocks_first"  # [blocks, 2, 128, 8, 128]: K and V pages interleave


def kv_cache_layout(backend_module: object) -> str | None:
    """The paged KV cache layout the backend allocates, read from its own shape rule.

    ``TritonAttentionBackend.get_kv_cache_shape`` is asked for a cache of 3
    blocks: the axis of length 2 that sits next to the one of length 3 tells
    K/V-first from blocks-first.  None when the backend offers no such rule
    or its answer fits neither layout.
    """
    backend = getattr(backend_module, "TritonAttentionBackend", None)
    rule = getattr(backend, "get_kv_cache_shape", None)
    if not callable(rule):
        return None
    try:
        shape = tuple(int(x) for x in rule(3, 128, 8, 128))
    except Exception:
        return None
    if len(shape) == 5 and shape[:2] == (2, 3):
        return KV_FIRST
    if len(shape) == 5 and shape[:2] == (3, 2):
        return BLOCKS_FIRST
    return None


def _split_kv(kv_cache: object, layout: str | None) -> tuple[object, object]:
    """(key cache, value cache) views of a layer's KV cache, or (None, None) when they cannot be found.

    A blocks-first cache splits on dim 1; its K and V views step two pages
    per block, which the op's contiguous page layout does not take, so the
    router falls back with ``kv_cache_unsupported``.  Without a layout from
    the backend, a 5-D cache counts as K/V-first only when that reading is
    unambiguous (dim 0 is 2 and dim 1 is not): a 2-block cache could be
    either and is refused.
    """
    if isinstance(kv_cache, (tuple, list)) and len(kv_cache) == 2:
        return kv_cache[0], kv_cache[1]
    shape = tuple(getattr(kv_cache, "shape", ()))
    if len(shape) != 5:
        return None, None
    if layout == KV_FIRST and shape[0] == 2:
        return kv_cache[0], kv_cache[1]
    if layout == BLOCKS_FIRST and shape[1] == 2:
        return kv_cache[:, 0], kv_cache[:, 1]
    if layout is None and shape[0] == 2 and shape[1] != 2:
        return kv_cache[0], kv_cache[1]
    return None, None


def _capturing(metadata: object) -> bool:
    if _STORE.get(metadata, _CAPTURE_ATTR):
        return True
    try:
        import torch

        return bool(torch.cuda.is_available() and torch.cuda.is_current_stream_capturing())
    except Exception:
        return True


def _wrap_builder(builder_cls: type) -> list[tuple[object, str, object]]:
    original_build = builder_cls.build
    original_capture = getattr(builder_cls, "build_for_cudagraph_capture", None)

    @functools.wraps(original_build)
    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        metadata = original_build(self, common_prefix_len, common_attn_metadata, fast_build)
        config = config_of(self)
        if not config.enabled:
            return metadata
        step = _current_step()
        try:
            plan = plan_from_common(common_attn_metadata, config.kernel,
                                    step.prompt_lens if step is not None else None)
        except Exception:
            runtime_stats().record_runtime_error(stage="metadata_build")
            if config.strict:
                raise
            logger.exception("TriangleMix metadata planning failed; vLLM's attention stays in use")
            plan = _missing_plan(config.kernel)
        _STORE.put(metadata, _PLAN_ATTR, _Routing(plan, config))
        return metadata

    wrapped = [(builder_cls, "build", build)]
    if callable(original_capture):
        @functools.wraps(original_capture)
        def build_for_cudagraph_capture(self, common_attn_metadata):
            metadata = original_capture(self, common_attn_metadata)
            _STORE.put(metadata, _CAPTURE_ATTR, True)
            return metadata

        wrapped.append((builder_cls, "build_for_cudagraph_capture", build_for_cudagraph_capture))
    return wrapped


def _wrap_impl(impl_cls: type, backend_module: object) -> list[tuple[object, str, object]]:
    original = impl_cls.forward
    layout = kv_cache_layout(backend_module)

    @functools.wraps(original)
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                output_block_scale=None):
        def vllm_forward():
            return original(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                            output_block_scale)

        if attn_metadata is None or output is None:
            return vllm_forward()
        routing = _STORE.get(attn_metadata, _PLAN_ATTR)
        config = routing.config if isinstance(routing, _Routing) else config_of(self)
        layer_name = str(getattr(layer, "layer_name", ""))
        if not config.enabled or not config.kernel.uses_layer(layer_name):
            return vllm_forward()
        if isinstance(routing, _Routing):
            plan = routing.plan
        else:
            # Metadata that did not come through the patched builder: no plan, so no direct launch.
            plan = _missing_plan(config.kernel)
            _STORE.put(attn_metadata, _PLAN_ATTR, _Routing(plan, config))
        heads, kv_heads = int(getattr(self, "num_heads", 0)), int(getattr(self, "num_kv_heads", 0))
        size = int(getattr(self, "head_size", 0))
        split = getattr(self, _KV_SPLIT_ATTR, None)
        if split is not None and split[0] is kv_cache:
            key_cache, value_cache = split[1], split[2]
        else:
            key_cache, value_cache = _split_kv(kv_cache, layout)
            setattr(self, _KV_SPLIT_ATTR, (kv_cache, key_cache, value_cache))
        features = LayerFeatures(
            num_heads=heads, num_kv_heads=kv_heads, head_size=size,
            causal=bool(getattr(attn_metadata, "causal", True)),
            tensor_parallel_size=_tp_world_size(backend_module) or 0, context_parallel=False,
            sliding_window=_sliding_window(self), sinks=getattr(self, "sinks", None),
            alibi_slopes=getattr(self, "alibi_slopes", None), attn_type=str(getattr(self, "attn_type", "decoder")),
            unsupported_mode=_unsupported_mode(self, output_scale, output_block_scale, attn_metadata))
        # vLLM may pad the token dimension; the direct path sees the chunk's own rows only.
        rows = plan.requests[0].query_len if plan.direct else int(getattr(query, "shape", (0,))[0])
        q_rows = leading_rows(_heads(query, heads, size), rows)
        out_rows = leading_rows(_heads(output, heads, size), rows)

        def write_kv():
            kv_write = OPS.kv_write
            if kv_write is None:
                from .cache import reshape_and_cache as kv_write
            kv_write(leading_rows(_heads(key, kv_heads, size), rows), leading_rows(_heads(value, kv_heads, size), rows),
                     key_cache, value_cache, leading_rows(attn_metadata.slot_mapping, rows))

        router = _router_of(self, config)
        router.prefill_attention(
            layer_name=layer_name, plan=plan, query=q_rows, key_cache=key_cache, value_cache=value_cache,
            block_table=getattr(attn_metadata, "block_table", None), output=out_rows,
            softmax_scale=float(getattr(self, "scale")), features=features, capturing=_capturing(attn_metadata),
            fallback=vllm_forward, before_direct=write_kv)
        return output

    return [(impl_cls, "forward", forward)]


def _wrap_runner(runner_cls: type) -> list[tuple[object, str, object]]:
    original = runner_cls._prepare_inputs

    @functools.wraps(original)
    def _prepare_inputs(self, scheduler_output):
        previous = _current_step()
        _STEP.value = _StepPrompt(runner_prompt(self), next(_STEP_TOKENS))
        try:
            return original(self, scheduler_output)
        finally:
            _STEP.value = previous

    return [(runner_cls, "_prepare_inputs", _prepare_inputs)]


# ------------------------------------------------------------------ patching
def preflight(backend_module: object, runner_module: object | None = None) -> tuple[type, type, type | None]:
    """The classes to patch, after checking every wrapped method against the allowlist."""
    builder_cls = getattr(backend_module, BUILDER_CLASS, None)
    impl_cls = getattr(backend_module, IMPL_CLASS, None)
    if not isinstance(builder_cls, type) or not isinstance(impl_cls, type):
        raise UnsupportedFramework("unsupported_version: the Triton attention builder or impl class is missing")
    _check("builder.build", getattr(builder_cls, "build", None))
    capture = getattr(builder_cls, "build_for_cudagraph_capture", None)
    if capture is not None:
        _check("builder.build_for_cudagraph_capture", capture)
    _check("impl.forward", getattr(impl_cls, "forward", None))
    runner_cls = None
    if runner_module is not None:
        runner_cls = getattr(runner_module, RUNNER_CLASS, None)
        if not isinstance(runner_cls, type):
            raise UnsupportedFramework("unsupported_version: GPUModelRunner is missing")
        _check("runner._prepare_inputs", getattr(runner_cls, "_prepare_inputs", None))
    return builder_cls, impl_cls, runner_cls


def _restore(saved: list[tuple[object, str, object]]) -> None:
    for owner, name, value in reversed(saved):
        if value is _MISSING:
            try:
                delattr(owner, name)
            except AttributeError:
                pass
        else:
            setattr(owner, name, value)


def patch_modules(backend_module: object, runner_module: object | None = None) -> bool:
    """Wrap the seam's methods (once); all-or-nothing.  Returns False when they were already wrapped."""
    builder_cls, impl_cls, runner_cls = preflight(backend_module, runner_module)
    owners = [c for c in (builder_cls, impl_cls, runner_cls) if c is not None]
    if all(vars(c).get(_MARK, False) for c in owners):
        return False
    plan: list[tuple[object, str, object]] = []
    if not vars(builder_cls).get(_MARK, False):
        plan += _wrap_builder(builder_cls) + [(builder_cls, _MARK, True)]
    if not vars(impl_cls).get(_MARK, False):
        plan += _wrap_impl(impl_cls, backend_module) + [(impl_cls, _MARK, True)]
    if runner_cls is not None and not vars(runner_cls).get(_MARK, False):
        plan += _wrap_runner(runner_cls) + [(runner_cls, _MARK, True)]
    applied: list[tuple[object, str, object]] = []  # (owner, name, previous value) of each attribute set
    try:
        for owner, name, value in plan:
            previous = vars(owner).get(name, _MISSING)
            setattr(owner, name, value)
            applied.append((owner, name, previous))
    except Exception:
        _restore(applied)
        raise
    return True


def register() -> None:
    """vLLM ``general_plugins`` entry point: patch the Triton attention backend and the GPU model runner.

    Any failure leaves vLLM's own attention in place; it is counted and
    logged, and raised when ``VLLM_ASCEND_TRIANGLE_MIX_STRICT`` is set.
    """
    global _REGISTERED
    with _PATCH_LOCK:
        if _REGISTERED:
            return
        try:
            backend = importlib.import_module(BACKEND_MODULE)
            runner = importlib.import_module(RUNNER_MODULE)
            patch_modules(backend, runner)
        except UnsupportedFramework:
            runtime_stats().record_runtime_error(stage="unsupported_version")
            if _strict_env():
                raise
            logger.warning("TriangleMix seam rejected the installed vLLM (reason=unsupported_version); "
                           "its attention stays in use", exc_info=True)
            return
        except Exception:
            runtime_stats().record_runtime_error(stage="plugin_register")
            if _strict_env():
                raise
            logger.exception("TriangleMix seam could not patch vLLM; its attention stays in use")
            return
        _REGISTERED = True


__all__ = ["register", "patch_modules", "preflight", "plan_from_common", "runner_prompt", "UnsupportedFramework",
           "SIGNATURES", "OPS"]
