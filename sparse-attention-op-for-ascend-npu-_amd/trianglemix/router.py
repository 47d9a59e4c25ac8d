"""Per-layer prefill routing: TriangleMix direct launch or dense fallback.

Engine-independent restatement of the reference's patched
``forward_fused_infer_attention`` decision
(package/src/vllm_ascend_trianglemix/plugin.py:1406-1535) and its gates
(``_dispatch_reason`` :1275-1324, ``_model_reason`` :1243-1272,
``_validate_query`` :1134-1167, ``_validate_static_kv`` :1106-1131,
``_validate_block_table`` :1170-1192), with the dense paged causal companion
kernel in the role of the official FIA kernel.

Order of the gates: not enabled / layer not selected / no plan -> dense
without counters; graph capture; plan not direct (the planner's reason);
native adapter not ready; model features (tensor / context parallel,
non-causal, geometry, sliding window, sinks, ALiBi, encoder); query/output;
KV cache; block table.  Any reason -> counters + dense.  A failing direct
launch is counted as ``runtime_error_stage:direct_launch`` and re-raised in
strict mode, else it falls back with ``DIRECT_LAUNCH_ERROR``.
"""

from __future__ import annotations

import logging
import math
import time
from dataclasses import dataclass
from typing import Any, Callable

from .config import PluginConfig, device_gate_profile, resolve_plugin_config
from .counters import log_if_due
from .kernel import (
    SUPPORTED_CACHE_BLOCK_SIZE,
    SUPPORTED_HEAD_SIZE,
    SUPPORTED_KV_HEADS,
    SUPPORTED_QUERY_HEADS,
    dense_paged_causal_attention,
    extract_layer_index,
    triangle_direct_after_gates,
)
from .native import routed_fast_path, triangle_mix_adapter_loaded
from .planning import FallbackReason, TriangleBatchPlan
from .stats import TriangleMixRuntimeStats, runtime_stats

logger = logging.getLogger("trianglemix.router")


@dataclass(frozen=True)
class LayerFeatures:
    """Model/parallel facts the reference reads from the vLLM backend."""

    num_heads: int = SUPPORTED_QUERY_HEADS
    num_kv_heads: int = SUPPORTED_KV_HEADS
    head_size: int = SUPPORTED_HEAD_SIZE
    causal: bool = True
    tensor_parallel_size: int = 1
    context_parallel: bool = False
    sliding_window: Any = None
    sinks: Any = None
    alibi_slopes: Any = None
    attn_type: str = "DECODER"
    # an engine feature the op does not implement (quantised output or KV
    # cache, shared KV, soft-capped logits, cascade attention)
    unsupported_mode: bool = False


def _dtype_name(dtype: object) -> str:
    return str(dtype).rsplit(".", 1)[-1]


def _contiguous(t: object) -> bool:
    fn = getattr(t, "is_contiguous", None)
    return bool(callable(fn) and fn())


def _shape(t: object) -> tuple[int, ...]:
    shape = getattr(t, "shape", ())
    # torch.Size is already a tuple of ints; anything else is normalised
    return shape if type(shape).__name__ == "Size" else tuple(int(x) for x in shape)


def leading_rows(t: Any, n: int) -> Any:
    """The first ``n`` rows of ``t`` (``t`` itself when it has exactly ``n``: no view to build per call)."""
    return t if t.shape[0] == n else t[:n]


def _model_reason(features: LayerFeatures, config: PluginConfig) -> FallbackReason:
    if features.tensor_parallel_size != 1:
        return FallbackReason.TENSOR_PARALLEL
    if features.context_parallel:
        return FallbackReason.CONTEXT_PARALLEL
    if not features.causal:
        return FallbackReason.NON_CAUSAL
    if not config.kernel.has_supported_geometry:
        return FallbackReason.GEOMETRY_UNSUPPORTED
    if (features.sliding_window is not None or features.sinks is not None or features.alibi_slopes is not None
            or features.unsupported_mode or "ENCODER" in features.attn_type.upper()):
        return FallbackReason.MODEL_UNSUPPORTED
    return FallbackReason.NONE


def _query_reason(features: LayerFeatures, query: object, output: object, plan: TriangleBatchPlan) -> FallbackReason:
    shape = _shape(query)
    if (len(shape) != 3 or shape[1:] != (SUPPORTED_QUERY_HEADS, SUPPORTED_HEAD_SIZE)
            or shape[0] != plan.requests[0].query_len or _dtype_name(getattr(query, "dtype", None)) != "bfloat16"
            or not _contiguous(query) or features.num_heads != SUPPORTED_QUERY_HEADS
            or features.num_kv_heads != SUPPORTED_KV_HEADS or features.head_size != SUPPORTED_HEAD_SIZE):
        return FallbackReason.QUERY_UNSUPPORTED
    oshape = _shape(output)
    if (not oshape or oshape[0] < shape[0] or _dtype_name(getattr(output, "dtype", None)) != "bfloat16"
            or getattr(output, "device", None) != getattr(query, "device", None) or not _contiguous(output)):
        return FallbackReason.QUERY_UNSUPPORTED
    return FallbackReason.NONE


def _kv_reason(key_cache: object, value_cache: object, query: object) -> FallbackReason:
    if key_cache is None or value_cache is None:
        return FallbackReason.KV_CACHE_UNSUPPORTED
    ks, vs = _shape(key_cache), _shape(value_cache)
    if (len(ks) != 4 or ks[1:] != (SUPPORTED_CACHE_BLOCK_SIZE, SUPPORTED_KV_HEADS, SUPPORTED_HEAD_SIZE) or vs != ks
            or _dtype_name(getattr(key_cache, "dtype", None)) != "bfloat16"
            or _dtype_name(getattr(value_cache, "dtype", None)) != "bfloat16"
            or getattr(key_cache, "device", None) != getattr(value_cache, "device", None)
            or not _contiguous(key_cache) or not _contiguous(value_cache)
            or getattr(key_cache, "device", None) != getattr(query, "device", None)):
        return FallbackReason.KV_CACHE_UNSUPPORTED
    return FallbackReason.NONE


def _block_table_reason(block_table: object, query: object, seq_len: int) -> FallbackReason:
    if block_table is None:
        return FallbackReason.BLOCK_TABLE_UNSUPPORTED
    shape = _shape(block_table)
    need = math.ceil(seq_len / SUPPORTED_CACHE_BLOCK_SIZE)
    if (len(shape) != 2 or shape[0] != 1 or shape[1] < need
            or _dtype_name(getattr(block_table, "dtype", None)) != "int32"
            or getattr(block_table, "device", None) != getattr(query, "device", None)
            or not _contiguous(block_table)):
        return FallbackReason.BLOCK_TABLE_UNSUPPORTED
    return FallbackReason.NONE


_TORCH_TYPES: tuple | None = None  # (torch.Tensor, torch.bfloat16, torch.int32) once torch is imported


def _torch_types() -> tuple:
    global _TORCH_TYPES
    if _TORCH_TYPES is None:
        import torch

        _TORCH_TYPES = (torch.Tensor, torch.bfloat16, torch.int32)
    return _TORCH_TYPES


def _tensor_reason(features: LayerFeatures, query, output, key_cache, value_cache, block_table,
                   query_len: int, seq_len: int) -> FallbackReason:
    """The query / output, KV cache and block table gates for torch tensors whose query is on a GPU, with
    the same predicates and order as ``_query_reason``, ``_kv_reason`` and ``_block_table_reason`` but read
    straight from the tensors (each routed call pays these checks).  Devices compare by index: with the
    query on a GPU, a tensor on the same device has the same index and any other tensor another index
    (-1 off the GPU)."""
    _, bf16, i32 = _torch_types()
    qs = query.shape
    if (len(qs) != 3 or qs[1] != SUPPORTED_QUERY_HEADS or qs[2] != SUPPORTED_HEAD_SIZE or qs[0] != query_len
            or query.dtype is not bf16 or not query.is_contiguous() or features.num_heads != SUPPORTED_QUERY_HEADS
            or features.num_kv_heads != SUPPORTED_KV_HEADS or features.head_size != SUPPORTED_HEAD_SIZE):
        return FallbackReason.QUERY_UNSUPPORTED
    device = query.get_device()
    os_ = output.shape
    if (not os_ or os_[0] < qs[0] or output.dtype is not bf16 or output.get_device() != device
            or not output.is_contiguous()):
        return FallbackReason.QUERY_UNSUPPORTED
    ks = key_cache.shape
    if (len(ks) != 4 or ks[1] != SUPPORTED_CACHE_BLOCK_SIZE or ks[2] != SUPPORTED_KV_HEADS
            or ks[3] != SUPPORTED_HEAD_SIZE or value_cache.shape != ks or key_cache.dtype is not bf16
            or value_cache.dtype is not bf16 or key_cache.get_device() != device
            or value_cache.get_device() != device or not key_cache.is_contiguous()
            or not value_cache.is_contiguous()):
        return FallbackReason.KV_CACHE_UNSUPPORTED
    bs = block_table.shape
    if (len(bs) != 2 or bs[0] != 1 or bs[1] < -(-seq_len // SUPPORTED_CACHE_BLOCK_SIZE)
            or block_table.dtype is not i32 or block_table.get_device() != device
            or not block_table.is_contiguous()):
        return FallbackReason.BLOCK_TABLE_UNSUPPORTED
    return FallbackReason.NONE


def _all_gpu_tensors(query, output, key_cache, value_cache, block_table) -> bool:
    tensor = _torch_types()[0]
    return (type(query) is tensor and type(output) is tensor and type(key_cache) is tensor
            and type(value_cache) is tensor and type(block_table) is tensor and query.is_cuda)


# tensor_gate's result codes (csrc/trianglemix_torch.cpp)
_GATE_CODES = (FallbackReason.NONE, FallbackReason.QUERY_UNSUPPORTED, FallbackReason.KV_CACHE_UNSUPPORTED,
               FallbackReason.BLOCK_TABLE_UNSUPPORTED)


def _call_reason(config: PluginConfig, plan: TriangleBatchPlan, features: LayerFeatures, capturing: bool,
                 native_ready: bool) -> FallbackReason:
    """The gates before the tensor gates: capture, the planner, the adapter, the model."""
    if capturing:
        return FallbackReason.GRAPH_CAPTURE
    if not plan.direct:
        return plan.primary_reason
    if not native_ready:
        return FallbackReason.ADAPTER_UNAVAILABLE
    return _model_reason(features, config)


def _head_counts_supported(features: LayerFeatures) -> bool:
    return (features.num_heads == SUPPORTED_QUERY_HEADS and features.num_kv_heads == SUPPORTED_KV_HEADS
            and features.head_size == SUPPORTED_HEAD_SIZE)


def dispatch_reason(*, config: PluginConfig, plan: TriangleBatchPlan, features: LayerFeatures, query: object,
                    output: object, key_cache: object, value_cache: object, block_table: object,
                    capturing: bool, native_ready: bool) -> FallbackReason:
    """First failing gate for a selected layer, or ``FallbackReason.NONE``."""
    reason = _call_reason(config, plan, features, capturing, native_ready)
    if reason is not FallbackReason.NONE:
        return reason
    tensor = _torch_types()[0]
    if (type(query) is tensor and type(output) is tensor and type(key_cache) is tensor
            and type(value_cache) is tensor and type(block_table) is tensor and query.is_cuda):
        request = plan.requests[0]
        fast = routed_fast_path()
        if fast is None:
            return _tensor_reason(features, query, output, key_cache, value_cache, block_table, request.query_len,
                                  request.seq_len)
        # the same gates in one native call (the adapter's tensor_gate); the layer's head counts stay here
        if not _head_counts_supported(features):
            return FallbackReason.QUERY_UNSUPPORTED
        return _GATE_CODES[fast.tensor_gate(query, output, key_cache, value_cache, block_table, request.query_len,
                                            request.seq_len)]
    for reason in (_query_reason(features, query, output, plan), _kv_reason(key_cache, value_cache, query)):
        if reason is not FallbackReason.NONE:
            return reason
    return _block_table_reason(block_table, query, plan.requests[0].seq_len)


def device_plugin_config(vllm_config: object | None, device: object | None = None) -> PluginConfig:
    """``resolve_plugin_config`` with the plan gates measured on the GPU this process runs on (the
    ``mi355x`` profile on gfx950: every chunk with a sparse middle goes direct) unless the configuration or
    the environment names a ``gate_profile`` (``"reference"`` keeps the reference's 910B gates)."""
    return resolve_plugin_config(vllm_config, default_gate_profile=device_gate_profile(device))


class TriangleMixRouter:
    """Routes one layer's prefill attention for the current scheduler step.

    ``direct_fn`` / ``dense_fn`` default to the gfx950 ops (the direct one
    without the Python pre-checks the router's gates already made); tests
    substitute them to force failure paths on the CPU.
    """

    def __init__(self, config: PluginConfig, *, stats: TriangleMixRuntimeStats | None = None,
                 direct_fn: Callable[..., Any] = triangle_direct_after_gates,
                 dense_fn: Callable[..., Any] = dense_paged_causal_attention,
                 native_ready: Callable[[], bool] = triangle_mix_adapter_loaded) -> None:
        self.config = config
        self.stats = stats if stats is not None else runtime_stats()
        self.stats.configure(config.stats_recent_capacity, config.stats_log_interval)
        self._direct = direct_fn
        self._dense = dense_fn
        self._native_ready = native_ready
        # With the default ops, GPU tensors launch through the adapter's routed-call entry points.
        self._native_direct = direct_fn is triangle_direct_after_gates
        self._native_dense = dense_fn is dense_paged_causal_attention
        self._layers: dict[str, tuple[bool, int | None]] = {}  # layer name -> (selected, layer index)
        self._ready = False  # the adapter was seen loaded (it stays loaded)

    def _layer(self, layer_name: str) -> tuple[bool, int | None]:
        known = self._layers.get(layer_name)
        if known is None:
            known = (self.config.kernel.uses_layer(layer_name), extract_layer_index(layer_name))
            if len(self._layers) < 4096:
                self._layers[layer_name] = known
        return known

    def _dense_fallback(self, *, query, key_cache, value_cache, block_table, seq_len: int, output, scale: float):
        if self._native_dense and type(query) is _torch_types()[0] and query.is_cuda:
            fast = routed_fast_path()
            if fast is not None:
                fast.launch_dense(query, key_cache, value_cache, block_table, seq_len, scale, output)
                return output
        view = output[: query.shape[0]]
        return self._dense(query=query, key_cache=key_cache, value_cache=value_cache, block_table=block_table,
                           seq_len=seq_len, output=view, softmax_scale=scale)

    def _log_if_due(self) -> None:
        log_if_due(self.stats, logger)

    def _launch_failed(self, plan: TriangleBatchPlan, layer_index: int | None, layer_name: str,
                       dense: Callable[[], Any]):
        """A failing direct launch (called from its ``except``): counted, raised in strict mode, else the
        fallback path."""
        self.stats.record_runtime_error(stage="direct_launch")
        if self.config.strict:
            raise
        logger.exception("TriangleMix direct launch failed at layer %s; using the fallback path", layer_name)
        self._count_fallback(plan, layer_index, FallbackReason.DIRECT_LAUNCH_ERROR)
        return dense()

    def _count_fallback(self, plan: TriangleBatchPlan, layer_index: int | None, reason: FallbackReason) -> None:
        # Graph-capture metadata is a reusable dummy, not a scheduled request.
        if reason is not FallbackReason.GRAPH_CAPTURE:
            self.stats.record_planner_decision(plan)
        self.stats.record_layer_fallback(
            plan_id=plan.plan_id, layer_index=layer_index, reason=reason,
            request_indices=tuple(r.request_index for r in plan.requests[:plan.batch_size]))
        self._log_if_due()

    def prefill_attention(self, *, layer_name: str, plan: TriangleBatchPlan | None, query, key_cache, value_cache,
                          block_table, output, softmax_scale: float, features: LayerFeatures = LayerFeatures(),
                          capturing: bool = False, fallback: Callable[[], Any] | None = None,
                          before_direct: Callable[[], None] | None = None):
        """Attention of one layer for the step's chunk, written into ``output``.

        ``fallback`` replaces the dense companion kernel as the non-direct
        path (an engine passes its own attention call); ``before_direct`` runs
        once the direct path is chosen, right before the launch (an engine
        writes the chunk's K/V into the cache there).  A failure in either
        one, like a failing launch, is counted and falls back.
        """
        def dense():
            if fallback is not None:
                return fallback()
            if plan is None:
                raise ValueError("dense fallback needs the chunk's seq_len from a plan")
            return self._dense_fallback(query=query, key_cache=key_cache, value_cache=value_cache,
                                        block_table=block_table, output=output, scale=softmax_scale,
                                        seq_len=plan.requests[0].seq_len)

        if not self.config.enabled or plan is None:
            return dense()
        selected, layer_index = self._layer(layer_name)
        if not selected:
            return dense()
        if not self._ready:
            self._ready = bool(self._native_ready())
        request = plan.requests[0]
        reason = _call_reason(self.config, plan, features, capturing, self._ready)
        if (reason is FallbackReason.NONE and before_direct is None and self._native_direct
                and _head_counts_supported(features) and _all_gpu_tensors(query, output, key_cache, value_cache,
                                                                          block_table)):
            fast = routed_fast_path()
            if fast is not None:
                # the tensor gates and, when they pass, the launch in one native call
                started = time.perf_counter_ns()
                try:
                    code = fast.route_sparse(query, output, key_cache, value_cache, block_table, request.query_len,
                                             request.seq_len, request.prompt_len, float(softmax_scale))
                except Exception:
                    return self._launch_failed(plan, layer_index, layer_name, dense)
                if code:
                    self._count_fallback(plan, layer_index, _GATE_CODES[code])
                    return dense()
                self.stats.record_direct_launch(plan, layer_index=layer_index,
                                                host_enqueue_ns=time.perf_counter_ns() - started)
                self._log_if_due()
                return output
        if reason is FallbackReason.NONE:
            reason = dispatch_reason(config=self.config, plan=plan, features=features, query=query, output=output,
                                     key_cache=key_cache, value_cache=value_cache, block_table=block_table,
                                     capturing=capturing, native_ready=self._ready)
        if reason is not FallbackReason.NONE:
            self._count_fallback(plan, layer_index, reason)
            return dense()
        rows = request.query_len
        started = time.perf_counter_ns()
        try:
            if before_direct is not None:
                before_direct()
            fast = routed_fast_path() if self._native_direct and query.is_cuda else None
            if fast is not None:  # the gates passed: five torch tensors on the query's GPU, query of `rows` rows
                fast.launch_sparse(query, key_cache, value_cache, block_table, request.seq_len, request.prompt_len,
                                   float(softmax_scale), output)
            else:
                self._direct(query=leading_rows(query, rows), key_cache=key_cache, value_cache=value_cache,
                             block_table=block_table, seq_len=request.seq_len, prompt_len=request.prompt_len,
                             output=leading_rows(output, rows),
                             softmax_scale=float(softmax_scale), config=self.config.kernel)
        except Exception:
            return self._launch_failed(plan, layer_index, layer_name, dense)
        enqueue_ns = time.perf_counter_ns() - started
        self.stats.record_direct_launch(plan, layer_index=layer_index, host_enqueue_ns=enqueue_ns)
        self._log_if_due()
        return output
