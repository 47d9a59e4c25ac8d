"""TriangleMix paged sparse prefill attention for AMD MI355X (gfx950).

Host-side package around ``libtrianglemix.so`` (hand-written HIP kernels, C
ABI in ``include/trianglemix.h``) and ``_trianglemix_torch.so`` (the
``torch.ops.trianglemix`` / ``torch.ops.trianglemix_reference`` operators).

Modules mirror the reference's plugin package ``vllm_ascend_trianglemix``:
``kernel`` (op wrapper, span math), ``planning`` (per-step plan, fallback
reasons), ``config``, ``stats`` (counters), ``native`` (library bootstrap),
plus ``router`` (per-layer routing), ``vllm_rocm`` (the vLLM-ROCm seam:
``register`` patches vLLM v1's Triton attention backend), ``counters``
(structured counter log and its run aggregator), ``cache`` (paged KV write), ``calibrate``
(crossover gates), ``cabi`` (C ABI binding) and ``workload`` (seeded
synthetic chunks, work accounting).
"""

from .kernel import (  # noqa: F401
    TriangleMixConfig,
    TriangleSparseSpan,
    dense_paged_causal_attention,
    estimate_tile_counts,
    extract_layer_index,
    parse_layer_indices,
    triangle_direct_eligible,
    triangle_direct_paged_attention,
    triangle_saved_qk,
    triangle_sparse_span,
)
from .native import ensure_native_loaded, native_status  # noqa: F401
from .planning import FallbackReason, build_batch_plan  # noqa: F401
from .config import PluginConfig, resolve_plugin_config  # noqa: F401
from .stats import TriangleMixRuntimeStats, runtime_stats, stats_snapshot  # noqa: F401
