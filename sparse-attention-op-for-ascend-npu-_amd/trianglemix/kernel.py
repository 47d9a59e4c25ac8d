"""Single-launch paged TriangleMix prefill attention: Python op wrapper.

Host-side mirror of the reference's op layer
(package/src/vllm_ascend_trianglemix/kernel.py), same names, argument meaning
and errors:

* fixed-geometry constants and ``TriangleMixConfig`` (kernel.py:39-104)
* ``TriangleSparseSpan`` / ``triangle_sparse_span`` / ``triangle_saved_qk`` /
  ``triangle_direct_eligible`` (kernel.py:107-269)
* layer-name parsing (kernel.py:145-177)
* ``_validate_direct_tensors`` / ``triangle_direct_paged_attention``
  (kernel.py:342-489): the whole chunk goes through one launch of
  ``torch.ops.trianglemix.triangle_paged_sparse_attention.out``
* ``estimate_tile_counts`` (kernel.py:492-522)

plus the dense paged causal companion ``dense_paged_causal_attention`` that
replaces the reference's official FIA fallback, and
``triangle_direct_after_gates``, the router's launch of a call that passed its
gates (the public function without the Python re-checks).  There is no CPU path: the
ops exist only for ROCm device tensors and the native adapter must be loaded.
"""

from __future__ import annotations

import functools
import math
import re
from dataclasses import dataclass

SUPPORTED_HEAD_SIZE = 128
SUPPORTED_CACHE_BLOCK_SIZE = 128
SUPPORTED_QUERY_HEADS = 32
SUPPORTED_KV_HEADS = 8
SUPPORTED_SINK_TOKENS = 8
SUPPORTED_LOCAL_WINDOW = 512
SUPPORTED_LAST_ROWS = 128
DEFAULT_BLOCK_M = 32
DEFAULT_BLOCK_N = 512


@dataclass(frozen=True)
class TriangleMixConfig:
    """Runtime configuration for direct paged TriangleMix attention."""

    enabled: bool
    layer_indices: frozenset[int]
    sink_tokens: int = SUPPORTED_SINK_TOKENS
    local_window: int = SUPPORTED_LOCAL_WINDOW
    last_rows: int = SUPPORTED_LAST_ROWS
    direct_min_seq_len: int = 0
    direct_min_sparse_rows: int = 128
    direct_min_saved_qk: int = 913_152
    direct_split_min_sparse_rows: int = 192
    direct_split_min_saved_qk: int = 1_299_264

    def __post_init__(self) -> None:
        if self.sink_tokens <= 0:
            raise ValueError("TriangleMix sink_tokens must be positive")
        if self.local_window < 0:
            raise ValueError("TriangleMix local_window must be non-negative")
        if self.last_rows <= 0:
            raise ValueError("TriangleMix last_rows must be positive")
        for name in ("direct_min_seq_len", "direct_min_sparse_rows", "direct_min_saved_qk",
                     "direct_split_min_sparse_rows", "direct_split_min_saved_qk"):
            if getattr(self, name) < 0:
                raise ValueError(f"TriangleMix {name} must be non-negative")

    @property
    def has_supported_geometry(self) -> bool:
        """Whether the fixed compiled kernel geometry matches this config."""
        return (self.sink_tokens == SUPPORTED_SINK_TOKENS
                and self.local_window == SUPPORTED_LOCAL_WINDOW
                and self.last_rows == SUPPORTED_LAST_ROWS)

    def uses_layer(self, layer_name: str) -> bool:
        index = extract_layer_index(layer_name)
        return index is not None and index in self.layer_indices


@dataclass(frozen=True)
class TriangleSparseSpan:
    """Absolute-coordinate plan of one scheduler prefill chunk.

    Rows ``[q0, q1)`` are computed; ``[s0, s1)`` is the sparse middle.
    """

    q0: int
    q1: int
    s0: int
    s1: int

    @property
    def query_rows(self) -> int:
        return self.q1 - self.q0

    @property
    def sparse_rows(self) -> int:
        return max(0, self.s1 - self.s0)

    @property
    def has_sparse_middle(self) -> bool:
        return self.s0 < self.s1

    @property
    def has_dense_prefix(self) -> bool:
        return self.has_sparse_middle and self.q0 < self.s0

    @property
    def has_dense_tail(self) -> bool:
        return self.has_sparse_middle and self.s1 < self.q1

    @property
    def is_split(self) -> bool:
        return self.has_dense_prefix or self.has_dense_tail

    @property
    def saved_qk(self) -> int:
        return triangle_saved_qk(self.s0, self.s1)


_LAYER_RE = re.compile(r"(?:^|\.)layers\.(\d+)(?:\.|$)")


@functools.lru_cache(maxsize=4096)
def extract_layer_index(layer_name: str) -> int | None:
    """Transformer layer index of a vLLM layer name (``model.layers.7.attn``); memoised, as the names of one
    model repeat every step."""
    match = _LAYER_RE.search(layer_name)
    return int(match.group(1)) if match else None


def parse_layer_indices(value: str) -> frozenset[int]:
    """Parse ``"5,7,10,15-35"`` into a set of indices (ranges inclusive)."""
    out: set[int] = set()
    for item in (part.strip() for part in value.split(",")):
        if not item:
            continue
        if "-" in item:
            lo_text, hi_text = item.split("-", 1)
            lo, hi = int(lo_text), int(hi_text)
            if lo < 0 or hi < lo:
                raise ValueError(f"Invalid TriangleMix layer range: {item!r}")
            out.update(range(lo, hi + 1))
        else:
            index = int(item)
            if index < 0:
                raise ValueError(f"Invalid TriangleMix layer index: {item!r}")
            out.add(index)
    return frozenset(out)


def triangle_streaming_start(config: TriangleMixConfig) -> int:
    """First absolute query row whose attended keys leave a gap (521)."""
    return config.sink_tokens + config.local_window + 1


def triangle_sparse_span(*, query_len: int, seq_len: int, prompt_len: int,
                         config: TriangleMixConfig) -> TriangleSparseSpan:
    if query_len < 0:
        raise ValueError("TriangleMix query_len must be non-negative")
    if seq_len < query_len:
        raise ValueError("TriangleMix seq_len must be at least query_len")
    if prompt_len < seq_len:
        raise ValueError("TriangleMix prompt_len must be at least seq_len")
    q0, q1 = seq_len - query_len, seq_len
    s0 = max(q0, triangle_streaming_start(config))
    s1 = min(q1, max(0, prompt_len - config.last_rows))
    return TriangleSparseSpan(q0=q0, q1=q1, s0=s0, s1=s1)


def triangle_sparse_query_rows(*, query_len: int, seq_len: int, prompt_len: int,
                               config: TriangleMixConfig) -> int:
    return triangle_sparse_span(query_len=query_len, seq_len=seq_len, prompt_len=prompt_len,
                                config=config).sparse_rows


def triangle_saved_qk(sparse_start: int, sparse_end: int) -> int:
    """Causal QK pairs skipped by sparse rows ``[sparse_start, sparse_end)``.

    Sparse row q keeps 521 of its q+1 causal keys, so it skips q-520; the sum
    of that arithmetic series is the closed form below.
    """
    if sparse_end <= sparse_start:
        return 0
    rows = sparse_end - sparse_start
    return rows * (sparse_start + sparse_end - 1041) // 2


def triangle_direct_eligible(*, query_len: int, seq_len: int, prompt_len: int,
                             config: TriangleMixConfig) -> bool:
    """Geometry and crossover gates for a structurally valid call."""
    if not config.has_supported_geometry:
        return False
    span = triangle_sparse_span(query_len=query_len, seq_len=seq_len, prompt_len=prompt_len, config=config)
    if not span.has_sparse_middle:
        return False
    if seq_len < config.direct_min_seq_len:
        return False
    if span.sparse_rows < config.direct_min_sparse_rows:
        return False
    if span.saved_qk < config.direct_min_saved_qk:
        return False
    if span.is_split and (span.sparse_rows < config.direct_split_min_sparse_rows
                          or span.saved_qk < config.direct_split_min_saved_qk):
        return False
    return True


def _validate_direct_tensors(*, query, key_cache, value_cache, block_table, output, seq_len: int) -> None:
    """Python pre-check of the op contract; raises ValueError (kernel.py:342-416)."""
    import torch

    if query.ndim != 3 or tuple(query.shape[1:]) != (SUPPORTED_QUERY_HEADS, SUPPORTED_HEAD_SIZE):
        raise ValueError("TriangleMix query must be [Tq, 32, 128]")
    if query.dtype != torch.bfloat16:
        raise ValueError("TriangleMix query must be BF16")
    if output.shape != query.shape or output.dtype != query.dtype:
        raise ValueError("TriangleMix output must match query shape and dtype")
    tail = (SUPPORTED_CACHE_BLOCK_SIZE, SUPPORTED_KV_HEADS, SUPPORTED_HEAD_SIZE)
    if key_cache.ndim != 4 or tuple(key_cache.shape[1:]) != tail or value_cache.shape != key_cache.shape:
        raise ValueError("TriangleMix KV caches must be [pages, 128, 8, 128]")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise ValueError("TriangleMix query and KV cache dtypes must match")
    if block_table.ndim != 2 or block_table.shape[0] != 1 or block_table.dtype != torch.int32:
        raise ValueError("TriangleMix block table must be INT32 [1, max_pages]")
    if not all(t.is_contiguous() for t in (query, key_cache, value_cache, block_table, output)):
        raise ValueError("TriangleMix tensors must be contiguous")
    if any(t.device != query.device for t in (key_cache, value_cache, block_table, output)):
        raise ValueError("TriangleMix tensors must share one device")
    if block_table.shape[1] < math.ceil(seq_len / SUPPORTED_CACHE_BLOCK_SIZE):
        raise ValueError("TriangleMix block table is too short for seq_len")


def _run_triangle_single_launch_out(*, query, key_cache, value_cache, block_table, query_start: int,
                                    seq_len: int, prompt_len: int, softmax_scale: float, output) -> None:
    """Run the whole query chunk through one launch of the gfx950 kernel."""
    import torch

    torch.ops.trianglemix.triangle_paged_sparse_attention.out(
        query, key_cache, value_cache, block_table, query_start, seq_len, prompt_len, softmax_scale, out=output)


def triangle_direct_paged_attention(*, query, key_cache, value_cache, block_table, seq_len: int,
                                    prompt_len: int, output, softmax_scale: float, config: TriangleMixConfig):
    """Dense prefix, sparse middle and dense tail of one chunk in one launch."""
    from .native import require_adapter

    span = triangle_sparse_span(query_len=query.shape[0], seq_len=seq_len, prompt_len=prompt_len, config=config)
    if not config.has_supported_geometry:
        raise ValueError("TriangleMix operator geometry does not match config")
    if not span.has_sparse_middle:
        raise ValueError("TriangleMix direct path requires a non-empty sparse middle")
    _validate_direct_tensors(query=query, key_cache=key_cache, value_cache=value_cache,
                             block_table=block_table, output=output, seq_len=seq_len)
    require_adapter()
    _run_triangle_single_launch_out(query=query, key_cache=key_cache, value_cache=value_cache,
                                    block_table=block_table, query_start=span.q0, seq_len=span.q1,
                                    prompt_len=prompt_len, softmax_scale=softmax_scale, output=output)
    return output


_SPARSE_OUT = None  # torch.ops.trianglemix.triangle_paged_sparse_attention.out, looked up once


def triangle_direct_after_gates(*, query, key_cache, value_cache, block_table, seq_len: int, prompt_len: int,
                                output, softmax_scale: float, config: TriangleMixConfig):
    """The router's direct launch: ``triangle_direct_paged_attention`` without its Python pre-checks.

    Only for a call that passed the router's gates (``router.dispatch_reason``):
    the planner's sparse-middle gate, the geometry gate, the adapter gate and
    the query / output / KV cache / block table gates cover every check of the
    public function, so repeating them on each of a step's layer calls is
    host time the GPU waits for.  The op still validates every tensor in C++
    before it launches.
    """
    global _SPARSE_OUT
    op = _SPARSE_OUT
    if op is None:
        import torch

        op = _SPARSE_OUT = torch.ops.trianglemix.triangle_paged_sparse_attention.out
    op(query, key_cache, value_cache, block_table, seq_len - query.shape[0], seq_len, prompt_len, softmax_scale,
       out=output)
    return output


def dense_paged_causal_attention(*, query, key_cache, value_cache, block_table, seq_len: int, output,
                                 softmax_scale: float):
    """Dense causal paged prefill of one chunk (rows [seq_len-Tq, seq_len)).

    The companion kernel for unselected layers and fallbacks; same tiles and
    launch path as the sparse kernel, with no sparse rows.
    """
    import torch

    from .native import require_adapter

    if seq_len < query.shape[0]:
        raise ValueError("TriangleMix seq_len must be at least query_len")
    _validate_direct_tensors(query=query, key_cache=key_cache, value_cache=value_cache,
                             block_table=block_table, output=output, seq_len=seq_len)
    require_adapter()
    torch.ops.trianglemix.dense_paged_causal_attention.out(
        query, key_cache, value_cache, block_table, seq_len - query.shape[0], seq_len, softmax_scale, out=output)
    return output


def estimate_tile_counts(seq_len: int, config: TriangleMixConfig, block_m: int = DEFAULT_BLOCK_M,
                         block_n: int = DEFAULT_BLOCK_N) -> tuple[int, int]:
    """Theoretical ``(triangle, dense)`` full-prompt QK tile counts (kernel.py:492-522)."""
    if seq_len < 0:
        raise ValueError("seq_len must be non-negative")
    if block_m <= 0 or block_n <= 0:
        raise ValueError("block sizes must be positive")
    triangle = dense = 0
    start = triangle_streaming_start(config)
    for q_lo in range(0, seq_len, block_m):
        q_hi = min(seq_len, q_lo + block_m)
        causal_tiles = -(-q_hi // block_n)
        dense += causal_tiles
        if q_hi <= start:
            triangle += causal_tiles
            continue
        sink_tiles = -(-config.sink_tokens // block_n)
        local_lo = max(config.sink_tokens, q_lo - config.local_window)
        local_tiles = causal_tiles - local_lo // block_n
        triangle += sink_tiles + max(0, local_tiles)
    return triangle, dense
