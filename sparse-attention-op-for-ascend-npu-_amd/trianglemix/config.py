"""Typed TriangleMix configuration: additional_config > environment > defaults.

Mirror of package/src/vllm_ascend_trianglemix/config.py: the same keys,
precedence (``additional_config["trianglemix"]`` first, then the
``VLLM_ASCEND_TRIANGLE_MIX_*`` environment variables kept as the
compatibility interface, then defaults) and strict boolean coercion
(:16-29).  The environment names are kept verbatim so existing deployments
switch without edits.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Mapping

from .kernel import TriangleMixConfig, parse_layer_indices

_TRUE = frozenset({"1", "true", "yes", "on"})
_FALSE = frozenset({"0", "false", "no", "off"})


def _coerce_bool(value: object, *, name: str) -> bool:
    if isinstance(value, bool):
        return value
    if isinstance(value, int) and value in (0, 1):
        return bool(value)
    if isinstance(value, str):
        text = value.strip().lower()
        if text in _TRUE:
            return True
        if text in _FALSE:
            return False
    raise ValueError(f"TriangleMix {name} must be a boolean, got {value!r}")


def _mapping(value: object) -> Mapping[str, Any]:
    return value if isinstance(value, Mapping) else {}


def _value(section: Mapping[str, Any], name: str, env_name: str, default: Any) -> Any:
    if name in section:
        return section[name]
    env = os.getenv(env_name)
    if env is None:
        return default
    if isinstance(default, bool):
        return _coerce_bool(env, name=env_name)
    if isinstance(default, int):
        return int(env)
    return env


@dataclass(frozen=True)
class PluginConfig:
    """Process configuration shared by the planner and the router."""

    kernel: TriangleMixConfig
    strict: bool = False
    stats_recent_capacity: int = 256
    stats_log_interval: int = 0

    @property
    def enabled(self) -> bool:
        return self.kernel.enabled and bool(self.kernel.layer_indices)


_ENV = "VLLM_ASCEND_TRIANGLE_MIX_"

# (config key, environment variable, default, TriangleMixConfig field)
_INT_KEYS = (
    ("sink_tokens", _ENV + "SINK_TOKENS", 8, "sink_tokens"),
    ("local_window", _ENV + "LOCAL_WINDOW", 512, "local_window"),
    ("last_rows", _ENV + "LAST_ROWS", 128, "last_rows"),
    ("min_seq_len", _ENV + "DIRECT_MIN_SEQ_LEN", 0, "direct_min_seq_len"),
    ("min_sparse_rows", _ENV + "DIRECT_MIN_SPARSE_ROWS", 128, "direct_min_sparse_rows"),
    ("min_saved_qk", _ENV + "DIRECT_MIN_SAVED_QK", 913_152, "direct_min_saved_qk"),
    ("split_min_sparse_rows", _ENV + "DIRECT_SPLIT_MIN_SPARSE_ROWS", 192, "direct_split_min_sparse_rows"),
    ("split_min_saved_qk", _ENV + "DIRECT_SPLIT_MIN_SAVED_QK", 1_299_264, "direct_split_min_saved_qk"),
)


def resolve_plugin_config(vllm_config: object | None) -> PluginConfig:
    """Resolve typed config, preferring ``additional_config.trianglemix``."""
    additional = _mapping(getattr(vllm_config, "additional_config", None))
    section = _mapping(additional.get("trianglemix", additional))
    layers = _value(section, "layers", _ENV + "LAYERS", "")
    layers_text = ",".join(str(x) for x in layers) if isinstance(layers, (list, tuple, set)) else str(layers)
    ints = {field: int(_value(section, key, env, default)) for key, env, default, field in _INT_KEYS}
    kernel = TriangleMixConfig(
        enabled=_coerce_bool(_value(section, "enabled", "VLLM_ASCEND_ENABLE_TRIANGLE_MIX", False), name="enabled"),
        layer_indices=parse_layer_indices(layers_text),
        **ints,
    )
    recent = int(_value(section, "stats_recent_capacity", _ENV + "STATS_RECENT_CAPACITY", 256))
    interval = int(_value(section, "stats_log_interval", _ENV + "STATS_LOG_INTERVAL", 0))
    if recent < 0 or interval < 0:
        raise ValueError("TriangleMix stats capacities must be non-negative")
    return PluginConfig(
        kernel=kernel,
        strict=_coerce_bool(_value(section, "strict", _ENV + "STRICT", False), name="strict"),
        stats_recent_capacity=recent,
        stats_log_interval=interval,
    )
