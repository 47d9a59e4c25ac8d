"""Typed TriangleMix configuration: additional_config > environment > defaults.

Mirror of package/src/vllm_ascend_trianglemix/config.py: the same keys,
precedence (``additional_config["trianglemix"]`` first, then the
``VLLM_ASCEND_TRIANGLE_MIX_*`` environment variables kept as the
compatibility interface, then defaults) and strict boolean coercion
(:16-29).  The environment names are kept verbatim so existing deployments
switch without edits.

One key is this build's own: ``gate_profile`` (environment
``VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE``) names a crossover profile measured
by ``trianglemix.calibrate`` -- a name under ``trianglemix/gate_profiles/``
(``"mi355x"`` ships) or a JSON path.  Its gates replace the defaults of the
five ``direct_*`` gate keys; explicit keys and environment variables still
win.  Unset, the reference's 910B-measured defaults apply unchanged.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path
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


_GATE_FIELDS = ("direct_min_seq_len", "direct_min_sparse_rows", "direct_min_saved_qk",
                "direct_split_min_sparse_rows", "direct_split_min_saved_qk")
GATE_PROFILE_DIR = Path(__file__).resolve().parent / "gate_profiles"


def load_gate_profile(name_or_path: str) -> dict[str, int]:
    """The five ``direct_*`` gates of a calibration profile (a shipped name or a JSON path)."""
    text = str(name_or_path).strip()
    path = Path(text) if text.endswith(".json") else GATE_PROFILE_DIR / f"{text}.json"
    if not path.is_file():
        raise ValueError(f"TriangleMix gate_profile {name_or_path!r} not found ({path})")
    gates = json.loads(path.read_text()).get("gates", {})
    missing = [f for f in _GATE_FIELDS if f not in gates]
    if missing:
        raise ValueError(f"TriangleMix gate_profile {name_or_path!r} lacks {missing}")
    return {f: int(gates[f]) for f in _GATE_FIELDS}


def resolve_plugin_config(vllm_config: object | None) -> PluginConfig:
    """Resolve typed config, preferring ``additional_config.trianglemix``."""
    additional = _mapping(getattr(vllm_config, "additional_config", None))
    section = _mapping(additional.get("trianglemix", additional))
    layers = _value(section, "layers", _ENV + "LAYERS", "")
    layers_text = ",".join(str(x) for x in layers) if isinstance(layers, (list, tuple, set)) else str(layers)
    profile = str(_value(section, "gate_profile", _ENV + "GATE_PROFILE", "") or "")
    profile_gates = load_gate_profile(profile) if profile else {}
    ints = {field: int(_value(section, key, env, profile_gates.get(field, default)))
            for key, env, default, field in _INT_KEYS}
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
