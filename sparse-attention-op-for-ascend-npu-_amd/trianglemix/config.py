"""Typed TriangleMix configuration: additional_config > environment > defaults.

The keys, their precedence (``additional_config["trianglemix"]`` first --
or the whole ``additional_config`` when it has no ``trianglemix`` section --
then the ``VLLM_ASCEND_TRIANGLE_MIX_*`` environment variables, then defaults),
the boolean spellings and the error messages are the reference's contract
(package/src/vllm_ascend_trianglemix/config.py); the environment names are
kept verbatim so existing deployments switch without edits.  Golden results
of the reference for a set of inputs pin it (tests/test_policy_golden.py).

Every setting is one ``_Setting`` row (key, environment variable,
default, kind); ``_Source`` looks a row up in the section, then the
environment, and parses it by kind.  Rows resolve in table order, so with
several bad values the first row's error is the one raised.

One key is this build's own: ``gate_profile`` (environment
``VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE``) names a crossover profile measured
by ``trianglemix.calibrate`` -- a name under ``trianglemix/gate_profiles/``
(``"mi355x"`` ships) or a JSON path; ``"reference"`` names the reference's
own gates.  Its gates replace the defaults of the five ``direct_*`` gate
keys; explicit keys and environment variables still win.  Unset,
``resolve_plugin_config`` takes its ``default_gate_profile`` argument, whose
default keeps the reference's 910B-measured gates; the engine seam and
``router.device_plugin_config`` pass ``device_gate_profile()``, the profile
measured on the GPU they run on (``"mi355x"`` on gfx950).
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Mapping, NamedTuple

from .kernel import TriangleMixConfig, parse_layer_indices

# Accepted spellings of a boolean (after strip + lower-case).
_BOOL_WORDS = {"1": True, "true": True, "yes": True, "on": True,
               "0": False, "false": False, "no": False, "off": False}


def _as_bool(value: object, label: str) -> bool:
    """``value`` as a boolean: a bool, the integers 0 / 1, or one of ``_BOOL_WORDS``; else ValueError."""
    if isinstance(value, bool):
        return value
    if isinstance(value, int) and value in (0, 1):
        return value == 1
    word = value.strip().lower() if isinstance(value, str) else None
    if word in _BOOL_WORDS:
        return _BOOL_WORDS[word]
    raise ValueError(f"TriangleMix {label} must be a boolean, got {value!r}")


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


class _Setting(NamedTuple):
    key: str                 # additional_config key
    env: str                 # environment variable
    default: Any
    kind: str                # "bool", "int", "layers" or "text"
    field: str | None = None  # TriangleMixConfig field, when the setting is one


# Resolution order (the order errors surface in): the kernel settings, then the stats
# settings, then ``strict``.
_KERNEL_SETTINGS = (
    _Setting("enabled", "VLLM_ASCEND_ENABLE_TRIANGLE_MIX", False, "bool", "enabled"),
    _Setting("layers", _ENV + "LAYERS", "", "layers", "layer_indices"),
    _Setting("sink_tokens", _ENV + "SINK_TOKENS", 8, "int", "sink_tokens"),
    _Setting("local_window", _ENV + "LOCAL_WINDOW", 512, "int", "local_window"),
    _Setting("last_rows", _ENV + "LAST_ROWS", 128, "int", "last_rows"),
    _Setting("min_seq_len", _ENV + "DIRECT_MIN_SEQ_LEN", 0, "int", "direct_min_seq_len"),
    _Setting("min_sparse_rows", _ENV + "DIRECT_MIN_SPARSE_ROWS", 128, "int", "direct_min_sparse_rows"),
    _Setting("min_saved_qk", _ENV + "DIRECT_MIN_SAVED_QK", 913_152, "int", "direct_min_saved_qk"),
    _Setting("split_min_sparse_rows", _ENV + "DIRECT_SPLIT_MIN_SPARSE_ROWS", 192, "int",
             "direct_split_min_sparse_rows"),
    _Setting("split_min_saved_qk", _ENV + "DIRECT_SPLIT_MIN_SAVED_QK", 1_299_264, "int",
             "direct_split_min_saved_qk"),
)
_RECENT_CAPACITY = _Setting("stats_recent_capacity", _ENV + "STATS_RECENT_CAPACITY", 256, "int")
_LOG_INTERVAL = _Setting("stats_log_interval", _ENV + "STATS_LOG_INTERVAL", 0, "int")
_STRICT = _Setting("strict", _ENV + "STRICT", False, "bool")
_GATE_PROFILE = _Setting("gate_profile", _ENV + "GATE_PROFILE", "", "text")


class _Source:
    """One ``additional_config`` section backed by the environment."""

    def __init__(self, vllm_config: object | None) -> None:
        additional = getattr(vllm_config, "additional_config", None)
        additional = additional if isinstance(additional, Mapping) else {}
        section = additional.get("trianglemix", additional)
        self.section: Mapping[str, Any] = section if isinstance(section, Mapping) else {}

    def get(self, setting: _Setting, default: Any = None) -> Any:
        """The setting's value, parsed by kind.  Section values are taken as given, environment strings
        are parsed first; ``default`` (when given) replaces the row's default."""
        default = setting.default if default is None else default
        if setting.key in self.section:
            raw, label = self.section[setting.key], setting.key
        elif setting.env in os.environ:
            text = os.environ[setting.env]
            # environment text becomes the default's type; errors name the variable
            raw = (_as_bool(text, setting.env) if setting.kind == "bool"
                   else int(text) if setting.kind == "int" else text)
            label = setting.key
        else:
            raw, label = default, setting.key
        if setting.kind == "bool":
            return _as_bool(raw, label)
        if setting.kind == "int":
            return int(raw)
        if setting.kind == "layers":
            text = ",".join(str(x) for x in raw) if isinstance(raw, (list, tuple, set)) else str(raw)
            return parse_layer_indices(text)
        return raw


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


# GPU architecture -> the gate profile measured on it.
_DEVICE_PROFILES = {"gfx950": "mi355x"}
REFERENCE_PROFILE = "reference"  # the reference's own (910B-measured) gates


def device_gate_profile(device: object | None = None) -> str:
    """The gate profile measured on the GPU ``device`` (default: the current one), or "" when none was."""
    try:
        import torch

        if not torch.cuda.is_available():
            return ""
        arch = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
        name = str(getattr(arch, "gcnArchName", "")).split(":")[0]
    except Exception:
        return ""
    return _DEVICE_PROFILES.get(name, "")


def resolve_plugin_config(vllm_config: object | None, *, default_gate_profile: str = "") -> PluginConfig:
    """Resolve the typed configuration, preferring ``additional_config.trianglemix``.

    ``default_gate_profile`` applies when neither the section nor the
    environment names a ``gate_profile``; by default the reference's gates.
    """
    source = _Source(vllm_config)
    profile = str(source.get(_GATE_PROFILE, default_gate_profile or None) or "").strip()
    profile_gates = load_gate_profile(profile) if profile and profile != REFERENCE_PROFILE else {}
    kernel = TriangleMixConfig(**{s.field: source.get(s, profile_gates.get(s.field)) for s in _KERNEL_SETTINGS})
    recent, interval = source.get(_RECENT_CAPACITY), source.get(_LOG_INTERVAL)
    if recent < 0 or interval < 0:
        raise ValueError("TriangleMix stats capacities must be non-negative")
    return PluginConfig(kernel=kernel, strict=source.get(_STRICT), stats_recent_capacity=recent,
                        stats_log_interval=interval)
