"""Crossover calibration of the plan gates (``trianglemix.calibrate``) and gate profiles in the config.

CPU only:

* ``fit_gates`` on synthetic points: the smallest gate from which every
  measured chunk passing it keeps the sparse path within the margin;
* the shipped MI355X profile is self-consistent (refitting its own points with
  its margin reproduces its gates, and its gates never send a measured chunk
  to a path more than the margin slower);
* ``gate_profile`` in the plugin config: the profile's gates replace the
  reference defaults, explicit keys and environment variables still win, an
  unknown profile is an error, and without it the reference defaults stay.
"""

from __future__ import annotations

import json

import pytest

from trianglemix import calibrate as CAL
from trianglemix.config import GATE_PROFILE_DIR, load_gate_profile, resolve_plugin_config


def _p(saved, rows, split, us_sparse, us_dense, q0=0):
    return CAL.Point(4096, 512, q0, 512, rows, saved, split, us_sparse, us_dense)


def test_fit_gates_picks_smallest_safe_thresholds():
    pts = [
        _p(0, 0, False, 10.0, 9.0),            # no sparse middle: never routed, ignored
        _p(50_000, 512, False, 12.0, 10.0),    # loses
        _p(300_000, 512, False, 9.0, 9.5),     # wins
        _p(2_000_000, 512, False, 8.0, 12.0),  # wins
        _p(100, 503, True, 10.5, 10.0),        # split, loses by 5 %
        _p(900_000, 503, True, 9.0, 11.0),     # split, wins
    ]
    g = CAL.fit_gates(pts, margin=0.02)
    assert g["direct_min_saved_qk"] == 300_000
    assert g["direct_split_min_saved_qk"] == 900_000
    assert g["direct_min_seq_len"] == 0
    # with a margin above the split loss it disappears
    assert CAL.fit_gates(pts, margin=0.06)["direct_split_min_saved_qk"] == 0
    # every point the fitted gates route to the sparse path is within the margin
    for p in pts:
        if CAL.passes(p, g):
            assert p.us_sparse <= p.us_dense * 1.02


def test_all_winning_points_give_zero_gates():
    pts = [_p(s, 256, split, 5.0, 9.0) for s in (10, 10_000, 10**6) for split in (False, True)]
    assert CAL.fit_gates(pts, 0.0) == {k: 0 for k in CAL.GATE_NAMES}


def test_route_cases_cover_every_chunk():
    cases = list(CAL.route_cases([1000], [256]))
    assert [c[2] for c in cases] == [0, 256, 512, 768]
    assert cases[-1][3] == 1000 - 768


def test_shipped_mi355x_profile_is_self_consistent():
    prof = json.loads((GATE_PROFILE_DIR / "mi355x.json").read_text())
    fields = set(CAL.Point.__dataclass_fields__)
    pts = [CAL.Point(**{k: v for k, v in p.items() if k in fields}) for p in prof["points"]]
    assert len(pts) >= 200 and prof["device"].startswith("gfx950")
    assert CAL.fit_gates(pts, prof["margin"]) == prof["gates"]
    assert prof["reference_gates"] == CAL.REFERENCE_GATES
    for p in pts:
        if CAL.passes(p, prof["gates"]):
            assert p.us_sparse <= p.us_dense * (1 + prof["margin"]), p
    # the fitted gates route the measured chunks at least as fast as the reference gates
    assert CAL.routed_time_us(pts, prof["gates"]) <= CAL.routed_time_us(pts, CAL.REFERENCE_GATES)


class _VllmConfig:
    def __init__(self, section):
        self.additional_config = {"trianglemix": section}


def test_gate_profile_replaces_reference_defaults(monkeypatch):
    for name in ("GATE_PROFILE", "DIRECT_MIN_SAVED_QK", "DIRECT_MIN_SPARSE_ROWS"):
        monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_" + name, raising=False)
    gates = load_gate_profile("mi355x")
    cfg = resolve_plugin_config(_VllmConfig({"enabled": True, "layers": "5", "gate_profile": "mi355x"})).kernel
    for field, value in gates.items():
        assert getattr(cfg, field) == value
    # explicit keys still win over the profile
    cfg2 = resolve_plugin_config(_VllmConfig({"gate_profile": "mi355x", "min_saved_qk": 7})).kernel
    assert cfg2.direct_min_saved_qk == 7
    # and so does the environment
    monkeypatch.setenv("VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SPARSE_ROWS", "33")
    cfg3 = resolve_plugin_config(_VllmConfig({"gate_profile": "mi355x"})).kernel
    assert cfg3.direct_min_sparse_rows == 33
    # the profile can also come from the environment, by path
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_DIRECT_MIN_SPARSE_ROWS")
    monkeypatch.setenv("VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE", str(GATE_PROFILE_DIR / "mi355x.json"))
    cfg4 = resolve_plugin_config(_VllmConfig({})).kernel
    assert cfg4.direct_split_min_saved_qk == gates["direct_split_min_saved_qk"]


def test_without_profile_reference_defaults_stay(monkeypatch):
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE", raising=False)
    cfg = resolve_plugin_config(_VllmConfig({})).kernel
    assert (cfg.direct_min_saved_qk, cfg.direct_split_min_saved_qk) == (913_152, 1_299_264)


def test_unknown_profile_is_an_error():
    with pytest.raises(ValueError, match="not found"):
        resolve_plugin_config(_VllmConfig({"gate_profile": "no_such_gpu"}))


def test_device_default_profile_and_reference_opt_out(monkeypatch):
    """The engine seam and ``router.device_plugin_config`` default to the profile measured on the GPU they run
    on; ``resolve_plugin_config`` alone keeps the reference's gates.  A configured or environment profile wins
    over the device default, and ``"reference"`` names the reference's own gates."""
    from trianglemix import config as C
    from trianglemix import router as R

    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE", raising=False)
    gates = load_gate_profile("mi355x")
    dev = resolve_plugin_config(_VllmConfig({}), default_gate_profile="mi355x").kernel
    assert all(getattr(dev, f) == v for f, v in gates.items())
    ref = resolve_plugin_config(_VllmConfig({"gate_profile": "reference"}), default_gate_profile="mi355x").kernel
    assert (ref.direct_min_saved_qk, ref.direct_split_min_saved_qk) == (913_152, 1_299_264)
    monkeypatch.setenv("VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE", "reference")
    env = resolve_plugin_config(_VllmConfig({}), default_gate_profile="mi355x").kernel
    assert env.direct_min_saved_qk == 913_152
    monkeypatch.delenv("VLLM_ASCEND_TRIANGLE_MIX_GATE_PROFILE")
    # the device lookup: gfx950 -> mi355x; no GPU (this container) -> none, so the reference gates
    assert C._DEVICE_PROFILES["gfx950"] == "mi355x" and (GATE_PROFILE_DIR / "mi355x.json").is_file()
    monkeypatch.setattr(C, "device_gate_profile", lambda device=None: "mi355x")
    monkeypatch.setattr(R, "device_gate_profile", lambda device=None: "mi355x")
    assert R.device_plugin_config(_VllmConfig({})).kernel.direct_min_saved_qk == gates["direct_min_saved_qk"]
    monkeypatch.setattr(R, "device_gate_profile", lambda device=None: "")
    assert R.device_plugin_config(_VllmConfig({})).kernel.direct_min_saved_qk == 913_152


def test_device_gate_profile_without_a_gpu():
    import torch

    from trianglemix.config import device_gate_profile
    if not torch.cuda.is_available():
        assert device_gate_profile() == ""
