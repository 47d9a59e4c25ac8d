"""Write ``policy_snapshots.json`` from the reference's plugin layer.

Imports package/src/vllm_ascend_trianglemix/{kernel,planning,stats,config}.py
from the reference checkout (this container only; the reference never
travels) and records what they return for the scenario in ``policy_ops.py``:
plan records for every ``PLAN_CASES`` input, the result of every stats
operation (snapshots, structured-log payloads, counters, errors) and the
resolved configuration (or error) of every ``CONFIG_CASES`` input.

Usage: ``python tests/golden/make_policy_snapshots.py [--reference /root/reference]``
"""

from __future__ import annotations

import argparse
import importlib
import json
import sys
import types
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

import policy_ops  # noqa: E402


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    src = Path(args.reference) / "package" / "src"
    if not (src / "vllm_ascend_trianglemix" / "stats.py").is_file():
        raise SystemExit(f"reference plugin layer not found under {src}")
    sys.path.insert(0, str(src))
    mods = types.SimpleNamespace(**{name: importlib.import_module(f"vllm_ascend_trianglemix.{name}")
                                    for name in ("kernel", "planning", "stats", "config")})
    data = {
        "source": "package/src/vllm_ascend_trianglemix/{kernel,planning,stats,config}.py of the reference, "
                  "driven by tests/golden/policy_ops.py (make_policy_snapshots.py)",
        "planning": policy_ops.run_planning(mods),
        "stats": policy_ops.run_stats(mods),
        "config": policy_ops.run_config(mods),
    }
    out = HERE / "policy_snapshots.json"
    out.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    print(f"wrote {out} ({out.stat().st_size} bytes): {len(data['planning'])} plans, {len(data['stats'])} stats ops, "
          f"{len(data['config'])} config cases")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
