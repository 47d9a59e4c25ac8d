"""Fit the launch planner's costs to the forced-plan sweep (``tests/plan_sweep_mi355x.json``).

The planner (``choose_plan`` in ``sparse-attention-op-for-ascend-npu-_amd/csrc/trianglemix_capi.cpp``)
simulates the greedy dispatch of a plan's items onto a shape's slots: an item costs ``item_fixed +
per_iteration * ceil(tiles / KV parts)``, a split row block completes ``merge_fixed + merge_per_piece *
pieces`` after its last piece, and the plan takes its latest slot or split row block.  This script
restates that simulation (in C, compiled here with gcc, for speed) and

* without arguments: reports, per regime, the time the plans chosen under the costs in the C++ source lose
  to each geometry's fastest measured plan, on the fitted and on the held-out geometries;
* with ``--fit``: searches the costs of the two fitted regimes (TriangleMix chunks of at most 16 row
  blocks: quarters / halves; chunks of 17 row blocks or more: halves / KV whole) that minimise the summed
  relative loss on the geometries not held out (Nelder-Mead from many random starts), and reports them with
  their losses on both sets: the cross-check;
* with ``--fit --all``: the same search over every geometry, which is how the costs in the C++ source were
  made (after the cross-check held up).

The dense companion's chunks of at most 16 row blocks keep a fixed rule and integer costs (not fitted).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import re
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import plan_sweep  # noqa: E402

CAPI = HERE.parent / "sparse-attention-op-for-ascend-npu-_amd" / "csrc" / "trianglemix_capi.cpp"
SLOTS = {4: 16, 2: 32, 1: 64}

_SIM_C = r"""
#include <stdint.h>
// plan j: shape parameters prm[6*sh[j] .. +6] = (fixed, per_iteration, merge_fixed, merge_per_piece,
// slots, parts); row blocks rt[rb0[j] .. rb1[j]); tiles per item T[j].
void simulate(int nplans, const int* sh, const int* rb0, const int* rb1, const int* T, const int* rt,
              const double* prm, double* out) {
  double heap[128];
  for (int j = 0; j < nplans; ++j) {
    const double* p = prm + 6 * sh[j];
    const int slots = (int)p[4], parts = (int)p[5];
    for (int i = 0; i < slots; ++i) heap[i] = 0.0;
    double merged = 0.0;
    for (int r = rb0[j]; r < rb1[j]; ++r) {
      const int n = rt[r], k = (n + T[j] - 1) / T[j];
      double last = 0.0;
      for (int i = 0; i < k; ++i) {
        const int size = (int)((int64_t)(i + 1) * n / k - (int64_t)i * n / k);
        const double cost = p[0] + p[1] * (double)((size + parts - 1) / parts);
        const double v = heap[0] + cost;
        int a = 0;
        for (;;) {
          int l = 2 * a + 1, rr = l + 1, m = a;
          double mv = v;
          if (l < slots && heap[l] < mv) m = l, mv = heap[l];
          if (rr < slots && heap[rr] < mv) m = rr, mv = heap[rr];
          if (m == a) break;
          heap[a] = heap[m];
          a = m;
        }
        heap[a] = v;
        if (v > last) last = v;
      }
      if (k > 1 && last + p[2] + p[3] * k > merged) merged = last + p[2] + p[3] * k;
    }
    double end = merged;
    for (int i = 0; i < slots; ++i) if (heap[i] > end) end = heap[i];
    out[j] = end;
  }
}
"""


def _sim_lib():
    """The simulation built from _SIM_C into a temporary directory, loaded, and the directory removed (the
    loaded library stays mapped)."""
    with tempfile.TemporaryDirectory(prefix="plan_fit_") as tmp:
        d = Path(tmp)
        (d / "sim.c").write_text(_SIM_C)
        subprocess.run(["gcc", "-O2", "-shared", "-fPIC", str(d / "sim.c"), "-o", str(d / "sim.so")], check=True)
        return ctypes.CDLL(str(d / "sim.so"))


def source_costs() -> dict[str, list[float]]:
    """PlanModel constants of the C++ planner: name -> [fixed, per_iteration, merge_fixed, merge_per_piece]."""
    costs = {}
    for name, body in re.findall(r"constexpr PlanModel (k\w+)\{([^}]*)\}", CAPI.read_text()):
        vals = [float(x) for x in body.split(",")]
        costs[name] = vals[2:]
    return costs


# regime -> (shapes in the planner's order: (KV parts, cost name, smallest T, T from the ladder only))
REGIMES = {
    "small": [(4, "kSmallQuarters", 32, True), (2, "kSmallHalves", 24, False)],
    "large": [(2, "kLargeHalves", 16, False), (1, "kLargeWhole", 16, False)],
}


def regime_of(g) -> str | None:
    rbs = -(-g["query_tokens"] // 32)
    if rbs >= 17:
        return "large"
    return "small" if g["prompt_len"] else None


class Regime:
    """Every candidate plan of one regime's geometries, packed for the C simulation."""

    def __init__(self, lib, geoms, shapes):
        self.lib, self.shapes = lib, shapes
        sh, rb0, rb1, T, rt, us, gid = [], [], [], [], [], [], []
        self.best = []
        for gi, g in enumerate(geoms):
            tiles = plan_sweep.row_tiles(g["query_start"], g["query_tokens"], g["seq_len"], g["prompt_len"])
            off = len(rt)
            rt += tiles
            self.best.append(min(p[3] for p in g["plans"]))
            for si, (parts, _, lo, ladder) in enumerate(shapes):
                for p in g["plans"]:
                    if p[0] == parts and p[1] >= lo and (not ladder or p[1] <= 128):
                        sh.append(si); rb0.append(off); rb1.append(off + len(tiles)); T.append(p[1])
                        us.append(p[3]); gid.append(gi)
        a = lambda x: np.ascontiguousarray(np.array(x, dtype=np.int32))
        self.sh, self.rb0, self.rb1, self.T, self.rt = a(sh), a(rb0), a(rb1), a(T), a(rt)
        self.us, self.gid, self.best = np.array(us), np.array(gid), np.array(self.best)
        self.n, self.ng = len(sh), len(geoms)

    def losses(self, costs: list[float]) -> np.ndarray:
        """Per geometry: time of the plan the costs choose minus the fastest measured (us)."""
        prm = np.zeros(6 * len(self.shapes))
        for si, (parts, _, _, _) in enumerate(self.shapes):
            prm[6 * si:6 * si + 4] = costs[4 * si:4 * si + 4]
            prm[6 * si + 4], prm[6 * si + 5] = SLOTS[parts], parts
        out = np.zeros(self.n)
        ptr = lambda x: x.ctypes.data_as(ctypes.c_void_p)
        self.lib.simulate(ctypes.c_int(self.n), ptr(self.sh), ptr(self.rb0), ptr(self.rb1), ptr(self.T),
                          ptr(self.rt), ptr(np.ascontiguousarray(prm)), ptr(out))
        chosen = np.full(self.ng, -1)
        pred = np.full(self.ng, np.inf)
        for j in range(self.n):  # first strictly smaller: earlier shapes and larger T win ties
            g = self.gid[j]
            if out[j] < pred[g]:
                pred[g], chosen[g] = out[j], j
        return self.us[chosen] - self.best


def fit(reg: Regime, start: list[float], restarts: int, seed: int) -> list[float]:
    from scipy.optimize import minimize

    rng = np.random.default_rng(seed)
    objective = lambda x: float((reg.losses(np.abs(x)) / reg.best).sum()) + 1e-4 * float(np.abs(x).sum())
    best = (objective(np.array(start)), np.array(start))
    for _ in range(restarts):
        x0 = np.array([rng.uniform(0, 12), rng.uniform(0.3, 2), rng.uniform(0, 8), rng.uniform(0, 3)] * 2)
        r = minimize(objective, x0, method="Nelder-Mead", options={"maxfev": 2000})
        if r.fun < best[0]:
            best = (r.fun, np.abs(r.x))
    return [round(float(v), 3) for v in best[1]]


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--sweep", default=str(HERE / "plan_sweep_mi355x.json"))
    ap.add_argument("--fit", action="store_true")
    ap.add_argument("--all", action="store_true", help="with --fit: fit on every geometry, held out or not")
    ap.add_argument("--restarts", type=int, default=60)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()
    lib = _sim_lib()
    sweep = json.loads(Path(args.sweep).read_text())["geometries"]
    src = source_costs()
    for name, shapes in REGIMES.items():
        sets = {held: [g for g in sweep if regime_of(g) == name and g["held_out"] == held] for held in (False, True)}
        regs = {held: Regime(lib, gs, shapes) for held, gs in sets.items()}
        costs = [c for _, cname, _, _ in shapes for c in src[cname]]
        if args.fit:
            costs = fit(Regime(lib, sets[False] + sets[True], shapes) if args.all else regs[False], costs,
                        args.restarts, args.seed)
            print(f"{name}: fitted costs " + ", ".join(f"{cname}{{{', '.join(map(str, costs[4 * i:4 * i + 4]))}}}"
                                                       for i, (_, cname, _, _) in enumerate(shapes)))
        for held, reg in regs.items():
            loss = reg.losses(costs)
            print(f"{name} ({'held-out set' if held else 'fit set'}, {reg.ng} geometries): lose {loss.sum():.2f} us of "
                  f"{reg.best.sum():.1f} ({100 * loss.sum() / reg.best.sum():.2f} %), worst "
                  f"{100 * (loss / reg.best).max():.1f} %")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
