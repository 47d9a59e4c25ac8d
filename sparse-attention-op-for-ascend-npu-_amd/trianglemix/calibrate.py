"""Crossover calibration of the direct-path gates on this GPU.

The plan gates of ``TriangleMixConfig`` (``direct_min_seq_len``,
``direct_min_sparse_rows``, ``direct_min_saved_qk``,
``direct_split_min_sparse_rows``, ``direct_split_min_saved_qk``; the
reference's defaults in kernel.py:62-66 were measured on Ascend 910B) decide
whether a chunk runs the sparse kernel or falls back to dense attention.  This
module re-measures the crossover on the local GPU the way the reference's
crossover harness does (release_validation/installed_wheel_crossover.py:44-75:
every scheduler chunk of every (prompt length, chunk size) cell, the sparse
and the dense path timed in ABBA order) and fits each gate as the smallest
value from which the sparse path is never slower than the dense one by more
than ``margin``.

Run on the GPU::

    python -m trianglemix.calibrate --out trianglemix/gate_profiles/mi355x.json

The written profile holds the fitted gates, the reference gates, the margin and
every measured point; ``config.resolve_plugin_config`` takes its gates when the
plugin config sets ``gate_profile`` to the profile's name or path.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
from dataclasses import asdict, dataclass
from pathlib import Path

from .kernel import TriangleMixConfig, triangle_sparse_span

REFERENCE_GATES = {
    "direct_min_seq_len": 0,
    "direct_min_sparse_rows": 128,
    "direct_min_saved_qk": 913_152,
    "direct_split_min_sparse_rows": 192,
    "direct_split_min_saved_qk": 1_299_264,
}
GATE_NAMES = tuple(REFERENCE_GATES)


@dataclass(frozen=True)
class Point:
    prompt_len: int
    chunk: int
    query_start: int
    query_tokens: int
    sparse_rows: int
    saved_qk: int
    split: bool
    us_sparse: float
    us_dense: float

    @property
    def speedup(self) -> float:
        return self.us_dense / self.us_sparse


def route_cases(lengths, chunk_sizes):
    """(prompt_len, chunk, query_start, query_tokens) of every scheduler chunk of every cell."""
    for prompt_len in lengths:
        for chunk in chunk_sizes:
            for q0 in range(0, prompt_len, chunk):
                yield prompt_len, chunk, q0, min(chunk, prompt_len - q0)


def fit_gates(points, margin: float) -> dict[str, int]:
    """Smallest gate values from which every measured chunk that passes them runs the sparse path no slower
    than ``(1 + margin)`` x the dense path.  Chunks without a sparse middle never take the sparse path."""
    ok = lambda p: p.us_sparse <= p.us_dense * (1.0 + margin)  # noqa: E731

    def smallest(values_ok):
        # values_ok: [(value, ok)]; the smallest v with every value >= v ok (0 if all ok)
        bad = [v for v, good in values_ok if not good]
        if not bad:
            return 0
        worst = max(bad)
        above = [v for v, _ in values_ok if v > worst]
        return min(above) if above else worst + 1

    whole = [p for p in points if p.sparse_rows > 0 and not p.split]
    split = [p for p in points if p.sparse_rows > 0 and p.split]
    gates = {"direct_min_seq_len": 0}
    gates["direct_min_saved_qk"] = smallest([(p.saved_qk, ok(p)) for p in whole])
    gates["direct_min_sparse_rows"] = smallest(
        [(p.sparse_rows, ok(p)) for p in whole if p.saved_qk >= gates["direct_min_saved_qk"]])
    gates["direct_split_min_saved_qk"] = smallest(
        [(p.saved_qk, ok(p)) for p in split if p.sparse_rows >= gates["direct_min_sparse_rows"]])
    gates["direct_split_min_sparse_rows"] = smallest(
        [(p.sparse_rows, ok(p)) for p in split if p.saved_qk >= gates["direct_split_min_saved_qk"]])
    return gates


def passes(p: Point, gates: dict[str, int]) -> bool:
    if p.sparse_rows <= 0 or p.prompt_len < gates["direct_min_seq_len"]:
        return False
    if p.sparse_rows < gates["direct_min_sparse_rows"] or p.saved_qk < gates["direct_min_saved_qk"]:
        return False
    if p.split and (p.sparse_rows < gates["direct_split_min_sparse_rows"]
                    or p.saved_qk < gates["direct_split_min_saved_qk"]):
        return False
    return True


def routed_time_us(points, gates) -> float:
    """Attention time of all measured chunks when each takes the path the gates choose."""
    return sum(p.us_sparse if passes(p, gates) else p.us_dense for p in points)


def measure(lengths, chunk_sizes, reps: int, seed: int, log=print):
    import torch

    from . import native
    from .workload import SCALE, make_cache, make_query

    native.load_hip_library()
    native.load_triangle_mix_adapter()
    dev = torch.device("cuda:0")
    sparse_op = torch.ops.trianglemix.triangle_paged_sparse_attention.out
    dense_op = torch.ops.trianglemix.dense_paged_causal_attention.out
    config = TriangleMixConfig(enabled=True, layer_indices=frozenset())
    points = []
    by_len = {}
    for prompt_len, chunk, q0, tq in route_cases(lengths, chunk_sizes):
        if prompt_len not in by_len:
            by_len.clear()
            k, v, bt = make_cache(prompt_len, seed, std=1.0)
            q = make_query(prompt_len, seed + 1, std=1.0)
            by_len[prompt_len] = (k.to(dev), v.to(dev), bt.to(dev), q.to(dev))
        kd, vd, btd, qd = by_len[prompt_len]
        seq = q0 + tq
        query = qd[q0:seq]
        out = torch.empty_like(query)
        span = triangle_sparse_span(query_len=tq, seq_len=seq, prompt_len=prompt_len, config=config)

        def run_sparse():
            sparse_op(query, kd, vd, btd, q0, seq, prompt_len, SCALE, out=out)

        def run_dense():
            dense_op(query, kd, vd, btd, q0, seq, SCALE, out=out)

        def window(fn):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(reps):
                fn()
            e.record()
            torch.cuda.synchronize()
            return s.elapsed_time(e) * 1000.0 / reps

        run_sparse()
        run_dense()
        torch.cuda.synchronize()
        ts, td = [], []
        for order in ("sd", "ds"):  # ABBA
            for which in order:
                (ts if which == "s" else td).append(window(run_sparse if which == "s" else run_dense))
        p = Point(prompt_len, chunk, q0, tq, span.sparse_rows, span.saved_qk if span.has_sparse_middle else 0,
                  span.is_split, round(statistics.mean(ts), 3), round(statistics.mean(td), 3))
        points.append(p)
        log(f"L={prompt_len} chunk={chunk} q0={q0} tq={tq} sparse_rows={p.sparse_rows} saved={p.saved_qk} "
            f"split={p.split} sparse={p.us_sparse:.2f}us dense={p.us_dense:.2f}us x{p.speedup:.2f}")
    return points


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--lengths", default="1024,2048,4096,8192,16384")
    ap.add_argument("--chunks", default="256,512,1024,2048")
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--margin", type=float, default=0.05,
                    help="noise allowance: the same chunk geometry varies by ~5%% between runs")
    ap.add_argument("--seed", type=int, default=11)
    ap.add_argument("--name", default="mi355x")
    ap.add_argument("--out", default=None, help="write the profile JSON here")
    ap.add_argument("--summary", default=None, metavar="MD", help="also write a markdown summary here")
    ap.add_argument("--refit", default=None, metavar="PROFILE",
                    help="refit the points of an existing profile with --margin (no GPU needed)")
    args = ap.parse_args(argv)
    if args.refit:
        old = json.loads(Path(args.refit).read_text())
        fields = set(Point.__dataclass_fields__)
        points = [Point(**{k: v for k, v in p.items() if k in fields}) for p in old["points"]]
        device, reps = old["device"], old.get("reps", args.reps)
    else:
        import torch

        lengths = [int(x) for x in args.lengths.split(",")]
        chunks = [int(x) for x in args.chunks.split(",")]
        points = measure(lengths, chunks, args.reps, args.seed, log=lambda s: print(s, flush=True))
        device, reps = torch.cuda.get_device_properties(0).gcnArchName, args.reps
    gates = fit_gates(points, args.margin)

    profile = {
        "name": args.name,
        "device": device,
        "reps": reps,
        "method": "every scheduler chunk of each (prompt_len, chunk) cell; sparse vs dense ABBA, "
                  f"{reps} launches per window; gate = smallest value from which sparse <= dense x "
                  f"(1 + {args.margin})",
        "margin": args.margin,
        "gates": gates,
        "reference_gates": REFERENCE_GATES,
        "routed_us": {
            "fitted_gates": round(routed_time_us(points, gates), 2),
            "reference_gates": round(routed_time_us(points, REFERENCE_GATES), 2),
            "always_dense": round(sum(p.us_dense for p in points), 2),
        },
        "points": [dict(asdict(p), speedup=round(p.speedup, 4)) for p in points],
    }
    print(json.dumps({k: profile[k] for k in ("name", "device", "gates", "reference_gates", "routed_us")}),
          flush=True)
    if args.out:
        Path(args.out).write_text(json.dumps(profile, indent=1) + "\n")
    if args.summary:
        command = "python -m trianglemix.calibrate " + " ".join(argv if argv is not None else sys.argv[1:])
        Path(args.summary).write_text(summary_markdown(profile, points, command))
    return 0


def summary_markdown(profile, points, command: str) -> str:
    """Per-cell medians of the sweep plus the fitted and reference gates."""
    lines = [f"# Crossover sweep: sparse vs dense companion, {profile['device']}", "",
             "The points were measured on one MI355X by `python -m trianglemix.calibrate --out "
             "trianglemix/gate_profiles/mi355x.json` (package directory); this summary was written by:", "",
             "```", command, "```", "",
             f"Method: {profile['method']}.", "",
             "| gate | fitted | reference (910B) |", "|---|---:|---:|"]
    for g in GATE_NAMES:
        lines.append(f"| `{g}` | {profile['gates'][g]:,} | {profile['reference_gates'][g]:,} |")
    r = profile["routed_us"]
    lines += ["", f"Sum over the {len(points)} measured chunks when each takes the path the gates choose: "
              f"fitted gates {r['fitted_gates']:.0f} µs, reference gates {r['reference_gates']:.0f} µs, "
              f"always dense {r['always_dense']:.0f} µs.", "",
              "| prompt | chunk | chunks | with sparse rows | min speedup | median speedup | max speedup |",
              "|---:|---:|---:|---:|---:|---:|---:|"]
    cells = {}
    for p in points:
        cells.setdefault((p.prompt_len, p.chunk), []).append(p)
    for (L, c), ps in sorted(cells.items()):
        sp = [p.speedup for p in ps if p.sparse_rows > 0]
        if sp:
            lines.append(f"| {L} | {c} | {len(ps)} | {len(sp)} | {min(sp):.2f} | {statistics.median(sp):.2f} | "
                         f"{max(sp):.2f} |")
        else:
            lines.append(f"| {L} | {c} | {len(ps)} | 0 | - | - | - |")
    losers = [p for p in points if p.sparse_rows > 0 and p.us_sparse > p.us_dense * (1 + profile["margin"])]
    lines += ["", f"Chunks with sparse rows where the sparse path is more than {profile['margin']:.0%} slower: "
              f"{len(losers)}" + ("" if not losers else " -- " + "; ".join(
                  f"L={p.prompt_len} chunk={p.chunk} q0={p.query_start} ({p.sparse_rows} sparse rows, saved "
                  f"{p.saved_qk:,}, split={p.split}): {p.us_sparse:.1f} vs {p.us_dense:.1f} µs" for p in losers)), ""]
    return "\n".join(lines)


if __name__ == "__main__":
    sys.exit(main())
