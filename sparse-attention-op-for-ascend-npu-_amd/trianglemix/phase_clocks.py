"""Where a chunk's time goes: per-wave phase clocks of the attention kernel.

A diagnostic, not part of the op: the phase-clock build of the library
(``python build.py --phase-clocks`` -> ``libtrianglemix_phase_clocks.so``,
the same kernels compiled with ``TRIANGLEMIX_PHASE_CLOCKS``) stores the
100 MHz ``s_memrealtime`` clock from lane 0 of every wave at the phases
below.  This module runs one chunk on ``cuda:0`` through that library (20
warm-up launches, then the launch that is read) and prints, per phase, the
distribution over waves of the time since the earliest wave started, plus
the median length of each loop iteration::

    python -m trianglemix.phase_clocks --qs 4096 --tq 512 --prompt 8192
    python -m trianglemix.phase_clocks --qs 7680 --tq 512 --dense   # the dense companion

The stamps sit between phases, and each stamp waits for the scalar clock
read, so the instrumented kernel runs a few percent slower than the product.
"""

from __future__ import annotations

import argparse
import ctypes
import sys
from pathlib import Path

PHASES = {
    0: "entry",            # kernel arguments read
    1: "block table",      # the item's page numbers have landed
    2: "prologue",         # Q and K of the first tile landed, first barrier passed
    3: "first QK",         # first tile's scores, mask and row max
    **{4 + i: f"iteration {i}" for i in range(8)},  # start of loop iteration i (after its barrier)
    12: "loop end",
    13: "parts merged",    # the KV parts merged through LDS
    14: "stored",          # unsplit row block: output written
    16: "partial stored",  # split row block: partial written through
    17: "arrived",         # split row block: arrival counted
    18: "first batch",     # last arriver: first batch of partials merged
    19: "merged",          # last arriver: every partial merged
    15: "split stored",    # last arriver: output written
}
WORKGROUPS, WAVES, SLOTS = 4096, 8, 32


def library_path() -> Path:
    return Path(__file__).resolve().parent / "libtrianglemix_phase_clocks.so"


def run(qs: int, tq: int, prompt: int, seed: int = 7, dense: bool = False):
    """Per-wave clocks (µs since the earliest wave's entry, NaN where a wave did not pass a phase)."""
    import numpy as np
    import torch

    from . import cabi, native
    from .workload import SCALE, make_cache, make_query

    path = library_path()
    if not path.is_file():
        raise FileNotFoundError(f"{path} is missing: build it with `python build.py --phase-clocks`")
    native.load_hip_library(str(path))
    lib = ctypes.CDLL(str(path))
    lib.tm_phase_clocks_read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    seq = qs + tq
    parts, _, items = cabi.chunk_plan(tq, qs, seq, None if dense else prompt)
    workgroups = items * (16 if parts == 4 else 8)
    if workgroups > WORKGROUPS:
        raise ValueError(f"{workgroups} workgroups: the phase clocks cover {WORKGROUPS}")
    dev = torch.device("cuda:0")
    k, v, bt = make_cache(seq, seed, std=1.0)
    q = make_query(tq, seed + 1, std=1.0)
    kd, vd, btd, qd = k.to(dev), v.to(dev), bt.to(dev), q.to(dev)
    out = torch.empty_like(qd)

    def launch():
        if dense:
            cabi.dense_paged_causal_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, scale=SCALE)
        else:
            cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                                 scale=SCALE)

    for _ in range(20):
        launch()
    torch.cuda.synchronize()
    if lib.tm_phase_clocks_clear() != 0:
        raise RuntimeError("tm_phase_clocks_clear failed")
    launch()
    torch.cuda.synchronize()
    buf = np.zeros(WORKGROUPS * WAVES * SLOTS, dtype=np.uint64)
    if lib.tm_phase_clocks_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("tm_phase_clocks_read failed")
    t = buf.reshape(WORKGROUPS * WAVES, SLOTS)[: workgroups * WAVES].astype(np.float64)
    t0 = t[:, 0][t[:, 0] > 0].min()
    return np.where(t > 0, (t - t0) / 100.0, np.nan), (parts, items, workgroups)


def main(argv=None) -> int:
    import warnings

    import numpy as np

    warnings.simplefilter("ignore", RuntimeWarning)  # phases no wave of a chunk reaches are all-NaN columns

    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--qs", type=int, default=4096, help="query_start")
    ap.add_argument("--tq", type=int, default=512, help="query tokens")
    ap.add_argument("--prompt", type=int, default=8192, help="prompt_len")
    ap.add_argument("--dense", action="store_true", help="the dense paged causal companion (prompt_len unused)")
    a = ap.parse_args(argv)
    rel, (parts, items, workgroups) = run(a.qs, a.tq, a.prompt, dense=a.dense)
    what = "dense companion" if a.dense else f"prompt={a.prompt}"
    print(f"chunk qs={a.qs} tq={a.tq} {what}: KV parts {parts}, {items} items per KV head, "
          f"{workgroups} workgroups; µs since the earliest wave's entry")
    print(f"{'phase':>16} {'waves':>6} {'min':>7} {'p50':>7} {'p90':>7} {'max':>7}")
    for slot, name in PHASES.items():
        col = rel[:, slot]
        n = int(np.sum(~np.isnan(col)))
        if n:
            print(f"{name:>16} {n:6d} {np.nanmin(col):7.2f} {np.nanmedian(col):7.2f} "
                  f"{np.nanpercentile(col, 90):7.2f} {np.nanmax(col):7.2f}")
    starts = rel[:, 3:12]
    with np.errstate(all="ignore"):
        d = np.nanmedian(np.diff(starts, axis=1), axis=0)
    print("iteration lengths, median over waves (µs):", " ".join(f"{x:.2f}" for x in d if not np.isnan(x)))
    return 0


if __name__ == "__main__":
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    raise SystemExit(main())
