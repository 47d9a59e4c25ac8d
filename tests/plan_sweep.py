"""Forced-plan sweep on MI355X: writes ``tests/plan_sweep_mi355x.json``, the measurements the launch
planner's costs are fitted to (``tests/plan_fit.py``) and checked against (``tests/test_boundary_abi.py``).

Every candidate plan (KV parts 4 / 2 / 1 x tiles per item: each whole-piece cut of the longest row above
128 tiles, then 128, 124, ..., 16) of each geometry whose split layout fits the workspace bound, one plan
per distinct (KV parts, pieces per row block), is forced through the diagnostic library's
``tm_plan_override`` and timed: 3 warm-up + 20 launches between HIP events, in forward, reverse and
forward order over the plans, keeping each plan's fastest.  Inputs are seeded N(0, 1) bf16 with a random
page table, generated on the GPU.  Geometries marked ``held_out`` were not used for the first fit, only
to check it.

Run on the GPU box from the repository root after ``python sparse-attention-op-for-ascend-npu-_amd/build.py
--plan-override``:

    python tests/plan_sweep.py --out gpurun_out/plan_sweep_mi355x.json
"""

from __future__ import annotations

import argparse
import ctypes
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "sparse-attention-op-for-ascend-npu-_amd"

# (query_start, query_tokens, seq_len, prompt_len); prompt_len 0 = dense companion.
FIT = [
    (2357, 512, 2869, 2869), (7680, 512, 8192, 8192), (4096, 512, 4608, 8192), (0, 512, 512, 8192),
    (512, 512, 1024, 8192), (0, 2048, 2048, 8320), (2048, 2048, 4096, 8320), (4096, 2048, 6144, 8320),
    (8192, 128, 8320, 8320), (14336, 2048, 16384, 32768), (30720, 2048, 32768, 32768),
    (129024, 2048, 131072, 131072), (65536, 2048, 67584, 131072), (2048, 512, 2560, 2560),
    (3072, 512, 3584, 3584), (3584, 512, 4096, 4096), (4608, 512, 5120, 5120), (5632, 512, 6144, 6144),
    (11776, 512, 12288, 12288), (15872, 512, 16384, 16384), (32256, 512, 32768, 32768), (2560, 309, 2869, 2869),
    (12288, 96, 12384, 12384), (2613, 256, 2869, 2869), (3072, 1024, 4096, 4096), (7936, 256, 8192, 8192),
    (5120, 1024, 6144, 6144), (16128, 256, 16384, 16384), (9728, 512, 10240, 10240), (6272, 2048, 8320, 8320),
    (14336, 2048, 16384, 16384), (0, 2048, 2048, 2048), (0, 4096, 4096, 4096), (8192, 1024, 9216, 32768),
    (1024, 1024, 2048, 2048), (0, 1024, 1024, 1024),
    (3584, 512, 4096, 0), (7680, 512, 8192, 0), (7936, 256, 8192, 0), (8064, 128, 8192, 0), (5632, 256, 5888, 0),
    (15872, 512, 16384, 0), (4096, 1024, 5120, 0), (11776, 256, 12032, 0), (3072, 512, 3584, 0),
    (4096, 512, 4608, 0), (0, 512, 512, 0), (1024, 512, 1536, 0), (2048, 512, 2560, 0), (6144, 2048, 8192, 0),
    (30720, 2048, 32768, 0), (0, 2048, 2048, 0),
]
HELD_OUT = [
    (2488, 512, 3000, 3000), (3988, 512, 4500, 4500), (6488, 512, 7000, 7000), (8488, 512, 9000, 9000),
    (19488, 512, 20000, 20000), (24064, 512, 24576, 24576), (7808, 384, 8192, 8192), (7744, 448, 8192, 8192),
    (256, 512, 768, 8192), (1000, 300, 1300, 4000), (9800, 200, 10000, 10000), (6000, 64, 6064, 6064),
    (40448, 512, 40960, 40960), (2816, 256, 3072, 8192),
    (7168, 1024, 8192, 8192), (10976, 1024, 12000, 12000), (15360, 1024, 16384, 16384),
    (31744, 1024, 32768, 32768), (8464, 1536, 10000, 10000), (8192, 2048, 10240, 10240),
    (18432, 2048, 20480, 20480), (63488, 2048, 65536, 65536), (12288, 4096, 16384, 16384),
    (16384, 4096, 20480, 32768), (0, 3000, 3000, 3000), (0, 6144, 6144, 6144), (0, 12288, 12288, 12288),
    (4096, 1024, 5120, 32768),
    (8192, 1024, 9216, 0), (3000, 700, 3700, 0), (20000, 2048, 22048, 0), (12288, 4096, 16384, 0),
    (1536, 512, 2048, 0), (6000, 256, 6256, 0), (0, 1024, 1024, 0),
]


def row_tiles(qs: int, tq: int, seq: int, prompt: int) -> list[int]:
    """Tiles per row block in issue order (heaviest first), as csrc/trianglemix_kernel.h row_block_tiles."""
    sb, se = (521, max(0, prompt - 128)) if prompt else (0, 0)
    nrb = (tq + 31) // 32
    out = []
    for o in range(nrb):
        tb = qs + 32 * (nrb - 1 - o)
        te = min(tb + 32, seq)
        last = (te - 1) // 32
        first = (tb - 512) // 32 if tb >= sb and te <= se else 0
        out.append(last + 1 if first <= 0 else 1 + last - first + 1)
    return out


def pieces(rt: list[int], tiles: int) -> tuple[int, ...]:
    return tuple((n + tiles - 1) // tiles for n in rt)


def fits(rt: list[int], tiles: int) -> bool:
    """The split layout's arrival words and partials fit the 64 MiB workspace bound."""
    before = split_row_blocks = split_items = 0
    for o, n in enumerate(rt):
        p = (n + tiles - 1) // tiles
        before += p
        if p > 1:
            split_row_blocks, split_items = o + 1, before
    return split_row_blocks <= 512 and split_items <= 124


def candidates(rt: list[int]) -> list[tuple[int, int, int]]:
    """(KV parts, tiles per item, items per KV head), one per distinct (KV parts, pieces)."""
    longest = max(rt)
    ts: list[int] = []
    k = 1
    while longest > 128:
        tk = -(-longest // k)
        if tk <= 128:
            break
        if not ts or tk != ts[-1]:
            ts.append(tk)
        k += 1
    ts += list(range(128, 15, -4))
    seen, out = set(), []
    for parts in (4, 2, 1):
        for tiles in ts:
            if not fits(rt, tiles) or (parts, pieces(rt, tiles)) in seen:
                continue
            seen.add((parts, pieces(rt, tiles)))
            out.append((parts, tiles, sum(pieces(rt, tiles))))
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", default=str(ROOT / "gpurun_out" / "plan_sweep_mi355x.json"))
    args = ap.parse_args()
    sys.path.insert(0, str(PKG))
    import torch

    from trianglemix import native
    from trianglemix.workload import SCALE

    path = PKG / "trianglemix" / "libtrianglemix_plan_override.so"
    if not path.is_file():
        raise SystemExit(f"{path} is not built: python {PKG / 'build.py'} --plan-override")
    lib = native._declare(ctypes.CDLL(str(path)))
    lib.tm_plan_override.restype = None
    lib.tm_plan_override.argtypes = [ctypes.c_int32, ctypes.c_int32]
    dev = torch.device("cuda:0")
    workspace = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev).manual_seed(5)
    out = {"method": __doc__.split("\n\n")[1].replace("\n", " "), "geometries": []}
    t0 = time.time()
    for gi, ((qs, tq, seq, prompt), held) in enumerate([(g, False) for g in FIT] + [(g, True) for g in HELD_OUT]):
        logical = (seq + 127) // 128
        pages = logical + 7
        table = torch.randperm(pages, generator=gen, device=dev)[:logical].to(torch.int32).view(1, -1)
        kc = torch.randn(pages, 128, 8, 128, generator=gen, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(pages, 128, 8, 128, generator=gen, device=dev, dtype=torch.bfloat16)
        q = torch.randn(tq, 32, 128, generator=gen, device=dev, dtype=torch.bfloat16)
        o = torch.empty_like(q)
        stream = torch.cuda.current_stream().cuda_stream

        def launch():
            if prompt:
                r = lib.tm_triangle_paged_sparse_attention(
                    q.data_ptr(), kc.data_ptr(), vc.data_ptr(), table.data_ptr(), o.data_ptr(), tq, pages, logical,
                    qs, seq, prompt, SCALE, workspace.data_ptr(), workspace.numel(), stream)
            else:
                r = lib.tm_dense_paged_causal_attention(
                    q.data_ptr(), kc.data_ptr(), vc.data_ptr(), table.data_ptr(), o.data_ptr(), tq, pages, logical,
                    qs, seq, SCALE, workspace.data_ptr(), workspace.numel(), stream)
            if r != 0:
                raise RuntimeError(lib.tm_last_error().decode())

        rt = row_tiles(qs, tq, seq, prompt)
        cands = candidates(rt)
        lib.tm_plan_override(0, 0)
        launch()
        torch.cuda.synchronize()
        reference = o.clone()
        for _ in range(200 if gi == 0 else 20):  # clock warm-up
            launch()
        times = {c: [] for c in cands}
        worst = 0.0
        for rnd in range(3):
            for c in (cands if rnd % 2 == 0 else cands[::-1]):
                lib.tm_plan_override(c[0], c[1])
                for _ in range(3):
                    launch()
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                for _ in range(20):
                    launch()
                e.record()
                torch.cuda.synchronize()
                times[c].append(s.elapsed_time(e) * 1000.0 / 20)
                if rnd == 0:  # every plan computes the same attention (up to split rounding)
                    worst = max(worst, (o.float() - reference.float()).abs().max().item())
        lib.tm_plan_override(0, 0)
        if worst > 3e-2:
            raise RuntimeError(f"plans of {(qs, tq, seq, prompt)} differ by {worst}")
        out["geometries"].append({"query_start": qs, "query_tokens": tq, "seq_len": seq, "prompt_len": prompt,
                                  "held_out": held, "plans": [[*c, round(min(times[c]), 2)] for c in cands]})
        best = min(out["geometries"][-1]["plans"], key=lambda p: p[3])
        print(f"[{gi}] {qs}+{tq}/{seq}/{prompt}: {len(cands)} plans, fastest {best}, largest difference "
              f"{worst:.4f}, {time.time() - t0:.0f} s", flush=True)
        del kc, vc, q, o, table
        torch.cuda.empty_cache()
    Path(args.out).parent.mkdir(parents=True, exist_ok=True)
    Path(args.out).write_text("{\n \"method\": " + json.dumps(out["method"]) + ",\n \"geometries\": [\n" +
                              ",\n".join("  " + json.dumps(g) for g in out["geometries"]) + "\n ]\n}\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
