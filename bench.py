"""Benchmark: TriangleMix sparse prefill attention on one MI355X.

Workload (the headline configuration): Qwen3-8B attention geometry (Hq=32, Hkv=8,
D=128, bf16, page 128), one request, prompt L=8192 prefilled in 16 chunks of
512.  One *step* = the 16 chunk launches of the sparse kernel, in order, over
one paged K/V cache (random block-table permutation) that already holds the
whole prompt's K/V; all inputs are resident in HBM before timing.  Every
chunk is one kernel launch.

Reported JSON line (rank 0 only):

* ``value`` -- mean microseconds per chunk of the sparse kernel over the K
  timed steps (HIP-graph replay of the 16 launches, HIP events on the launch
  stream); the K steps run in windows that alternate with the dense
  companion's in ABBA order, and ``timing`` gives the windows' median,
  inter-quartile range, p10 and Tukey-fence outliers beside the mean;
* ``roofline`` -- bf16 MFMA bound: algorithmic FLOPs per launch
  (4*D*Hq*attended pairs) / average launch duration, vs 2.5 PFLOP/s;
  ``traffic`` is the rocprofv3 FETCH+WRITE bytes per launch when a summary
  for this workload exists under profiles/, else null;
* ``plans`` -- each chunk's launch plan: [KV parts, tiles per work item, work
  items per KV head];
* ``dense`` -- the same 16 chunks through the dense paged causal companion
  kernel, and the attention-time cut of sparse vs dense;
* ``library_dense`` -- the same 16 chunks through PyTorch's own dense
  attention (``scaled_dot_product_attention``, flash backend: AOTriton's
  kernels on ROCm), causal lower-right, GQA in the kernel, on K/V gathered
  into contiguous (1, Hkv, S, D) tensors outside the timed region (the
  library gets no page table to follow), one HIP graph per step: a dense
  baseline that is not this repository's own kernel;
* ``kv_write`` -- the paged KV write upstream of the attention
  (``trianglemix::reshape_and_cache``): one chunk's fresh K/V into its pages,
  and the whole prompt in one call, with HBM GB/s against 8 TB/s;
* ``cpu_baseline`` -- the fp32 PyTorch CPU masked-attention restatement of the
  reference's oracle (``oracle.attention.attention_torch``) over all 16
  chunks on this host's cores (``torch.set_num_threads(os.cpu_count())``):
  one warm-up pass, then the median of 3 passes;
* ``legs`` -- the other BASELINE configurations, measured in the same run:
  config 1 (one launch: rows 2357..2868 of a 2869-token prompt), config 3
  (L=8320 in chunks of 2048, 1 % of K entries +-8, with max/mean-abs error vs
  the fp32 oracle on row subsets), config 4 (whole prefills at L=32768 and
  131072, chunk 2048, sparse vs dense) and config 5 (36 layers through the
  plan / router layer with the router's default gates on this GPU -- the
  MI355X profile on gfx950 -- and with the reference's gates, vs all dense,
  with the counters).

``--gpus N`` with N > 1 is refused: this build runs on one GPU.

Detailed single-workload runs (one JSON line each, not the headline):
``--workload config1 | config3`` (same legs as the headline, that chunk set),
``--workload config4`` (the whole long-context curve, L = 1024 .. 131072, and
the crossover; each L also through PyTorch's own dense attention), ``--workload config5`` (the layer stack with both gate sets,
the structured counter log and the vLLM-ROCm seam).
"""

from __future__ import annotations

import argparse
import json
import logging
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG_ROOT = ROOT / "sparse-attention-op-for-ascend-npu-_amd"
for _p in (ROOT, PKG_ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "sparse-prefill attn µs/chunk + MFMA %peak, Qwen3-8B GQA, L=8192 chunk 512"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
TRAFFIC_SUMMARY = ROOT / "profiles" / "triangle_config2_traffic.md"


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prompt", type=int, default=8192)
    ap.add_argument("--chunk", type=int, default=512)
    ap.add_argument("--seed", type=int, default=7)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-legs", action="store_true", help="headline only (skip the config 1/3/4/5 legs)")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of a HIP graph")
    ap.add_argument("--only", choices=("sparse", "dense"), help="run one kernel only (for profiling)")
    ap.add_argument("--workload", choices=("config1", "config2", "config3", "config4", "config5", "host"),
                    default="config2", help="host: host time per call of each API level (one middle chunk)")
    ap.add_argument("--outliers", type=float, default=None, help="fraction of K entries set to +-8")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run 5 plain device copies of MIB MiB (scales rocprofv3 FETCH/WRITE_SIZE)")
    return ap.parse_args()


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this build measures one MI355X "
              "(the op has no cross-GPU path)", file=sys.stderr)
        return 2

    import torch

    from trianglemix import native

    if args.workload == "config4":
        return config4_curve(args)
    if args.workload == "config5":
        return config5_stack(args)
    if args.workload == "host":
        return host_overhead(args)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    native.load_hip_library()
    native.load_triangle_mix_adapter()
    headline = args.workload == "config2" and args.prompt == 8192 and args.chunk == 512 and not args.outliers
    if args.workload == "config3":
        args.prompt, args.chunk = 8320, 2048
        args.outliers = 0.01 if args.outliers is None else args.outliers
    if args.workload == "config1":
        args.prompt, args.chunk = 2869, 512
    line = chunk_set_line(args, headline)
    if headline and args.only is None and not args.no_legs:
        line["legs"] = headline_legs(args)
    print(json.dumps(line), flush=True)
    return 0


def timing_stats(window_ms: list[float]) -> dict:
    """Median, inter-quartile range, p10 and Tukey-fence outliers of per-window ms/step (as the reference
    reports its cells, harness/npu_harness_common.py:663-722)."""
    xs = sorted(window_ms)
    n = len(xs)

    def q(f):  # linear interpolation between closest ranks
        pos = f * (n - 1)
        lo = int(pos)
        hi = min(lo + 1, n - 1)
        return xs[lo] + (xs[hi] - xs[lo]) * (pos - lo)

    q1, q3 = q(0.25), q(0.75)
    iqr = q3 - q1
    return {"windows": n, "median_ms": round(statistics.median(xs), 5), "q1_ms": round(q1, 5),
            "q3_ms": round(q3, 5), "iqr_ms": round(iqr, 5), "p10_ms": round(q(0.10), 5),
            "tukey_outliers": sum(1 for x in xs if x < q1 - 1.5 * iqr or x > q3 + 1.5 * iqr)}


def abba(run_a, run_b, steps: int, windows: int):
    """Time ``steps`` calls of run_a and of run_b in ``windows`` windows each, alternating A B B A A B ...;
    every window is bracketed by events and a device synchronisation.  Returns (total ms of A, per-window
    ms/step of A, total ms of B, per-window ms/step of B)."""
    import torch

    windows = max(2, min(windows, steps))
    sizes = [steps // windows + (1 if i < steps % windows else 0) for i in range(windows)]
    out = {"a": [0.0, []], "b": [0.0, []]}

    def window(run, n, key):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(n):
            run()
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e)
        out[key][0] += ms
        out[key][1].append(ms / n)

    for i, n in enumerate(sizes):
        order = (("a", run_a), ("b", run_b)) if i % 2 == 0 else (("b", run_b), ("a", run_a))
        for key, run in order:
            if run is not None:
                window(run, n, key)
    return out["a"][0], out["a"][1], out["b"][0], out["b"][1]


def chunk_plans(chunks) -> list[list[int]]:
    """Per chunk, the TriangleMix launch plan the library takes: [KV parts, tiles per work item, work items per
    KV head] (4 / 2 / 1 = KV quarters / halves / whole)."""
    from trianglemix import cabi

    return [list(cabi.chunk_plan(c.query_tokens, c.query_start, c.seq_len, c.prompt_len)) for c in chunks]


def chunk_set_line(args, headline: bool) -> dict:
    """The JSON line of one chunk set (config 2 by default; config 1 or 3 with --workload)."""
    import torch

    from trianglemix.workload import (SCALE, Chunk, chunk_bytes, chunk_flops, executed_flops, kv_bytes,
                                      make_cache, make_query, prompt_chunks)

    dev = torch.device("cuda:0")
    chunks = [Chunk(2357, 2869, 2869)] if args.workload == "config1" else prompt_chunks(args.prompt, args.chunk)
    k, v, bt = make_cache(args.prompt, args.seed, std=1.0, outlier_frac=args.outliers or 0.0)
    qfull = make_query(args.prompt, args.seed + 1, std=1.0)
    kd, vd, btd = k.to(dev), v.to(dev), bt.to(dev)
    m = measure_chunk_set(chunks, qfull, kd, vd, btd, args.steps, args.warmup,
                          graph=not args.no_graph and len(chunks) > 1, only=args.only, per_chunk=True)
    ms_sparse, ms_dense = m["ms_sparse"], m["ms_dense"]
    n = len(chunks)
    alg_flops = sum(chunk_flops(c) for c in chunks)
    exe_flops = sum(executed_flops(c) for c in chunks)
    dense_flops = sum(chunk_flops(c, dense=True) for c in chunks)
    alg_bytes = sum(chunk_bytes(c) for c in chunks)
    kvb = sum(kv_bytes(c) for c in chunks)
    us_per_chunk = ms_sparse * 1000.0 / n
    achieved_tflops = alg_flops / (ms_sparse * 1e-3) / 1e12

    if args.copy_calibration > 0:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    traffic = read_traffic_summary() if headline else None
    kv_write = kv_write_bench(args, chunks, k, v, bt, dev) if args.only is None and headline else None
    library = None
    if args.only is None and (headline or args.workload == "config3"):
        library = library_dense(chunks, qfull, k, v, bt, kd, vd, btd, args.steps, ms_sparse, ms_dense)
    errors = None
    if args.workload == "config3" and args.only is None:
        errors = oracle_errors(chunks, qfull, k, v, bt, m["outputs"])
    cpu = None
    if not args.no_cpu_baseline and args.only is None:
        cpu = cpu_baseline(chunks, qfull, k, v, bt, SCALE)

    workload = (f"config2: one request, L={args.prompt}, chunked prefill {args.chunk} x {n} chunks, "
                "Hq=32 Hkv=8 D=128 page=128, one layer")
    if args.workload == "config1":
        workload = ("config1: one launch, rows 2357..2868 of a 2869-token prompt (384 sparse rows + 128-row "
                    "dense tail), Hq=32 Hkv=8 D=128 page=128, one layer")
    if args.workload == "config3":
        workload = (f"config3: one request, L={args.prompt}, chunked prefill {args.chunk} x {n} chunks, "
                    f"{args.outliers:.0%} of K entries +-8, Hq=32 Hkv=8 D=128 page=128, one layer")
    return {
        "metric": METRIC if headline else f"sparse-prefill attn µs/chunk + MFMA %peak ({args.workload})",
        "value": round(us_per_chunk, 3),
        "unit": "us/chunk",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_sparse, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, random page table)",
        "config": {
            "workload": workload,
            "timing": (f"HIP-graph replay of the {n} launches" if not args.no_graph and n > 1
                       else "back-to-back eager launches")
                      + f"; {args.steps} timed steps in ABBA windows with the dense companion",
        },
        "timing": m["sparse_stats"],
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved_tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "alg_flops_per_launch": alg_flops // n,
            "alg_bytes_per_launch": alg_bytes // n,
            "executed_tile_tflops": round(exe_flops / (ms_sparse * 1e-3) / 1e12, 2),
            "executed_tile_frac": round(exe_flops / (ms_sparse * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "kv_hbm_gbs": round(kvb / (ms_sparse * 1e-3) / 1e9, 1),
        },
        "per_chunk_us": m["per_chunk_us"],
        "plans": chunk_plans(chunks),
        "dense": {
            "ms_per_step": round(ms_dense, 5),
            "us_per_chunk": round(ms_dense * 1000.0 / n, 3),
            "alg_tflops": round(dense_flops / (ms_dense * 1e-3) / 1e12, 2) if ms_dense == ms_dense else None,
            "attention_time_cut": round(1.0 - ms_sparse / ms_dense, 4) if ms_dense == ms_dense else None,
            "timing": m["dense_stats"],
        },
        "library_dense": library,
        "errors_vs_fp32": errors,
        "kv_write": kv_write,
        "cpu_baseline": cpu,
    }


def measure_chunk_set(chunks, qfull, kd, vd, btd, steps, warmup, *, graph=True, only=None, per_chunk=False):
    """Sparse vs dense over one chunk set: every chunk launch of a step captured in one HIP graph (each
    replay checked against the eager result), ``warmup`` untimed steps, then ``steps`` timed steps of each
    in ABBA windows.  Returns ms/step means, window statistics, eager per-chunk µs and the sparse outputs."""
    import torch

    from trianglemix.workload import SCALE

    dev = kd.device
    qs = [qfull[c.query_start:c.seq_len].contiguous().to(dev) for c in chunks]
    outs = [torch.empty_like(q) for q in qs]
    sparse_op = torch.ops.trianglemix.triangle_paged_sparse_attention.out
    dense_op = torch.ops.trianglemix.dense_paged_causal_attention.out

    def sparse_step():
        for c, q, o in zip(chunks, qs, outs):
            sparse_op(q, kd, vd, btd, c.query_start, c.seq_len, c.prompt_len, SCALE, out=o)

    def dense_step():
        for c, q, o in zip(chunks, qs, outs):
            dense_op(q, kd, vd, btd, c.query_start, c.seq_len, SCALE, out=o)

    sparse_step()
    torch.cuda.synchronize()
    eager_sparse = [o.clone() for o in outs]
    dense_step()
    torch.cuda.synchronize()
    eager_dense = [o.clone() for o in outs]

    def make_runner(step, reference):
        if not graph:
            return step
        g = graph_of(step)
        for _ in range(3):  # every replay must reproduce the eager result
            for o in outs:
                o.zero_()
            g.replay()
            torch.cuda.synchronize()
            for o, ref in zip(outs, reference):
                if not torch.equal(o, ref):
                    raise RuntimeError("graph replay differs from eager launches")
        return g.replay

    run_sparse = make_runner(sparse_step, eager_sparse) if only != "dense" else None
    run_dense = make_runner(dense_step, eager_dense) if only != "sparse" else None
    for _ in range(warmup):
        if run_sparse:
            run_sparse()
        if run_dense:
            run_dense()
    torch.cuda.synchronize()
    windows = max(2, min(10, steps // 5 * 2))
    tot_s, win_s, tot_d, win_d = abba(run_sparse, run_dense, steps, windows)
    ms_sparse = tot_s / steps if win_s else float("nan")
    ms_dense = tot_d / steps if win_d else float("nan")

    per_chunk_us = []
    if per_chunk and only != "dense":  # eager, 20 back-to-back launches per chunk
        for c, q, o in zip(chunks, qs, outs):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(20):
                sparse_op(q, kd, vd, btd, c.query_start, c.seq_len, c.prompt_len, SCALE, out=o)
            e.record()
            torch.cuda.synchronize()
            per_chunk_us.append(round(s.elapsed_time(e) * 1000.0 / 20, 2))
    return {"ms_sparse": ms_sparse, "ms_dense": ms_dense,
            "sparse_stats": timing_stats(win_s) if win_s else None,
            "dense_stats": timing_stats(win_d) if win_d else None,
            "per_chunk_us": per_chunk_us, "outputs": eager_sparse}


def oracle_errors(chunks, qfull, k, v, bt, outs, rows: int = 32) -> dict:
    """max / mean-abs error vs the fp32 oracle on the first and last ``rows`` rows of every chunk."""
    import numpy as np

    from oracle.attention import attention_torch, error_metrics
    from trianglemix.workload import SCALE

    worst = {"max_abs": 0.0, "mean_abs": 0.0}
    checked = 0
    for c, o in zip(chunks, outs):
        n = c.query_tokens
        for r0, r1 in sorted({(0, min(rows, n)), (max(0, n - rows), n)}):
            exp = attention_torch(qfull[c.query_start + r0:c.query_start + r1], k, v, bt, c.query_start + r0,
                                  c.seq_len, c.prompt_len, SCALE)
            m = error_metrics(o[r0:r1].float().cpu().numpy(), exp.float().numpy())
            worst["max_abs"] = max(worst["max_abs"], m["max_abs"])
            worst["mean_abs"] = max(worst["mean_abs"], m["mean_abs"])
            checked += r1 - r0
    return {"max_abs": float(np.float32(worst["max_abs"])), "worst_window_mean_abs": worst["mean_abs"],
            "rows_checked": checked, "tolerance": {"max_abs": 2e-2, "mean_abs": 2e-3}}


def headline_legs(args) -> dict:
    """BASELINE configs 1, 3, 4 (L = 32768, 131072) and 5, measured after the headline (bounded)."""
    import torch

    from trianglemix.workload import Chunk, chunk_flops, executed_flops, make_cache, make_query, prompt_chunks

    dev = torch.device("cuda:0")
    legs = {}
    for name, prompt, chunk, outliers in (("config1", 2869, 512, 0.0), ("config3", 8320, 2048, 0.01)):
        chunks = [Chunk(2357, 2869, 2869)] if name == "config1" else prompt_chunks(prompt, chunk)
        k, v, bt = make_cache(prompt, args.seed, std=1.0, outlier_frac=outliers)
        qfull = make_query(prompt, args.seed + 1, std=1.0)
        # one launch: back-to-back eager launches (a one-kernel graph replay mostly times the graph launch)
        m = measure_chunk_set(chunks, qfull, k.to(dev), v.to(dev), bt.to(dev), 20, 5, graph=len(chunks) > 1,
                              per_chunk=True)
        n = len(chunks)
        flops = sum(chunk_flops(c) for c in chunks)
        leg = {"us_per_chunk": round(m["ms_sparse"] * 1000.0 / n, 3),
               "per_chunk_us": m["per_chunk_us"],
               "plans": chunk_plans(chunks),
               "mfma_frac": round(flops / (m["ms_sparse"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
               "executed_tile_frac": round(sum(executed_flops(c) for c in chunks) / (m["ms_sparse"] * 1e-3) / 1e12
                                           / PEAK_BF16_TFLOPS, 4),
               "dense_us_per_chunk": round(m["ms_dense"] * 1000.0 / n, 3),
               "attention_time_cut": round(1.0 - m["ms_sparse"] / m["ms_dense"], 4),
               "timing": m["sparse_stats"]}
        if name == "config3":
            leg["errors_vs_fp32"] = oracle_errors(chunks, qfull, k, v, bt, m["outputs"])
        legs[name] = leg
        del m
        torch.cuda.empty_cache()
    legs["config4"] = long_context_points(args.seed, (32768, 131072))
    legs["config5"] = layer_stack_summary(args.seed)
    return legs


def sdpa_chunks(chunks, qs, ks, vs, between):
    """PyTorch's own dense attention over a chunk sequence: ``scaled_dot_product_attention`` restricted to
    its flash backend (AOTriton's kernels on ROCm; the memory-efficient backend if flash is refused), mask
    ``causal_lower_right`` (row i of a chunk sees keys <= query_start + i, as the dense companion does),
    GQA handled by the kernel.  ``qs[i]`` is chunk i's (1, Hq, T, D) query and ``ks[i]`` / ``vs[i]`` its
    (1, Hkv, S, D) keys and values, all contiguous.  Returns (run, eager outputs, facts): ``run`` replays
    one HIP graph of all the calls (three replays are first checked against the eager outputs, each after
    ``between()`` has run eagerly) or, if capture is refused, makes the calls eagerly; ``run`` is None when
    no fused backend accepts the chunks."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from torch.nn.attention.bias import causal_lower_right

    from trianglemix.workload import SCALE

    masks = [causal_lower_right(c.seq_len - c.query_start, c.seq_len) for c in chunks]
    outs = [None] * len(chunks)

    def calls(backend):
        with sdpa_kernel([backend]):
            for i in range(len(chunks)):
                outs[i] = F.scaled_dot_product_attention(qs[i], ks[i], vs[i], attn_mask=masks[i], scale=SCALE,
                                                         enable_gqa=True)

    backend, refused = None, {}
    for b in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            calls(b)
            torch.cuda.synchronize()
            backend = b
            break
        except RuntimeError as e:
            refused[b.name] = str(e).splitlines()[0][:200]
    facts = {"impl": None if backend is None else
             (f"torch.nn.functional.scaled_dot_product_attention, {backend.name} backend (AOTriton on ROCm), "
              "causal_lower_right, enable_gqa; Q/K/V contiguous (gathered from the pages before timing)"),
             "refused_backends": refused or None}
    if backend is None:
        facts["error"] = "no fused SDPA backend accepted the chunks"
        return None, None, facts
    eager = [o.clone() for o in outs]
    run, graphed = (lambda: calls(backend)), True
    try:
        g = graph_of(run)
        for _ in range(3):
            for o in outs:
                o.zero_()
            between()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            if not all(torch.equal(o, e) for o, e in zip(outs, eager)):
                raise RuntimeError("graph replay differs from eager calls")
        run = g.replay
    except RuntimeError:
        graphed = False
    facts["graph"] = graphed
    return run, eager, facts


def library_dense(chunks, qfull, k, v, bt, kd, vd, btd, steps, ms_sparse, ms_dense) -> dict:
    """The same chunks through PyTorch's own dense attention (``sdpa_chunks``), on Q/K/V gathered into
    contiguous tensors before timing, timed in windows of its own; its largest output difference from the
    dense companion."""
    import torch

    from trianglemix.workload import SCALE, chunk_flops

    dev = kd.device
    order = bt[0].long()
    kc, vc = k[order].flatten(0, 1), v[order].flatten(0, 1)  # (pages * page, Hkv, D) in logical order
    qs = [qfull[c.query_start:c.seq_len].to(dev).permute(1, 0, 2).contiguous().unsqueeze(0) for c in chunks]
    ks = [kc[:c.seq_len].to(dev).permute(1, 0, 2).contiguous().unsqueeze(0) for c in chunks]
    vs = [vc[:c.seq_len].to(dev).permute(1, 0, 2).contiguous().unsqueeze(0) for c in chunks]
    dense_op = torch.ops.trianglemix.dense_paged_causal_attention.out
    ours = [torch.empty(c.seq_len - c.query_start, qfull.shape[1], qfull.shape[2], dtype=qfull.dtype, device=dev)
            for c in chunks]

    def dense_calls():
        for c, q, o in zip(chunks, qs, ours):
            dense_op(q[0].permute(1, 0, 2).contiguous(), kd, vd, btd, c.query_start, c.seq_len, SCALE, out=o)

    run, eager, facts = sdpa_chunks(chunks, qs, ks, vs, dense_calls)
    if run is None:
        return facts
    dense_calls()
    torch.cuda.synchronize()
    max_abs = max((e[0].permute(1, 0, 2).float() - o.float()).abs().max().item() for e, o in zip(eager, ours))
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    tot, win, _, _ = abba(run, None, steps, max(2, min(10, steps // 5 * 2)))
    ms = tot / steps
    dense_flops = sum(chunk_flops(c, dense=True) for c in chunks)
    return {
        **facts,
        "ms_per_step": round(ms, 5),
        "us_per_chunk": round(ms * 1000.0 / len(chunks), 3),
        "alg_tflops": round(dense_flops / (ms * 1e-3) / 1e12, 2),
        "dense_companion_speedup": round(ms / ms_dense, 3) if ms_dense == ms_dense else None,
        "sparse_speedup": round(ms / ms_sparse, 3) if ms_sparse == ms_sparse else None,
        "max_abs_vs_dense_companion": max_abs,
        "timing": timing_stats(win),
    }


def graph_of(step):
    """HIP graph of ``step`` (captured after one eager warm-up on the capture stream)."""
    import torch

    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    return graph


def median_ms(run, reps: int, windows: int = 3) -> float:
    """Median over ``windows`` of the mean time of ``reps`` back-to-back calls (ms per call)."""
    import torch

    times = []
    for _ in range(windows):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            run()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e) / reps)
    return statistics.median(times)


def long_context_points(seed: int, lengths, library: bool = False) -> list[dict]:
    """Whole prefills (chunk 2048), sparse vs dense, one HIP graph of the chunk launches per L; the sparse
    graph's timing windows, then the dense graph's; with ``library``, then PyTorch's own dense attention
    over the same chunks (``sdpa_chunks``, on contiguous copies of each chunk's Q/K/V)."""
    import torch

    from trianglemix.workload import SCALE, chunk_flops, prompt_chunks

    dev = torch.device("cuda:0")
    sparse_op = torch.ops.trianglemix.triangle_paged_sparse_attention.out
    dense_op = torch.ops.trianglemix.dense_paged_causal_attention.out
    chunk = 2048
    curve = []
    for L in lengths:
        g = torch.Generator(device=dev).manual_seed(seed + L)
        logical = (L + 127) // 128
        pages = logical + 7
        table = torch.randperm(pages, generator=g, device=dev)[:logical].to(torch.int32).view(1, -1)
        kc = torch.randn(pages, 128, 8, 128, generator=g, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(pages, 128, 8, 128, generator=g, device=dev, dtype=torch.bfloat16)
        q = torch.randn(L, 32, 128, generator=g, device=dev, dtype=torch.bfloat16)
        out = torch.empty_like(q)
        chunks = prompt_chunks(L, chunk)

        def sparse_step():
            for c in chunks:
                sparse_op(q[c.query_start:c.seq_len], kc, vc, table, c.query_start, c.seq_len, L, SCALE,
                          out=out[c.query_start:c.seq_len])

        def dense_step():
            for c in chunks:
                dense_op(q[c.query_start:c.seq_len], kc, vc, table, c.query_start, c.seq_len, SCALE,
                         out=out[c.query_start:c.seq_len])

        # The sparse prefill is timed first, in windows of its own, and the dense one after it: at these
        # lengths a dense window runs 10-150 ms at full power, and a short sparse window right after one
        # (as ABBA order would put it) runs at a lowered clock.
        # The sparse prefill also gets a warm-up of a third of its timed replays (its windows follow the
        # previous leg's dense work) and more replays than the dense one: they cost little.
        reps = 4 if L >= 131072 else (10 if L >= 32768 else 40)
        reps_s = 3 * reps
        gs = graph_of(sparse_step)
        for _ in range(reps):
            gs.replay()
        tot_s, win_s, _, _ = abba(gs.replay, None, reps_s, 4)
        gd = graph_of(dense_step)
        gd.replay()
        tot_d, win_d, _, _ = abba(gd.replay, None, reps, 4)
        ms_s, ms_d = tot_s / reps_s, tot_d / reps
        fs = sum(chunk_flops(c) for c in chunks)
        fd = sum(chunk_flops(c, dense=True) for c in chunks)
        point = {"L": L, "chunks": len(chunks), "sparse_ms": round(ms_s, 4), "dense_ms": round(ms_d, 4),
                 "speedup": round(ms_d / ms_s, 3), "sparse_gflop": round(fs / 1e9, 2),
                 "dense_gflop": round(fd / 1e9, 2), "sparse_tflops": round(fs / (ms_s * 1e-3) / 1e12, 1),
                 "dense_tflops": round(fd / (ms_d * 1e-3) / 1e12, 1),
                 "sparse_us_per_chunk": round(ms_s * 1000.0 / len(chunks), 2),
                 "sparse_window_iqr_ms": timing_stats(win_s)["iqr_ms"]}
        if library:
            point["library"] = library_prefill(chunks, q, kc, vc, table, out, gd.replay, reps, ms_d)
        curve.append(point)
        print(f"# config4 L={L}: sparse {ms_s:.3f} ms dense {ms_d:.3f} ms x{ms_d / ms_s:.2f}", file=sys.stderr,
              flush=True)
        del kc, vc, q, out, gs, gd
        torch.cuda.empty_cache()
    return curve


def library_prefill(chunks, q, kc, vc, table, dense_out, between, reps: int, ms_dense: float) -> dict:
    """One whole prefill through PyTorch's own dense attention (``sdpa_chunks``): each chunk's Q/K/V copied
    into contiguous tensors before timing, then ``reps`` timed replays; the largest difference of its
    outputs from the dense companion's (``dense_out``, all rows of the prompt)."""
    import torch

    kl = kc[table[0].long()].flatten(0, 1)  # (pages * page, Hkv, D) in logical order
    vl = vc[table[0].long()].flatten(0, 1)
    qs = [q[c.query_start:c.seq_len].permute(1, 0, 2).contiguous().unsqueeze(0) for c in chunks]
    ks = [kl[:c.seq_len].permute(1, 0, 2).contiguous().unsqueeze(0) for c in chunks]
    vs = [vl[:c.seq_len].permute(1, 0, 2).contiguous().unsqueeze(0) for c in chunks]
    del kl, vl
    run, eager, facts = sdpa_chunks(chunks, qs, ks, vs, between)
    if run is None:
        return facts
    max_abs = max((e[0].permute(1, 0, 2).float() - dense_out[c.query_start:c.seq_len].float()).abs().max().item()
                  for c, e in zip(chunks, eager))
    run()
    torch.cuda.synchronize()
    tot, _, _, _ = abba(run, None, reps, min(4, reps))
    ms = tot / reps
    del qs, ks, vs, eager
    return {**facts, "ms": round(ms, 4), "vs_dense_companion": round(ms / ms_dense, 3),
            "max_abs_vs_dense_companion": max_abs}


def config4_curve(args) -> int:
    """Long-context curve (chunk 2048): whole-prefill sparse vs dense attention time per L, and the crossover."""
    from trianglemix import native

    native.load_hip_library()
    native.load_triangle_mix_adapter()
    curve = long_context_points(args.seed, (1024, 2048, 4096, 8192, 16384, 32768, 131072), library=True)
    wins = [p["L"] for p in curve if p["sparse_ms"] < p["dense_ms"]]
    line = {
        "metric": "long-context prefill attention, sparse vs dense (config4, chunk 2048)",
        "value": next(p["sparse_ms"] for p in curve if p["L"] == 32768),
        "unit": "ms/prefill at L=32768",
        "n_gpus": 1,
        "higher_is_better": False,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V from the GPU generator, random page table)",
        "config": {"workload": "config4: one request per L, chunked prefill of 2048, Hq=32 Hkv=8 D=128 page=128, "
                               "one layer; each prefill is one HIP graph of its chunk launches, timed in windows of "
                               "its own (sparse first, then dense, then PyTorch's own dense attention on "
                               "contiguous copies of each chunk's Q/K/V: `library`)"},
        "curve": curve,
        "crossover_L": min(wins) if wins else None,
        "crossover_note": "smallest measured L whose whole sparse prefill beats the dense one; L=1024 is one "
                          "1024-row chunk, whose one-kernel graph replay is dominated by the graph launch (the "
                          "eager crossover sweep of trianglemix.calibrate measures that chunk at x1.02)",
    }
    print(json.dumps(line), flush=True)
    return 0


def _stand_in_vllm(prompt_len: int):
    """A stand-in vLLM v1 Triton backend and GPU model runner with the signatures the seam allowlists.

    Its own forward does what vLLM's Triton path does for a prefill chunk:
    write the step's K/V into the paged cache, then attend -- here with the
    gfx950 KV write and the dense companion kernel.  No vLLM is installed on
    these machines; the stand-in lets the seam run a whole engine step loop.
    """
    import types

    import torch

    class Metadata:
        def __init__(self, common):
            self.num_actual_tokens = int(common.query_start_loc_cpu[-1])
            self.seq_len = int(common.seq_lens_cpu[0])
            self.block_table = common.block_table_tensor
            self.slot_mapping = common.slot_mapping
            self.causal = True
            self.use_cascade = False

    class TritonAttentionMetadataBuilder:
        def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
            self.vllm_config = vllm_config

        def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
            return Metadata(common_attn_metadata)

        def build_for_cudagraph_capture(self, common_attn_metadata):
            return self.build(0, common_attn_metadata)

    class TritonAttentionImpl:
        def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes, sliding_window, kv_cache_dtype,
                     logits_soft_cap=None, attn_type="decoder", kv_sharing_target_layer_name=None, sinks=None):
            self.num_heads, self.head_size, self.scale, self.num_kv_heads = num_heads, head_size, scale, num_kv_heads
            self.alibi_slopes, self.sinks, self.logits_soft_cap = alibi_slopes, sinks, logits_soft_cap
            self.sliding_window = (-1, -1)
            self.kv_cache_dtype, self.attn_type = kv_cache_dtype, attn_type
            self.kv_sharing_target_layer_name = kv_sharing_target_layer_name

        def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                    output_block_scale=None):
            kc, vc = kv_cache.unbind(0)
            n, seq = attn_metadata.num_actual_tokens, attn_metadata.seq_len
            torch.ops.trianglemix.reshape_and_cache(key[:n], value[:n], kc, vc, attn_metadata.slot_mapping[:n])
            torch.ops.trianglemix.dense_paged_causal_attention.out(
                query[:n], kc, vc, attn_metadata.block_table, seq - n, seq, self.scale, out=output[:n])
            return output

    class GPUModelRunner:
        def __init__(self, builder):
            self.builder = builder
            self.input_batch = types.SimpleNamespace(num_reqs=1, num_prompt_tokens=[prompt_len])
            self.speculative_config = None

        def _prepare_inputs(self, scheduler_output):
            return {"layers": self.builder.build(0, scheduler_output)}, None

    class TritonAttentionBackend:
        @staticmethod
        def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, cache_dtype_str="auto"):
            return (2, num_blocks, block_size, num_kv_heads, head_size)

    backend = types.SimpleNamespace(TritonAttentionMetadataBuilder=TritonAttentionMetadataBuilder,
                                    TritonAttentionImpl=TritonAttentionImpl,
                                    TritonAttentionBackend=TritonAttentionBackend,
                                    get_tensor_model_parallel_world_size=lambda: 1)
    return backend, types.SimpleNamespace(GPUModelRunner=GPUModelRunner)


def vllm_seam_stack(qs, kcs, vcs, table, chunks, selected: str, prompt_len: int) -> dict:
    """The config-5 stack through the vLLM-ROCm seam on a stand-in backend: ms/prefill with the seam routing
    the selected layers, and with the feature off (every layer on the stand-in's own path); both write every
    chunk's K/V, as an engine does."""
    import types

    import torch

    from trianglemix import vllm_rocm
    from trianglemix.cache import chunk_slot_mapping
    from trianglemix.stats import runtime_stats
    from trianglemix.workload import SCALE

    backend, runner_mod = _stand_in_vllm(prompt_len)
    vllm_rocm.patch_modules(backend, runner_mod)
    layers = len(qs)
    rows = torch.arange(prompt_len, device=table.device)
    slots = table[0].long()[rows // 128] * 128 + rows % 128
    # fresh K/V of every token: the values already in the cache, so every run attends the same data
    kv = [(k.view(-1, 8, 128)[slots].contiguous(), v.view(-1, 8, 128)[slots].contiguous()) for k, v in zip(kcs, vcs)]
    caches = [torch.stack([k, v]) for k, v in zip(kcs, vcs)]
    outs = [torch.empty_like(q) for q in qs]
    commons = [types.SimpleNamespace(
        query_start_loc_cpu=torch.tensor([0, c.query_tokens], dtype=torch.int32),
        seq_lens_cpu=torch.tensor([c.seq_len], dtype=torch.int32), num_reqs=1, causal=True,
        block_table_tensor=table, slot_mapping=chunk_slot_mapping(table, c.query_start, c.query_tokens))
        for c in chunks]
    names = [types.SimpleNamespace(layer_name=f"model.layers.{i}.self_attn.attn") for i in range(layers)]
    result = {}
    for name, enabled in (("seam", True), ("seam_feature_off", False)):
        cfg = types.SimpleNamespace(additional_config={"trianglemix": {"enabled": enabled, "layers": selected}})
        builder = backend.TritonAttentionMetadataBuilder(None, [], cfg, table.device)
        runner = runner_mod.GPUModelRunner(builder)
        impls = [backend.TritonAttentionImpl(32, 128, SCALE, 8, None, None, "auto") for _ in range(layers)]

        def prefill():
            for c, common in zip(chunks, commons):
                md = runner._prepare_inputs(common)[0]["layers"]
                sl = slice(c.query_start, c.seq_len)
                for i in range(layers):
                    impls[i].forward(names[i], qs[i][sl], kv[i][0][sl], kv[i][1][sl], caches[i], md, outs[i][sl])

        prefill()  # warm-up
        torch.cuda.synchronize()
        runtime_stats().snapshot(reset=True)
        ms = median_ms(prefill, 1)
        counters = runtime_stats().snapshot()["counters"]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prefill()  # host time to issue one prefill (the GPU drains behind it)
        host_ms = (time.perf_counter() - t0) * 1e3
        torch.cuda.synchronize()
        result[name] = {"ms_per_prefill": round(ms, 3), "host_issue_ms_per_prefill": round(host_ms, 3),
                        "single_launch": counters.get("single_launch", 0), "layer_fia": counters.get("layer_fia", 0)}
    result["attention_time_cut"] = round(1 - result["seam"]["ms_per_prefill"]
                                         / result["seam_feature_off"]["ms_per_prefill"], 4)
    return result


class LayerStack:
    """36 attention layers at config-2 geometry (own Q / K / V per layer, one random page table), prefilled
    chunk by chunk through the plan / router layer."""

    L, CHUNK, LAYERS, SELECTED = 8192, 512, 36, "5,7,10,15-35"

    def __init__(self, seed: int):
        import torch

        from trianglemix.workload import prompt_chunks

        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev).manual_seed(seed)
        logical = self.L // 128
        pages = logical + 7
        self.table = torch.randperm(pages, generator=g, device=dev)[:logical].to(torch.int32).view(1, -1)
        shape = (pages, 128, 8, 128)
        self.kcs = [torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(self.LAYERS)]
        self.vcs = [torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(self.LAYERS)]
        self.qs = [torch.randn(self.L, 32, 128, generator=g, device=dev, dtype=torch.bfloat16)
                   for _ in range(self.LAYERS)]
        self.outs = [torch.empty_like(x) for x in self.qs]
        self.chunks = prompt_chunks(self.L, self.CHUNK)

    def config(self, enabled: bool, profile: str = "", log_interval: int = 0):
        """The stack's plugin config: the gate profile measured on this GPU (the router's default), or the
        named one ("reference": the reference's own gates)."""
        from trianglemix.router import device_plugin_config

        section = {"enabled": enabled, "layers": self.SELECTED, "stats_log_interval": log_interval}
        if profile:
            section["gate_profile"] = profile

        class _Vllm:
            additional_config = {"trianglemix": section}

        return device_plugin_config(_Vllm())

    def prefill(self, router, cfg) -> None:
        from trianglemix.planning import build_batch_plan
        from trianglemix.workload import SCALE

        for c in self.chunks:
            plan = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[c.query_tokens],
                                    seq_lens=[c.seq_len], prompt_lens=[self.L], num_decodes=0, num_prefills=1,
                                    config=cfg.kernel)
            for i in range(self.LAYERS):
                router.prefill_attention(layer_name=f"model.layers.{i}.self_attn.attn", plan=plan,
                                         query=self.qs[i][c.query_start:c.seq_len], key_cache=self.kcs[i],
                                         value_cache=self.vcs[i], block_table=self.table,
                                         output=self.outs[i][c.query_start:c.seq_len], softmax_scale=SCALE)

    def run(self, variants, windows: int = 3) -> dict:
        """ms per prefill (median of ``windows``, variants interleaved A B .. B A), stats snapshot and router
        log lines of each (name, enabled, gate profile, stats_log_interval) variant."""
        import torch

        from trianglemix.router import TriangleMixRouter
        from trianglemix.stats import TriangleMixRuntimeStats

        class _Lines(logging.Handler):
            def __init__(self):
                super().__init__()
                self.lines = []

            def emit(self, record):
                self.lines.append(record.getMessage())

        state = {}
        for name, enabled, profile, interval in variants:
            cfg = self.config(enabled, profile, interval)
            stats = TriangleMixRuntimeStats()
            router = TriangleMixRouter(cfg, stats=stats)
            self.prefill(router, cfg)  # warm-up
            torch.cuda.synchronize()
            stats.snapshot(reset=True)
            state[name] = (cfg, stats, router, _Lines(), [])
        router_log = logging.getLogger("trianglemix.router")
        level = router_log.level
        router_log.setLevel(logging.INFO)
        try:
            names = [v[0] for v in variants]
            for w in range(windows):
                for name in (names if w % 2 == 0 else names[::-1]):
                    cfg, stats, router, handler, times = state[name]
                    router_log.addHandler(handler)
                    try:
                        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        torch.cuda.synchronize()
                        s.record()
                        self.prefill(router, cfg)
                        e.record()
                        torch.cuda.synchronize()
                        times.append(s.elapsed_time(e))
                    finally:
                        router_log.removeHandler(handler)
        finally:
            router_log.setLevel(level)
        return {name: {"ms_per_prefill": round(statistics.median(times), 3), "windows_ms": [round(t, 3) for t in times],
                       "stats": stats.snapshot(reset=False), "log_lines": handler.lines}
                for name, (cfg, stats, router, handler, times) in state.items()}


def layer_stack_summary(seed: int) -> dict:
    """Config 5 leg of the default run: the router's default gates (those measured on this GPU) and the
    reference's gates vs every layer dense, with the counters."""
    import torch

    from trianglemix.config import device_gate_profile
    from trianglemix.workload import chunk_flops

    stack = LayerStack(seed)
    res = stack.run((("trianglemix", True, "", 0), ("reference_gates", True, "reference", 0),
                     ("all_dense", False, "", 0)))
    sel = stack.config(True).kernel.layer_indices
    tm = res["trianglemix"]["stats"]
    ref = res["reference_gates"]
    out = {
        "workload": f"L={stack.L}, chunked prefill {stack.CHUNK} x {len(stack.chunks)}, {stack.LAYERS} layers, "
                    f"layers {stack.SELECTED} sparse; eager, median of 3 interleaved prefills",
        "gates": device_gate_profile() or "reference",
        "ms_per_prefill": res["trianglemix"]["ms_per_prefill"],
        "reference_gates": {
            "ms_per_prefill": ref["ms_per_prefill"],
            "attention_time_cut": round(1 - ref["ms_per_prefill"] / res["all_dense"]["ms_per_prefill"], 4),
            "counters": {k: v for k, v in ref["stats"]["counters"].items() if not k.endswith("_ns")},
            "fallback_reasons": ref["stats"]["fallback_reasons"],
        },
        "all_dense_ms_per_prefill": res["all_dense"]["ms_per_prefill"],
        "attention_time_cut": round(1 - res["trianglemix"]["ms_per_prefill"] / res["all_dense"]["ms_per_prefill"], 4),
        "gflop": {"routed": round(sum(chunk_flops(c, dense=(i not in sel)) for c in stack.chunks
                                      for i in range(stack.LAYERS)) / 1e9, 1),
                  "all_dense": round(sum(chunk_flops(c, dense=True) for c in stack.chunks) * stack.LAYERS / 1e9, 1)},
        "counters": {k: v for k, v in tm["counters"].items() if not k.endswith("_ns")},
        "fallback_reasons": tm["fallback_reasons"],
    }
    del stack
    torch.cuda.empty_cache()
    return out


def host_overhead(args) -> int:
    """Host time per call of one config-2 middle chunk at each API level, beside the kernel's device time.

    Each level is called 100 times back to back with no synchronisation inside the timed loop, so the time
    is what the host spends per call; events around the same calls give the rate the GPU sees (the larger
    of host and device time).  The device time comes from a HIP graph of 16 launches.
    """
    import torch

    from trianglemix import cabi, kernel, native
    from trianglemix.planning import build_batch_plan
    from trianglemix.router import TriangleMixRouter, device_plugin_config
    from trianglemix.stats import TriangleMixRuntimeStats
    from trianglemix.workload import SCALE, make_cache, make_query

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    native.load_hip_library()
    native.load_triangle_mix_adapter()
    dev = torch.device("cuda:0")
    qs, tq, prompt = 4096, 512, 8192
    seq = qs + tq
    k, v, bt = make_cache(seq, args.seed, std=1.0)
    q = make_query(tq, args.seed + 1, std=1.0)
    kd, vd, btd, qd = k.to(dev), v.to(dev), bt.to(dev), q.to(dev)
    out = torch.empty_like(qd)

    def router_for(layers: str):
        class _Vllm:
            additional_config = {"trianglemix": {"enabled": True, "layers": layers}}

        cfg = device_plugin_config(_Vllm())
        return cfg, TriangleMixRouter(cfg, stats=TriangleMixRuntimeStats())

    cfg, router = router_for("0-35")
    _, dense_router = router_for("5")
    plan = build_batch_plan(state_name="ChunkedPrefill", cumulative_query_ends=[tq], seq_lens=[seq],
                            prompt_lens=[prompt], num_decodes=0, num_prefills=1, config=cfg.kernel)
    routed = dict(plan=plan, query=qd, key_cache=kd, value_cache=vd, block_table=btd, output=out, softmax_scale=SCALE)
    levels = {
        "torch_op": lambda: torch.ops.trianglemix.triangle_paged_sparse_attention.out(
            qd, kd, vd, btd, qs, seq, prompt, SCALE, out=out),
        "c_abi_ctypes": lambda: cabi.triangle_paged_sparse_attention(
            qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt, scale=SCALE),
        "python_op": lambda: kernel.triangle_direct_paged_attention(
            query=qd, key_cache=kd, value_cache=vd, block_table=btd, seq_len=seq, prompt_len=prompt, output=out,
            softmax_scale=SCALE, config=cfg.kernel),
        "router_direct": lambda: router.prefill_attention(layer_name="model.layers.5.self_attn.attn", **routed),
        "router_dense_layer": lambda: dense_router.prefill_attention(layer_name="model.layers.6.self_attn.attn",
                                                                     **routed),
    }
    result = {}
    for name, fn in levels.items():
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        host = []
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(100):
                fn()
            host.append((time.perf_counter() - t0) * 1e4)
            torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(100):
            fn()
        e.record()
        torch.cuda.synchronize()
        result[name] = {"host_us_per_call": round(statistics.median(host), 2),
                        "stream_us_per_call": round(s.elapsed_time(e) * 10, 2)}
    graph = graph_of(lambda: [levels["torch_op"]() for _ in range(16)])
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(10):
        graph.replay()
    e.record()
    torch.cuda.synchronize()
    print(json.dumps({
        "metric": "host time per attention call (one middle chunk, L=8192 chunk 512)", "unit": "us/call",
        "n_gpus": 1, "higher_is_better": False, "data": "synthetic",
        "config": {"workload": "host: qs=4096 tq=512 prompt=8192, 100 calls per level, median of 5 windows"},
        "levels": result, "device_us_per_call": round(s.elapsed_time(e) * 1000 / 160, 2),
    }), flush=True)
    return 0


def config5_stack(args) -> int:
    """36 layers x config 2 through the plan / router layer; counters from the stats snapshot."""
    from trianglemix import native
    from trianglemix.config import device_gate_profile
    from trianglemix.counters import aggregate as counters_aggregate
    from trianglemix.counters import report_status, scan_events
    from trianglemix.workload import chunk_flops

    native.load_hip_library()
    native.load_triangle_mix_adapter()
    stack = LayerStack(args.seed)
    chunks, L, layers = stack.chunks, stack.L, stack.LAYERS
    results = stack.run((("trianglemix", True, "", 0),
                         ("trianglemix_reference_gates", True, "reference", 0),
                         ("all_dense", False, "", 0),
                         ("trianglemix_logged", True, "", len(chunks))), windows=1)
    # the structured log of the logged run, aggregated the way a run's worker logs are
    logged = results["trianglemix_logged"]
    report = counters_aggregate(scan_events("\n".join(logged["log_lines"]), source="config5"))
    structured_log = {
        "stats_log_interval": len(chunks),
        "events": report["event_count"],
        "status": report_status(report),
        "aggregate_equals_snapshot": (report["aggregate"]["counters"] == logged["stats"]["counters"]
                                      and report["aggregate"]["layers"] == logged["stats"]["layers"]),
        "ms_per_prefill": logged["ms_per_prefill"],
        "logging_overhead": round(logged["ms_per_prefill"] / results["trianglemix"]["ms_per_prefill"] - 1, 4),
    }
    sel = stack.config(True).kernel.layer_indices
    gflop = sum(chunk_flops(c, dense=(i not in sel)) for c in chunks for i in range(layers)) / 1e9
    dense_gflop = sum(chunk_flops(c, dense=True) for c in chunks) * layers / 1e9
    tm = results["trianglemix"]["stats"]
    line = {
        "metric": "36-layer prefill attention through the plan / router layer (config5)",
        "value": results["trianglemix"]["ms_per_prefill"],
        "unit": "ms/prefill (36 layers x 16 chunks, eager)",
        "n_gpus": 1,
        "higher_is_better": False,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V per layer from the GPU generator, random page table)",
        "config": {"workload": f"config5: L={L}, chunked prefill {stack.CHUNK} x {len(chunks)}, {layers} layers, "
                               f"layers {stack.SELECTED} sparse",
                   "gates": (device_gate_profile() or "reference") + " (the router's default on this GPU)"},
        "all_dense_ms_per_prefill": results["all_dense"]["ms_per_prefill"],
        "reference_gates": {
            "ms_per_prefill": results["trianglemix_reference_gates"]["ms_per_prefill"],
            "attention_time_cut": round(1 - results["trianglemix_reference_gates"]["ms_per_prefill"]
                                        / results["all_dense"]["ms_per_prefill"], 4),
            "counters": results["trianglemix_reference_gates"]["stats"]["counters"],
            "fallback_reasons": results["trianglemix_reference_gates"]["stats"]["fallback_reasons"],
        },
        "attention_time_cut": round(1 - results["trianglemix"]["ms_per_prefill"]
                                    / results["all_dense"]["ms_per_prefill"], 4),
        "gflop": {"routed": round(gflop, 1), "all_dense": round(dense_gflop, 1)},
        "counters": tm["counters"],
        "fallback_reasons": tm["fallback_reasons"],
        "routing": tm["performance"],
        "structured_log": structured_log,
        "vllm_seam": vllm_seam_stack(stack.qs, stack.kcs, stack.vcs, stack.table, chunks, stack.SELECTED, L),
    }
    print(json.dumps(line), flush=True)
    return 0


def kv_write_bench(args, chunks, k, v, bt, dev):
    """Paged KV write: µs and HBM GB/s for one chunk and for the whole prompt (checked against the cache)."""
    import torch

    from trianglemix.cache import chunk_slot_mapping

    table = bt[0].tolist()
    logical = torch.tensor([table[t // 128] * 128 + t % 128 for t in range(args.prompt)], dtype=torch.int64)
    k_tok = k.view(-1, 8, 128)[logical].to(dev)  # each token's fresh K / V, in logical order
    v_tok = v.view(-1, 8, 128)[logical].to(dev)
    btd = bt.to(dev)
    kc = torch.zeros(k.shape, dtype=k.dtype, device=dev)
    vc = torch.zeros_like(kc)
    op = torch.ops.trianglemix.reshape_and_cache
    slots = [chunk_slot_mapping(btd, c.query_start, c.query_tokens) for c in chunks]
    for c, sl in zip(chunks, slots):  # fill chunk by chunk, as the prefill does
        op(k_tok[c.query_start:c.seq_len], v_tok[c.query_start:c.seq_len], kc, vc, sl)
    torch.cuda.synchronize()
    if not (torch.equal(kc.view(-1, 8, 128)[logical.to(dev)], k_tok) and
            torch.equal(vc.view(-1, 8, 128)[logical.to(dev)], v_tok)):
        raise RuntimeError("paged KV write does not reproduce the cache")

    def per_call_us(fn, reps=50):
        fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1000.0 / reps

    c0, s0 = chunks[len(chunks) // 2], slots[len(chunks) // 2]
    # eager calls: bound by the host's enqueue rate (one torch op per chunk)
    us_chunk = per_call_us(lambda: op(k_tok[c0.query_start:c0.seq_len], v_tok[c0.query_start:c0.seq_len], kc, vc, s0))
    all_slots = chunk_slot_mapping(btd, 0, args.prompt)
    us_prompt = per_call_us(lambda: op(k_tok, v_tok, kc, vc, all_slots))

    # device time: every chunk's write replayed as one HIP graph, as a captured prefill step would run them
    def all_chunks():
        for c, sl in zip(chunks, slots):
            op(k_tok[c.query_start:c.seq_len], v_tok[c.query_start:c.seq_len], kc, vc, sl)

    graph = graph_of(all_chunks)
    us_chunk_graph = per_call_us(graph.replay, reps=20) / len(chunks)
    torch.cuda.synchronize()
    if not (torch.equal(kc.view(-1, 8, 128)[logical.to(dev)], k_tok) and
            torch.equal(vc.view(-1, 8, 128)[logical.to(dev)], v_tok)):
        raise RuntimeError("paged KV write replayed from a graph does not reproduce the cache")
    moved = lambda tokens: tokens * 8 * 128 * 2 * 2 * 2  # K and V rows, read and written
    gbs_chunk = moved(c0.query_tokens) / (us_chunk * 1e-6) / 1e9
    gbs_prompt = moved(args.prompt) / (us_prompt * 1e-6) / 1e9
    return {
        "chunk_tokens": c0.query_tokens,
        "us_per_chunk": round(us_chunk, 2),
        "gbs_chunk": round(gbs_chunk, 1),
        "us_per_chunk_graph": round(us_chunk_graph, 2),
        "gbs_chunk_graph": round(moved(c0.query_tokens) / (us_chunk_graph * 1e-6) / 1e9, 1),
        "prompt_tokens": args.prompt,
        "us_prompt": round(us_prompt, 2),
        "gbs_prompt": round(gbs_prompt, 1),
        "peak_gbs": PEAK_HBM_GBS,
        "frac_hbm_prompt": round(gbs_prompt / PEAK_HBM_GBS, 4),
        # the repeated whole-prompt calls move the same 67 MB, which stays in the 256 MB Infinity Cache:
        # the rate is algorithmic bytes over time and can exceed the HBM figure
        "note": "algorithmic bytes / time; repeated calls keep the working set in the Infinity Cache",
    }


def read_traffic_summary():
    """HBM bytes per launch of the attention kernel from the committed rocprofv3 summary, or None."""
    if not TRAFFIC_SUMMARY.is_file():
        return None
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            try:
                return int(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline(chunks, qfull, k, v, bt, scale):
    """fp32 PyTorch CPU oracle over all chunks on every core of this host: one warm-up pass, median of 3."""
    import torch

    from oracle.attention import attention_torch

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    print(f"# cpu_baseline: torch.set_num_threads({threads}) (os.cpu_count()); "
          f"{len(os.sched_getaffinity(0))} cores in this process's affinity mask", file=sys.stderr, flush=True)

    def one_pass():
        t0 = time.perf_counter()
        for c in chunks:
            attention_torch(qfull[c.query_start:c.seq_len], k, v, bt, c.query_start, c.seq_len, c.prompt_len, scale)
        return time.perf_counter() - t0

    warm = one_pass()
    passes = [one_pass() for _ in range(3)]
    per_chunk_us = statistics.median(passes) / len(chunks) * 1e6
    return {
        "value": round(per_chunk_us, 1),
        "unit": "us/chunk",
        "cores": threads,
        "kind": "port",
        "sample": (f"all {len(chunks)} chunks of the same workload (same seeded inputs), fp32 torch CPU oracle; "
                   f"one warm-up pass ({warm:.2f} s), then the median of 3 passes "
                   f"({', '.join(f'{x:.2f}' for x in passes)} s)"),
    }


if __name__ == "__main__":
    raise SystemExit(main())
