"""Benchmark: TriangleMix sparse prefill attention on one MI355X.

Workload (the headline configuration): Qwen3-8B attention geometry (Hq=32, Hkv=8,
D=128, bf16, page 128), one request, prompt L=8192 prefilled in 16 chunks of
512.  One *step* = the 16 chunk launches of the sparse kernel, in order, over
one paged K/V cache (random block-table permutation) that already holds the
whole prompt's K/V; all inputs are resident in HBM before timing.

Reported JSON line (rank 0 only):

* ``value`` -- mean microseconds per chunk of the sparse kernel (graph
  replay of the 16 launches, HIP events on the launch stream);
* ``roofline`` -- bf16 MFMA bound: algorithmic FLOPs per launch
  (4*D*Hq*attended pairs) / average launch duration, vs 2.5 PFLOP/s;
  ``traffic`` is the rocprofv3 FETCH+WRITE bytes per launch when a summary
  for this workload exists under profiles/, else null;
* ``dense`` -- the same 16 chunks through the dense paged causal companion
  kernel, and the attention-time cut of sparse vs dense (ABBA order);
* ``kv_write`` -- the paged KV write upstream of the attention
  (``trianglemix::reshape_and_cache``): one chunk's fresh K/V into its pages,
  and the whole prompt in one call, with HBM GB/s against 8 TB/s (it moves
  each token's 2 KB K row and 2 KB V row in and out);
* ``cpu_baseline`` -- the fp32 PyTorch CPU masked-attention restatement of the
  reference's oracle (``oracle.attention.attention_torch``) over all 16
  chunks, median of 2 passes after a warm-up, on this host's cores.

``--gpus N`` with N > 1 is refused: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
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
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead of a HIP graph")
    ap.add_argument("--only", choices=("sparse", "dense"), help="run one kernel only (for profiling)")
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
    from trianglemix.workload import (SCALE, chunk_bytes, chunk_flops, executed_flops, kv_bytes, make_cache,
                                      make_query, prompt_chunks)

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    native.load_hip_library()
    native.load_triangle_mix_adapter()
    dev = torch.device("cuda:0")
    chunks = prompt_chunks(args.prompt, args.chunk)

    k, v, bt = make_cache(args.prompt, args.seed, std=1.0)
    qfull = make_query(args.prompt, args.seed + 1, std=1.0)
    kd, vd, btd = k.to(dev), v.to(dev), bt.to(dev)
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

    # Eager reference results for the graph replay checks.
    sparse_step()
    torch.cuda.synchronize()
    eager_sparse = [o.clone() for o in outs]
    dense_step()
    torch.cuda.synchronize()
    eager_dense = [o.clone() for o in outs]

    def make_runner(step, reference):
        if args.no_graph:
            return step
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            step()  # warm the allocator on the capture stream
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                step()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        for _ in range(3):  # every replay must reproduce the eager result
            for o in outs:
                o.zero_()
            graph.replay()
            torch.cuda.synchronize()
            for o, ref in zip(outs, reference):
                if not torch.equal(o, ref):
                    raise RuntimeError("graph replay differs from eager launches")
        return graph.replay

    run_sparse = make_runner(sparse_step, eager_sparse)
    run_dense = make_runner(dense_step, eager_dense)

    def timed(run, steps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            run()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps  # ms per step

    for _ in range(args.warmup):
        if args.only != "dense":
            run_sparse()
        if args.only != "sparse":
            run_dense()
    torch.cuda.synchronize()

    # ABBA: sparse, dense, dense, sparse -- the timed region is the 2K sparse steps.
    sparse_ms, dense_ms = [], []
    half = max(1, args.steps // 2)
    for order in ("sd", "ds"):
        for which in order:
            if which == "s" and args.only != "dense":
                sparse_ms.append(timed(run_sparse, half))
            if which == "d" and args.only != "sparse":
                dense_ms.append(timed(run_dense, half))
    ms_sparse = statistics.mean(sparse_ms) if sparse_ms else float("nan")
    ms_dense = statistics.mean(dense_ms) if dense_ms else float("nan")

    # Per-chunk kernel durations (eager, R back-to-back launches per chunk).
    per_chunk_us = []
    if args.only != "dense":
        reps = 20
        for c, q, o in zip(chunks, qs, outs):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(reps):
                sparse_op(q, kd, vd, btd, c.query_start, c.seq_len, c.prompt_len, SCALE, out=o)
            e.record()
            torch.cuda.synchronize()
            per_chunk_us.append(round(s.elapsed_time(e) * 1000.0 / reps, 2))

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

    traffic = read_traffic_summary()

    kv_write = kv_write_bench(args, chunks, k, v, bt, dev) if args.only is None else None

    cpu = None
    if not args.no_cpu_baseline and args.only is None:
        cpu = cpu_baseline(chunks, qfull, k, v, bt, SCALE)

    line = {
        "metric": METRIC,
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
            "workload": f"config2: one request, L={args.prompt}, chunked prefill {args.chunk} x {n} chunks, "
                        "Hq=32 Hkv=8 D=128 page=128, one layer",
            "timing": "HIP-graph replay of the 16 launches" if not args.no_graph else "eager launches",
        },
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
            "kv_hbm_gbs": round(kvb / (ms_sparse * 1e-3) / 1e9, 1),
        },
        "per_chunk_us": per_chunk_us,
        "dense": {
            "ms_per_step": round(ms_dense, 5),
            "us_per_chunk": round(ms_dense * 1000.0 / n, 3),
            "alg_tflops": round(dense_flops / (ms_dense * 1e-3) / 1e12, 2) if ms_dense == ms_dense else None,
            "attention_time_cut": round(1.0 - ms_sparse / ms_dense, 4) if ms_dense == ms_dense else None,
        },
        "kv_write": kv_write,
        "cpu_baseline": cpu,
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
    us_chunk = per_call_us(lambda: op(k_tok[c0.query_start:c0.seq_len], v_tok[c0.query_start:c0.seq_len], kc, vc, s0))
    all_slots = chunk_slot_mapping(btd, 0, args.prompt)
    us_prompt = per_call_us(lambda: op(k_tok, v_tok, kc, vc, all_slots))
    moved = lambda tokens: tokens * 8 * 128 * 2 * 2 * 2  # K and V rows, read and written
    gbs_chunk = moved(c0.query_tokens) / (us_chunk * 1e-6) / 1e9
    gbs_prompt = moved(args.prompt) / (us_prompt * 1e-6) / 1e9
    return {
        "chunk_tokens": c0.query_tokens,
        "us_per_chunk": round(us_chunk, 2),
        "gbs_chunk": round(gbs_chunk, 1),
        "prompt_tokens": args.prompt,
        "us_prompt": round(us_prompt, 2),
        "gbs_prompt": round(gbs_prompt, 1),
        "peak_gbs": PEAK_HBM_GBS,
        "frac_hbm_prompt": round(gbs_prompt / PEAK_HBM_GBS, 4),
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
    """fp32 PyTorch CPU oracle over all chunks (bounded: ~2 passes of ~6 s)."""
    import torch

    from oracle.attention import attention_torch

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    mid = chunks[len(chunks) // 2]
    attention_torch(qfull[mid.query_start:mid.seq_len], k, v, bt, mid.query_start, mid.seq_len, mid.prompt_len,
                    scale)  # warm-up
    passes = []
    for _ in range(2):
        t0 = time.perf_counter()
        for c in chunks:
            attention_torch(qfull[c.query_start:c.seq_len], k, v, bt, c.query_start, c.seq_len, c.prompt_len,
                            scale)
        passes.append(time.perf_counter() - t0)
    per_chunk_us = statistics.median(passes) / len(chunks) * 1e6
    return {
        "value": round(per_chunk_us, 1),
        "unit": "us/chunk",
        "cores": threads,
        "kind": "port",
        "sample": f"all {len(chunks)} chunks of the same workload, fp32 torch CPU oracle, median of 2 passes",
    }


if __name__ == "__main__":
    raise SystemExit(main())
