"""Seeded random long-context chunk geometries on the GPU against the fp32 oracle.

The companion of test_gpu_random_geometry.py for longer sequences: 48 chunks
drawn from a fixed seed with L up to 20,000 and chunks of up to 2,048 rows.
The draws include tiny queries deep into a prompt, chunk sizes one off 128 /
256 / 512, 1,000-2,048-row chunks, last chunks whose dense tail splits over
KV, unaligned medium chunks, and prompts longer than the sequence.  Chunks of
more than 256 rows are compared on a row subset (the first and last 64 rows
and the rows within 32 of the sparse start at 521), which keeps the CPU
oracle cheap; the oracle of a row subset equals the same rows of the whole
chunk (a contiguous query range with its own query_start / seq_len).  Every
fifth case also runs the dense companion and every seventh repeats the call
and requires identical bytes.  Tolerances: max-abs 2e-2, mean-abs 2e-3,
relative L2 2e-2 vs fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from trianglemix import cabi
from trianglemix.workload import SCALE, make_inputs

MAX_ABS, MEAN_ABS, REL_L2 = 2e-2, 2e-3, 2e-2


def _cases(n=48, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 8
        if kind == 0:    # tiny queries deep into a prompt
            seq, tq = int(rng.integers(1, 20000)), int(rng.integers(1, 40))
        elif kind == 1:  # chunk sizes one off the row-block / page multiples
            seq, tq = int(rng.integers(512, 20000)), int(rng.choice([127, 128, 129, 255, 256, 257, 511, 512, 513]))
        elif kind == 2:  # large chunks
            seq, tq = int(rng.integers(2048, 20000)), int(rng.integers(1000, 2049))
        elif kind == 3:  # last chunks: the dense tail splits over KV
            seq, tq = int(rng.integers(4000, 20000)), int(rng.integers(64, 1024))
        elif kind == 4:  # around the sparse start and the window edge
            seq = int(rng.integers(500, 1200))
            tq = int(rng.integers(1, seq + 1))
        elif kind == 5:  # whole prompts
            seq = int(rng.integers(1, 4000))
            tq = seq
        elif kind == 6:  # unaligned medium chunks
            seq, tq = int(rng.integers(3000, 12000)), int(rng.integers(200, 900))
        else:
            seq, tq = int(rng.integers(8000, 20000)), int(rng.integers(1, 2049))
        tq = max(1, min(tq, seq))
        prompt = seq if rng.random() < 0.5 else seq + int(rng.integers(1, 6000))
        out.append((i, seq - tq, tq, seq, prompt))
    return out


CASES = _cases()


def _checked_rows(qs, tq):
    """Contiguous [a, b) row runs of the chunk that are compared with the oracle."""
    if tq <= 256:
        return [(0, tq)]
    rows = sorted(set(range(64)) | set(range(tq - 64, tq)) | {r for r in range(tq) if abs(qs + r - 521) < 32})
    runs, start = [], rows[0]
    for a, b in zip(rows, rows[1:] + [None]):
        if b is None or b != a + 1:
            runs.append((start, a + 1))
            start = b
    return runs


def _oracle(q, k, v, bt, qs, prompt, runs, dense=False):
    return torch.cat([OA.attention_torch(q[a:b].contiguous(), k, v, bt, qs + a, qs + b, prompt, SCALE, dense=dense)
                      for a, b in runs])


def _picked(out, runs):
    return torch.cat([out[a:b] for a, b in runs])


def test_row_subset_oracle_equals_whole_chunk():
    """The oracle of a contiguous row range equals those rows of the whole chunk (CPU)."""
    qs, tq, seq, prompt = 700, 300, 1000, 1500
    q, k, v, bt = make_inputs(qs, tq, seq, 3, std=1.0)
    full = OA.attention_torch(q, k, v, bt, qs, seq, prompt, SCALE)
    runs = _checked_rows(qs, tq)
    assert torch.equal(_picked(full, runs), _oracle(q, k, v, bt, qs, prompt, runs))


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[f"L{c[0]}_qs{c[1]}_tq{c[2]}_seq{c[3]}_p{c[4]}" for c in CASES])
def test_random_long_geometry_matches_oracle(gpu, case):
    i, qs, tq, seq, prompt = case
    print(f"case {case}", flush=True)
    q, k, v, bt = make_inputs(qs, tq, seq, 5000 + i, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    out = torch.full_like(qd, float("nan"))
    cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                         scale=SCALE)
    torch.cuda.synchronize()
    runs = _checked_rows(qs, tq)
    m = OA.error_metrics(_picked(out.cpu(), runs).float().numpy(), _oracle(q, k, v, bt, qs, prompt, runs).float().numpy())
    assert m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, m
    if i % 7 == 0:
        again = torch.full_like(qd, float("nan"))
        cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, again, query_start=qs, seq_len=seq, prompt_len=prompt,
                                             scale=SCALE)
        torch.cuda.synchronize()
        assert torch.equal(out, again)
    if i % 5 == 0:
        dense = torch.full_like(qd, float("nan"))
        cabi.dense_paged_causal_attention(qd, kd, vd, btd, dense, query_start=qs, seq_len=seq, scale=SCALE)
        torch.cuda.synchronize()
        md = OA.error_metrics(_picked(dense.cpu(), runs).float().numpy(),
                              _oracle(q, k, v, bt, qs, prompt, runs, dense=True).float().numpy())
        assert md["finite"] and md["max_abs"] <= MAX_ABS and md["mean_abs"] <= MEAN_ABS, md
