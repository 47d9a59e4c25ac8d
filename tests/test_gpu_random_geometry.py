"""Seeded random chunk geometries on the GPU against the fp32 oracle.

Beyond the reference's boundary matrix: 36 chunks drawn from a fixed seed,
biased toward the edges of the mask and the schedule.  The draws cover
query lengths of 1-3 and 31-33 tokens, chunks that start mid-page, rows next
to the sparse start (521), prompts much longer than the sequence (no dense
tail yet), and last chunks whose dense tail forces KV splits.  Every tenth
case also runs the dense companion against the causal oracle.  The tolerances
are the project's (max-abs 2e-2, mean-abs 2e-3, relative L2 2e-2 vs fp32).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from trianglemix import cabi
from trianglemix.workload import SCALE, make_inputs

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS, REL_L2 = 2e-2, 2e-3, 2e-2


def _cases(n=36, seed=20261201):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 6
        if kind == 0:    # tiny queries anywhere
            seq = int(rng.integers(1, 3000))
            tq = int(rng.choice([1, 2, 3]))
        elif kind == 1:  # ragged around the row block
            seq = int(rng.integers(40, 3000))
            tq = int(rng.choice([31, 32, 33, 63, 65]))
        elif kind == 2:  # around the sparse start
            seq = int(rng.integers(500, 560))
            tq = int(rng.integers(1, min(seq, 96)))
        elif kind == 3:  # mid-page starts, medium chunks
            seq = int(rng.integers(600, 3200))
            tq = int(rng.integers(100, min(seq, 700)))
        elif kind == 4:  # whole short prompts
            seq = int(rng.integers(1, 900))
            tq = seq
        else:            # long rows: last chunks with a dense tail that splits
            seq = int(rng.integers(2500, 3600))
            tq = int(rng.integers(64, 300))
        tq = max(1, min(tq, seq))
        qs = seq - tq
        prompt = seq if rng.random() < 0.4 else seq + int(rng.integers(1, 3000))
        out.append((i, qs, tq, seq, prompt))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[f"g{c[0]}_qs{c[1]}_tq{c[2]}_seq{c[3]}_p{c[4]}" for c in CASES])
def test_random_geometry_matches_oracle(gpu, case):
    i, qs, tq, seq, prompt = case
    print(f"case {case}", flush=True)
    q, k, v, bt = make_inputs(qs, tq, seq, 1000 + i, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    out = torch.full_like(qd, float("nan"))
    cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                         scale=SCALE)
    torch.cuda.synchronize()
    expected = OA.attention_torch(q, k, v, bt, qs, seq, prompt, SCALE)
    m = OA.error_metrics(out.float().cpu().numpy(), expected.float().numpy())
    assert m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, m
    if i % 10 == 0:
        dense = torch.full_like(qd, float("nan"))
        cabi.dense_paged_causal_attention(qd, kd, vd, btd, dense, query_start=qs, seq_len=seq, scale=SCALE)
        torch.cuda.synchronize()
        expected_dense = OA.attention_torch(q, k, v, bt, qs, seq, prompt, SCALE, dense=True)
        md = OA.error_metrics(dense.float().cpu().numpy(), expected_dense.float().numpy())
        assert md["finite"] and md["max_abs"] <= MAX_ABS and md["mean_abs"] <= MEAN_ABS, md
