"""Seeded random chunks whose launch plans split long rows, in every workgroup shape, against the fp32
oracle on the GPU.

The planner cuts long rows (a prompt's dense tail, the dense companion's causal rows) into pieces merged
inside the launch, as KV quarters, KV halves or KV whole, depending on the chunk (csrc/trianglemix_capi.cpp
choose_plan, fitted to tests/plan_sweep_mi355x.json).  64 chunks drawn from a fixed seed -- last chunks of
prompts of 6000-24000 tokens, whole prompts, and a fifth of them through the dense companion -- cover each
shape with and without split items (the draw is checked on the CPU); their outputs are compared with the
fp32 oracle on row subsets (the first and last 64 rows and the rows near the sparse start; every row of a
chunk of at most 256 rows).  Tolerances: max-abs 2e-2, mean-abs 2e-3, relative L2 2e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_random_geometry_long import _checked_rows, _oracle, _picked
from trianglemix import cabi
from trianglemix.workload import SCALE, make_inputs

MAX_ABS, MEAN_ABS, REL_L2 = 2e-2, 2e-3, 2e-2


def _cases(n=64, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        if i % 2 == 0:   # last chunks of long prompts: dense-tail rows split
            seq = int(rng.integers(6000, 24000))
            tq = int(rng.choice([64, 128, 256, 512, 1024, 2048, 3000]))
        elif i % 4 == 1:  # whole prompts
            seq = int(rng.integers(1000, 16000))
            tq = seq
        else:             # chunks ending anywhere, of any size
            seq = int(rng.integers(600, 24000))
            tq = int(rng.integers(1, min(seq, 4096) + 1))
        tq = max(1, min(tq, seq))
        prompt = seq if rng.random() < 0.6 else seq + int(rng.integers(1, 8000))
        dense = bool(rng.random() < 0.2)
        out.append((i, seq - tq, tq, seq, prompt, dense))
    return out


CASES = _cases()


def _plan(case):
    _, qs, tq, seq, prompt, dense = case
    p = None if dense else prompt
    return cabi.chunk_plan(tq, qs, seq, p)[0], cabi.workspace_size(tq, qs, seq, p) > 0


def test_draw_covers_every_shape_with_split_items():
    """The seeded draw holds split plans of all three shapes for the TriangleMix op, and split plans of the
    dense companion (CPU)."""
    plans = {(_plan(c), c[5]) for c in CASES}
    for parts in (4, 2, 1):
        assert ((parts, True), False) in plans, parts
    assert any(split and dense for (_, split), dense in plans)


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[f"r{c[0]}_qs{c[1]}_tq{c[2]}_seq{c[3]}_p{c[4]}{'_dense' if c[5] else ''}"
                                             for c in CASES])
def test_random_split_plan_matches_oracle(gpu, case):
    i, qs, tq, seq, prompt, dense = case
    print(f"case {case} plan {cabi.chunk_plan(tq, qs, seq, None if dense else prompt)}", flush=True)
    q, k, v, bt = make_inputs(qs, tq, seq, 9000 + i, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    out = torch.full_like(qd, float("nan"))
    if dense:
        cabi.dense_paged_causal_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, scale=SCALE)
    else:
        cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                             scale=SCALE)
    torch.cuda.synchronize()
    runs = _checked_rows(qs, tq)
    got = _picked(out.cpu(), runs).float()
    expected = _oracle(q, k, v, bt, qs, seq if dense else prompt, runs, dense=dense)
    assert torch.isfinite(got).all()
    d = (got - expected).abs()
    rel = (d.norm() / expected.norm().clamp_min(1e-12)).item()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS and rel <= REL_L2, (d.max().item(), rel)
