"""Long-context correctness: BASELINE config 4 (L = 32768 and 131072, chunk 2048).

At L = 131072 a dense-tail row attends 131072 keys = 4096 tiles: the
TriangleMix op splits those rows over the GPU (sixteen pieces of 256 tiles,
merged inside the launch) and the dense companion runs each of its 64 row
blocks as one item of ~4096 tiles; the position, row-index and page
arithmetic run at sizes no other test reaches.  The reference pins its
longest case the same way (operator/tests/npu_v2_correctness.py:53-216,
``long_random_paged_8192``) and keeps an exact on-device reference
(operator/op_kernel/triangle_paged_sparse_attention.cpp:22-322); here the
fp32 oracle runs on the GPU in its blocked form, so whole chunks are checked.

* Oracle parity (N(0,1) bf16, random page table) on EVERY row of the
  prompt's last chunk and of a middle chunk, for the TriangleMix op, and of
  the dense companion's last chunk; tolerances as everywhere (max-abs 2e-2,
  mean-abs 2e-3, rel-L2 2e-2), the mean also per 32-row block.
* The exact mask identity over the WHOLE last chunk (KV whole, dense-tail rows in pieces) and a whole
  middle chunk at L = 32768 (KV whole: four-wave workgroups, two per CU,
  one wave per head over every tile): Q = 0 weighs every
  attended key 1/|S|, and one-hot residue V rows turn each output row into
  the residue histogram of its key set (8 moduli), so one added, dropped or
  shifted key of any row changes the output.  Counts and sums are exact
  integers in fp32; bf16 rounding of count/|S| (half an ulp) is the only
  difference allowed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import geometry as OG
from trianglemix import cabi
from trianglemix.workload import SCALE, make_cache, make_query

pytestmark = pytest.mark.gpu

CHUNK = 2048
MAX_ABS, MEAN_ABS, REL_L2 = 2e-2, 2e-3, 2e-2


def _check_all_rows(label, got, qd, kd, vd, btd, qs, seq, prompt, dense=False):
    assert torch.isfinite(got.float()).all(), label
    expected = OA.attention_torch_blocked(qd, kd, vd, btd, qs, seq, prompt, SCALE, dense=dense, max_scores=1 << 27)
    d = (got.float() - expected).abs()
    per_block = d.reshape(-1, 32 * 32 * 128).mean(1)  # 2048 rows = 64 row blocks of 32
    m = {"max_abs": d.max().item(), "mean_abs": d.mean().item(),
         "relative_l2": (d.norm() / expected.norm().clamp_min(1e-12)).item(),
         "worst_block_mean_abs": per_block.max().item()}
    print(f"{label}: {m}", flush=True)
    assert m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, (label, m)
    assert m["worst_block_mean_abs"] <= MEAN_ABS, (label, m)


def _sparse(gpu, qd, kd, vd, btd, qs, seq, prompt):
    out = torch.full_like(qd, float("nan"))
    cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                         scale=SCALE)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("L", [32768, 131072])
def test_long_context_rows_match_oracle(gpu, L):
    prompt = L
    k, v, bt = make_cache(L, 700 + L // 1024, std=1.0)
    kd, vd, btd = k.to(gpu), v.to(gpu), bt.to(gpu)
    del k, v
    for label, qs in (("last", L - CHUNK), ("middle", L // 2)):
        seq = qs + CHUNK
        qd = make_query(CHUNK, 900 + qs // 1024, std=1.0).to(gpu)
        plan = cabi.chunk_plan(CHUNK, qs, seq, prompt)
        print(f"L={L} {label} chunk qs={qs} plan={plan} "
              f"workspace={cabi.workspace_size(CHUNK, qs, seq, prompt)}", flush=True)
        # both run as KV whole (four-wave workgroups, two per CU); the last chunk cuts its dense-tail rows
        # into pieces merged inside the launch
        assert plan[0] == 1, plan
        got = _sparse(gpu, qd, kd, vd, btd, qs, seq, prompt)
        _check_all_rows(f"L={L} {label} rows {qs}..{seq - 1}", got, qd, kd, vd, btd, qs, seq, prompt)
    assert cabi.workspace_size(CHUNK, L - CHUNK, L, prompt) > cabi.WORKSPACE_COUNTER_BYTES  # dense tail split


@pytest.mark.parametrize("L", [32768, 131072])
def test_long_context_dense_companion_rows_match_oracle(gpu, L):
    """The dense companion's last 2048-row chunk: 64 row blocks of up to 1024 (L = 32768) or 4096 tiles
    (L = 131072), each one work item, no split and no workspace."""
    qs, seq = L - CHUNK, L
    k, v, bt = make_cache(L, 750 + L // 1024, std=1.0)
    qd, kd, vd, btd = make_query(CHUNK, 950 + L // 1024, std=1.0).to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    del k, v
    plan = cabi.chunk_plan(CHUNK, qs, seq, None)
    print(f"L={L} dense chunk qs={qs} plan={plan} workspace={cabi.workspace_size(CHUNK, qs, seq, None)}", flush=True)
    assert plan[2] == CHUNK // 32
    out = torch.full_like(qd, float("nan"))
    cabi.dense_paged_causal_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, scale=SCALE)
    torch.cuda.synchronize()
    _check_all_rows(f"L={L} dense rows {qs}..{seq - 1}", out, qd, kd, vd, btd, qs, seq, seq, dense=True)


def _residue_histogram(intervals, m):
    """Count of keys k in the union of ``intervals`` with k % m == d, for d in 0..127."""
    d = np.arange(128)
    hist = np.zeros(128, dtype=np.int64)
    for b, e in intervals:
        # keys k in [b, e) with k = d (mod m): floor((e-1-d)/m) - floor((b-1-d)/m)
        hist += (e - 1 - d) // m - (b - 1 - d) // m
    hist[d >= m] = 0
    return hist


@pytest.mark.parametrize("L,where", [(32768, "last"), (131072, "last"), (32768, "middle")])
def test_long_context_mask_identity_whole_chunk(gpu, L, where):
    """Every row of a 2048-row chunk: the last one (KV whole, dense-tail rows split over KV) and a middle
    one (KV whole)."""
    qs = L - CHUNK if where == "last" else L // 2
    seq, prompt = qs + CHUNK, L
    print(f"mask identity L={L} {where} chunk qs={qs} plan={cabi.chunk_plan(CHUNK, qs, seq, prompt)}", flush=True)
    _, _, bt = make_cache(L, 800 + L // 1024)
    pages = int(bt.max()) + 1
    moduli = [128, 127, 125, 123, 121, 119, 113, 109]
    table = bt[0].tolist()
    tok = torch.arange(seq)
    v = torch.zeros(pages, 128, 8, 128, dtype=torch.bfloat16)
    for h, m in enumerate(moduli):
        onehot = torch.nn.functional.one_hot(tok % m, 128).to(torch.bfloat16).reshape(-1, 128, 128)
        full = seq // 128
        v[torch.tensor(table[:full]), :, h] = onehot[:full]
        if seq % 128:
            v[table[full], :seq % 128, h] = onehot.reshape(-1, 128)[full * 128:seq]
    k = torch.zeros_like(v)
    q = torch.zeros(CHUNK, 32, 128, dtype=torch.bfloat16)
    actual = _sparse(gpu, q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu), qs, seq, prompt).float().cpu().numpy()
    expected = np.zeros((CHUNK, 32, 128))
    for r in range(CHUNK):
        ivs = OG.selected_intervals(qs + r, seq, prompt)
        n = sum(e - b for b, e in ivs)
        for h, m in enumerate(moduli):
            expected[r, 4 * h:4 * h + 4] = _residue_histogram(ivs, m) / n
    # the histograms' own check: every row's counts add up to |S|
    assert all(_residue_histogram(OG.selected_intervals(qs + r, seq, prompt), 128).sum() ==
               sum(e - b for b, e in OG.selected_intervals(qs + r, seq, prompt)) for r in (0, CHUNK - 1))
    tol = np.maximum(np.abs(expected) * 2.0 ** -8, 1e-30)
    bad = np.abs(actual - expected) > tol
    assert not bad.any(), f"{bad.sum()} mismatching entries, first at {np.argwhere(bad)[0]}"
