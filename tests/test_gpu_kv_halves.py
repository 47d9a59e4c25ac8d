"""The KV-halves workgroup shape on the GPU.

Chunks of more than 16 row blocks (513 query tokens and up), and chunks of
at least 4 row blocks whose long dense rows split over KV, run a different
workgroup shape from the others: the four query heads of a GQA group per
workgroup and the item's K/V tiles cut into two halves (instead of two heads
and four quarters).  These cases pin that shape against the fp32 oracle: the
first chunk of a prompt (dense prefix, sparse start), the shape boundary at
512 / 513 query tokens, ragged and mid-page chunks, long chunks whose dense
tail splits over KV, short split chunks on either side of the 4-row-block
bound, a chunk whose prompt extends past the sequence (no dense tail yet),
32-row blocks that hold a single live row, and the dense companion.
Tolerances are the project's (max-abs 2e-2, mean-abs 2e-3, relative L2 2e-2
vs fp32).
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as OA
from trianglemix import cabi
from trianglemix.workload import SCALE, make_inputs

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS, REL_L2 = 2e-2, 2e-3, 2e-2
HALVES_MIN_ROW_BLOCKS = 17  # chunks of at least this many 32-row blocks take the KV-halves shape

# (name, query_start, query_tokens, seq_len, prompt_len, seed)
CASES = [
    ("first_chunk_1024", 0, 1024, 1024, 8192, 71),
    ("quarters_side_512", 1000, 512, 1512, 4000, 72),
    ("halves_side_513_one_live_row", 1000, 513, 1513, 4000, 73),
    ("halves_993_one_live_row", 1000, 993, 1993, 4000, 80),
    ("split_tail_3_row_blocks_quarters", 12200, 96, 12296, 12296, 82),
    ("split_tail_4_row_blocks_halves", 12200, 128, 12328, 12328, 83),
    ("split_tail_8_row_blocks_halves", 8000, 256, 8256, 8256, 84),
    ("ragged_1057_mid_page", 1333, 1057, 2390, 2390, 74),
    ("chunk_2048_no_tail_yet", 2048, 2048, 4096, 8192, 75),
    ("last_chunk_1024_split_tail", 7168, 1024, 8192, 8192, 76),
    ("last_chunk_2048_16k_split_tail", 14336, 2048, 16384, 16384, 77),
    ("whole_prompt_1500", 0, 1500, 1500, 1500, 78),
    ("prompt_past_sequence_1111", 3000, 1111, 4111, 9000, 79),
    # split-candidate chunks that stay KV quarters (one round of workgroups, shorter items)
    ("quarters_kept_last_chunk_2048_prompt", 1536, 512, 2048, 2048, 85),
    ("quarters_kept_tail_309_rows", 2560, 309, 2869, 2869, 86),
]


def _row_blocks(tq: int) -> int:
    return (tq + 31) // 32


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_kv_halves_matches_oracle(gpu, case):
    name, qs, tq, seq, prompt, seed = case
    print(f"case {name} qs={qs} tq={tq} seq={seq} prompt={prompt} row_blocks={_row_blocks(tq)}", flush=True)
    q, k, v, bt = make_inputs(qs, tq, seq, seed, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    out = torch.full_like(qd, float("nan"))
    cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                         scale=SCALE)
    torch.cuda.synchronize()
    expected = OA.attention_torch(q, k, v, bt, qs, seq, prompt, SCALE)
    m = OA.error_metrics(out.float().cpu().numpy(), expected.float().numpy())
    print(f"{name}: {m}", flush=True)
    assert m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, m


@pytest.mark.parametrize("qs,tq,seq", [(0, 1024, 1024), (1900, 1100, 3000), (5000, 2048, 7048), (0, 600, 600)])
def test_kv_halves_dense_companion(gpu, qs, tq, seq):
    assert _row_blocks(tq) >= HALVES_MIN_ROW_BLOCKS
    print(f"dense qs={qs} tq={tq} seq={seq}", flush=True)
    q, k, v, bt = make_inputs(qs, tq, seq, 900 + tq, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    out = torch.full_like(qd, float("nan"))
    cabi.dense_paged_causal_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, scale=SCALE)
    torch.cuda.synchronize()
    expected = OA.attention_torch(q, k, v, bt, qs, seq, seq, SCALE, dense=True)
    m = OA.error_metrics(out.float().cpu().numpy(), expected.float().numpy())
    print(f"dense {qs}+{tq}: {m}", flush=True)
    assert m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, m


def test_kv_halves_deterministic_across_calls(gpu):
    """Two launches of one split chunk give identical bytes (fixed merge order)."""
    qs, tq, seq, prompt = 7168, 1024, 8192, 8192
    q, k, v, bt = make_inputs(qs, tq, seq, 81, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    a = torch.full_like(qd, float("nan"))
    b = torch.full_like(qd, float("nan"))
    for out in (a, b):
        cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                             scale=SCALE)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


# Dense-companion chunks of at most 16 row blocks whose rows all split: KV
# halves once the chunk holds at least 2048 tiles per KV head, KV quarters
# below that.
DENSE_SPLIT_CASES = [
    (7680, 512, 8192),    # 16 row blocks, ~3970 tiles: halves
    (12000, 256, 12256),  # 8 row blocks, ~3040 tiles: halves
    (12200, 128, 12328),  # 4 row blocks, ~1540 tiles: quarters
    (5000, 512, 5512),    # 16 row blocks, ~2650 tiles: halves
]


@pytest.mark.parametrize("qs,tq,seq", DENSE_SPLIT_CASES)
def test_dense_split_chunks_either_shape(gpu, qs, tq, seq):
    print(f"dense split qs={qs} tq={tq} seq={seq} row_blocks={_row_blocks(tq)}", flush=True)
    q, k, v, bt = make_inputs(qs, tq, seq, 700 + tq, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    out = torch.full_like(qd, float("nan"))
    cabi.dense_paged_causal_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, scale=SCALE)
    torch.cuda.synchronize()
    expected = OA.attention_torch(q, k, v, bt, qs, seq, seq, SCALE, dense=True)
    m = OA.error_metrics(out.float().cpu().numpy(), expected.float().numpy())
    print(f"dense split {qs}+{tq}: {m}", flush=True)
    assert m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, m
