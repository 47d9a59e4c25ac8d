"""The no-allocation entry point against the workspace entry point.

``tm_triangle_paged_sparse_attention_noalloc`` runs the same kernel with its
split-KV scratch (arrival counters + partials) in a static per-GPU array
instead of a caller workspace.  Two calls in a row -- the second one smaller
-- whose dense-tail rows split over KV, so the scratch is used by both and the
second finds it as the first left it; each must be bit-identical to the
workspace entry point on the same inputs.  A chunk needing more scratch than
the array holds is refused before any HIP call.
"""

from __future__ import annotations

import pytest
import torch

from trianglemix import cabi
from trianglemix.workload import SCALE, make_cache, make_query

pytestmark = pytest.mark.gpu


def test_noalloc_matches_workspace_entry_point(gpu):
    seq = 8192
    k, v, bt = make_cache(seq, 501, std=1.0)
    kd, vd, btd = k.to(gpu), v.to(gpu), bt.to(gpu)
    # second call smaller: 128 instead of 512 rows, fewer split items
    for qs, tq in [(7680, 512), (8064, 128)]:
        need = cabi.workspace_size(tq, qs, seq, seq)
        print(f"noalloc qs={qs} tq={tq} scratch bytes needed={need}", flush=True)
        assert need > cabi.WORKSPACE_COUNTER_BYTES  # split row blocks: counters and partials in use
        q = make_query(tq, qs, std=1.0).to(gpu)
        a = torch.full_like(q, float("nan"))
        b = torch.full_like(q, float("nan"))
        cabi.triangle_paged_sparse_attention_noalloc(q, kd, vd, btd, a, query_start=qs, seq_len=seq,
                                                     prompt_len=seq, scale=SCALE)
        cabi.triangle_paged_sparse_attention(q, kd, vd, btd, b, query_start=qs, seq_len=seq, prompt_len=seq,
                                             scale=SCALE)
        torch.cuda.synchronize()
        assert torch.isfinite(a.float()).all(), (qs, tq)
        assert torch.equal(a, b), (qs, tq)


def test_noalloc_refuses_oversized_chunk(gpu):
    # a dense 2048-row chunk ending at L = 131072 splits every row: far more scratch than 64 MiB
    qs, tq = 131072 - 2048, 2048
    assert cabi.workspace_size(tq, qs, 131072, 131072) > 64 << 20
    q = torch.empty((tq, 32, 128), dtype=torch.bfloat16, device=gpu)
    kv = torch.empty((1, 128, 8, 128), dtype=torch.bfloat16, device=gpu)
    bt = torch.zeros((1, 1024), dtype=torch.int32, device=gpu)
    out = torch.empty_like(q)
    with pytest.raises(cabi.TriangleMixError) as err:
        cabi.triangle_paged_sparse_attention_noalloc(q, kv, kv, bt, out, query_start=qs, seq_len=131072,
                                                     prompt_len=131072, scale=SCALE)
    assert err.value.status == cabi.TM_ERR_WORKSPACE
    assert "no-allocation" in str(err.value)
