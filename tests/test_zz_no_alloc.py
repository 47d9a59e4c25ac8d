"""The no-allocation entry point against the workspace entry point.

``tm_triangle_paged_sparse_attention_noalloc`` runs the same kernel with its
split-KV scratch (arrival counters + partials) in a static per-GPU array
instead of a caller workspace.  Two calls in a row -- the second one smaller
-- whose dense-tail rows split over KV, so the scratch is used by both and the
second finds it as the first left it; each must be bit-identical to the
workspace entry point on the same inputs.  The array holds the largest
workspace any chunk needs, so the largest BASELINE chunk runs too.
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


def test_noalloc_serves_the_largest_baseline_chunk(gpu):
    """The config-4 last chunk at L = 131072 needs the most split scratch of the BASELINE chunks (its four
    dense-tail row blocks in eight pieces each, 17 MB): within the 64 MiB array, bit-identical to the
    workspace entry point, twice in a row on the array the first call left."""
    seq, tq = 131072, 2048
    qs = seq - tq
    need = cabi.workspace_size(tq, qs, seq, seq)
    print(f"noalloc L={seq} last chunk scratch bytes needed={need}", flush=True)
    assert cabi.WORKSPACE_COUNTER_BYTES < need <= 64 << 20
    k, v, bt = make_cache(seq, 502, std=1.0)
    kd, vd, btd = k.to(gpu), v.to(gpu), bt.to(gpu)
    del k, v
    q = make_query(tq, 503, std=1.0).to(gpu)
    b = torch.full_like(q, float("nan"))
    cabi.triangle_paged_sparse_attention(q, kd, vd, btd, b, query_start=qs, seq_len=seq, prompt_len=seq, scale=SCALE)
    for repeat in range(2):
        a = torch.full_like(q, float("nan"))
        cabi.triangle_paged_sparse_attention_noalloc(q, kd, vd, btd, a, query_start=qs, seq_len=seq, prompt_len=seq,
                                                     scale=SCALE)
        torch.cuda.synchronize()
        assert torch.isfinite(a.float()).all(), repeat
        assert torch.equal(a, b), repeat
