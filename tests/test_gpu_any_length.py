"""Chunks of any length, with a workspace that does not grow with the work.

The reference accepts any query length (its fast path grid-strides the
tasks, operator/op_kernel/triangle_paged_fia_fast_path.h:234-236), takes a
fixed workspace (operator/op_host/triangle_paged_sparse_attention.cpp:264,
306) and routes whole-prompt PrefillNoCache steps direct
(package/src/vllm_ascend_trianglemix/planning.py:79-83).  Here a work item of
any length runs in one workgroup (its page table refills 64 tiles at a time
inside the loop), rows split across workgroups only for load balance, and no
workspace exceeds 64 MiB.  Checks, all through the C ABI:

* a whole 40960-token prompt (query_start 0, Tq = seq_len = prompt_len)
  through the TriangleMix op and the dense companion, EVERY row against the
  fp32 oracle (its blocked form, run on the GPU), and the exact mask identity
  over every row;
* chunks whose plans hold items of 129-512 tiles in both workgroup shapes,
  for both ops -- item ends on either side of the 64-tile table blocks --
  every row against the oracle;
* a split chunk on a workspace holding garbage (all 0xFF, random bytes, the
  words an interrupted launch would leave) is bit-identical to one on a fresh
  workspace, and so is a repeat on the same workspace;
* one workspace carried through a sequence of split chunks of different
  shapes (the library keeps one arrival tag per workspace, and each chunk's
  arrival words sit at positions another chunk's used) gives every chunk the
  bits of a fresh workspace, and so do 80 workspaces used in turn (more than
  the library's table of tags holds);
* split chunks in flight on two streams at once through the torch ops (one
  adapter workspace per stream) equal the same calls run alone.

Tolerances as everywhere: max-abs 2e-2, mean-abs 2e-3, rel-L2 2e-2.
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

MAX_ABS, MEAN_ABS, REL_L2 = 2e-2, 2e-3, 2e-2


def _run(gpu, qd, kd, vd, btd, qs, seq, prompt, workspace=None):
    out = torch.full_like(qd, float("nan"))
    if prompt is None:
        cabi.dense_paged_causal_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, scale=SCALE,
                                          workspace=workspace)
    else:
        cabi.triangle_paged_sparse_attention(qd, kd, vd, btd, out, query_start=qs, seq_len=seq, prompt_len=prompt,
                                             scale=SCALE, workspace=workspace)
    torch.cuda.synchronize()
    return out


def _check_all_rows(label, got, qd, kd, vd, btd, qs, seq, prompt):
    assert torch.isfinite(got.float()).all(), label
    expected = OA.attention_torch_blocked(qd, kd, vd, btd, qs, seq, seq if prompt is None else prompt, SCALE,
                                          dense=prompt is None, max_scores=1 << 27)
    d = (got.float() - expected).abs()
    m = {"max_abs": d.max().item(), "mean_abs": d.mean().item(),
         "relative_l2": (d.norm() / expected.norm().clamp_min(1e-12)).item()}
    # the worst 32-row window as well as the whole chunk: a wrong row block cannot hide in the mean
    per_block = d.reshape(-1)[: (d.shape[0] // 32) * 32 * 32 * 128].reshape(-1, 32 * 32 * 128).mean(1)
    m["worst_block_mean_abs"] = per_block.max().item() if per_block.numel() else m["mean_abs"]
    print(f"{label}: {m}", flush=True)
    assert m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS and m["relative_l2"] <= REL_L2, (label, m)
    assert m["worst_block_mean_abs"] <= MEAN_ABS, (label, m)


L_WHOLE = 40960


@pytest.mark.parametrize("dense", [False, True], ids=["triangle", "dense"])
def test_whole_prompt_every_row_matches_oracle(gpu, dense):
    """PrefillNoCache: the whole 40960-token prompt in one call (refused before items could hold more than
    128 tiles: its dense-tail rows hold 1280)."""
    L = L_WHOLE
    prompt = None if dense else L
    parts, tiles, items = cabi.chunk_plan(L, 0, L, prompt)
    need = cabi.workspace_size(L, 0, L, prompt)
    print(f"whole prompt L={L} dense={dense}: plan parts={parts} tiles/item={tiles} items/head={items} "
          f"workspace={need}", flush=True)
    assert tiles > 128 and need <= cabi.MAX_WORKSPACE_BYTES
    k, v, bt = make_cache(L, 4096 + dense, std=1.0)
    q = make_query(L, 4097 + dense, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    del q, k, v
    got = _run(gpu, qd, kd, vd, btd, 0, L, prompt)
    _check_all_rows(f"whole prompt L={L} dense={dense}", got, qd, kd, vd, btd, 0, L, prompt)


def _residue_histograms(qs, tq, seq, prompt, moduli):
    """[tq, 8, 128]: per row and modulus m, the count of attended keys k with k % m == d, over |S|."""
    d = np.arange(128)
    out = np.zeros((tq, len(moduli), 128))
    for r in range(tq):
        ivs = OG.selected_intervals(qs + r, seq, prompt)
        n = sum(e - b for b, e in ivs)
        for h, m in enumerate(moduli):
            hist = np.zeros(128)
            for b, e in ivs:
                hist += (e - 1 - d) // m - (b - 1 - d) // m
            hist[d >= m] = 0
            out[r, h] = hist / n
    return out


def test_whole_prompt_mask_identity(gpu):
    """Q = 0 weighs every attended key 1/|S|; one-hot residue V rows (8 moduli, one per KV head) turn each
    output row into the residue histogram of its key set, so an added, dropped or shifted key in any of the
    40960 rows changes the output beyond bf16 rounding."""
    L = prompt = seq = L_WHOLE
    _, _, bt = make_cache(L, 4100)
    pages = int(bt.max()) + 1
    moduli = [128, 127, 125, 123, 121, 119, 113, 109]
    tok = torch.arange(seq)
    logical = torch.zeros(seq, 8, 128, dtype=torch.bfloat16)
    for h, m in enumerate(moduli):
        logical[:, h] = torch.nn.functional.one_hot(tok % m, 128).to(torch.bfloat16)
    v = torch.zeros(pages, 128, 8, 128, dtype=torch.bfloat16)
    v[bt[0, :seq // 128].long()] = logical.reshape(-1, 128, 8, 128)
    qd = torch.zeros(L, 32, 128, dtype=torch.bfloat16, device=gpu)
    vd = v.to(gpu)
    actual = _run(gpu, qd, torch.zeros_like(vd), vd, bt.to(gpu), 0, seq, prompt).float().cpu().numpy()
    expected = np.repeat(_residue_histograms(0, L, seq, prompt, moduli), 4, axis=1)  # 4 query heads per KV head
    tol = np.maximum(np.abs(expected) * 2.0 ** -8, 1e-30)
    bad = np.abs(actual - expected) > tol
    assert not bad.any(), f"{bad.sum()} mismatching entries, first at {np.argwhere(bad)[0]}"


# (query_tokens, seq_len, dense) -> chunks at the end of a prompt of seq_len tokens whose plans hold items
# of more than 128 tiles; the comment gives (KV parts, tiles per item, items per KV head).
LONG_ITEMS = [
    (200, 32768, False),   # (2, 171, 32): the dense tail in pieces of 170-171 tiles
    (512, 40000, False),   # (2, 157, 44): BASELINE-sized chunk, pieces of 156-157 tiles
    (1024, 65536, False),  # (2, 256, 60): pieces of exactly four table blocks
    (512, 4200, True),     # (4, 132, 16): pieces of 129-132 tiles -- a few tiles into table block 2
    (200, 9000, True),     # (4, 141, 14)
    (96, 24576, True),     # (4, 154, 15)
    (96, 32768, True),     # (4, 205, 15)
    (200, 24576, True),    # (2, 192, 28): pieces of exactly three table blocks
    (512, 12345, True),    # (2, 193, 32): one tile past three table blocks
    (512, 20000, True),    # (2, 313, 32)
    (512, 24576, True),    # (2, 384, 32): six table blocks
    (256, 32768, True),    # (2, 256, 32)
    (640, 16384, True),    # (1, 171, 60): KV whole, rows of 493-512 tiles in three pieces
    (2048, 12345, True),   # (1, 386, 64): KV whole, rows of 323-386 tiles unsplit
]


@pytest.mark.parametrize("tq,seq,dense", LONG_ITEMS, ids=[f"{'dense' if d else 'tri'}-{t}of{s}" for t, s, d in LONG_ITEMS])
def test_items_longer_than_128_tiles_match_oracle(gpu, tq, seq, dense):
    qs = seq - tq
    prompt = None if dense else seq
    parts, tiles, items = cabi.chunk_plan(tq, qs, seq, prompt)
    print(f"long items: qs={qs} tq={tq} seq={seq} dense={dense} plan=({parts}, {tiles}, {items})", flush=True)
    assert tiles > 128
    k, v, bt = make_cache(seq, 310 + tq, std=1.0)
    q = make_query(tq, 311 + seq, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    got = _run(gpu, qd, kd, vd, btd, qs, seq, prompt)
    _check_all_rows(f"long items {tq}of{seq} dense={dense}", got, qd, kd, vd, btd, qs, seq, prompt)


@pytest.mark.parametrize("dense", [False, True], ids=["triangle", "dense"])
def test_workspace_contents_do_not_matter(gpu, dense):
    """A split chunk (the config-2 last chunk; for the dense companion its 512-row chunk) gives the same bits
    on a fresh zeroed workspace, on one of all-0xFF bytes, on random bytes, on one whose arrival words look
    like an interrupted launch's (another epoch, counts below the split count) and on the same workspace
    again -- the arrival words carry their launch's tag, so none is mistaken for an arrival of this one."""
    qs, tq, seq = 7680, 512, 8192
    prompt = None if dense else seq
    need = cabi.workspace_size(tq, qs, seq, prompt)
    print(f"workspace contents: dense={dense} need={need}", flush=True)
    assert need > cabi.WORKSPACE_COUNTER_BYTES
    k, v, bt = make_cache(seq, 61 + dense, std=1.0)
    q = make_query(tq, 62 + dense, std=1.0)
    qd, kd, vd, btd = q.to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    gen = torch.Generator(device="cpu").manual_seed(5)
    stale = torch.zeros(cabi.WORKSPACE_COUNTER_BYTES // 8, dtype=torch.int64)
    stale[:] = (torch.randint(1, 1 << 40, (stale.numel(),), generator=gen) << 16) + torch.randint(
        0, 3, (stale.numel(),), generator=gen)
    workspaces = {
        "zeros": torch.zeros(need, dtype=torch.uint8, device=gpu),
        "0xff": torch.full((need,), 0xFF, dtype=torch.uint8, device=gpu),
        "random": torch.randint(0, 256, (need,), generator=gen, dtype=torch.uint8).to(gpu),
        "interrupted": torch.cat([stale.view(torch.uint8),
                                  torch.zeros(need - cabi.WORKSPACE_COUNTER_BYTES, dtype=torch.uint8)]).to(gpu),
    }
    reference = _run(gpu, qd, kd, vd, btd, qs, seq, prompt, workspaces["zeros"])
    assert torch.isfinite(reference.float()).all()
    for name, ws in workspaces.items():
        for repeat in range(2):  # the second call finds the words the first left
            got = _run(gpu, qd, kd, vd, btd, qs, seq, prompt, ws)
            assert torch.equal(got, reference), (name, repeat)


# (query_start, query_tokens, seq_len, prompt_len or None for the dense companion): split chunks of both
# workgroup shapes, two to eight splits per row, dense-tail and dense rows
SHARED_WORKSPACE_CHUNKS = [
    (7680, 512, 8192, 8192),     # KV quarters, three splits per dense-tail row
    (7680, 512, 8192, None),     # dense companion, every row split
    (8192, 128, 8320, 8320),     # KV quarters, four splits per row
    (6144, 2048, 8192, 8192),    # KV halves, split dense-tail rows among unsplit sparse ones
    (16256, 128, 16384, 16384),  # long dense-tail rows
    (7680, 512, 8192, 8192),     # the first chunk again, on words the others left
]


def test_one_workspace_across_split_chunks_of_different_shapes(gpu):
    """One workspace through a sequence of split chunks whose arrival words overlap one another's (the
    layout depends on the split row blocks and the workgroup shape): every chunk equals its run on a fresh
    workspace, bit for bit.  The library keeps one arrival tag per workspace and each completed launch
    leaves its words at (tag, 0), so a later chunk meets clean words of its own tag, words another shape
    left and never-touched words at once."""
    need = max(cabi.workspace_size(tq, qs, seq, prompt) for qs, tq, seq, prompt in SHARED_WORKSPACE_CHUNKS)
    assert 0 < need <= cabi.MAX_WORKSPACE_BYTES
    shared = torch.full((need,), 0xFF, dtype=torch.uint8, device=gpu)
    caches = {}
    for i, (qs, tq, seq, prompt) in enumerate(SHARED_WORKSPACE_CHUNKS):
        print(f"shared workspace: chunk {i} qs={qs} tq={tq} seq={seq} prompt={prompt}", flush=True)
        assert cabi.workspace_size(tq, qs, seq, prompt) > cabi.WORKSPACE_COUNTER_BYTES, "the chunk must split"
        if seq not in caches:
            k, v, bt = make_cache(seq, 80 + seq % 97, std=1.0)
            caches[seq] = (k.to(gpu), v.to(gpu), bt.to(gpu))
        kd, vd, btd = caches[seq]
        qd = make_query(tq, 90 + i % 5, std=1.0).to(gpu)
        fresh = torch.zeros(cabi.workspace_size(tq, qs, seq, prompt), dtype=torch.uint8, device=gpu)
        expected = _run(gpu, qd, kd, vd, btd, qs, seq, prompt, fresh)
        assert torch.isfinite(expected.float()).all(), i
        for repeat in range(2):
            got = _run(gpu, qd, kd, vd, btd, qs, seq, prompt, shared)
            assert torch.equal(got, expected), (i, repeat)


def test_more_workspaces_than_the_tag_table_holds(gpu):
    """The library keeps one arrival tag per workspace address in a table of 64 slots; 80 workspaces used
    in turn, twice over, evict one another's entries (an evicted address gets a fresh tag, so its words
    from the first pass are foreign in the second).  Every call equals the run on a fresh workspace."""
    qs, tq, seq = 7680, 512, 8192
    need = cabi.workspace_size(tq, qs, seq, seq)
    assert need > cabi.WORKSPACE_COUNTER_BYTES
    k, v, bt = make_cache(seq, 95, std=1.0)
    qd, kd, vd, btd = make_query(tq, 96, std=1.0).to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    expected = _run(gpu, qd, kd, vd, btd, qs, seq, seq, torch.zeros(need, dtype=torch.uint8, device=gpu))
    workspaces = [torch.empty(need, dtype=torch.uint8, device=gpu) for _ in range(80)]
    for sweep in range(2):
        print(f"tag table: pass {sweep} over {len(workspaces)} workspaces", flush=True)
        for i, ws in enumerate(workspaces):
            got = _run(gpu, qd, kd, vd, btd, qs, seq, seq, ws)
            assert torch.equal(got, expected), (sweep, i)


def test_captured_split_chunk_replays_bit_identical(gpu):
    """The torch adapter's capture path: a split chunk (the config-2 last chunk) captured into a HIP graph
    through torch.ops takes its workspace from the capture's own memory.  Each replay, with eager calls of
    the same op (on the stream's own workspace) between the replays, is bit-identical to the eager result:
    the replays share one launch tag and find the arrival words cleared by the replay before."""
    qs, tq, seq = 7680, 512, 8192
    assert cabi.workspace_size(tq, qs, seq, seq) > cabi.WORKSPACE_COUNTER_BYTES
    k, v, bt = make_cache(seq, 71, std=1.0)
    qd, kd, vd, btd = make_query(tq, 72, std=1.0).to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    op = torch.ops.trianglemix.triangle_paged_sparse_attention.out
    eager = torch.empty_like(qd)
    op(qd, kd, vd, btd, qs, seq, seq, SCALE, out=eager)
    other_q = make_query(tq, 73, std=1.0).to(gpu)
    other_eager = torch.empty_like(qd)
    op(other_q, kd, vd, btd, qs, seq, seq, SCALE, out=other_eager)
    torch.cuda.synchronize()
    print("graph capture of the config-2 last chunk", flush=True)
    graph_out = torch.empty_like(qd)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            op(qd, kd, vd, btd, qs, seq, seq, SCALE, out=graph_out)
    torch.cuda.current_stream().wait_stream(side)
    for replay in range(3):
        graph_out.fill_(float("nan"))
        graph.replay()
        between = torch.full_like(qd, float("nan"))
        op(other_q, kd, vd, btd, qs, seq, seq, SCALE, out=between)  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(graph_out, eager), replay
        assert torch.equal(between, other_eager), replay


def test_split_chunks_on_two_streams_at_once(gpu):
    """Two streams running split chunks through the torch ops at the same time: the adapter keeps one
    workspace per (device, stream), so calls in flight on different streams never share arrival words or
    partials.  Four rounds, each enqueuing the TriangleMix op's last config-2 chunk on one stream and the
    dense companion's on the other with no synchronisation between them; every output is bit-identical to
    the same call run alone."""
    qs, tq, seq = 7680, 512, 8192
    assert cabi.workspace_size(tq, qs, seq, seq) > cabi.WORKSPACE_COUNTER_BYTES
    assert cabi.workspace_size(tq, qs, seq, None) > cabi.WORKSPACE_COUNTER_BYTES
    k, v, bt = make_cache(seq, 61, std=1.0)
    kd, vd, btd = k.to(gpu), v.to(gpu), bt.to(gpu)
    queries = [make_query(tq, 62 + i, std=1.0).to(gpu) for i in range(4)]
    sparse_op = torch.ops.trianglemix.triangle_paged_sparse_attention.out
    dense_op = torch.ops.trianglemix.dense_paged_causal_attention.out
    alone_sparse, alone_dense = [], []
    for qd in queries:
        alone_sparse.append(torch.empty_like(qd))
        sparse_op(qd, kd, vd, btd, qs, seq, seq, SCALE, out=alone_sparse[-1])
        alone_dense.append(torch.empty_like(qd))
        dense_op(qd, kd, vd, btd, qs, seq, SCALE, out=alone_dense[-1])
    torch.cuda.synchronize()
    got_sparse = [torch.full_like(qd, float("nan")) for qd in queries]
    got_dense = [torch.full_like(qd, float("nan")) for qd in queries]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    print("two streams: 4 rounds of a split sparse and a split dense chunk", flush=True)
    for i, qd in enumerate(queries):
        first, second = (streams[0], streams[1]) if i % 2 == 0 else (streams[1], streams[0])
        with torch.cuda.stream(first):
            sparse_op(qd, kd, vd, btd, qs, seq, seq, SCALE, out=got_sparse[i])
        with torch.cuda.stream(second):
            dense_op(qd, kd, vd, btd, qs, seq, SCALE, out=got_dense[i])
    torch.cuda.synchronize()
    for i in range(len(queries)):
        assert torch.equal(got_sparse[i], alone_sparse[i]), ("sparse", i)
        assert torch.equal(got_dense[i], alone_dense[i]), ("dense", i)


def test_router_routes_a_whole_long_prompt_direct(gpu):
    """Through the routing layer with the real ops: a whole-prompt PrefillNoCache step of 40960 tokens on a
    selected layer is launched direct (no fallback counted) and is bit-identical to the op called directly;
    the same step on an unselected layer runs the dense companion, bit-identical to it."""
    from trianglemix.config import resolve_plugin_config
    from trianglemix.planning import build_batch_plan
    from trianglemix.router import TriangleMixRouter
    from trianglemix.stats import TriangleMixRuntimeStats

    class _Vllm:
        additional_config = {"trianglemix": {"enabled": True, "layers": "1"}}

    L = L_WHOLE
    cfg = resolve_plugin_config(_Vllm())
    plan = build_batch_plan(state_name="PrefillNoCache", cumulative_query_ends=[L], seq_lens=[L], prompt_lens=[L],
                            num_decodes=0, num_prefills=1, config=cfg.kernel)
    assert plan.direct
    stats = TriangleMixRuntimeStats()
    router = TriangleMixRouter(cfg, stats=stats)
    k, v, bt = make_cache(L, 4200, std=1.0)
    qd, kd, vd, btd = make_query(L, 4201, std=1.0).to(gpu), k.to(gpu), v.to(gpu), bt.to(gpu)
    print(f"router whole prompt L={L}", flush=True)
    for layer, sparse in ((1, True), (0, False)):
        got = torch.full_like(qd, float("nan"))
        router.prefill_attention(layer_name=f"model.layers.{layer}.self_attn.attn", plan=plan, query=qd,
                                 key_cache=kd, value_cache=vd, block_table=btd, output=got, softmax_scale=SCALE)
        want = _run(gpu, qd, kd, vd, btd, 0, L, L if sparse else None)
        assert torch.equal(got, want), layer
    counters = stats.snapshot()["counters"]
    assert counters["layer_direct"] == 1 and counters.get("layer_fia", 0) == 0
    assert counters.get("runtime_error_stage:direct_launch", 0) == 0
