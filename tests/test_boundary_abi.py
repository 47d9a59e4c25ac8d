"""The drop-in boundary on the CPU: the C-ABI library and the torch adapter.

No kernel runs here.  Checks:

* ``libtrianglemix.so`` loads and exports every function ``include/trianglemix.h``
  declares, with the declared ABI version and status strings;
* every validation error of the launch entry points is returned before any
  HIP call (fake, never-dereferenced pointers; the attributes are invalid, so
  no launch is attempted);
* the workspace-size entry points: zero when no row block is split, the
  arrival words plus whole partial records of the split row blocks' items
  otherwise, never more than TM_MAX_WORKSPACE_BYTES, and -1 for exactly the
  attributes the launch refuses;
* the torch adapter registers the reference's exact schema strings
  (operator/torch_adapter/triangle_paged_attention_torch.cpp:264-296) plus the
  ``npu_triangle_paged_sparse_attention`` alias, shape-infers on the Meta
  device, and has no CPU kernel (a CPU call fails loudly instead of falling
  back).
"""

from __future__ import annotations

import ctypes
import json
import re
import sys
from pathlib import Path

import pytest
import torch

from trianglemix import cabi, native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "trianglemix.h"
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
PARTIAL_BYTES = 4 * 64 * 66 * 4  # fp32 partial record of one (row block, kv head, split) item
COUNTER_BYTES = 65536            # arrival words at the front of a non-empty workspace (TM_WORKSPACE_COUNTER_BYTES)
MAX_WORKSPACE = 64 << 20         # TM_MAX_WORKSPACE_BYTES


def _items(need: int) -> int:
    """Split items per KV head a workspace size accounts for (0: no split, no workspace)."""
    if need == 0:
        return 0
    assert need > COUNTER_BYTES and (need - COUNTER_BYTES) % (8 * PARTIAL_BYTES) == 0, need
    return (need - COUNTER_BYTES) // (8 * PARTIAL_BYTES)


@pytest.fixture(scope="module")
def lib():
    if not native.HIP_LIBRARY.is_file() or not native.TORCH_ADAPTER.is_file():
        import importlib.util

        spec = importlib.util.spec_from_file_location("tm_build", native.PKG_DIR.parent / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build_all()
    return native.load_hip_library()


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tm_[a-z_]+)\s*\(", text)))


def test_header_functions_are_exported(lib):
    names = _declared_functions()
    assert names == sorted([
        "tm_abi_version", "tm_status_string", "tm_last_error",
        "tm_triangle_paged_sparse_attention", "tm_triangle_paged_sparse_attention_workspace_size",
        "tm_triangle_paged_sparse_attention_noalloc",
        "tm_dense_paged_causal_attention", "tm_dense_paged_causal_attention_workspace_size",
        "tm_chunk_plan", "tm_reshape_and_cache"])
    raw = ctypes.CDLL(str(native.HIP_LIBRARY))
    for name in names:
        assert getattr(raw, name) is not None, name


def test_product_library_has_no_phase_clocks():
    """The phase-clock instrumentation is compiled only into the diagnostic build (build.py --phase-clocks,
    its own file name)."""
    raw = ctypes.CDLL(str(native.HIP_LIBRARY))
    assert not hasattr(raw, "tm_phase_clocks_read") and not hasattr(raw, "tm_phase_clocks_clear")
    import importlib.util
    spec = importlib.util.spec_from_file_location("tm_build", native.PKG_DIR.parent / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert mod.PHASE_CLOCK_LIB.name == "libtrianglemix_phase_clocks.so" and mod.PHASE_CLOCK_LIB != native.HIP_LIBRARY


def test_product_library_has_no_plan_override():
    """Forcing the launch plan is compiled only into the sweep's diagnostic build (build.py --plan-override,
    its own file name)."""
    raw = ctypes.CDLL(str(native.HIP_LIBRARY))
    assert not hasattr(raw, "tm_plan_override")
    import importlib.util
    spec = importlib.util.spec_from_file_location("tm_build", native.PKG_DIR.parent / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert mod.PLAN_OVERRIDE_LIB.name == "libtrianglemix_plan_override.so" and mod.PLAN_OVERRIDE_LIB != native.HIP_LIBRARY


def test_abi_version_and_status_strings(lib):
    m = re.search(r"#define\s+TM_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert lib.tm_abi_version() == int(m.group(1)) == native.ABI_VERSION
    for name, value in (("TM_WORKSPACE_COUNTER_BYTES", COUNTER_BYTES), ("TM_MAX_WORKSPACE_BYTES", MAX_WORKSPACE)):
        assert int(re.search(rf"#define\s+{name}\s+(\d+)", HEADER.read_text()).group(1)) == value
    assert (cabi.WORKSPACE_COUNTER_BYTES, cabi.MAX_WORKSPACE_BYTES) == (COUNTER_BYTES, MAX_WORKSPACE)
    for code, name in [(0, "TM_OK"), (1, "TM_ERR_INVALID_ARGUMENT"), (2, "TM_ERR_UNSUPPORTED"),
                       (3, "TM_ERR_WORKSPACE"), (4, "TM_ERR_LAUNCH"), (99, "TM_ERR_UNKNOWN")]:
        assert lib.tm_status_string(code).decode() == name
        if code < 5:
            assert re.search(rf"#define\s+{name}\s+{code}\b", HEADER.read_text())


# fake device addresses, far apart; never dereferenced because every call below fails validation
Q, K, V, BT, OUT, WS = (0x10_0000_0000 * (i + 1) for i in range(6))
GOOD = dict(query=Q, key=K, value=V, table=BT, out=OUT, tq=512, pages=71, cols=64, qs=4096, seq=4608, prompt=8192,
            scale=0.08838834764831845, ws=0, ws_bytes=0)


def _sparse(lib, **over):
    a = dict(GOOD, **over)
    return lib.tm_triangle_paged_sparse_attention(a["query"], a["key"], a["value"], a["table"], a["out"], a["tq"],
                                                  a["pages"], a["cols"], a["qs"], a["seq"], a["prompt"], a["scale"],
                                                  a["ws"], a["ws_bytes"], None)


@pytest.mark.parametrize("over,status,msg", [
    (dict(query=None), 1, "non-null"),
    (dict(out=None), 1, "non-null"),
    (dict(tq=0, qs=4608), 1, "Tq > 0"),
    (dict(qs=4000), 1, "query_start \\+ Tq == seq_len"),
    (dict(prompt=4000), 1, "prompt_len"),
    (dict(scale=0.0), 1, "scale"),
    (dict(scale=float("nan")), 1, "scale"),
    (dict(scale=float("inf")), 1, "scale"),
    (dict(pages=0), 1, "pages > 0"),
    (dict(pages=(1 << 22) + 1), 2, "limit is 4194304"),
    (dict(cols=35), 1, "block_table lacks"),
    (dict(out=Q + 1024), 1, "must not overlap"),
    (dict(out=K + 4096), 1, "must not overlap"),
    (dict(out=BT), 1, "must not overlap"),
    (dict(ws=0, ws_bytes=4096), 3, "inconsistent"),
    (dict(ws_bytes=-1, ws=WS), 3, "inconsistent"),
    (dict(tq=512, qs=(1 << 30), seq=(1 << 30) + 512, prompt=(1 << 30) + 512, cols=(1 << 23) + 4), 2, "exceed"),
])
def test_sparse_entry_validation_errors(lib, over, status, msg):
    assert _sparse(lib, **over) == status
    assert re.search(msg, lib.tm_last_error().decode()), lib.tm_last_error()


def test_small_workspace_is_rejected_before_launch(lib):
    need = lib.tm_triangle_paged_sparse_attention_workspace_size(512, 7680, 8192, 8192)
    assert need > 0
    assert _sparse(lib, qs=7680, seq=8192, ws=WS, ws_bytes=need - 1) == 3
    assert "smaller than" in lib.tm_last_error().decode()
    assert _sparse(lib, qs=7680, seq=8192, ws=OUT - 16, ws_bytes=need) == 3  # workspace overlapping out
    assert "overlap" in lib.tm_last_error().decode()
    assert _sparse(lib, qs=7680, seq=8192, ws=WS + 8, ws_bytes=need) == 3  # 64-bit arrival words need alignment
    assert "16-byte aligned" in lib.tm_last_error().decode()


def test_dense_entry_validation_errors(lib):
    r = lib.tm_dense_paged_causal_attention(Q, K, V, BT, OUT, 512, 71, 64, 4000, 4608, 0.088, 0, 0, None)
    assert r == 1 and "query_start + Tq" in lib.tm_last_error().decode()
    r = lib.tm_dense_paged_causal_attention(Q, K, V, BT, None, 512, 71, 64, 4096, 4608, 0.088, 0, 0, None)
    assert r == 1


KW_GOOD = dict(key=0x10000, value=0x20000, kc=0x1000000, vc=0x2000000, slots=0x3000, tokens=512, ks=1024, vs=1024,
               pages=71)


def _kv_write(lib, **over):
    a = dict(KW_GOOD, **over)
    return lib.tm_reshape_and_cache(a["key"], a["value"], a["kc"], a["vc"], a["slots"], a["tokens"], a["ks"],
                                    a["vs"], a["pages"], None)


@pytest.mark.parametrize("over,status,msg", [
    (dict(tokens=-1), 1, "num_tokens"),
    (dict(pages=0), 1, "pages > 0"),
    (dict(pages=(1 << 22) + 1), 2, "limit is 4194304"),
    (dict(key=None), 1, "non-null"),
    (dict(slots=None), 1, "non-null"),
    (dict(ks=1000), 1, "row stride"),
    (dict(vs=1028), 1, "row stride"),
    (dict(value=0x20004), 1, "16-byte aligned"),
    (dict(vc=0x1000000 + 71 * 256 * 1024 - 16), 1, "must not overlap"),   # caches overlap
    (dict(key=0x1000000 + 4096), 1, "must not overlap"),                  # source inside the key cache
    (dict(slots=0x2000000 + 64), 1, "must not overlap"),                  # slot mapping inside the value cache
])
def test_kv_write_validation_errors(lib, over, status, msg):
    assert _kv_write(lib, **over) == status
    assert re.search(msg, lib.tm_last_error().decode()), lib.tm_last_error()


def test_kv_write_without_tokens_enqueues_nothing(lib):
    # no pointer is dereferenced and no HIP call is made for an empty chunk
    assert _kv_write(lib, tokens=0, key=None, value=None, slots=None) == 0


def test_noalloc_refuses_what_the_workspace_entry_point_refuses(lib):
    # fake (never dereferenced) pointers: the refusal happens before any HIP call
    fake = ctypes.c_void_p(0x1000)
    r = lib.tm_triangle_paged_sparse_attention_noalloc(fake, fake, fake, fake, fake, 512, 64, 64, 4096, 4000, 8192,
                                                       0.088, None)
    assert r == 1 and "Tq == seq_len" in lib.tm_last_error().decode()
    # its 64 MiB array holds the largest workspace any chunk needs (the config-4 last chunk at L = 131072 needed
    # ~100 MB when rows had to split every 4096 keys; it needs 17 MB now), so it accepts every valid chunk
    assert 0 < lib.tm_triangle_paged_sparse_attention_workspace_size(2048, 129024, 131072, 131072) <= MAX_WORKSPACE


def test_workspace_sizes(lib):
    ws = lib.tm_triangle_paged_sparse_attention_workspace_size
    dws = lib.tm_dense_paged_causal_attention_workspace_size
    # sparse middle chunks: every row block holds few tiles -> no split, no workspace
    assert ws(512, 4096, 4608, 8192) == 0
    assert ws(5, 250, 255, 2048) == 0
    # long rows (dense tail, dense companion) are split over KV when the chunk has too few row blocks to fill
    # the GPU -> arrival words + whole partial records of the split items for 8 KV heads
    for n in (ws(512, 7680, 8192, 8192), dws(512, 7680, 8192)):
        assert n > 0 and _items(n) > 0
    # a 2048-row chunk already fills the GPU with row blocks: no split, however long its rows (an item takes
    # any number of tiles)
    assert dws(2048, 2048, 4096) == 0
    assert dws(2048, 6272, 8320) == 0
    assert dws(2048, 129024, 131072) == 0  # 1.1 GB when an item held at most 128 tiles
    # only the split row blocks' items have partial records: the config-2 last chunk splits its 4 dense-tail
    # row blocks in 3 (12 records), not its 12 sparse ones (24 items in all)
    assert _items(ws(512, 7680, 8192, 8192)) == 12 and cabi.chunk_plan(512, 7680, 8192, 8192)[2] == 24
    # invalid attributes -> -1 with a message
    assert ws(0, 0, 0, 0) == -1 and lib.tm_last_error().decode()
    assert ws(512, 4096, 4608, 4000) == -1
    assert dws(512, 4000, 4608) == -1


# (query_tokens, query_start, seq_len, prompt_len): chunks and whole prompts up to L = 131072, ragged and
# mid-page, including every BASELINE configuration's chunks and whole-prompt calls of any length
AGREE_GRID = sorted({
    *[(c, s, s + c, L) for L in (2869, 8192, 8320, 32768, 40960, 131072) for c in (1, 32, 128, 512, 2048)
      for s in (0, max(0, L - c - 4096), L - c) if s + c <= L],
    *[(L, 0, L, L) for L in (1, 31, 521, 1000, 4096, 8320, 32768, 32769, 40960, 65536, 131072)],
    (512, 2357, 2869, 2869), (100, 500, 600, 700), (300, 97, 397, 5000), (77, 8243, 8320, 8320),
})


def test_workspace_size_agrees_with_the_launch_over_a_grid(lib):
    """For every geometry: the size query, the plan query and the launch accept or refuse alike; an accepted
    call's workspace stays within TM_MAX_WORKSPACE_BYTES and holds the split items' partials; and a launch
    given one byte less is refused for its workspace, while one given the full size passes the size check
    (it then stops at an overlap check, so nothing is launched on these fake pointers)."""
    parts, tiles, items = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    for tq, qs, seq, prompt in AGREE_GRID + [(512, 4000, 4608, 8192), (0, 0, 0, 0), (512, 4096, 4608, 4000)]:
        for dense in (0, 1):
            need = (lib.tm_dense_paged_causal_attention_workspace_size(tq, qs, seq) if dense
                    else lib.tm_triangle_paged_sparse_attention_workspace_size(tq, qs, seq, prompt))
            size_msg = lib.tm_last_error().decode()
            plan = lib.tm_chunk_plan(dense, tq, qs, seq, prompt, ctypes.byref(parts), ctypes.byref(tiles),
                                     ctypes.byref(items))
            assert (need >= 0) == (plan == 0), (tq, qs, seq, prompt, dense)
            pages = -(-max(seq, 1) // 128) + 1
            a = dict(query=Q, key=K, value=V, table=BT, out=OUT, tq=tq, pages=pages, cols=pages, qs=qs, seq=seq,
                     prompt=prompt, scale=0.0883883, ws=WS, ws_bytes=max(need - 1, 0))

            def launch(**over):
                b = dict(a, **over)
                if dense:
                    return lib.tm_dense_paged_causal_attention(b["query"], b["key"], b["value"], b["table"],
                                                               b["out"], b["tq"], b["pages"], b["cols"], b["qs"],
                                                               b["seq"], b["scale"], b["ws"], b["ws_bytes"], None)
                return lib.tm_triangle_paged_sparse_attention(
                    b["query"], b["key"], b["value"], b["table"], b["out"], b["tq"], b["pages"], b["cols"], b["qs"],
                    b["seq"], b["prompt"], b["scale"], b["ws"], b["ws_bytes"], None)

            if need < 0:
                assert launch(ws=0, ws_bytes=0) == plan != 0
                assert lib.tm_last_error().decode() == size_msg
                continue
            assert need <= MAX_WORKSPACE
            assert _items(need) <= items.value and tiles.value >= 1 and parts.value in (1, 2, 4)
            if need > 0:
                assert launch() == 3 and "smaller than" in lib.tm_last_error().decode()
                assert launch(ws=OUT, ws_bytes=need) == 3 and "overlap" in lib.tm_last_error().decode()


def test_cabi_workspace_size_wrapper(lib):
    assert cabi.workspace_size(512, 4096, 4608, 8192) == 0
    with pytest.raises(cabi.TriangleMixError):
        cabi.workspace_size(512, 4000, 4608, 8192)


# ------------------------------------------------------------ torch adapter

@pytest.fixture(scope="module")
def adapter(lib):
    native.load_triangle_mix_adapter()
    return torch.ops


def test_adapter_schemas_match_reference(adapter):
    schemas = KATS["op_schemas"]
    got = {
        "trianglemix_reference::triangle_paged_sparse_attention":
            adapter.trianglemix_reference.triangle_paged_sparse_attention.default._schema,
        "trianglemix_reference::triangle_paged_sparse_attention_workspace_size":
            adapter.trianglemix_reference.triangle_paged_sparse_attention_workspace_size.default._schema,
        "trianglemix::triangle_paged_sparse_attention.out":
            adapter.trianglemix.triangle_paged_sparse_attention.out._schema,
    }
    for name, schema in got.items():
        assert str(schema) == schemas[name], name
    alias = str(adapter.trianglemix.npu_triangle_paged_sparse_attention.default._schema)
    assert "Tensor(a!) out) -> Tensor(a!)" in alias and "int prompt_len, float scale" in alias
    # the paged KV write keeps vLLM's reshape_and_cache argument order (bf16 caches, no scales)
    assert str(adapter.trianglemix.reshape_and_cache.default._schema) == (
        "trianglemix::reshape_and_cache(Tensor key, Tensor value, Tensor(a!) key_cache, Tensor(b!) value_cache, "
        "Tensor slot_mapping) -> ()")


def test_adapter_load_is_idempotent_and_refuses_second_path(adapter, tmp_path):
    assert native.load_triangle_mix_adapter() == native.load_triangle_mix_adapter()
    other = tmp_path / "other.so"
    other.write_bytes(b"")
    with pytest.raises(RuntimeError, match="refusing"):
        native.load_triangle_mix_adapter(other)
    assert native.native_status().ready


def test_meta_shape_inference(adapter):
    q = torch.empty(512, 32, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(71, 128, 8, 128, dtype=torch.bfloat16, device="meta")
    bt = torch.empty(1, 64, dtype=torch.int32, device="meta")
    out = adapter.trianglemix_reference.triangle_paged_sparse_attention(q, k, k, bt, 4096, 4608, 8192, 0.088)
    assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.device.type == "meta"
    o2 = torch.empty_like(q)
    assert adapter.trianglemix.triangle_paged_sparse_attention.out(q, k, k, bt, 4096, 4608, 8192, 0.088,
                                                                    out=o2) is o2


def test_cpu_tensors_have_no_kernel(adapter):
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(2, 128, 8, 128, dtype=torch.bfloat16)
    bt = torch.zeros(1, 2, dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        adapter.trianglemix.triangle_paged_sparse_attention.out(q, k, k, bt, 0, 4, 1024, 0.088,
                                                                 out=torch.empty_like(q))
    with pytest.raises(NotImplementedError):
        adapter.trianglemix_reference.dense_paged_causal_attention(q, k, k, bt, 0, 4, 0.088)
    kv = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        adapter.trianglemix.reshape_and_cache(kv, kv, k, k.clone(), torch.zeros(4, dtype=torch.int64))


# ------------------------------------------------------------ launch planner
# Measured on MI355X (tests/plan_sweep.py): for 87 chunk geometries (TriangleMix and dense-companion chunks
# of 64-12288 rows at prompts of 1024-131072 tokens) every forced (KV parts, tiles per item) plan was timed.
# The planner's costs were fitted to the 52 geometries not marked held_out, checked on the other 35, then
# fitted on all 87 (tests/plan_fit.py).
SWEEP = json.loads((Path(__file__).parent / "plan_sweep_mi355x.json").read_text())
sys.path.insert(0, str(Path(__file__).parent))
import plan_sweep  # noqa: E402


def _loss(g):
    """(time of the planned plan, fastest measured time) for a sweep geometry, plans matched by KV parts and
    pieces per row block."""
    qs, tq, seq, prompt = g["query_start"], g["query_tokens"], g["seq_len"], g["prompt_len"]
    rt = plan_sweep.row_tiles(qs, tq, seq, prompt)
    parts, tiles, items = cabi.chunk_plan(tq, qs, seq, prompt or None)
    assert items == sum(plan_sweep.pieces(rt, tiles))
    times = {(p[0], plan_sweep.pieces(rt, p[1])): p[3] for p in g["plans"]}
    assert (parts, plan_sweep.pieces(rt, tiles)) in times, (g["query_start"], parts, tiles)  # a measured plan
    return times[(parts, plan_sweep.pieces(rt, tiles))], min(times.values())


@pytest.mark.parametrize("g", SWEEP["geometries"],
                         ids=[f"{g['query_start']}+{g['query_tokens']}/{g['seq_len']}/{g['prompt_len']}"
                              for g in SWEEP["geometries"]])
def test_planned_plan_is_near_the_fastest_measured(lib, g):
    """The planner's choice is the fastest measured plan or close to it: at worst 9.3 % slower (the last
    1024 rows of a 16384-token prompt), and within 1 % on 70 of the 87 chunks."""
    planned, fastest = _loss(g)
    assert planned <= 1.10 * fastest


def test_planner_loss_over_the_sweep(lib):
    """Summed over the 87 geometries the planned plans lose 43.5 us of the 6,533 us the chunks take at their
    fastest (0.67 %): 12.8 us over the 52 first fitted on, 30.8 us over the 35 held out of that fit."""
    fit = [_loss(g) for g in SWEEP["geometries"] if not g["held_out"]]
    held = [_loss(g) for g in SWEEP["geometries"] if g["held_out"]]
    assert len(fit) == 52 and len(held) == 35
    lost = sum(p - f for p, f in fit + held)
    assert lost <= 0.0075 * sum(f for _, f in fit + held), lost
    assert sum(p - f for p, f in held) <= 0.01 * sum(f for _, f in held)


def test_plan_fit_restates_the_planner(lib):
    """tests/plan_fit.py's restated simulation, with the costs parsed from the C++ source, chooses the plan
    the library chooses (same KV parts and pieces) for every sweep geometry the fitted regimes cover."""
    import plan_fit
    sim = plan_fit._sim_lib()
    src = plan_fit.source_costs()
    for name, shapes in plan_fit.REGIMES.items():
        geoms = [g for g in SWEEP["geometries"] if plan_fit.regime_of(g) == name]
        reg = plan_fit.Regime(sim, geoms, shapes)
        costs = [c for _, cname, _, _ in shapes for c in src[cname]]
        loss = reg.losses(costs)
        for g, lost in zip(geoms, loss):
            planned, fastest = _loss(g)
            assert planned - fastest == pytest.approx(lost, abs=1e-6), g["query_start"]


# (query_start, query_tokens, seq_len, prompt_len) -> (KV parts, tiles per item, items per KV head)
# for the BASELINE configurations' split chunks.
BASELINE_PLANS = [
    ((2357, 512, 2869, 2869), (4, 84, 20)),        # config 1: quarters, dense-tail rows in two pieces
    ((7680, 512, 8192, 8192), (4, 124, 24)),       # config 2, last chunk: quarters in 1.5 rounds
    ((4096, 512, 4608, 8192), (4, 128, 16)),       # config 2, a middle chunk: one item per row block, no split
    ((6272, 2048, 8320, 8320), (1, 20, 112)),      # the last 2048 rows of an 8320-token prompt
    ((2048, 2048, 4096, 8320), (1, 128, 64)),      # config 3, a middle chunk: KV whole, 512 workgroups in one round
    ((0, 2048, 2048, 8320), (1, 128, 64)),         # config 3, the first chunk (dense rows of at most 17 tiles)
    ((14336, 2048, 16384, 32768), (1, 128, 64)),   # config 4, a middle chunk at L = 32768
    ((0, 2048, 2048, 2048), (1, 28, 72)),          # a whole 2048-token prompt: KV whole, its 64-tile tail in 3 pieces
    ((8192, 1024, 9216, 32768), (2, 128, 32)),     # 32 row blocks: too few for two KV-whole workgroups per CU
    ((8192, 128, 8320, 8320), (4, 84, 16)),        # config 3, last chunk
    ((30720, 2048, 32768, 32768), (1, 68, 124)),   # config 4, last chunk at L = 32768: tail rows in 16 pieces
    ((129024, 2048, 131072, 131072), (1, 256, 124)),  # config 4, last chunk at L = 131072: tail rows in 16 pieces
    ((0, 40960, 40960, 40960), (1, 640, 1284)),    # a whole 40960-token prompt: tail rows in two pieces
]


@pytest.mark.parametrize("geom,plan", BASELINE_PLANS, ids=[str(g) for g, _ in BASELINE_PLANS])
def test_baseline_config_plans(lib, geom, plan):
    qs, tq, seq, prompt = geom
    parts, tiles, items = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    assert lib.tm_chunk_plan(0, tq, qs, seq, prompt, ctypes.byref(parts), ctypes.byref(tiles), ctypes.byref(items)) == 0
    assert (parts.value, tiles.value, items.value) == plan


def test_chunk_plan_rejects_what_the_entry_points_reject(lib):
    parts, tiles, items = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    assert lib.tm_chunk_plan(0, 512, 4000, 4608, 8192, ctypes.byref(parts), ctypes.byref(tiles),
                             ctypes.byref(items)) == 1
    assert "Tq == seq_len" in lib.tm_last_error().decode()
    assert lib.tm_chunk_plan(0, 512, 4096, 4608, 8192, None, ctypes.byref(tiles), ctypes.byref(items)) == 1
    assert cabi.chunk_plan(512, 4096, 4608, 8192) == (4, 128, 16)
    assert cabi.chunk_plan(512, 7680, 8192, None) == (2, 128, 32)


def _row_block_tiles(tb: int, te: int, sparse_begin: int, sparse_end: int) -> int:
    """Tiles of 32 keys a row block [tb, te) visits (csrc/trianglemix_kernel.h row_block_tiles)."""
    last = (te - 1) // 32
    if tb >= sparse_begin and te <= sparse_end and sparse_end > 0 and (tb - 512) // 32 > 0:
        return 1 + last - (tb - 512) // 32 + 1  # the sink tile + the window's tiles
    return last + 1


def _items_at(T: int, qs: int, tq: int, seq: int, prompt: int | None) -> tuple[int, int]:
    sparse_begin, sparse_end = (521, max(0, prompt - 128)) if prompt else (0, 0)
    tiles = [_row_block_tiles(tb, min(tb + 32, seq), sparse_begin, sparse_end) for tb in range(qs, seq, 32)]
    return sum(tiles), sum(-(-n // T) for n in tiles)


def test_long_chunk_plan_skips_the_simulation_and_takes_the_largest_items(lib):
    """A chunk with more than 4096 candidate items (total tiles / 32, the smallest split) is not simulated:
    its tiles spread over one item per slot -- T is the smallest candidate of at least total / slots tiles
    (csrc/trianglemix_capi.cpp choose_plan), which for such a chunk is the longest row: no split.
    Pinned for the dense companion's last 2048-row chunk of a 131072-token prompt (64 row blocks of
    4033-4096 tiles): 64 items of whole rows, no workspace (2048 items and 1.1 GB of partials when an item
    held at most 128 tiles).  The TriangleMix chunk at the same place has 17458 tiles (sparse rows of 18
    tiles, four dense-tail rows of 4096) and stays below the bound: it is simulated, and splits its tail."""
    qs, tq, seq = 129024, 2048, 131072
    total, items = _items_at(4096, qs, tq, seq, None)
    assert total // 32 > 4096 and -(-total // 32) > 4096  # the shortcut applies: one slot's share > any row
    assert cabi.chunk_plan(tq, qs, seq, None) == (2, 4096, 64) and items == 64
    assert lib.tm_dense_paged_causal_attention_workspace_size(tq, qs, seq) == 0
    sparse_total, _ = _items_at(128, qs, tq, seq, 131072)
    assert sparse_total == 17458 and sparse_total // 32 <= 4096
    assert cabi.chunk_plan(tq, qs, seq, 131072) == (1, 256, 124)  # four tail rows in 16 pieces + 60 sparse


def test_whole_prompts_plan_without_refusal(lib):
    """Whole-prompt calls (PrefillNoCache: query_start 0, Tq = seq_len = prompt_len) of any length are
    accepted.  The dense companion plans one item per row block: a prompt has so many row blocks that no row
    needs splitting.  The TriangleMix op runs KV whole and splits at most its four dense-tail row blocks, where
    that balances the slots, within a few tens of MB of workspace.  The planning stays cheap on the host even
    at L = 131072 (4096 row blocks, simulated for the TriangleMix op)."""
    import time
    for L in (32769, 40960, 65536, 131072):
        row_blocks = -(-L // 32)
        for prompt in (L, None):
            t0 = time.perf_counter()
            parts, tiles, items = cabi.chunk_plan(L, 0, L, prompt)
            assert time.perf_counter() - t0 < 0.1
            assert parts == (1 if prompt else 2) and items >= row_blocks
        assert cabi.chunk_plan(L, 0, L, None)[2] == row_blocks
        assert lib.tm_dense_paged_causal_attention_workspace_size(L, 0, L) == 0
        # only row blocks holding dense-tail rows (the last 128 tokens: four or five row blocks) split
        _, tiles, items = cabi.chunk_plan(L, 0, L, L)
        pieces = plan_sweep.pieces(plan_sweep.row_tiles(0, L, L, L), tiles)  # issue order: last row block first
        assert items == sum(pieces) and all(p == 1 for p in pieces[5:])
        assert _items(cabi.workspace_size(L, 0, L, L)) == sum(p for p in pieces if p > 1)
        assert cabi.workspace_size(L, 0, L, L) <= 64 << 20


def test_routed_fast_path_gate_equals_the_python_gates(adapter):
    """The adapter library is also the Python module of the routed-call fast path.  Its ``tensor_gate`` names
    the same first failing gate as the router's Python ``_tensor_reason`` for a well-formed call and one broken
    property at a time (CPU tensors here: the gates compare devices with each other, so everything but a
    device mismatch is covered; tests/test_gpu_router_gates.py covers those on the GPU)."""
    from trianglemix import router as R

    fast = native.routed_fast_path()
    assert fast is not None and {"tensor_gate", "launch_sparse", "launch_dense"} <= set(dir(fast))
    tq, seq = 64, 700
    bf = torch.bfloat16
    base = dict(query=torch.zeros(tq, 32, 128, dtype=bf), output=torch.zeros(tq + 3, 32, 128, dtype=bf),
                key_cache=torch.zeros(7, 128, 8, 128, dtype=bf), value_cache=torch.zeros(7, 128, 8, 128, dtype=bf),
                block_table=torch.zeros(1, 6, dtype=torch.int32))
    cases = [{}, {"query": base["query"].half()}, {"query": torch.zeros(tq + 1, 32, 128, dtype=bf)},
             {"query": torch.zeros(tq, 32, 256, dtype=bf)[:, :, :128]}, {"query": torch.zeros(tq, 4096, dtype=bf)},
             {"output": torch.zeros(tq - 1, 32, 128, dtype=bf)}, {"output": torch.zeros((), dtype=bf)},
             {"output": torch.zeros(tq, 32, 128)}, {"key_cache": torch.zeros(7, 64, 8, 128, dtype=bf)},
             {"value_cache": torch.zeros(8, 128, 8, 128, dtype=bf)}, {"value_cache": base["value_cache"].half()},
             {"key_cache": torch.zeros(7, 128, 16, 128, dtype=bf)[:, :, ::2]},
             {"block_table": torch.zeros(1, 5, dtype=torch.int32)}, {"block_table": torch.zeros(1, 6, dtype=torch.int64)},
             {"block_table": torch.zeros(2, 6, dtype=torch.int32)},
             {"block_table": torch.zeros(1, 12, dtype=torch.int32)[:, ::2]}]
    seen = set()
    for change in cases:
        t = {**base, **change}
        args = (t["query"], t["output"], t["key_cache"], t["value_cache"], t["block_table"])
        py = R._tensor_reason(R.LayerFeatures(), *args, tq, seq)
        assert R._GATE_CODES[fast.tensor_gate(*args, tq, seq)] is py, (change.keys(), py)
        seen.add(py)
    assert len(seen) == 4  # every reason reached, and the well-formed call passes
