"""Pins the floating-point oracle (``oracle/attention.py``) before it is trusted.

* the reference's sentinels (shared softmax at q=521 with a poisoned token 8,
  GQA head map; the small joint-softmax 4.6 vs forbidden 11);
* Q = 0 closed form: every output row is the mean of V over the row's keys,
  with the keys taken from the set-builder form of the mask (independent of
  the oracle's interval code);
* a library routine: ``torch.nn.functional.scaled_dot_product_attention``
  with an explicit boolean mask over an identity page table;
* page-permutation invariance (test_triangle_v2_reference.py:150-226);
* float64 numpy vs float32 torch agreement;
* online softmax over any split == joint softmax, and a fully masked block
  leaves the state unchanged (test_boundary_mask_alignment_design.py:743-822);
* planted oracle mistakes (dropped window key, transposed head map, two
  separately normalised softmaxes) fail these checks.
"""

from __future__ import annotations

import json
import math
import random
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import geometry as G
from trianglemix.workload import SCALE, make_inputs

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
SENT = KATS["sentinels"]


def _setbuilder(q, seq_len, prompt_len):
    dense = not (521 <= q < max(0, prompt_len - 128))
    return [k for k in range(min(q + 1, seq_len)) if dense or k < 8 or q - k <= 512]


def _set_logical(cache, table, tokens, value):
    for t in tokens:
        pp, off = G.physical_location(t, table.view(-1).tolist())
        cache[pp, off].fill_(value)


def _shared_softmax_inputs():
    s = SENT["shared_softmax"]
    g = torch.Generator().manual_seed(2201)
    pages = math.ceil(s["seq_len"] / 128)
    from trianglemix.workload import noncontiguous_block_table
    table = noncontiguous_block_table(pages, pages + 5, g)
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(pages + 5, 128, 8, 128, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    _set_logical(v, table, range(8), s["v_sink"])
    _set_logical(v, table, (8,), s["v_token8"])
    _set_logical(v, table, range(9, 522), s["v_local"])
    return q, k, v, table, s


def test_shared_softmax_sentinel():
    q, k, v, table, s = _shared_softmax_inputs()
    for out in (OA.attention_torch(q, k, v, table, s["query_start"], s["seq_len"], s["prompt_len"], SCALE),
                torch.from_numpy(OA.attention_np(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                                 table.numpy(), s["query_start"], s["seq_len"], s["prompt_len"],
                                                 SCALE))):
        assert torch.allclose(out.double(), torch.full_like(out.double(), s["joint_expected"]), atol=1e-6)
        assert abs(float(out[0, 0, 0]) - s["forbidden_two_softmax"]) > 1.0
    assert s["joint_expected"] == pytest.approx((8 * 10.0 + 513.0) / 521.0, abs=1e-12)


def test_gqa_sentinel():
    s = SENT["gqa"]
    g = torch.Generator().manual_seed(2202)
    from trianglemix.workload import noncontiguous_block_table
    table = noncontiguous_block_table(1, 4, g)
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(4, 128, 8, 128, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    pp = int(table[0, 0])
    for h in range(8):
        v[pp, 0, h].fill_(float(h + 1))
    out = OA.attention_torch(q, k, v, table, s["query_start"], s["seq_len"], s["prompt_len"], 1.0)
    assert out[0, :, 0].tolist() == [float(x) for x in s["expected_per_query_head"]]


def test_small_joint_vs_two_softmax():
    s = SENT["joint_vs_two_softmax_small"]
    vals = [[float(x)] for x in s["values"]]
    joint = OA.joint_softmax_weighted_sum(s["scores"], vals)
    b0 = s["blocks"][0]
    online = OA.online_softmax_weighted_sum([(s["scores"][:b0], vals[:b0]), (s["scores"][b0:], vals[b0:])])
    assert joint[0] == pytest.approx(s["joint_expected"]) and online[0] == pytest.approx(joint[0])
    two = (OA.joint_softmax_weighted_sum(s["scores"][:b0], vals[:b0])[0]
           + OA.joint_softmax_weighted_sum(s["scores"][b0:], vals[b0:])[0])
    assert two == s["forbidden_two_softmax"]


def test_online_equals_joint_over_random_splits():
    rng = random.Random(7)
    for _ in range(50):
        n = rng.randint(1, 40)
        scores = [rng.uniform(-30, 30) for _ in range(n)]
        vals = [[rng.uniform(-5, 5), rng.uniform(-5, 5)] for _ in range(n)]
        cuts = sorted(rng.sample(range(1, n), min(n - 1, rng.randint(0, 4)))) if n > 1 else []
        blocks, prev = [], 0
        for c in cuts + [n]:
            blocks.append((scores[prev:c], vals[prev:c]))
            prev = c
        assert OA.online_softmax_weighted_sum(blocks) == pytest.approx(OA.joint_softmax_weighted_sum(scores, vals))


def test_fully_masked_block_leaves_state_unchanged():
    vals = [[1.0], [2.0], [3.0]]
    base = OA.online_softmax_weighted_sum([([0.5, 1.5, -2.0], vals)])
    masked = OA.online_softmax_weighted_sum([([0.5, 1.5, -2.0], vals), ([-3.4028e38] * 2, [[1e6], [-1e6]])])
    assert masked == base


@pytest.mark.parametrize("query_start,query_tokens,prompt_len", [
    (500, 40, 1024), (880, 32, 1024), (1018, 5, 2048), (0, 12, 64), (1023, 1, 1024)])
def test_zero_query_gives_mean_of_selected_values(query_start, query_tokens, prompt_len):
    seq_len = query_start + query_tokens
    _, k, v, table = make_inputs(query_start, query_tokens, seq_len, seed=11)
    q = torch.zeros(query_tokens, 32, 128, dtype=torch.bfloat16)
    out = OA.attention_np(q.float().numpy(), k.float().numpy(), v.float().numpy(), table.numpy(),
                          query_start, seq_len, prompt_len, SCALE)
    lv = v.float()[table.view(-1).long()].reshape(-1, 8, 128)[:seq_len].double().numpy()
    for r in range(query_tokens):
        keys = _setbuilder(query_start + r, seq_len, prompt_len)
        expect = np.repeat(lv[keys].mean(axis=0), 4, axis=0)  # kv head h//4
        np.testing.assert_allclose(out[r], expect, rtol=0, atol=1e-12)


def test_matches_sdpa_with_boolean_mask():
    query_start, tq, prompt_len = 480, 64, 1024  # rows cross sparse_begin 521
    seq_len = query_start + tq
    q, k, v, table = make_inputs(query_start, tq, seq_len, seed=21, std=1.0)
    ours = OA.attention_torch(q, k, v, table, query_start, seq_len, prompt_len, SCALE)
    lk = k.float()[table.view(-1).long()].reshape(-1, 8, 128)[:seq_len]
    lv = v.float()[table.view(-1).long()].reshape(-1, 8, 128)[:seq_len]
    mask = torch.zeros(tq, seq_len, dtype=torch.bool)
    for r in range(tq):
        mask[r, _setbuilder(query_start + r, seq_len, prompt_len)] = True
    qh = q.float().permute(1, 0, 2)                           # [32, tq, 128]
    kh = lk.permute(1, 0, 2).repeat_interleave(4, 0)          # [32, seq, 128]
    vh = lv.permute(1, 0, 2).repeat_interleave(4, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, attn_mask=mask, scale=SCALE)
    torch.testing.assert_close(ours, ref.permute(1, 0, 2), rtol=0, atol=2e-6)


def test_page_permutation_invariance():
    query_start, tq, prompt_len = 600, 16, 2048
    seq_len = query_start + tq
    q, k, v, table = make_inputs(query_start, tq, seq_len, seed=31, std=1.0)
    pages = table.numel()
    ident = torch.arange(pages, dtype=torch.int32).view(1, -1)
    k2, v2 = k[table.view(-1).long()].clone(), v[table.view(-1).long()].clone()
    a = OA.attention_torch(q, k, v, table, query_start, seq_len, prompt_len, SCALE)
    b = OA.attention_torch(q, k2, v2, ident, query_start, seq_len, prompt_len, SCALE)
    assert torch.equal(a, b)


def test_float64_and_float32_oracles_agree():
    query_start, tq, prompt_len = 890, 12, 1024  # sparse rows and dense tail rows
    seq_len = query_start + tq
    q, k, v, table = make_inputs(query_start, tq, seq_len, seed=41, std=1.0)
    a = OA.attention_torch(q, k, v, table, query_start, seq_len, prompt_len, SCALE).double().numpy()
    b = OA.attention_np(q.float().numpy(), k.float().numpy(), v.float().numpy(), table.numpy(),
                        query_start, seq_len, prompt_len, SCALE)
    np.testing.assert_allclose(a, b, atol=2e-6, rtol=0)
    ad = OA.attention_torch(q, k, v, table, query_start, seq_len, prompt_len, SCALE, dense=True).double().numpy()
    bd = OA.attention_np(q.float().numpy(), k.float().numpy(), v.float().numpy(), table.numpy(),
                         query_start, seq_len, prompt_len, SCALE, dense=True)
    np.testing.assert_allclose(ad, bd, atol=2e-6, rtol=0)
    assert np.abs(a - ad).max() > 1e-3  # sparse rows do differ from dense


def test_error_metrics():
    m = OA.error_metrics(np.array([1.0, 2.0, 4.0]), np.array([1.0, 2.5, 4.0]))
    assert m == {"finite": True, "max_abs": 0.5, "mean_abs": pytest.approx(1 / 6),
                 "relative_l2": pytest.approx(0.5 / math.sqrt(1 + 6.25 + 16))}
    assert not OA.error_metrics(np.array([np.nan]), np.array([0.0]))["finite"]


def test_planted_mistakes_fail(monkeypatch):
    """Mistakes planted in the oracle are caught by the checks above."""
    q, k, v, table, s = _shared_softmax_inputs()
    good = G.selected_intervals

    # 1. window edge off by one (token q-512 dropped): Q=0 closed form breaks
    def short_window(qq, seq_len, prompt_len):
        return tuple((b + 1, e) if b > 8 else (b, e) for b, e in good(qq, seq_len, prompt_len))

    monkeypatch.setattr(G, "selected_intervals", short_window)
    _, kk, vv, tt = make_inputs(600, 4, 604, seed=11)
    out = OA.attention_np(np.zeros((4, 32, 128)), kk.float().numpy(), vv.float().numpy(), tt.numpy(), 600, 604,
                          2048, SCALE)
    lv = vv.float()[tt.view(-1).long()].reshape(-1, 8, 128)[:604].double().numpy()
    expect = np.repeat(lv[_setbuilder(600, 604, 2048)].mean(axis=0), 4, axis=0)
    assert np.abs(out[0] - expect).max() > 1e-6
    monkeypatch.setattr(G, "selected_intervals", good)

    # 2. token 8 leaking in (sink of 9): the shared-softmax sentinel moves
    def leaky_sink(qq, seq_len, prompt_len):
        return tuple((0, 9) if (b, e) == (0, 8) else (b, e) for b, e in good(qq, seq_len, prompt_len))

    monkeypatch.setattr(G, "selected_intervals", leaky_sink)
    out = OA.attention_torch(q, k, v, table, s["query_start"], s["seq_len"], s["prompt_len"], SCALE)
    assert abs(float(out[0, 0, 0]) - s["joint_expected"]) > s["tolerance"]
    monkeypatch.setattr(G, "selected_intervals", good)

    # 3. two separately normalised softmaxes: 11, not 1.138
    sink = OA.joint_softmax_weighted_sum([0.0] * 8, [[10.0]] * 8)[0]
    local = OA.joint_softmax_weighted_sum([0.0] * 513, [[1.0]] * 513)[0]
    assert abs(sink + local - s["joint_expected"]) > s["tolerance"]


# ---------------------------------------------------------------- the blocked restatement
# ``attention_torch_blocked`` runs the same softmax for many rows at once (and on the GPU, where the long
# whole-chunk parity tests use it).  Pinned here: its mask predicate against the set-builder form over every
# row of several prompts, a planted off-by-one that this check catches, and its outputs against the per-row
# fp32 oracle and the float64 one, with blocks forced small enough that every kind of block boundary occurs.

@pytest.mark.parametrize("seq_len,prompt_len", [(700, 700), (1100, 5000), (1300, 1300), (650, 650), (520, 900)])
def test_attended_mask_equals_set_builder(seq_len, prompt_len):
    rows = torch.arange(0, seq_len)
    keys = torch.arange(0, seq_len)
    for dense in (False, True):
        mask = OA.attended_mask(rows, keys, seq_len, prompt_len, dense=dense)
        for q in range(seq_len):
            want = list(range(q + 1)) if dense else _setbuilder(q, seq_len, prompt_len)
            assert torch.nonzero(mask[q]).reshape(-1).tolist() == want, (q, dense)


def test_attended_mask_planted_window_off_by_one_is_caught():
    rows, keys = torch.arange(0, 1200), torch.arange(0, 1200)
    good = OA.attended_mask(rows, keys, 1200, 1200)
    q = rows.reshape(-1, 1)
    k = keys.reshape(1, -1)
    sparse = (q >= 521) & (q < 1200 - 128)
    bad = (k <= q) & (~sparse | (k < 8) | (k >= q - 511))  # one window key dropped
    assert not torch.equal(good, bad)
    assert torch.nonzero(good[700]).reshape(-1).tolist() == _setbuilder(700, 1200, 1200)


@pytest.mark.parametrize("qs,tq,seq,prompt,dense", [
    (500, 100, 600, 700, False),     # dense prefix rows, the sparse start, sparse rows
    (0, 700, 700, 700, False),       # a whole prompt: prefix, sparse middle, dense tail
    (2357, 512, 2869, 2869, False),
    (1000, 600, 1600, 5000, False),  # a prompt past the sequence: all sparse
    (0, 300, 300, 300, True),        # dense companion, whole prompt
    (1500, 233, 1733, 1733, True),   # dense companion, ragged chunk
])
def test_blocked_oracle_matches_per_row_oracles(qs, tq, seq, prompt, dense):
    q, k, v, bt = make_inputs(qs, tq, seq, 77 + qs)
    per_row = OA.attention_torch(q, k, v, bt, qs, seq, prompt, SCALE, dense=dense)
    for max_scores in (1 << 14, 1 << 20, 1 << 26):  # blocks of 1-2 rows up to the whole chunk
        blocked = OA.attention_torch_blocked(q, k, v, bt, qs, seq, prompt, SCALE, dense=dense,
                                             max_scores=max_scores)
        assert (blocked - per_row).abs().max().item() <= 4e-6, max_scores
    if tq <= 400:  # the float64 restatement is slow; the per-row fp32 one above covers the larger chunks
        ref64 = OA.attention_np(q.float().numpy(), k.float().numpy(), v.float().numpy(), bt.numpy(), qs, seq,
                                prompt, SCALE, dense=dense)
        assert np.abs(blocked.numpy() - ref64).max() <= 1e-4


def test_blocked_oracle_zero_query_is_the_mean_of_selected_values():
    qs, tq, seq, prompt = 400, 400, 800, 900
    _, k, v, bt = make_inputs(qs, tq, seq, 5)
    q = torch.zeros(tq, 32, 128, dtype=torch.bfloat16)
    got = OA.attention_torch_blocked(q, k, v, bt, qs, seq, prompt, SCALE, max_scores=1 << 16)
    lv = v[bt[0, :-(-seq // 128)].long()].reshape(-1, 8, 128)[:seq].double()
    for r in (0, 120, 121, 122, 399):
        keys = _setbuilder(qs + r, seq, prompt)
        want = lv[keys].mean(0).repeat_interleave(4, dim=0)
        assert torch.allclose(got[r].double(), want, atol=1e-5), r
