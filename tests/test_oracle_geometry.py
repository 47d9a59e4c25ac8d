"""Pins the integer oracle (``oracle/geometry.py``) before it is trusted.

Checks, in order of strength:

* the reference's own known-answer vectors (``tests/golden/reference_kats.json``,
  each entry naming its reference file:line);
* brute force against the set-builder form of the mask rule,
  ``k <= q and (dense(q) or k < 8 or q - k <= 512)``, which shares no code
  with the interval construction;
* "span intervals + per-row boundary mask == per-row intervals" over every
  q-tile of several chunks (test_query_span_contract.py:64-115 states this
  invariant for the reference);
* exact coverage of the query rows by the spans;
* the closed forms of saved-QK and attended pairs against direct counting.

A planted mistake in the oracle (a shifted window edge, a wrong sink size,
a dropped dense tail) fails at least one of these; ``test_planted_mistakes``
shows that on the CPU.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from oracle import geometry as G

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _setbuilder(q: int, seq_len: int, prompt_len: int) -> set[int]:
    dense = not (521 <= q < max(0, prompt_len - 128))
    return {k for k in range(min(q + 1, seq_len)) if dense or k < 8 or q - k <= 512}


@pytest.mark.parametrize("kat", KATS["row_intervals"], ids=lambda k: f"q{k['q']}_s{k['seq_len']}_p{k['prompt_len']}")
def test_row_interval_kats(kat):
    got = G.selected_intervals(kat["q"], kat["seq_len"], kat["prompt_len"])
    assert [list(iv) for iv in got] == kat["intervals"], kat["source"]


def test_token8_is_first_gap_and_row_has_521_keys():
    keys = G.selected_keys(521, 522, 2048)
    assert keys[:8] == list(range(8)) and keys[8:] == list(range(9, 522))
    assert len(keys) == 521 and 8 not in keys


@pytest.mark.parametrize("kat", KATS["dense_tail"])
def test_dense_tail_kat(kat):
    assert G.dense_tail_start(kat["prompt_len"]) == kat["sparse_end"]
    lo, hi = kat["dense_rows"]
    for q in range(lo, hi):
        assert G.selected_intervals(q, kat["prompt_len"], kat["prompt_len"]) == ((0, q + 1),)


@pytest.mark.parametrize("prompt_len", [1, 8, 520, 521, 600, 649, 650, 777, 1024, 1500])
def test_row_intervals_match_setbuilder_bruteforce(prompt_len):
    for q in range(prompt_len):
        for seq_len in (q + 1, prompt_len):
            got = G.selected_keys(q, seq_len, prompt_len)
            assert got == sorted(_setbuilder(q, seq_len, prompt_len)), (q, seq_len, prompt_len)
            assert all(G.attended(q, k, seq_len, prompt_len) == (k in got) for k in range(max(0, q - 520), q + 2))


@pytest.mark.parametrize("kat", KATS["span_schedules"], ids=lambda k: f"{k['q_begin']}_{k['q_end']}")
def test_span_schedule_kats(kat):
    dense, ivs = G.span_intervals(kat["q_begin"], kat["q_end"], kat["kv_len"], kat["sparse_begin"], kat["sparse_end"])
    assert dense == kat["dense"] and [list(iv) for iv in ivs] == kat["intervals"], kat["source"]
    if "virtual_tokens" in kat:
        assert sum(e - b for b, e in ivs) == kat["virtual_tokens"]


@pytest.mark.parametrize("kat", KATS["query_spans"], ids=lambda k: f"{k['query_start']}_{k['query_tokens']}")
def test_query_span_kats(kat):
    spans = G.split_query_spans(kat["query_start"], kat["query_tokens"], kat["sparse_begin"], kat["sparse_end"])
    assert [[s.begin, s.end, s.sparse] for s in spans] == kat["spans"], kat["source"]


@pytest.mark.parametrize("query_start,query_tokens,prompt_len", [
    (0, 1, 2048), (500, 65, 2048), (503, 67, 8320), (512, 32, 8320), (700, 31, 2048), (766, 35, 2048),
    (880, 32, 1024), (883, 30, 1024), (894, 4, 1024), (1023, 1, 1024), (2357, 512, 2869), (7680, 512, 8192),
])
def test_spans_cover_rows_and_intervals_plus_mask_equal_rows(query_start, query_tokens, prompt_len):
    seq_len = query_start + query_tokens
    sb, se = G.SPARSE_BEGIN, G.dense_tail_start(prompt_len)
    spans = G.split_query_spans(query_start, query_tokens, sb, se)
    rows = [q for s in spans for q in range(s.begin, s.end)]
    assert rows == list(range(query_start, seq_len))
    for s in spans:
        assert s.end - s.begin <= G.Q_TILE
        assert all(G.row_is_sparse(q, prompt_len) == s.sparse for q in range(s.begin, s.end))
        dense, ivs = G.span_intervals(s.begin, s.end, seq_len, sb, se)
        submitted = {k for b, e in ivs for k in range(b, e)}
        for q in range(s.begin, s.end):
            # per-row boundary mask applied to the span's submitted keys
            after = {k for k in submitted if k <= q and (dense or k < G.SINK or q - k <= G.WINDOW)}
            assert after == set(G.selected_keys(q, seq_len, prompt_len)), (s, q)


@pytest.mark.parametrize("kat", KATS["bsnd_address"])
def test_bsnd_address_kat(kat):
    pp, off = G.physical_location(kat["token"], kat["block_table"])
    assert pp == kat["physical_page"] and kat["token"] // G.PAGE_SIZE == kat["logical_page"]
    assert G.bsnd_element_offset(kat["token"], kat["kv_head"], kat["block_table"]) == kat["element_offset"]


def test_physical_location_rejects_short_table():
    with pytest.raises(ValueError):
        G.physical_location(3 * 128, [7, 2, 19])


@pytest.mark.parametrize("kat", [k for k in KATS["chunk_spans"] if "saved_qk" in k], ids=lambda k: str(k["saved_qk"]))
def test_saved_qk_bruteforce_kats(kat):
    q0 = kat["query_start"]
    assert G.saved_qk_bruteforce(q0, q0 + kat["query_tokens"], kat["prompt_len"]) == kat["saved_qk"]


def test_attended_pairs_closed_form_against_counting():
    # dense causal minus saved pairs
    for q0, q1, prompt in [(2357, 2869, 2869), (500, 900, 1024), (0, 2261, 2261), (4096, 4608, 8192)]:
        dense = sum(q + 1 for q in range(q0, q1))
        assert G.attended_pairs(q0, q1, q1, prompt) == dense - G.saved_qk_bruteforce(q0, q1, prompt)
    # config 1: 384 sparse rows of 521 keys + 128 tail rows
    assert G.attended_pairs(2357, 2869, 2869, 2869) == 384 * 521 + sum(q + 1 for q in range(2741, 2869))


def test_unique_kv_tokens():
    assert G.unique_kv_tokens(4096, 4608, 4608, 8192) == 8 + (4607 - (4096 - 512) + 1)
    assert G.unique_kv_tokens(0, 512, 512, 8192) == 512
    assert G.unique_kv_tokens(7680, 8192, 8192, 8192) == 8192


def test_planted_mistakes_fail(monkeypatch):
    """A shifted window edge or a dropped dense tail in the oracle is caught."""
    good = G.selected_intervals
    kat = KATS["row_intervals"]

    def off_by_one_window(q, seq_len, prompt_len):
        ivs = good(q, seq_len, prompt_len)
        return tuple((b + 1, e) if b > 8 else (b, e) for b, e in ivs)

    def no_dense_tail(q, seq_len, prompt_len):
        return good(q, seq_len, prompt_len + 128)

    for mistake in (off_by_one_window, no_dense_tail):
        failures = sum([list(map(list, mistake(k["q"], k["seq_len"], k["prompt_len"]))) != k["intervals"] for k in kat])
        assert failures > 0, mistake.__name__
