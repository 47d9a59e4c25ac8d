"""Pins the paged-KV-write oracle (``oracle/cache.py``) before it is trusted.

* ``chunk_slots`` against the reference's address known answer
  (test_project_contract.py:107-122: token 139, table [7, 2, 19], KV head 3
  -> element 273,792) and against ``geometry.bsnd_element_offset`` (itself
  pinned by that KAT) for every token of several page tables;
* ``reshape_and_cache`` against an independent formulation (one fancy
  assignment into the flattened ``[pages * 128, 8, 128]`` cache), with padding
  and out-of-range slots untouched;
* a planted mistake (page and offset swapped in the slot) fails both checks.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import cache as C
from oracle import geometry as G

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _slot_element_offset(slot: int, kv_head: int) -> int:
    return (slot * G.KV_HEADS + kv_head) * G.HEAD_DIM


@pytest.mark.parametrize("kat", KATS["bsnd_address"])
def test_chunk_slot_reproduces_reference_address_kat(kat):
    slot = int(C.chunk_slots(kat["block_table"], kat["token"], 1)[0])
    assert slot // C.PAGE_SIZE == kat["physical_page"]
    assert _slot_element_offset(slot, kat["kv_head"]) == kat["element_offset"]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_chunk_slots_match_bsnd_offsets_for_every_token(seed):
    rng = np.random.default_rng(seed)
    logical = 9
    table = [int(x) for x in rng.permutation(logical + 5)[:logical]]
    for q0, n in [(0, logical * 128), (300, 517), (1000, 1)]:
        slots = C.chunk_slots(table, q0, n)
        for i, slot in enumerate(slots):
            for h in (0, 7):
                assert _slot_element_offset(int(slot), h) == G.bsnd_element_offset(q0 + i, h, table)


def _random_case(seed, tokens=40, pages=6):
    rng = np.random.default_rng(seed)
    key = rng.standard_normal((tokens, 8, 128)).astype(np.float32)
    value = rng.standard_normal((tokens, 8, 128)).astype(np.float32)
    kc = rng.standard_normal((pages, 128, 8, 128)).astype(np.float32)
    vc = rng.standard_normal((pages, 128, 8, 128)).astype(np.float32)
    slots = rng.permutation(pages * 128)[:tokens].astype(np.int64)
    slots[3] = -1                     # padding
    slots[7] = pages * 128 + 5        # past the cache
    return key, value, kc, vc, slots


def _flat_reference(key, value, kc, vc, slots):
    kc, vc = kc.copy(), vc.copy()
    ok = (slots >= 0) & (slots < kc.shape[0] * 128)
    kc.reshape(-1, 8, 128)[slots[ok]] = key[ok]
    vc.reshape(-1, 8, 128)[slots[ok]] = value[ok]
    return kc, vc


@pytest.mark.parametrize("seed", [0, 1])
def test_reshape_and_cache_matches_flat_assignment(seed):
    key, value, kc, vc, slots = _random_case(seed)
    want_k, want_v = _flat_reference(key, value, kc, vc, slots)
    before_k, before_v = kc.copy(), vc.copy()
    C.reshape_and_cache(key, value, kc, vc, slots)
    assert np.array_equal(kc, want_k) and np.array_equal(vc, want_v)
    # padding / out-of-range tokens wrote nothing; every other cache row is untouched
    written = np.zeros(kc.shape[0] * 128, dtype=bool)
    ok = (slots >= 0) & (slots < kc.shape[0] * 128)
    written[slots[ok]] = True
    assert np.array_equal(kc.reshape(-1, 8, 128)[~written], before_k.reshape(-1, 8, 128)[~written])
    assert np.array_equal(vc.reshape(-1, 8, 128)[~written], before_v.reshape(-1, 8, 128)[~written])


def test_planted_mistake_is_caught():
    """Page and offset swapped (slot = offset * 128 + page): the checks above fail."""
    table = KATS["bsnd_address"][0]["block_table"]
    t = np.arange(139, 140, dtype=np.int64)
    tab = np.asarray(table, dtype=np.int64)
    wrong = (t % 128) * 128 + tab[t // 128]
    assert _slot_element_offset(int(wrong[0]), 3) != KATS["bsnd_address"][0]["element_offset"]
    key, value, kc, vc, slots = _random_case(3)
    want_k, _ = _flat_reference(key, value, kc, vc, slots)
    swapped = np.where(slots >= 0, (slots % 128) * 128 + slots // 128, slots)
    got_k, got_v = kc.copy(), vc.copy()
    C.reshape_and_cache(key, value, got_k, got_v, swapped)
    assert not np.array_equal(got_k, want_k)


def test_product_slot_mapping_matches_oracle():
    """``trianglemix.cache.chunk_slot_mapping`` (torch, the engine-side helper) equals the oracle's slots."""
    import torch

    from trianglemix.cache import chunk_slot_mapping

    table = torch.tensor([[7, 2, 19, 4, 11]], dtype=torch.int32)
    for q0, n in [(0, 640), (139, 1), (300, 211), (512, 0)]:
        got = chunk_slot_mapping(table, q0, n)
        assert got.dtype == torch.int64
        assert np.array_equal(got.numpy(), C.chunk_slots(table, q0, n))
    with pytest.raises(ValueError, match="lacks logical pages"):
        chunk_slot_mapping(table, 600, 41)
