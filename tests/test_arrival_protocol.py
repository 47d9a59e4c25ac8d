"""The split-merge arrival protocol of the attention kernel, checked over every interleaving on the CPU.

``csrc/trianglemix_kernel.hip`` counts the splits of a row block in one 64-bit word per (KV head, row block,
workgroup position): the launch's 48-bit epoch above a 16-bit count.  An arrival adds one (fetch-and-add);
if the word it added to carried another epoch, it installs its own epoch with a count of one, or counts
itself under an epoch another arrival installed, by compare-and-swap from the value last seen.  The arrival
whose count reaches the split count merges.  Workspace contents are arbitrary before a launch, so the
initial word may be anything.

This file models each arrival as the sequence of atomic steps the kernel performs (the kernel's two atomic
operations, each indivisible) and explores every interleaving of two and three arrivals from initial words
that are clean, cleared by a previous launch, carry another epoch at every count, or sit one below a carry
into the epoch field.  In every execution exactly one arrival must reach the split count, every arrival
must end in a bounded number of steps, and the word must end as (epoch, splits).  A planted variant that
skips the install step (trusting any word) fails on a foreign word.
"""

from __future__ import annotations

import itertools

SHIFT = 16
MASK64 = (1 << 64) - 1


def arrival(epoch: int, trust_any_word: bool = False):
    """Generator over one arrival's atomic steps; each ``yield`` hands an operation to the scheduler,
    which applies it to the shared word and sends back the old value (fetch-and-add) or (ok, current)."""
    old = yield ("add", 1)
    mine = (old + 1) & MASK64
    if (old >> SHIFT) != epoch and not trust_any_word:
        seen = mine
        while True:
            mine = seen + 1 if (seen >> SHIFT) == epoch else (epoch << SHIFT) + 1
            ok, cur = yield ("cas", seen, mine)
            if ok:
                break
            seen = cur
    return mine & ((1 << SHIFT) - 1)


def run_schedule(initial: int, epoch: int, n: int, order, trust_any_word=False):
    """Run n arrivals, picking the next to step from ``order`` (an iterator of arrival indices; exhausted
    or finished picks fall to the lowest unfinished one).  Returns (final word, counts seen)."""
    word = initial
    gens = [arrival(epoch, trust_any_word) for _ in range(n)]
    pending = [next(g) for g in gens]
    result = [None] * n
    steps = 0
    order = iter(order)
    while any(r is None for r in result):
        steps += 1
        assert steps < 100, "an arrival did not finish"
        live = [i for i in range(n) if result[i] is None]
        i = next(order, live[0])
        if result[i] is not None:
            i = live[0]
        op = pending[i]
        if op[0] == "add":
            reply = word
            word = (word + op[1]) & MASK64
        else:
            _, expected, desired = op
            ok = word == expected
            reply = (ok, word)
            if ok:
                word = desired
        try:
            pending[i] = gens[i].send(reply)
        except StopIteration as stop:
            result[i] = stop.value
    return word, result


EPOCH = 0x1234_5678_9ABC
INITIAL_WORDS = [0, (EPOCH - 1) << SHIFT, ((EPOCH + 7) << SHIFT) + 3, ((EPOCH - 1) << SHIFT) | 0xFFFF,
                 0xFFFF_FFFF_FFFF_FFFF, (0xDEAD_BEEF << SHIFT) + 1]


def _schedules(n, length):
    return itertools.product(range(n), repeat=length)


def test_every_interleaving_counts_each_arrival_once():
    for n in (2, 3):
        for initial in INITIAL_WORDS:
            for order in _schedules(n, 7 if n == 3 else 8):
                word, counts = run_schedule(initial, EPOCH, n, order)
                assert sorted(counts) == list(range(1, n + 1)), (n, hex(initial), order, counts)
                assert word == (EPOCH << SHIFT) + n, (n, hex(initial), order, hex(word))


def test_cleared_word_takes_one_atomic_after_the_first_arrival():
    # a word cleared by the previous launch: the first arrival installs the epoch (two atomics), every later
    # one is counted by its fetch-and-add alone
    word, counts = run_schedule(0, EPOCH, 3, [0, 0, 1, 2])
    assert counts == [1, 2, 3] and word == (EPOCH << SHIFT) + 3


def test_trusting_any_word_fails_on_a_foreign_word():
    # the planted variant counts from whatever the word held: right only when its count field happens to be
    # zero, wrong for an interrupted launch's word (count 3) and for garbage
    for initial in INITIAL_WORDS[1:]:
        _, counts = run_schedule(initial, EPOCH, 2, [0, 1], trust_any_word=True)
        assert (sorted(counts) == [1, 2]) == (initial & 0xFFFF == 0), hex(initial)
