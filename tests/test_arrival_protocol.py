"""The split-merge arrival protocol of the attention kernel, checked over every interleaving on the CPU.

``csrc/trianglemix_kernel.hip`` counts the splits of a row block in one 64-bit word per (KV head, row block,
workgroup position): the launch's 48-bit epoch above a 16-bit count.  An arrival adds one (fetch-and-add);
if the word it added to carried another epoch, it installs its own epoch with a count of one, or counts
itself under an epoch another arrival installed, by compare-and-swap from the value last seen.  The arrival
whose count reaches the split count merges, then leaves the word at (epoch, 0): the host keeps one epoch per
workspace address, so the next launch on that workspace (or the next replay of a captured one) finds its
words clean and counts each arrival with its fetch-and-add alone.  Workspace contents are otherwise
arbitrary before a launch, so the initial word may be anything.

This file models each arrival as the sequence of atomic steps the kernel performs (the kernel's two atomic
operations, each indivisible) and explores every interleaving of two and three arrivals from initial words
that are zero, left clean by a previous launch on the workspace (this epoch, count 0), carry another epoch
at every count, or sit one below a carry into the epoch field.  In every execution exactly one arrival must reach the split count, every arrival
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
    atomics = [0] * n
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
        atomics[i] += 1
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
    run_schedule.atomics = atomics
    return word, result


def merge_and_reset(word: int, epoch: int) -> int:
    """The last arrival's reset after its merge: the word is left at (epoch, 0)."""
    assert word & ((1 << SHIFT) - 1) != 0
    return epoch << SHIFT


EPOCH = 0x1234_5678_9ABC
INITIAL_WORDS = [0, EPOCH << SHIFT, (EPOCH - 1) << SHIFT, ((EPOCH + 7) << SHIFT) + 3, ((EPOCH - 1) << SHIFT) | 0xFFFF,
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


def test_a_word_left_by_the_previous_launch_takes_one_atomic_per_arrival():
    # launch 1 on a foreign word installs the epoch; its last arrival leaves (epoch, 0); launch 2 with the
    # same epoch (the same workspace) counts every arrival by its fetch-and-add alone, in every order
    word, counts = run_schedule(0xFFFF_FFFF_FFFF_FFFF, EPOCH, 3, [0, 1, 2, 0, 1, 2])
    assert sorted(counts) == [1, 2, 3]
    word = merge_and_reset(word, EPOCH)
    for order in _schedules(3, 6):
        final, counts = run_schedule(word, EPOCH, 3, order)
        assert sorted(counts) == [1, 2, 3] and final == (EPOCH << SHIFT) + 3, order
        assert run_schedule.atomics == [1, 1, 1], order


def test_a_word_left_for_another_workspace_is_foreign():
    # a word another workspace's launches left clean, (other epoch, 0), seen by this epoch: installed anew
    word, counts = run_schedule((EPOCH + 1) << SHIFT, EPOCH, 2, [0, 1, 0, 1])
    assert sorted(counts) == [1, 2] and word == (EPOCH << SHIFT) + 2
    assert sum(run_schedule.atomics) > 2


def test_trusting_any_word_fails_on_a_foreign_word():
    # the planted variant counts from whatever the word held: right only when its count field happens to be
    # zero, wrong for an interrupted launch's word (count 3) and for garbage
    for initial in INITIAL_WORDS[2:]:
        _, counts = run_schedule(initial, EPOCH, 2, [0, 1], trust_any_word=True)
        assert (sorted(counts) == [1, 2]) == (initial & 0xFFFF == 0), hex(initial)
