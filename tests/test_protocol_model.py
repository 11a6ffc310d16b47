"""A host model of the wide GEMM's stream-K hand-off (``wide_gemm_kernel``'s
``emit`` in ternel_amd/csrc/tq1_engine.hip), run over explicit interleavings.

Per split tile t with contributors q0..q1 (k = q1 - q0 + 1 workgroups):
  - a launch first reads the workspace's error word; if it is set, every
    contributor writes the tile as NaN and touches no counter (refusal);
  - otherwise each contributor adds 1 to ``arrivals[t]``; the one that reads
    k - 1 is the last; the others store their partial and, later, add 1 to
    ``published[t]``;
  - the last polls ``published[t]`` at most ``spin_limit + 1`` times; with
    k - 1 publications it sums the partials in workgroup order, writes the
    tile and returns both counters to zero; otherwise it writes NaN, sets the
    error word (2) and leaves the counters as they are.
The host zeroes the workspace after reading a set error word. The model checks
that no schedule, including publications that land after a give-up, makes a
later launch write a finite wrong tile.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import pytest

NAN = float("nan")


@dataclass
class Workspace:
    arrivals: dict[int, int] = field(default_factory=dict)
    published: dict[int, int] = field(default_factory=dict)
    error: int = 0

    def zero(self) -> None:
        self.arrivals.clear()
        self.published.clear()
        self.error = 0

    def clean(self) -> bool:
        return self.error == 0 and not any(self.arrivals.values()) and not any(self.published.values())


def launch(ws: Workspace, partials: list[float], order: list[int], polls_before: dict[int, int],
           spin_limit: int) -> float | None:
    """One launch of one split tile. ``order`` is the arrival order of the k
    contributors (indices into ``partials``, in workgroup order); a
    contributor's publication lands after ``polls_before[q]`` polls of the
    last arriver (0: before its first poll; larger than the spin limit: after
    it gave up). Returns the tile value written (None if no one wrote it)."""
    k = len(partials)
    if ws.error:  # refusal: every contributor writes NaN, counters untouched
        return NAN
    t = 0
    last = None
    for q in order:
        old = ws.arrivals.get(t, 0)
        ws.arrivals[t] = old + 1
        if old == k - 1:
            if last is not None:
                pytest.fail("two last arrivers")  # cannot happen from a zero counter
            last = q
    if last is None:
        return None
    # the last arriver polls; publications of the others land per the schedule
    late = []
    polls = 0
    got = False
    pending = sorted((polls_before[q], q) for q in range(k) if q != last)
    while polls <= spin_limit:
        while pending and pending[0][0] <= polls:
            ws.published[t] = ws.published.get(t, 0) + 1
            pending.pop(0)
        if ws.published.get(t, 0) >= k - 1:
            got = True
            break
        polls += 1
    late = pending  # publications that land after the last arriver left
    if not got:
        ws.error |= 2
        for _ in late:
            ws.published[t] = ws.published.get(t, 0) + 1
        return NAN
    total = partials[0]
    for v in partials[1:]:
        total += v
    ws.arrivals[t] = 0
    ws.published[t] = 0
    for _ in late:  # (none: the last arriver saw all of them)
        ws.published[t] = ws.published.get(t, 0) + 1
    return total


PARTIALS = [1.5, -2.25, 4.0]
EXACT = sum(PARTIALS)


@pytest.mark.parametrize("order", ([0, 1, 2], [2, 1, 0], [1, 2, 0]))
def test_a_clean_reduction_sums_in_workgroup_order_and_leaves_zeros(order) -> None:
    ws = Workspace()
    assert launch(ws, PARTIALS, order, {0: 0, 1: 3, 2: 7}, spin_limit=10) == EXACT
    assert ws.clean()


def test_a_give_up_writes_nan_sets_the_word_and_a_late_publication_stays_out_of_the_next_call() -> None:
    ws = Workspace()
    # contributor 0 publishes only after the last arriver (2) gave up
    assert math.isnan(launch(ws, PARTIALS, [0, 1, 2], {0: 50, 1: 0, 2: 0}, spin_limit=10))
    assert ws.error == 2
    assert ws.arrivals[0] == 3 and ws.published[0] == 2  # the late one landed after
    # the next launch finds the word set and refuses: NaN, counters untouched
    assert math.isnan(launch(ws, PARTIALS, [0, 1, 2], {0: 0, 1: 0, 2: 0}, spin_limit=10))
    assert ws.arrivals[0] == 3 and ws.published[0] == 2
    # the host reads the word and zeroes the workspace: the launch after is exact
    ws.zero()
    assert launch(ws, PARTIALS, [1, 0, 2], {0: 0, 1: 0, 2: 1}, spin_limit=10) == EXACT
    assert ws.clean()


def test_without_refusal_the_stale_counters_would_break_the_next_reduction() -> None:
    """Why a set word must be refused: from stale counters no contributor (or
    the wrong one) sees itself last, so the tile is not written or is summed
    from unpublished partials."""
    ws = Workspace()
    assert math.isnan(launch(ws, PARTIALS, [0, 1, 2], {0: 50, 1: 0, 2: 0}, spin_limit=10))
    ws.error = 0  # pretend the word was cleared but the counters were not
    assert launch(ws, PARTIALS, [0, 1, 2], {0: 0, 1: 0, 2: 0}, spin_limit=10) is None


@pytest.mark.parametrize("spin_limit", (-1, 0, 3))
def test_every_schedule_writes_the_exact_tile_or_nan(spin_limit) -> None:
    import itertools

    for order in itertools.permutations(range(3)):
        for delays in itertools.product((0, 1, 2, 5), repeat=3):
            ws = Workspace()
            value = launch(ws, PARTIALS, list(order), dict(enumerate(delays)), spin_limit)
            assert value == EXACT or math.isnan(value)
            if math.isnan(value):
                assert ws.error == 2
                ws.zero()
            assert ws.clean()
            assert launch(ws, PARTIALS, list(order), {0: 0, 1: 0, 2: 0}, max(spin_limit, 0)) == EXACT
