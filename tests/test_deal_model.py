"""A host model of how the select kernel deals a level's chain groups to its waves, checked
over random and exhaustive interleavings of the waves (CPU only).

The kernel (tree_select.hip, level_loop): each wave asks an LDS counter for a group index
(atomicAdd(&next, 1), one fetch in flight: the next index is requested when a group starts),
runs the group when the index is below the level's group count nb, and leaves the loop at the
first index >= nb.  The loop is bounded by nb + 1 iterations, and no barrier is inside it.

Properties checked for that deal, with up to 16 waves:
  * every interleaving terminates, each wave after at most nb + 1 fetches;
  * every group index below nb is run exactly once.

The same model is run on a two-pass form of the deal (large groups first, then small groups,
from one counter reset between the passes), the shape of an earlier variant that stalled its
first GPU test and whose source was not kept.  With the reset fenced by a barrier on both sides
it has the same two properties; with the reset done by one wave before the barrier that ends
the first pass, the model finds interleavings where a wave still in the first pass re-takes a
group, and where the second pass starts from a counter that is past its groups and runs none
of them.  A group left unrun leaves its members without a path length (the kernel writes it
only when the member's path ends), which every later kernel of the wave uses as a loop bound.
"""
import itertools
import random

import pytest


class Counter:
    def __init__(self):
        self.v = 0

    def fetch(self):
        old = self.v
        self.v += 1
        return old


def deal_wave(ctr, nb, ran):
    """One wave of the current deal, as a generator: yields before every shared access."""
    yield
    gnext = ctr.fetch()
    fetches = 1
    for _ in range(nb + 1):
        gi = gnext
        if gi >= nb:
            return fetches
        yield
        gnext = ctr.fetch()
        fetches += 1
        yield
        ran.append(gi)
    raise AssertionError("loop bound reached")  # the kernel's bound never ends the loop


def run(waves, order):
    """Steps the waves in the given order of wave indices (skipping finished or blocked waves
    by taking the next runnable one); returns the number of steps taken."""
    live = list(range(len(waves)))
    results = {}
    steps = 0
    blocked = 0
    i = 0
    while live:
        w = order(i, live)
        i += 1
        try:
            r = next(waves[w])
            if r == "blocked":
                blocked += 1
                if blocked > 1000 * len(live):
                    raise AssertionError("deadlock: every live wave waits")
                continue
            blocked = 0
        except StopIteration as e:
            results[w] = e.value
            live.remove(w)
        steps += 1
        if steps > 100_000:
            raise AssertionError("no termination")
    return results


def _random_order(seed):
    rng = random.Random(seed)
    return lambda i, live: rng.choice(live)


@pytest.mark.parametrize("nw,nb", [(16, 0), (16, 1), (16, 15), (16, 16), (16, 17), (16, 200),
                                   (4, 33)])
def test_current_deal_random_interleavings(nw, nb):
    for seed in range(300):
        ctr, ran = Counter(), []
        waves = [deal_wave(ctr, nb, ran) for _ in range(nw)]
        res = run(waves, _random_order(seed))
        assert sorted(ran) == list(range(nb)), seed
        assert all(f <= nb + 1 for f in res.values())
        assert ctr.v == nb + nw  # every wave's last fetch is its one index >= nb


def _all_orders(nw, length):
    """Every sequence of wave choices of the given length (taken modulo the live waves)."""
    for seq in itertools.product(range(nw), repeat=length):
        it = iter(seq)
        yield lambda i, live, it=it: live[next(it, 0) % len(live)]


@pytest.mark.parametrize("nw,nb", [(2, 3), (3, 2), (3, 3)])
def test_current_deal_exhaustive(nw, nb):
    """All interleavings of the first 8 steps (then the lowest live wave) for small sizes."""
    n = 0
    for order in _all_orders(nw, 8):
        ctr, ran = Counter(), []
        waves = [deal_wave(ctr, nb, ran) for _ in range(nw)]
        run(waves, order)
        assert sorted(ran) == list(range(nb))
        n += 1
    assert n == nw ** 8


# ---- the two-pass form --------------------------------------------------------------------
class Barrier:
    def __init__(self, nw):
        self.nw = nw
        self.arrived = 0
        self.gen = 0

    def wait(self):
        """Generator: arrive, then block until every wave has arrived."""
        gen = self.gen
        self.arrived += 1
        if self.arrived == self.nw:
            self.arrived = 0
            self.gen += 1
        while self.gen == gen:
            yield "blocked"


def two_pass_wave(wid, ctr, bar, big, small, ran, fenced):
    """Pass 1 over the large groups [0, big), pass 2 over the small ones [0, small), one
    counter.  fenced: barrier, reset by wave 0, barrier.  Else wave 0 resets the counter as it
    leaves pass 1, before the one barrier between the passes."""
    for pass_no, n in ((1, big), (2, small)):
        yield
        g = ctr.fetch()
        for _ in range(4 * (big + small) + 4):
            if g >= n:
                break
            yield
            ran.append((pass_no, g))
            yield
            g = ctr.fetch()
        if pass_no == 1:
            if fenced:
                yield from bar.wait()
                if wid == 0:
                    ctr.v = 0
                yield from bar.wait()
            else:
                if wid == 0:
                    ctr.v = 0
                yield from bar.wait()
    return 0


def _two_pass_outcomes(fenced, nw=4, big=3, small=5, seeds=400):
    bad = []
    for seed in range(seeds):
        ctr, bar, ran = Counter(), Barrier(nw), []
        waves = [two_pass_wave(w, ctr, bar, big, small, ran, fenced) for w in range(nw)]
        run(waves, _random_order(seed))
        want = sorted([(1, g) for g in range(big)] + [(2, g) for g in range(small)])
        if sorted(ran) != want:
            bad.append((seed, sorted(ran)))
    return bad


def test_two_pass_deal_fenced_reset_is_exact():
    assert _two_pass_outcomes(True) == []


def test_two_pass_deal_unfenced_reset_loses_groups():
    bad = _two_pass_outcomes(False)
    assert bad, "the model should find interleavings that re-take or skip groups"
    want2 = {(2, g) for g in range(5)}
    assert any(not want2 <= set(r) for _, r in bad), "some interleaving skips a pass-2 group"
    assert any(len(r) != len(set(r)) for _, r in bad), "some interleaving re-takes a group"
