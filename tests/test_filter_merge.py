"""The filtered search's merge of the walkers' two least keys into a list's pair (trench-gguf_amd/csrc/filter.cuh,
coop_filter's flush): each walker offers its least to the first slot with a returning atomic min, then the second
least of {the value it got back, its least, its second least} to the second slot. The flush issues the first slots'
atomics of all its trials before the second slots' (a trial outside the walker's list offers ~0u to both), so the
atomics of different walkers interleave in any order. Run here over random interleavings: the slots must end holding
the two least keys of all walkers, as a serial sort gives them, and the walker's own update must keep its two least."""
import numpy as np

NONE = 0xFFFFFFFF


def med3(a, b, c):
    return sorted((a, b, c))[1]


def walker_ops(r1, r2):
    """one walker's flush of one trial as (slot, value) atomic-min requests, each receiving the slot's old value"""
    o = yield (0, r1)
    yield (1, med3(o, r1, r2))


def merge(walkers, rng):
    slots = [NONE, NONE]
    gens = [walker_ops(*w) for w in walkers]
    pending = {i: next(g) for i, g in enumerate(gens)}
    while pending:
        i = int(rng.choice(sorted(pending)))
        slot, v = pending[i]
        old = slots[slot]
        slots[slot] = min(old, v)
        try:
            pending[i] = gens[i].send(old)
        except StopIteration:
            del pending[i]
    return slots


def test_two_least_survive_every_interleaving():
    rng = np.random.default_rng(7)
    for trial in range(4000):
        nw = int(rng.integers(1, 9))
        keys = rng.integers(0, 40, size=int(rng.integers(1, 3 * nw + 1))).tolist()    # ties included
        owner = rng.integers(0, nw, size=len(keys))
        walkers = []
        for w in range(nw):
            mine = sorted(k for k, o in zip(keys, owner) if o == w)[:2]
            walkers.append(tuple(mine + [NONE] * (2 - len(mine))))
        walkers += [(NONE, NONE)] * int(rng.integers(0, 3))       # walkers offering ~0u (trials outside their list)
        want = (sorted(keys) + [NONE] * 2)[:2]
        got = merge(walkers, rng)
        assert got == want, (trial, walkers, got, want)


def test_walker_update_keeps_its_two_least():
    """the walk's per-candidate update: r2 = med3(r1, r2, k), r1 = min(r1, k)"""
    rng = np.random.default_rng(8)
    for _ in range(2000):
        ks = rng.integers(0, 30, size=int(rng.integers(1, 12))).tolist()
        r1 = r2 = NONE
        for k in ks:
            r2 = med3(r1, r2, k)
            r1 = min(r1, k)
        assert [r1, r2] == (sorted(ks) + [NONE] * 2)[:2]
