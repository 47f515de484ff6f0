"""Pins of the expert-cache policy oracle (oracle/ecache_oracle.c, restating
src/ecache.c) by forms that do not share its code:

* a full-scan LFRU / LRU model.  The reference draws 16 victim candidates
  with x <- 1664525 x + 1013904223 (mod 2^32), slot x mod n_slots.  By the
  Hull-Dobell theorem (c odd, a - 1 divisible by 4) that generator has full
  period modulo every power of two, so for n_slots in {4, 8, 16} any 16
  consecutive draws visit every slot: the sampled choice must equal the
  textbook full-scan minimum.  A flipped comparison, a missing hit count, an
  unpinned last-used or held record fails it;
* known answers for hint / prefetch worked out from ecache.h's contract
  (depth and n_slots / 4 caps, fresh reads counted once, speculative reads
  not misses, demand reads queued ahead of speculative ones);
* invariants over random operation sequences with reads in flight.
"""
import numpy as np
import pytest

REC = 1000


class FullScan:
    """Textbook cache: empty slot first (lowest index), else the unpinned
    slot with the fewest hits, then the oldest use (LFRU), or the oldest use
    (LRU).  Pinned: the record handed out last, and held records."""

    def __init__(self, n_slots, policy):
        self.key = [None] * n_slots
        self.hits = [0] * n_slots
        self.last = [0] * n_slots
        self.policy = policy
        self.clock = 0
        self.last_used = -1
        self.held = set()
        self.n_hits = self.n_misses = self.n_evict = 0

    def _victim(self):
        for i, k in enumerate(self.key):
            if k is None:
                return i
        free = [i for i in range(len(self.key)) if i != self.last_used and i not in self.held]
        if not free:
            return -1
        if self.policy == 1:
            return min(free, key=lambda i: self.last[i])
        return min(free, key=lambda i: (self.hits[i], self.last[i]))

    def get(self, k):
        self.clock += 1
        self.last_used = -1
        if k in self.key:
            i = self.key.index(k)
            self.hits[i] += 1
            self.n_hits += 1
        else:
            i = self._victim()
            if i < 0:
                return -1
            if self.key[i] is not None:
                self.n_evict += 1
            self.key[i], self.hits[i] = k, 1
            self.n_misses += 1
        self.last[i] = self.clock
        self.last_used = i
        return i

    def hold(self, k):
        i = self.get(k)
        if i >= 0:
            self.held.add(i)
            self.last_used = -1
        return i

    def release(self):
        self.held.clear()


@pytest.mark.parametrize("n_slots", [4, 8, 16])
@pytest.mark.parametrize("policy", [0, 1])
def test_sampled_victims_equal_full_scan(orc, n_slots, policy):
    rng = np.random.default_rng(n_slots * 10 + policy)
    m = orc.ECacheModel(n_slots * REC, REC, policy)
    ref = FullScan(n_slots, policy)
    n_keys = n_slots * 3
    for step in range(3000):
        r = rng.random()
        if r < 0.08:
            m.release()
            ref.release()
            continue
        # a skewed key distribution: some records hot, most cold
        e = int(min(rng.zipf(1.3), n_keys)) - 1
        layer = e % 3
        if r < 0.2 and len(ref.held) < n_slots - 2:
            got, want = m.hold(layer, e), ref.hold((layer, e))
        else:
            got, want = m.get(layer, e), ref.get((layer, e))
        assert got == want, step
    st = m.stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (ref.n_hits, ref.n_misses, ref.n_evict)
    assert st["bytes_read"] == st["misses"] * REC


def test_hint_known_answers(orc):
    m = orc.ECacheModel(8 * REC, REC)          # 8 slots: hints capped at 8 / 4 = 2 ids
    m.io_start(4, 8)                           # depth capped at 2
    m.hint(0, [10, 11, 12])
    assert m.stats()["misses"] == 2 and m.stats()["prefetched"] == 2
    m.drain()
    a, b = m.get(0, 10), m.get(0, 11)
    st = m.stats()
    assert (st["hits"], st["misses"]) == (0, 2)             # fresh reads: counted once, as misses
    assert m.get(0, 10) == a and m.stats()["hits"] == 1     # the second get is a hit
    assert m.get(0, 12) not in (a, b) and m.stats()["misses"] == 3   # beyond the cap: a demand miss
    assert m.stats()["bytes_read"] == 3 * REC


def test_hint_depth_releases_one_read_per_get(orc):
    m = orc.ECacheModel(40 * REC, REC)         # 40 slots: up to 10 hinted ids
    m.io_start(2, 2)
    ids = list(range(100, 108))
    m.hint(3, ids)
    assert m.stats()["misses"] == 2                          # the first `depth` reads start now
    m.drain()
    for n, e in enumerate(ids):
        assert m.get(3, e) >= 0
        # each get releases one more read; the last ones find nothing left
        assert m.stats()["misses"] == min(len(ids), n + 3)
        m.drain()
    assert m.stats()["prefetched"] == len(ids) and m.stats()["hits"] == 0


def test_prefetch_is_speculative(orc):
    m = orc.ECacheModel(8 * REC, REC)
    m.io_start(1, 1)
    m.prefetch(5, [1, 2, -1, 2])                             # negative ids skipped, resident ones too
    st = m.stats()
    assert (st["spec_issued"], st["misses"], st["bytes_read"]) == (2, 0, 2 * REC)
    m.drain()
    m.get(5, 1)
    assert m.stats()["hits"] == 1                            # a speculative record is a hit when used


def test_demand_reads_jump_the_queue(orc):
    """A hint queued after a prefetch completes first: a get of the hinted
    record drains only the queue up to it, leaving the speculative read in
    flight (a slot still in flight is pinned)."""
    m = orc.ECacheModel(8 * REC, REC)
    m.io_start(1, 2)
    m.prefetch(1, [7])
    m.hint(0, [3])
    s3 = m.get(0, 3)
    s7 = m.lookup(1, 7)
    assert s3 >= 0 and s7 >= 0
    # fill the other slots with demand misses; the in-flight record survives
    for e in range(20, 30):
        assert m.get(2, e) != s7
    assert m.lookup(1, 7) == s7


def test_failed_reads(orc):
    m = orc.ECacheModel(4 * REC, REC, n_layer=2, n_expert=8)
    assert m.get(0, 9) == -1 and m.get(5, 0) == -1           # out of range: the read fails
    st = m.stats()
    assert st["misses"] == 2 and m.lookup(0, 9) == -1         # counted, slot given back
    m.io_start(1, 1)
    m.hint(0, [9])
    m.drain()
    assert m.get(0, 9) == -1 and m.lookup(0, 9) == -1        # a failed hinted read is dropped at get
    assert orc.ECacheModel(REC - 1, REC).stats()["n_slots"] == 0
    z = orc.ECacheModel(REC - 1, REC)                        # no cache: every get is a miss, no slot
    assert z.get(0, 1) == -1 and z.stats()["misses"] == 1
    assert orc.ECacheModel(2 * REC, REC).stats()["n_slots"] == 4     # at least 4 slots


def test_invariants_random_with_reads_in_flight(orc):
    rng = np.random.default_rng(7)
    for n_slots in (5, 12, 33):
        m = orc.ECacheModel(n_slots * REC, REC, policy=int(rng.integers(2)), n_layer=4, n_expert=64)
        m.io_start(4, 3)
        held = {}
        for _ in range(2000):
            r = rng.random()
            layer, e = int(rng.integers(5)), int(rng.integers(70))
            if r < 0.15:
                m.hint(layer, rng.integers(0, 70, int(rng.integers(1, 12))))
            elif r < 0.25:
                m.prefetch(layer, rng.integers(-2, 70, int(rng.integers(1, 6))))
            elif r < 0.3:
                m.release()
                held.clear()
            elif r < 0.35:
                m.drain()
            elif r < 0.45 and len(held) < n_slots // 2:
                s = m.hold(layer, e)
                if s >= 0:
                    held[s] = (layer, e)
            else:
                m.get(layer, e)
            st = m.stats()
            assert st["bytes_read"] == (st["misses"] + st["spec_issued"]) * REC
            for s, (hl, he) in held.items():
                assert m.lookup(hl, he) == s            # held records are never evicted
        keys = [(l, e) for l in range(5) for e in range(70) if m.lookup(l, e) >= 0]
        slots = [m.lookup(l, e) for l, e in keys]
        assert len(slots) == len(set(slots)) <= n_slots
