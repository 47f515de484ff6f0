"""Pins of the oracle's sampler (sampler.c:36-134, restated in
oracle/qma_oracle.c) against forms written from the definition:

* candidates: penalty per occurrence in last_tokens (negative logits
  multiplied, others divided), fp32 division by the temperature, then the k
  largest values in descending order -- numpy's stable argsort on distinct
  values;
* the pick: greedy and all-masked known answers, the top-p cut, and the
  draw's distribution against the softmax probabilities (chi-square), which
  a wrong normalisation, cut or cumulative comparison would fail.

The draw itself is xorshift64* (sampler.c:9-14, shifts 12/25/27, multiplier
0x2545F4914F6CDD1D): it is pinned here only through the uniformity of its
53-bit outputs; the exact stream is checked GPU against oracle."""
import numpy as np
import pytest


def _numpy_candidates(logits, temp, top_k, max_k, rp, last):
    l = logits.astype(np.float32).copy()
    for t in last:                                   # every occurrence, in order
        if 0 <= t < l.size:
            l[t] = l[t] * np.float32(rp) if l[t] < 0 else l[t] / np.float32(rp)
    if temp > 0:
        l = (l / np.float32(temp)).astype(np.float32)
    k = min(max(top_k, 1), l.size, max_k)
    order = np.argsort(-l.astype(np.float64), kind="stable")[:k]
    return order.astype(np.int32), l[order]


@pytest.mark.parametrize("temp,top_k,max_k,rp", [(0.7, 20, 40, 1.0), (1.3, 40, 40, 1.1), (0.0, 5, 40, 1.0),
                                                 (0.5, 64, 40, 1.3), (1.0, 0, 40, 1.0), (1.0, 300, 64, 1.0)])
def test_candidates_vs_numpy(orc, temp, top_k, max_k, rp):
    rng = np.random.default_rng(top_k + 7)
    logits = (rng.standard_normal(151936) * 3).astype(np.float32)
    last = list(rng.integers(0, 151936, 30)) + [5, 5, 5, -1, 151936 + 3]
    logits[5] = -2.0
    s = orc.make_sampler(temp=temp, top_k=top_k, repeat_penalty=rp, last=last)
    ids, lgs = orc.sampler_candidates(logits, s, max_k)
    want_ids, want_lgs = _numpy_candidates(logits, temp, top_k, max_k, rp, last[:64])
    assert list(ids) == list(want_ids)
    assert np.array_equal(lgs.view(np.uint32), want_lgs.view(np.uint32))


def test_penalty_known_answers(orc):
    """-2 penalised twice by 1.5 is -4.5; 3 penalised once is 2."""
    logits = np.full(10, -10.0, np.float32)
    logits[1], logits[2] = -2.0, 3.0
    s = orc.make_sampler(temp=0.0, top_k=2, repeat_penalty=1.5, last=[1, 2, 1])
    ids, lgs = orc.sampler_candidates(logits, s, 40)
    assert list(ids) == [2, 1] and list(lgs) == [2.0, -4.5]


def test_pick_known_answers(orc):
    ids = np.array([7, 3, 9], np.int32)
    s = orc.make_sampler(temp=0.0, seed=5)
    assert orc.sampler_pick(s, ids, [-1e30, 1.0, 2.0], 0.9) == 3      # greedy: first live
    assert s.seed == 5 and s.n_last == 0                              # no draw, no history
    s = orc.make_sampler(temp=1.0, seed=5)
    assert orc.sampler_pick(s, ids, [-1e30, -1e30, -1e30], 0.9) == 7  # all masked: the first
    assert s.seed == 5
    for seed in range(1, 40):                                         # top_p 0: only the first live
        s = orc.make_sampler(temp=1.0, seed=seed)
        assert orc.sampler_pick(s, ids, [-1e30, 1.0, 5.0], 0.0) == 3
        assert s.n_last == 1 and s.last_tokens[0] == 3 and s.seed != seed


def test_pick_distribution_matches_softmax(orc):
    """Draws over fixed candidates follow the softmax of the live ones up to
    the smallest prefix whose mass reaches top_p; the probabilities are not
    renormalised after that cut, so the draws beyond the kept mass fall to
    the last kept candidate (sampler.c:121-131)."""
    lg = np.array([2.0, 1.5, -1e30, 1.0, 0.2, -0.5], np.float32)
    ids = np.arange(6, dtype=np.int32)
    live = lg > -1e29
    p = np.where(live, np.exp(lg.astype(np.float64) - 2.0), 0.0)
    p /= p.sum()
    top_p = 0.85
    cut = np.searchsorted(np.cumsum(p), top_p) + 1        # first index where the mass reaches top_p
    s = orc.make_sampler(temp=1.0, seed=12345)
    n = 60000
    counts = np.zeros(6)
    for _ in range(n):
        counts[orc.sampler_pick(s, ids, lg, top_p)] += 1
        s.n_last = 0
    assert counts[cut:].sum() == 0 and counts[2] == 0
    q = p[:cut].copy()
    q[cut - 1] += 1.0 - q.sum()                          # the leftover mass
    exp = q * n
    keep = exp > 0
    chi2 = float(np.sum((counts[:cut][keep] - exp[keep]) ** 2 / exp[keep]))
    assert chi2 < 20.0, (counts, exp)


def test_draw_is_uniform(orc):
    """(r >> 11) / 2^53 of xorshift64* is uniform on [0, 1): seen through the
    pick over 10 equal candidates."""
    s = orc.make_sampler(temp=1.0, seed=99)
    ids = np.arange(10, dtype=np.int32)
    lg = np.zeros(10, np.float32)
    c = np.zeros(10)
    for _ in range(50000):
        c[orc.sampler_pick(s, ids, lg, 1.0)] += 1
        s.n_last = 0
    chi2 = float(np.sum((c - 5000) ** 2 / 5000))
    assert chi2 < 30.0, c


M64 = (1 << 64) - 1


def _xorshift64star(state, shifts=(12, 25, 27), mult=0x2545F4914F6CDD1D):
    """One step of xorshift64* as published (S. Vigna, "An experimental
    exploration of Marsaglia's xorshift generators, scrambled", ACM TOMS 42(4),
    2016): x ^= x >> 12; x ^= x << 25; x ^= x >> 27; output x * M mod 2^64.
    Written here from that description, not from the oracle; `shifts` and
    `mult` let the test plant the plausible mistakes below."""
    a, b, c = shifts
    x = state
    x ^= x >> a
    x = (x ^ (x << b)) & M64
    x ^= x >> c
    return x, (x * mult) & M64


def _kat(seed, steps, **kw):
    """States after each step and the pick each draw makes over 1024 equal
    candidates: rv = float32((r >> 11) / 2^53) and the cumulative sums k/1024
    are exact in float32, so the pick is floor(rv * 1024)."""
    states, picks, x = [], [], seed
    for _ in range(steps):
        x, r = _xorshift64star(x, **kw)
        rv = np.float32((r >> 11) * (1.0 / 9007199254740992.0))
        states.append(x)
        picks.append(int(np.floor(np.float64(rv) * 1024)))
    return states, picks


@pytest.mark.parametrize("seed", [1, 12345, 0x9E3779B97F4A7C15, 0xDEADBEEFCAFEF00D])
def test_rng_known_answers(orc, seed):
    """The oracle's draw (orc_rng_next, sampler.c:9-14, and the (r >> 11) / 2^53
    uniform of sampler.c:118) against xorshift64* from its publication: the
    state after every draw and every pick over 1024 equal candidates agree for
    32 draws.  The plausible mistakes -- the 25/27 shifts swapped, a left shift
    first, the multiplier's last digit changed, the uniform taken from r >> 12
    -- each give other states or picks, so this check tells them apart."""
    steps = 32
    s = orc.make_sampler(temp=1.0, seed=seed)
    ids = np.arange(1024, dtype=np.int32)
    got_states, got_picks = [], []
    for _ in range(steps):
        got_picks.append(orc.sampler_pick(s, ids, np.zeros(1024, np.float32), 1.0))
        got_states.append(int(s.seed))
        s.n_last = 0
    want_states, want_picks = _kat(seed, steps)
    assert got_states == want_states
    assert got_picks == want_picks
    for wrong in (dict(shifts=(12, 27, 25)), dict(shifts=(25, 12, 27)), dict(mult=0x2545F4914F6CDD1C)):
        ws, wp = _kat(seed, steps, **wrong)
        assert ws != got_states or wp != got_picks, wrong
    # the uniform from r >> 12 instead of r >> 11 halves rv: other picks
    x, wrong_picks = seed, []
    for _ in range(steps):
        x, r = _xorshift64star(x)
        wrong_picks.append(int(np.floor(np.float64(np.float32((r >> 12) * (1.0 / 9007199254740992.0))) * 1024)))
    assert wrong_picks != got_picks
