"""Device sampling (qmag_sampler_candidates_dev / qmag_sampler_sample_dev,
the sampler_candidates + sampler_pick pair of src/sampler.c:36-134 as
agent.c:935-955 calls it) against the oracle's restatement on the same
logits and sampler state.

Bar: candidates bit-exact (ids and values) when the logits are distinct; with
exact ties the values are still bit-exact and the device orders equal values
by ascending id, where the reference's order among them follows its heap
(checked as a set).  Picks, seeds and token histories equal step for step
over generation-length sequences (the pick's expf is the correctly rounded
one on both sides; a differing last bit could move a pick only if the draw
fell within ~1e-7 of a cumulative boundary)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V = 151936                       # the Qwen3.5 vocabulary (LM-head rows)


def _state(qm, orc, **kw):
    return qm.Sampler.init(**kw), orc.make_sampler(**kw)


def _check_candidates(qm, orc, logits, kw, max_k):
    sd, so = _state(qm, orc, **kw)
    d = qm.DBuf.from_array(logits)
    gi, gv = qm.sampler_candidates_dev(d.ptr, logits.size, sd, max_k)
    oi, ov = orc.sampler_candidates(logits, so, max_k)
    assert gi.size == oi.size
    # values equal as the reference compares them (-0 == +0; without zeros
    # this is bit equality), and every returned value is bit for bit its
    # id's scaled logit, the sign of a zero included
    assert np.array_equal(gv, ov)
    sc = _scaled(orc, logits, kw)
    assert np.array_equal(gv.view(np.uint32), sc[gi].view(np.uint32))
    if np.unique(ov).size == ov.size and (ov.size == 0 or np.count_nonzero(_scaled(orc, logits, kw) == ov[-1]) == 1):
        assert np.array_equal(gi, oi)
    else:
        for v in np.unique(ov):
            assert set(gi[gv == v]) <= set(np.flatnonzero(_scaled(orc, logits, kw) == v))
            assert set(oi[ov == v]) <= set(np.flatnonzero(_scaled(orc, logits, kw) == v))
    # the device's rule among equal values: ascending id
    for v in np.unique(gv):
        ids = gi[gv == v]
        assert list(ids) == sorted(ids)
    return gi, gv


def _scaled(orc, logits, kw):
    """The logits after the penalty and the temperature (sampler.c:47-58),
    used only to find which vocabulary positions share a candidate's value."""
    l = logits.astype(np.float32).copy()
    rp = np.float32(kw.get("repeat_penalty", 1.0))
    if rp != 1:
        for t in list(kw.get("last", ()))[:64]:
            if 0 <= t < l.size:
                l[t] = l[t] * rp if l[t] < 0 else l[t] / rp
    temp = np.float32(kw.get("temp", 0.7))
    if temp > 0:
        l = l / temp
    return l


@pytest.mark.parametrize("temp,top_k,max_k,rp", [(1.0, 20, 40, 1.1), (0.7, 40, 40, 1.0), (0.0, 5, 40, 1.3),
                                                 (1.0, 64, 64, 1.0), (1.0, 0, 40, 1.0), (1.3, 300, 64, 1.1)])
def test_candidates_vs_oracle(qm, orc, temp, top_k, max_k, rp):
    rng = np.random.default_rng(1000 + top_k)
    logits = (rng.standard_normal(V) * 3).astype(np.float32)
    top = np.argsort(-logits)[:8]
    # history: repeats, ids in the first and last chunk, the current top
    # ids, and ids out of range (skipped)
    last = list(rng.integers(0, V, 30)) + [5, 5, 5, V - 1, V - 1, -1, V + 3] + [int(t) for t in top]
    logits[5] = -2.0
    logits[V - 1] = 9.5
    kw = dict(temp=temp, top_k=top_k, repeat_penalty=rp, last=last)
    gi, _ = _check_candidates(qm, orc, logits, kw, max_k)
    assert gi.size == min(max(top_k, 1), max_k)


@pytest.mark.parametrize("n", [1, 3, 63, 64, 1000, 1024, 4095, 4097, 8191, 248320, 128 * 4096])
def test_candidates_vocab_edges(qm, orc, n):
    """Ragged vocabularies: k clamps to n_vocab (sampler.c:63-66), the last
    chunk is partial, the engine's own vocabulary (N_VOCAB, qma.h:33: 60 full
    chunks and one of 2,560), the largest vocabulary the device merge takes."""
    rng = np.random.default_rng(n)
    logits = rng.standard_normal(n).astype(np.float32)
    for top_k, max_k in ((40, 40), (64, 64), (1, 40)):
        gi, _ = _check_candidates(qm, orc, logits, dict(temp=0.8, top_k=top_k, repeat_penalty=1.0), max_k)
        assert gi.size == min(top_k, max_k, n)


def test_candidates_ties(qm, orc):
    """Logits on a coarse grid (thousands of exact ties): the values match
    bit for bit, the device takes the lowest ids of the boundary value."""
    rng = np.random.default_rng(3)
    logits = np.round(rng.standard_normal(V) * 4).astype(np.float32)
    gi, gv = _check_candidates(qm, orc, logits, dict(temp=0.0, top_k=40, repeat_penalty=1.0), 40)
    boundary = gv[-1]
    assert list(gi[gv == boundary]) == list(np.flatnonzero(logits == boundary)[:np.count_nonzero(gv == boundary)])


@pytest.mark.parametrize("temp", [1.0, 0.7, 0.0])
def test_candidates_signed_zero_boundary(qm, orc, temp):
    """The k-th value is zero, held by interleaved +0 and -0 logits: the
    reference's comparisons treat them as one value, so the device orders
    them by ascending id alone, and reports each one with its own sign."""
    rng = np.random.default_rng(17)
    n = 5000
    logits = -np.abs(rng.standard_normal(n)).astype(np.float32) - 1.0
    logits[rng.choice(n, 10, replace=False)] = 4.0 + rng.random(10).astype(np.float32)
    zeros = rng.choice(n, 200, replace=False)
    logits[zeros] = np.where(np.arange(200) % 3 == 0, np.float32(-0.0), np.float32(0.0))
    gi, gv = _check_candidates(qm, orc, logits, dict(temp=temp, top_k=40, repeat_penalty=1.0), 40)
    z = gi[gv == 0]
    assert z.size == 40 - np.count_nonzero(logits > 0)
    assert list(z) == list(np.flatnonzero(logits == 0)[:z.size])
    assert np.any(np.signbit(gv[gv == 0])) and not np.all(np.signbit(gv[gv == 0]))


def test_candidates_concentrated_chunk(qm, orc):
    """The large logits all on 16 threads of one chunk (ids t + 256m, t < 16):
    the k-th largest of the threads' maxima then lies among the small values,
    more than 128 keys reach that bound, and the exact radix selection takes
    over -- in the chunk and in the merge."""
    rng = np.random.default_rng(11)
    logits = rng.standard_normal(V).astype(np.float32)
    ids = (np.arange(16)[:, None] + 256 * np.arange(16)[None, :]).ravel() + 4096 * 7
    logits[ids] = (5.0 + rng.standard_normal(ids.size)).astype(np.float32)
    for top_k in (64, 40, 8):
        gi, _ = _check_candidates(qm, orc, logits, dict(temp=1.0, top_k=top_k, repeat_penalty=1.0), 64)
        assert set(gi.tolist()) <= set(ids.tolist())


def test_candidates_rejects(qm):
    s = qm.Sampler.init(top_k=40)
    d = qm.DBuf.from_array(np.zeros(128 * 4096 + 1, np.float32))
    for n, mk in ((128 * 4096 + 1, 40), (1000, 0), (1000, 65), (0, 40)):
        with pytest.raises(qm.QmagError, match="sampler"):
            qm.sampler_candidates_dev(d.ptr, n, s, mk)


@pytest.mark.parametrize("temp,top_k,top_p,rp", [(1.0, 20, 0.95, 1.1), (0.7, 40, 0.9, 1.0), (1.5, 64, 1.0, 1.3),
                                                 (0.3, 20, 0.1, 1.1), (0.0, 20, 0.95, 1.1)])
def test_sample_sequence_vs_oracle(qm, orc, temp, top_k, top_p, rp):
    """A 200-token generation: each step fresh logits (with the sampled
    tokens' logits raised, so the penalty matters), the device pair against
    the oracle pair; tokens, seeds and histories equal at every step."""
    rng = np.random.default_rng(int(temp * 10) + top_k)
    kw = dict(seed=12345 + top_k, temp=temp, top_k=top_k, top_p=top_p, repeat_penalty=rp)
    sd, so = _state(qm, orc, **kw)
    max_k = 64 if top_k > 40 else 40
    d = qm.DBuf(4 * V)
    for step in range(200):
        logits = (rng.standard_normal(V) * 2.5).astype(np.float32)
        for t in list(so.last_tokens)[:so.n_last]:
            logits[t] += 4.0
        d.upload(logits)
        gt = qm.sampler_sample_dev(d.ptr, V, sd, max_k, top_p)
        oi, ov = orc.sampler_candidates(logits, so, max_k)
        ot = orc.sampler_pick(so, oi, ov, top_p)
        assert gt == ot, step
        assert sd.seed == so.seed and sd.n_last == so.n_last, step
        assert list(sd.last_tokens)[:sd.n_last] == list(so.last_tokens)[:so.n_last], step
    if temp > 0:
        assert sd.n_last == 64                  # the history window filled and slid


def test_sample_all_masked(qm, orc):
    """Every candidate at or below -1e29 after the temperature: no draw, the
    first candidate (the device's lowest id among the equal values), the
    state untouched -- the all-masked answer of sampler_pick."""
    sd = qm.Sampler.init(seed=9, temp=0.7, top_k=20)
    d = qm.DBuf.from_array(np.full(5000, -1e30, np.float32))
    assert qm.sampler_sample_dev(d.ptr, 5000, sd, 40, 0.95) == 0
    assert sd.seed == 9 and sd.n_last == 0


@pytest.mark.parametrize("case", ["partly_masked", "one_inf", "masked_and_inf"])
def test_sample_edge_candidates_vs_oracle(qm, orc, case):
    """Candidate lists the pick's per-lane sums must treat as the reference's
    running sums do: fewer live logits than top_k (the masked ones, -1e30,
    fill the list's tail and are skipped), and a +Inf logit (its softmax term
    is NaN, so every probability is NaN: no cut, the pick falls to the last
    live candidate).  Tokens, seeds and histories equal the oracle's over a
    short sequence."""
    rng = np.random.default_rng({"partly_masked": 5, "one_inf": 6, "masked_and_inf": 7}[case])
    kw = dict(seed=777, temp=0.9, top_k=20, top_p=0.9, repeat_penalty=1.0)
    sd, so = _state(qm, orc, **kw)
    d = qm.DBuf(4 * V)
    for step in range(12):
        logits = (rng.standard_normal(V) * 2.0).astype(np.float32)
        if case != "one_inf":
            live = rng.choice(V, 11, replace=False)
            masked = np.full(V, -1e30, np.float32)
            masked[live] = logits[live]
            logits = masked
        if case != "partly_masked":
            logits[rng.integers(V)] = np.inf
        d.upload(logits)
        gt = qm.sampler_sample_dev(d.ptr, V, sd, 40, 0.9)
        oi, ov = orc.sampler_candidates(logits, so, 40)
        ot = orc.sampler_pick(so, oi, ov, 0.9)
        assert gt == ot, step
        assert sd.seed == so.seed and sd.n_last == so.n_last, step
        assert list(sd.last_tokens)[:sd.n_last] == list(so.last_tokens)[:so.n_last], step


def test_sample_after_recovery_reports_stale_logits(qm, orc):
    """A persistent decode launch queued before the sampler finds its abort
    word set (the test hook, as after an expired wait).  The sampler's status
    check re-runs that call, but the logits were meant to come from its
    output, so the sampler samples nothing, leaves the state unchanged and
    returns QMAG_ERR_REPLAYED; called again, it samples as the oracle does."""
    rl = qm.ResidentLayer(seed=3, layer=0)
    x = qm.DBuf.from_array(orc.fill_normal(12, 2048, 0.0, 1.0))
    out = qm.DBuf(4 * 2048)
    logits = (np.random.default_rng(41).standard_normal(5000) * 2.5).astype(np.float32)
    d = qm.DBuf.from_array(logits)
    kw = dict(seed=777, temp=0.8, top_k=20, top_p=0.9, repeat_penalty=1.0)
    sd, so = _state(qm, orc, **kw)
    r0 = qm.fused_recoveries()
    qm.arm_test_abort(1)
    qm.moe_ffn_dev(rl.c, x.ptr, out.ptr, 1)
    with pytest.raises(qm.QmagError, match="status -5"):
        qm.sampler_sample_dev(d.ptr, logits.size, sd, 40, 0.9)
    assert qm.fused_recoveries() == r0 + 1
    assert sd.seed == 777 and sd.n_last == 0
    gt = qm.sampler_sample_dev(d.ptr, logits.size, sd, 40, 0.9)
    oi, ov = orc.sampler_candidates(logits, so, 40)
    assert gt == orc.sampler_pick(so, oi, ov, 0.9)
    assert sd.seed == so.seed and sd.n_last == so.n_last == 1
    rl.close()


def test_sampling_random_parameters_vs_oracle(qm, orc):
    """Seeded random sampler states and logits: vocabularies of 1-20,000
    (and a few up to the 151,936 of the LM head), temperatures 0-1.7, top_k
    0-100 against max_k 1-64, top_p 0.05-1, repeat penalties below and above
    1 over histories with repeats and ids out of range; logits normal, tied
    (rounded, with +0 and -0), largely masked at -1e30, partly -inf, or
    wide.  Candidates as _check_candidates requires; when the candidate
    values are all distinct, the pick, seed and history equal the oracle's
    over four steps."""
    rng = np.random.default_rng(2025)
    for case in range(120):
        n = int(rng.integers(1, 200)) if case % 3 == 0 else int(rng.integers(200, 20000))
        if case % 40 == 39:
            n = V
        kind = str(rng.choice(["normal", "ties", "masked", "neginf", "wide"]))
        kw = dict(seed=int(rng.integers(1, 1 << 62)), temp=float(rng.choice([0.0, 0.2, 0.7, 1.0, 1.7])),
                  top_k=int(rng.choice([0, 1, 5, 20, 40, 64, 100])), top_p=float(rng.choice([0.05, 0.5, 0.9, 1.0])),
                  repeat_penalty=float(rng.choice([1.0, 1.1, 1.3, 0.8])))
        max_k = int(rng.choice([1, 8, 20, 40, 64]))
        last = [int(v) for v in rng.integers(-5, n + 5, int(rng.integers(0, 81)))]
        sd, so = _state(qm, orc, last=last, **kw)
        d = qm.DBuf(4 * n)
        for step in range(4):
            if kind == "normal":
                lg = (rng.standard_normal(n) * 2.5).astype(np.float32)
            elif kind == "ties":
                lg = np.round(rng.standard_normal(n) * 3).astype(np.float32)
            elif kind == "masked":
                lg = (rng.standard_normal(n) * 2).astype(np.float32)
                lg[rng.random(n) < 0.95] = -1e30
            elif kind == "neginf":
                lg = (rng.standard_normal(n) * 2).astype(np.float32)
                lg[rng.random(n) < 0.3] = -np.inf
            else:
                lg = (rng.standard_normal(n) * 200).astype(np.float32)
            d.upload(lg)
            gi, gv = qm.sampler_candidates_dev(d.ptr, n, sd, max_k)
            oi, ov = orc.sampler_candidates(lg, so, max_k)
            kwc = dict(kw, last=list(so.last_tokens)[:so.n_last])
            assert gi.size == oi.size and np.array_equal(gv, ov), (case, step)
            sc = _scaled(orc, lg, kwc)
            assert np.array_equal(gv.view(np.uint32), sc[gi].view(np.uint32)), (case, step)
            if np.unique(ov).size == ov.size and (ov.size == 0 or np.count_nonzero(sc == ov[-1]) == 1):
                assert np.array_equal(gi, oi), (case, step)
            if np.unique(ov).size != ov.size:
                continue                 # the pick among equal values follows each side's order
            gt = qm.sampler_sample_dev(d.ptr, n, sd, max_k, kw["top_p"])
            ot = orc.sampler_pick(so, oi, ov, kw["top_p"])
            assert gt == ot and sd.seed == so.seed and sd.n_last == so.n_last, (case, step)
            assert list(sd.last_tokens)[:sd.n_last] == list(so.last_tokens)[:so.n_last], (case, step)
        d.close()
