"""The HBM expert cache (qmag_ecache_*, the qma_ecache role of
src/ecache.h:95-123) and the paged MoE layer (qmag_moe_ffn_paged_dev, moe_ffn
with the cache on, nn.c:553-571, 677-694) on the GPU.

* Policy: the same operation sequences on the device cache and on the
  oracle's restatement of ecache.c give the same slot for every record and
  the same counters after every operation.  The reference's reader threads
  make in-flight timing part of its decisions; both sides drain the read
  queue before each operation, where the two are defined to agree.
* Records: every record handed out holds, in device memory, exactly the
  gate/up/down slabs the GGUF file stores for that (layer, expert) -- read
  through the GGUF fetch callback on reader threads and on the calling
  thread, and through a Python callback.
* The paged layer equals the resident launch sequence bit for bit (same
  kernels, experts addressed through the cache's slots), across evictions
  and with reader threads on.
"""
import ctypes as C

import numpy as np
import pytest

import gguf_writer as gw
from moe_fixtures import make_host_layer

pytestmark = pytest.mark.gpu


def _write(orc, path, n_layer, N, F, E, K):
    layers = [make_host_layer(orc, seed=300 + i, n_embd=N, n_ff=F, n_expert=E, n_used=K,
                              t_down=(14 if i % 2 == 0 else 12)) for i in range(n_layer)]
    gw.write_gguf(path, gw.qwen35moe_metadata(n_layer, N, E, K, F), gw.moe_model_tensors(layers))
    return layers


def _records(g, n_layer):
    """Expected record bytes per (layer, expert): gate | up | down slabs."""
    out = {}
    for il in range(n_layer):
        slabs = []
        for nm in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
            _, ne, data = g.tensor(f"blk.{il}.{nm}.weight")
            slabs.append(data.reshape(ne[2], -1))
        for e in range(slabs[0].shape[0]):
            out[(il, e)] = np.concatenate([s[e] for s in slabs])
    return out


@pytest.fixture(scope="module")
def small(orc, tmp_path_factory):
    path = tmp_path_factory.mktemp("ec") / "small.gguf"
    _write(orc, path, 2, 256, 256, 64, 4)
    return path


def _check_bytes(qm, recs, key, ptr, rec_bytes):
    want = recs[key]
    got = qm.d2h_ptr(ptr, np.uint8, want.size)
    assert np.array_equal(got, want), key


@pytest.mark.parametrize("n_slots,policy,nthreads", [(12, 0, 3), (9, 1, 1), (33, 0, 8)])
def test_policy_matches_oracle(qm, orc, small, n_slots, policy, nthreads):
    g = qm.Gguf(str(small))
    rec = g.expert_record_bytes()
    recs = _records(g, 2)
    c = qm.ECache(n_slots * rec, rec, policy, fetch=qm.gguf_fetch_fn(), user=g.h)
    m = orc.ECacheModel(n_slots * rec, rec, policy, n_layer=2, n_expert=64)
    c.io_start(nthreads, 3)
    m.io_start(nthreads, 3)
    base = c.slot_ptr(0)
    slot_bytes = c.stats()["slot_bytes"]
    rng = np.random.default_rng(n_slots + policy)
    try:
        for step in range(1500):
            c.drain()
            m.drain()
            r = rng.random()
            layer = int(rng.integers(3))                   # layer 2 does not exist: reads fail
            e = int(min(rng.zipf(1.2), 70)) - 1            # experts >= 64 do not exist
            if r < 0.12:
                ids = rng.integers(0, 66, int(rng.integers(1, 10)))
                c.hint(layer, ids)
                m.hint(layer, ids)
            elif r < 0.2:
                ids = rng.integers(-1, 66, int(rng.integers(1, 5)))
                c.prefetch(layer, ids)
                m.prefetch(layer, ids)
            elif r < 0.25:
                c.release()
                m.release()
            elif r < 0.255:
                c.clear()                                  # everything evicted, counters zeroed
                m.clear()
            else:
                hold = r < 0.35
                p = c.hold(layer, e) if hold else c.get(layer, e)
                s = m.hold(layer, e) if hold else m.get(layer, e)
                got = (p - base) // slot_bytes if p else -1
                assert got == s, (step, layer, e)
                if p:
                    _check_bytes(qm, recs, (layer, e), p, rec)
            assert c.stats()["hits"] == m.stats()["hits"], step
            cs, ms = c.stats(), m.stats()
            for k in orc.ECacheModel.FIELDS:
                assert cs[k] == ms[k], (step, k)
        c.drain()
        m.drain()
        for layer in range(3):
            for e in range(70):
                assert c.slot_of(layer, e) == m.lookup(layer, e), (layer, e)
    finally:
        c.close()
        g.close()


def test_python_fetch_callback(qm, orc, small):
    """Any fetch callback works, including one that reads from elsewhere than
    a GGUF mapping; records fetched by reader threads and by the calling
    thread land intact."""
    g = qm.Gguf(str(small))
    rec = g.expert_record_bytes()
    recs = _records(g, 2)
    calls = []

    def fetch(user, layer, expert, dst):
        calls.append((layer, expert))
        b = recs.get((layer, expert))
        if b is None:
            return -1
        C.memmove(dst, b.ctypes.data, b.size)
        return 0

    c = qm.ECache(6 * rec, rec, fetch=fetch)
    try:
        p = c.get(1, 5)                                   # synchronous read, calling thread
        _check_bytes(qm, recs, (1, 5), p, rec)
        assert c.get(1, 99) == 0 and c.stats()["misses"] == 2
        c.io_start(2, 2)
        c.hint(0, [3, 4, 6, 7])                          # capped at 6 / 4 = 1 id
        c.drain()
        for e in (3, 4):
            _check_bytes(qm, recs, (0, e), c.get(0, e), rec)
        assert (0, 3) in calls and (1, 99) in calls
    finally:
        c.close()
        g.close()


def test_paged_layer_equals_resident(qm, orc, tmp_path):
    """Two qwen35moe-shaped layers (hidden 2048, expert ff 512, 16 experts,
    top-8; Q6_K then Q4_K down) from a GGUF: the paged layer, its experts
    read into a 12-slot cache (evictions on nearly every token), equals the
    resident launch sequence bit for bit, synchronously and with 4 reader
    threads."""
    N, F, E, K = 2048, 512, 16, 8
    path = tmp_path / "m.gguf"
    _write(orc, path, 2, N, F, E, K)
    g = qm.Gguf(str(path))
    dev = [g.upload_moe_layer(il) for il in range(2)]
    paged = []
    for L in dev:                                       # router + shared resident, experts paged
        P_ = qm.MoeLayer()
        C.memmove(C.byref(P_), C.byref(L), C.sizeof(L))
        P_.gate_exps = P_.up_exps = P_.down_exps = None
        paged.append(P_)
    rec = g.expert_record_bytes()
    c = qm.ECache(12 * rec, rec, fetch=qm.gguf_fetch_fn(), user=g.h)
    qm.set_fused(False)
    try:
        for threads in (0, 4):
            if threads:
                c.io_start(threads, 3)
            for it in range(6):
                T = 1 if it % 2 == 0 else 3
                x = orc.fill_normal(900 + 10 * it + threads, T * N, 0.0, 1.0)
                xb = qm.DBuf.from_array(x)
                for il in range(2):
                    want = qm.DBuf(4 * T * N)
                    qm.moe_ffn_dev(dev[il], xb.ptr, want.ptr, T)
                    w_stage = qm.moe_last_stage(E, K, F, T)
                    got = qm.DBuf(4 * T * N)
                    c.moe_ffn_paged(paged[il], il, xb.ptr, got.ptr, T)
                    g_stage = qm.moe_last_stage(E, K, F, T)
                    assert np.array_equal(got.download(np.uint32), want.download(np.uint32)), (threads, it, il)
                    assert np.array_equal(g_stage["sel"], w_stage["sel"])
        st = c.stats()
        assert st["evictions"] > 0 and st["misses"] > 12
    finally:
        qm.set_fused(True)
        c.close()
        for L in dev:
            qm.Gguf.free_moe_layer(L)
        g.close()


def test_paged_layer_vs_oracle(qm, orc, tmp_path):
    """The paged layer (experts through the cache, nn.c:553-571 and 677-694)
    against the oracle's moe_ffn on the bytes the GGUF file holds, stage by
    stage: logits, selection and weights, the shared gate, h of every slot
    and the output (from the device's own h, as the staged check of the
    resident path does), for T = 1 and 3, with evictions between calls and
    with reader threads on.  Two qwen35moe-shaped layers, Q6_K then Q4_K
    down."""
    from test_gpu_moe import check_layer_staged
    N, F, E, K = 2048, 512, 16, 8
    path = tmp_path / "m.gguf"
    host = _write(orc, path, 2, N, F, E, K)
    g = qm.Gguf(str(path))
    dev = [g.upload_moe_layer(il) for il in range(2)]
    paged = []
    for L in dev:
        P_ = qm.MoeLayer()
        C.memmove(C.byref(P_), C.byref(L), C.sizeof(L))
        P_.gate_exps = P_.up_exps = P_.down_exps = None
        paged.append(P_)
    rec = g.expert_record_bytes()
    c = qm.ECache(10 * rec, rec, fetch=qm.gguf_fetch_fn(), user=g.h)

    def run_paged(il):
        def run(x, T):
            xb = qm.DBuf.from_array(x)
            ob = qm.DBuf(4 * T * N)
            c.moe_ffn_paged(paged[il], il, xb.ptr, ob.ptr, T)
            return ob.download(np.float32).reshape(T, N)
        return run

    try:
        for threads in (0, 3):
            if threads:
                c.io_start(threads, 2)
            for il, hl in enumerate(host):
                for T in (1, 3):
                    x = orc.fill_normal(700 + 10 * il + T + threads, T * N, 0.0, 1.0)
                    check_layer_staged(qm, orc, None, hl, x, T, run=run_paged(il))
        assert c.stats()["evictions"] > 0
    finally:
        c.close()
        for L in dev:
            qm.Gguf.free_moe_layer(L)
        g.close()


def test_paged_layer_rejects_small_records(qm, orc, small):
    g = qm.Gguf(str(small))
    L = g.upload_moe_layer(0)
    rec = g.expert_record_bytes()
    c = qm.ECache(8 * (rec - 256), rec - 256, fetch=qm.gguf_fetch_fn(), user=g.h)
    x = qm.DBuf.from_array(np.ones(256, np.float32))
    out = qm.DBuf(4 * 256)
    try:
        with pytest.raises(qm.QmagError, match="cannot hold"):
            c.moe_ffn_paged(L, 0, x.ptr, out.ptr, 1)
    finally:
        c.close()
        qm.Gguf.free_moe_layer(L)
        g.close()


def test_concurrent_gets_of_hinted_records(qm, orc, small):
    """The reference calls qma_ecache_get from its pool workers at once
    (nn.c:677-678); records a hint named are pinned for the generation, so
    their addresses stay valid while other threads get.  Four host threads
    get the hinted records of a layer concurrently (reader threads on) and
    every address holds the file's bytes."""
    import threading
    g = qm.Gguf(str(small))
    rec = g.expert_record_bytes()
    recs = _records(g, 2)
    c = qm.ECache(40 * rec, rec, fetch=qm.gguf_fetch_fn(), user=g.h)
    c.io_start(4, 4)
    errors = []
    try:
        for layer in range(2):
            ids = list(range(3 + layer, 3 + layer + 10))          # 10 = 40 slots / 4
            c.hint(layer, ids)
            got = {}

            def worker(tid):
                try:
                    for e in ids[tid::4] + ids[::-1][tid::4]:
                        p = c.get(layer, e)
                        if not p:
                            errors.append(("null", layer, e))
                        got.setdefault(e, set()).add(p)
                except Exception as exc:                     # surfaced below
                    errors.append(exc)

            th = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
            for t in th:
                t.start()
            for t in th:
                t.join()
            assert not errors, errors
            c.drain()
            for e, ps in got.items():
                assert len(ps) == 1, (layer, e, ps)                # one slot per record
                _check_bytes(qm, recs, (layer, e), next(iter(ps)), rec)
    finally:
        c.close()
        g.close()


def test_waiter_does_not_take_a_reclaimed_slot(qm, orc, small):
    """A get that waits for a record in flight must not return whatever the
    slot holds when it wakes.  The reader thread's fetch of one record fails
    after a delay while a second thread keeps asking for another record; the
    only slot it can claim is the failed one.  Whichever thread takes the lock
    first, the waiter for the failing record gets nothing (never the other
    record's slot), and the other record's bytes are its own."""
    import threading
    import time
    g = qm.Gguf(str(small))
    rec = g.expert_record_bytes()
    recs = _records(g, 2)
    FAIL = 7

    def fetch(user, layer, expert, dst):
        if expert == FAIL:
            time.sleep(0.03)
            return -1
        b = recs.get((layer, expert))
        if b is None:
            return -1
        C.memmove(dst, b.ctypes.data, b.size)
        return 0

    c = qm.ECache(4 * rec, rec, fetch=fetch)               # 4 slots
    c.io_start(1, 1)
    wrong = []
    try:
        for rnd in range(12):
            c.release()
            for e in (0, 1, 2):                             # three slots held: one victim left
                assert c.hold(0, e)
            c.prefetch(0, [FAIL])                           # the reader thread's read fails
            res = {}

            def waiter():
                res["a"] = c.hold(0, FAIL)

            def filler():
                t_end = time.time() + 2.0
                while time.time() < t_end:
                    p = c.hold(0, 20 + rnd)
                    if p:
                        res["c"] = p
                        return

            ta, tc = threading.Thread(target=waiter), threading.Thread(target=filler)
            ta.start()
            time.sleep(0.005)
            tc.start()
            ta.join()
            tc.join()
            if res.get("a"):
                wrong.append((rnd, res["a"]))
            assert res.get("c"), rnd
            _check_bytes(qm, recs, (0, 20 + rnd), res["c"], rec)
            c.drain()
    finally:
        c.close()
        g.close()
    assert not wrong, wrong


def test_gguf_fetch_needs_room_for_the_largest_record(qm, orc, tmp_path):
    """The fetch callback cannot be told the staging size.  The file's layers
    differ in down type (Q6_K, then Q4_K), so its records differ in size; a
    cache sized for the smaller one refuses the GGUF callback instead of
    letting it overrun the staging: no read starts, no slot is claimed."""
    N, F, E, K = 256, 256, 8, 2
    path = tmp_path / "mixed.gguf"
    _write(orc, path, 2, N, F, E, K)
    g = qm.Gguf(str(path))
    big = g.expert_record_bytes()
    small = big - (F * N // 256) * (210 - 144)          # a Q4_K-down layer's record
    c = qm.ECache(8 * small, small, fetch=qm.gguf_fetch_fn(), user=g.h)
    try:
        assert c.get(1, 3) == 0 and c.get(0, 3) == 0
        with pytest.raises(qm.QmagError, match="largest"):
            c.io_start(2, 2)
        st = c.stats()
        assert st["misses"] == 0 and st["bytes_read"] == 0
        assert all(c.slot_of(il, e) == -1 for il in range(2) for e in range(E))
    finally:
        c.close()
    ok = qm.ECache(8 * big, big, fetch=qm.gguf_fetch_fn(), user=g.h)
    try:
        assert ok.get(1, 3) != 0 and ok.get(0, 3) != 0
    finally:
        ok.close()
        g.close()


def test_gguf_fetch_bound_spans_layer_gaps(qm, orc, tmp_path):
    """A file whose expert layers have a gap (blk.0 and blk.2, no blk.1),
    the later layer's record the larger (Q6_K down against Q4_K): a cache
    sized for blk.0's record refuses the GGUF callback, since a fetch of
    blk.2 would overrun its staging."""
    N, F, E, K = 256, 256, 8, 2
    l0 = make_host_layer(orc, seed=150, n_embd=N, n_ff=F, n_expert=E, n_used=K, t_down=12)
    l2 = make_host_layer(orc, seed=152, n_embd=N, n_ff=F, n_expert=E, n_used=K, t_down=14)
    t2 = [(n.replace("blk.0.", "blk.2."), ty, d, b) for n, ty, d, b in gw.moe_model_tensors([l2])]
    path = tmp_path / "gap.gguf"
    gw.write_gguf(path, gw.qwen35moe_metadata(3, N, E, K, F), gw.moe_model_tensors([l0]) + t2)
    g = qm.Gguf(str(path))
    small = 2 * F * (N // 256) * 144 + N * (F // 256) * 144
    assert g.expert_record_bytes() == small + N * (F // 256) * (210 - 144)
    c = qm.ECache(8 * small, small, fetch=qm.gguf_fetch_fn(), user=g.h)
    try:
        assert c.get(2, 1) == 0
        with pytest.raises(qm.QmagError, match="largest"):
            c.io_start(2, 2)
        assert c.stats()["bytes_read"] == 0
    finally:
        c.close()
        g.close()


def test_clear_waits_for_reads_in_flight(qm, orc, small):
    """clear() while reader threads still fetch hinted records (a slow
    callback): it returns only once they have landed, leaves every slot
    empty and the counters zero, and later reads put the right bytes in the
    slots they claim."""
    import time
    g = qm.Gguf(str(small))
    rec = g.expert_record_bytes()
    recs = _records(g, 2)
    started = []

    def slow_fetch(user, layer, expert, dst):
        started.append((layer, expert))
        time.sleep(0.02)
        b = recs.get((layer, expert))
        if b is None:
            return -1
        C.memmove(dst, b.ctypes.data, b.size)
        return 0

    c = qm.ECache(40 * rec, rec, fetch=slow_fetch)
    try:
        c.io_start(4, 8)
        c.hint(0, list(range(10)))                       # 8 reads start at once
        c.prefetch(1, [20, 21, 22])
        c.clear()
        assert len(started) >= 8
        st = c.stats()
        assert (st["hits"], st["misses"], st["bytes_read"], st["prefetched"], st["spec_issued"]) == (0, 0, 0, 0, 0)
        assert all(c.slot_of(il, e) == -1 for il in range(2) for e in range(64))
        for e in (3, 30, 5):
            p = c.get(0, e)
            _check_bytes(qm, recs, (0, e), p, rec)
        assert c.stats()["misses"] == 3
    finally:
        c.close()
        g.close()
