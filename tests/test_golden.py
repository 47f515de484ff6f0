"""Committed golden fixtures (tests/golden/, written by make_golden.py from the
C oracle): the oracle must still reproduce them bit for bit, closed-form
known answers inside them are checked directly, and the HIP path is held
to them (Q8_K bit-exact; fp32 within 1e-4 of max|y|)."""
import hashlib
import os

import numpy as np
import pytest

from conftest import max_rel_err
from moe_fixtures import make_host_layer

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ---------------------------------------------------------------- CPU --

def test_golden_q8k_oracle(orc):
    g = load("q8k_cases.npz")
    xq, xd, xs = orc.q8k_quant(g["x"])
    assert np.array_equal(xq, g["xq"])
    assert np.array_equal(xd.view(np.uint32), g["xd"].view(np.uint32))
    assert np.array_equal(xs, g["xsum"])
    q = g["xq"].reshape(16, 256)
    d = g["xd"]
    # closed forms (q8k.c:34-85): zero block -> d = 1, q = 0
    assert d[0] == 1.0 and not q[0].any()
    # a lone spike maps to +-127 with d = amax / 127
    assert q[1, 7] == 127 and d[1] == np.float32(5.0) / np.float32(127.0)
    assert q[2, 200] == -127
    # d = 1 exactly: .5 ties round away from zero
    assert list(q[3, :8]) == [127, 3, -3, 1, -1, 2, -2, 127]
    # |q| <= 127 and xsum are the 16-lane sums
    assert np.abs(g["xq"].astype(np.int32)).max() <= 127
    assert np.array_equal(g["xq"].astype(np.int64).reshape(-1, 16).sum(axis=1), g["xsum"].astype(np.int64))


def test_golden_dots_oracle(orc):
    import oracle_np as onp
    g = load("dots.npz")
    n = int(g["n"])
    nb = n // 256
    xq, xd, xs = g["xq"], g["xd"], g["xsum"]
    r4, r6 = 144 * nb, 210 * nb
    rows = len(g["dot4"])
    for r in range(rows):
        w4 = g["w4"][r * r4:(r + 1) * r4]
        w6 = g["w6"][r * r6:(r + 1) * r6]
        assert np.float32(orc.q8k_dot(w4, 12, xq, xd, xs, n)) == g["dot4"][r]
        assert np.float32(orc.q8k_dot(w6, 14, xq, xd, xs, n)) == g["dot6"][r]
        # integer sums: the C oracle, the fixture and the independent numpy
        # field extraction agree exactly
        assert np.array_equal(orc.q4k_subsums(w4, xq, n), g["sub4"][r])
        assert np.array_equal(onp.q4k_subsums(w4, xq).reshape(-1), g["sub4"][r].reshape(-1))
        assert np.array_equal(orc.q6k_blocksums(w6, xq, n), g["bs6"][r])
    gu = orc.q8k_gateup(g["w4"][:r4], g["w4"][r4:2 * r4], xq, xd, xs, n)
    assert np.float32(gu[0]) == g["gateup"][0] and np.float32(gu[1]) == g["gateup"][1]
    assert g["gateup"][0] == g["dot4"][0] and g["gateup"][1] == g["dot4"][1]


def _moe_layer(orc, g):
    from make_golden import MOE_SHAPE
    hl = make_host_layer(orc, int(g["seed"]), **MOE_SHAPE)
    for k, a in hl.arrays.items():
        assert hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest() == g["sha_" + k].tobytes(), k
    return hl


def test_golden_moe_oracle(orc):
    import sys
    sys.path.insert(0, GOLD)
    g = load("moe_small.npz")
    hl = _moe_layer(orc, g)
    T = int(g["T"])
    out = orc.moe_ffn(hl, g["x"], T)
    assert np.array_equal(out.view(np.uint32), g["out"].view(np.uint32))
    n = hl.n_embd
    for t in range(T):
        s, w, _ = orc.moe_route(hl, g["x"][t * n:(t + 1) * n])
        assert np.array_equal(s, g["sel"][t])
        assert np.array_equal(w, g["w"][t])


# ---------------------------------------------------------------- GPU --

@pytest.mark.gpu
def test_golden_q8k_gpu(qm):
    g = load("q8k_cases.npz")
    x = g["x"]
    n = 256
    T = len(x) // n
    xb = qm.DBuf.from_array(x)
    xq, xd, xs = qm.DBuf(T * n), qm.DBuf(4 * T), qm.DBuf(2 * T * 16)
    qm.q8k_quant_dev(xb, n, T, xq, xd, xs)
    assert np.array_equal(xq.download(np.int8), g["xq"])
    assert np.array_equal(xd.download(np.float32).view(np.uint32), g["xd"].view(np.uint32))
    assert np.array_equal(xs.download(np.int16), g["xsum"])


@pytest.mark.gpu
@pytest.mark.parametrize("wtype,key,wkey", [(12, "dot4", "w4"), (14, "dot6", "w6")])
def test_golden_dots_gpu(qm, wtype, key, wkey):
    g = load("dots.npz")
    n = int(g["n"])
    rows = len(g[key])
    out = qm.DBuf(4 * rows)
    bufs = [qm.DBuf.from_array(a) for a in (g["xq"], g["xd"], g["xsum"], g[wkey])]
    qm.matmul_q8k_dev(*bufs, n, rows, 1, wtype, out)
    got = out.download(np.float32)
    assert max_rel_err(got, g[key]) <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [True, False])
def test_golden_moe_gpu(qm, orc, fused):
    import sys
    sys.path.insert(0, GOLD)
    g = load("moe_small.npz")
    hl = _moe_layer(orc, g)
    T = int(g["T"])
    rl = qm.ResidentLayer.from_host(hl)
    xb = qm.DBuf.from_array(g["x"])
    ob = qm.DBuf(4 * T * hl.n_embd)
    qm.set_fused(fused)
    try:
        qm.moe_ffn_dev(rl.c, xb.ptr, ob.ptr, T)
        qm.sync()
    finally:
        qm.set_fused(True)
    got = ob.download(np.float32).reshape(T, hl.n_embd)
    assert max_rel_err(got, g["out"].reshape(T, hl.n_embd)) <= TOL
    rl.close()
