"""Independent pins of oracle functions that no other check fixes.

Each oracle result is compared with an fp64 closed form within an analytic
bound on the fp32 rounding of the oracle's own evaluation order, and each
test also shows that a plausible mistake lies outside that bound, so the
bound discriminates.

* orc_moe_shared_gate (nn.c:452-454): sigmoid of sum_i wsh[i] * xq[i] * xd[i/256],
  the shared-expert gate on the dequantised Q8_K input.  The plausible
  mistakes: gating on the fp32 x itself (the fp32 path's form, nn.c:479), or
  on xq without its block scale.
* orc_dot_q4k_f32 / orc_dot_q6k_f32 (quants.c:80-133): dequantise-then-dot
  against sum_j deq(W)_j * x_j.  The plausible mistakes: a dropped min term,
  swapped nibble halves, a Q6_K sub-block scale taken from the wrong group.
"""
import numpy as np
import pytest

import oracle_np as onp

U = 2.0 ** -24          # unit roundoff of fp32


def _rand_q4k(rng, nb):
    """Random-byte Q4_K blocks with finite, moderate fp16 d and dmin."""
    raw = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    d = rng.uniform(1e-4, 1e-2, size=nb).astype(np.float16)
    dm = rng.uniform(1e-4, 1e-2, size=nb).astype(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    raw[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def _rand_q6k(rng, nb):
    raw = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    d = rng.uniform(1e-4, 1e-2, size=nb).astype(np.float16)
    raw[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


# ------------------------------------------------------------ shared gate --

def _sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def _gate_bound(wsh, xq, xd):
    """|computed - exact| for sigmoid(sum_i fl(fl(w_i * q_i) * d_i)) summed
    left to right in fp32: each term carries <= 2 roundings (2u|t_i|), each
    addition one rounding of the running sum (u|S_k|, S_k the exact partial
    sums); the sigmoid is 1/4-Lipschitz, and expf plus the final division
    add a few ulp of a value <= 1."""
    t = wsh.astype(np.float64) * xq.astype(np.float64) * np.repeat(xd.astype(np.float64), 256)
    S = np.cumsum(t)
    pre = U * (2.0 * np.sum(np.abs(t)) + np.sum(np.abs(S))) * 1.01
    return pre / 4.0 + 8 * U, float(S[-1])


def test_shared_gate_vs_fp64(orc):
    n = 2048
    wsh = orc.fill_normal(0x5A, n, 0.0, 0.02)
    outside_x, outside_noscale = 0, 0
    trials = 12
    for t in range(trials):
        x = orc.fill_normal(0x600 + t, n, 0.0, 1.0)
        xq, xd, _ = orc.q8k_quant(x)
        got = orc.moe_shared_gate(wsh, xq, xd, n)
        bound, pre64 = _gate_bound(wsh, xq, xd)
        ref = _sigmoid(pre64)
        assert abs(got - ref) <= bound, (t, got, ref, bound)
        # plausible mistakes lie outside the bound
        gate_x = _sigmoid(float(np.dot(wsh.astype(np.float64), x.astype(np.float64))))
        outside_x += abs(gate_x - ref) > bound
        gate_noscale = _sigmoid(float(np.dot(wsh.astype(np.float64), xq.astype(np.float64))))
        outside_noscale += abs(gate_noscale - ref) > bound
    # gating on fp32 x moves the pre-activation by ~N(0, 4e-3) here against a
    # bound of ~2e-5: it can fall inside by chance only rarely
    assert outside_x >= trials - 1
    assert outside_noscale == trials


def test_shared_gate_known_answers(orc):
    """Zero gate weights give sigmoid(0) = 0.5 exactly; a single nonzero
    weight gives sigmoid(w * q * d) for that element."""
    n = 512
    x = orc.fill_normal(0x61, n, 0.0, 1.0)
    xq, xd, _ = orc.q8k_quant(x)
    assert orc.moe_shared_gate(np.zeros(n, np.float32), xq, xd, n) == 0.5
    wsh = np.zeros(n, np.float32)
    i = 300                      # second 256-block: its own scale xd[1]
    wsh[i] = np.float32(0.75)
    pre = np.float32(np.float32(wsh[i] * np.float32(xq[i])) * xd[i // 256])
    want = np.float32(1.0) / (np.float32(1.0) + np.exp(-pre, dtype=np.float32))
    assert abs(orc.moe_shared_gate(wsh, xq, xd, n) - float(want)) <= 2 * U


# ---------------------------------------------------------- fp32 dots ----

def _q4k_terms(raw, x):
    """Per-element exact products and the term-magnitude bound of
    dot_q4_K_f32 (quants.c:80-105): w = fl(fl(d*sc)*q) - fl(dmin*m) carries
    <= 3 roundings relative to |d*sc*q| + |dmin*m|, times x one more."""
    d, dmin, sc, m, q = onp.q4k_fields(raw)
    sub = np.repeat(np.arange(8), 32)
    a = d[:, None].astype(np.float64) * sc[:, sub] * q
    b = dmin[:, None].astype(np.float64) * m[:, sub]
    xf = x.astype(np.float64).reshape(-1, 256)
    return ((a - b) * xf).reshape(-1), ((np.abs(a) + np.abs(b)) * np.abs(xf)).reshape(-1)


def _q4k_sum_bound(t):
    """Sum of |exact partial sums| in the reference's association: per
    super-block and 64-element group, s1 over the 32 low-nibble terms and s2
    over the 32 high-nibble terms (left to right), then acc += s1 + s2."""
    g = t.reshape(-1, 2, 32)                     # [group][lo/hi][l]
    inner = np.sum(np.abs(np.cumsum(g, axis=2)))
    pair = np.sum(g, axis=2).sum(axis=1)         # s1 + s2 per group
    outer = np.sum(np.abs(pair)) + np.sum(np.abs(np.cumsum(pair)))
    return inner + outer


def _q6k_terms(raw, x):
    d, sc, q = onp.q6k_fields(raw)
    xf = x.astype(np.float64).reshape(-1, 256)
    tt = d[:, None].astype(np.float64) * sc[:, np.arange(256) // 16] * q * xf
    return tt.reshape(-1)


def _q6k_order(nb):
    """Element order of dot_q6_K_f32's single running sum (quants.c:108-133):
    per block, per 128-half, per l < 32: elements l, l+32, l+64, l+96."""
    o = []
    for i in range(nb):
        for h in range(2):
            for l in range(32):
                o += [256 * i + 128 * h + l + 32 * k for k in range(4)]
    return np.array(o)


@pytest.mark.parametrize("nb", [1, 2, 8])
def test_dot_q4k_f32_vs_fp64(orc, nb):
    rng = np.random.default_rng(100 + nb)
    n = 256 * nb
    for _ in range(10):
        raw = _rand_q4k(rng, nb)
        x = rng.standard_normal(n).astype(np.float32)
        got = orc.dot_f32(raw, 12, x, n)
        t, mag = _q4k_terms(raw, x)
        ref = float(np.sum(t))
        bound = U * (4.0 * np.sum(mag) + _q4k_sum_bound(t)) * 1.01
        assert abs(got - ref) <= bound, (got, ref, bound)
        # plausible mistakes: no min term; low/high nibbles swapped
        d, dmin, sc, m, q = onp.q4k_fields(raw)
        sub = np.repeat(np.arange(8), 32)
        no_min = float(np.sum((d[:, None].astype(np.float64) * sc[:, sub] * q).reshape(-1) * x))
        assert abs(no_min - ref) > bound
        qs = q.reshape(-1, 4, 2, 32)[:, :, ::-1, :].reshape(-1, 256)
        swapped = float(np.sum((d[:, None].astype(np.float64) * sc[:, sub] * qs
                                - dmin[:, None].astype(np.float64) * m[:, sub]).reshape(-1) * x))
        assert abs(swapped - ref) > bound


@pytest.mark.parametrize("nb", [1, 2, 8])
def test_dot_q6k_f32_vs_fp64(orc, nb):
    rng = np.random.default_rng(200 + nb)
    n = 256 * nb
    order = _q6k_order(nb)
    for _ in range(10):
        raw = _rand_q6k(rng, nb)
        x = rng.standard_normal(n).astype(np.float32)
        got = orc.dot_f32(raw, 14, x, n)
        t = _q6k_terms(raw, x)
        ref = float(np.sum(t))
        # each term: d*sc, *q, *x: 3 roundings; then one running sum in order
        bound = U * (3.0 * np.sum(np.abs(t)) + np.sum(np.abs(np.cumsum(t[order])))) * 1.01
        assert abs(got - ref) <= bound, (got, ref, bound)
        # plausible mistake: the scale of the neighbouring 16-group
        d, sc, q = onp.q6k_fields(raw)
        wrong = d[:, None].astype(np.float64) * sc[:, (np.arange(256) // 16) ^ 1] * q
        assert abs(float(np.sum(wrong.reshape(-1) * x)) - ref) > bound


def test_dequant_rows_are_the_dot_weights(orc):
    """dequantize_row_* and the fp32 dots share one weight definition: the
    dot of a dequantised row with a one-hot x picks that weight exactly."""
    rng = np.random.default_rng(7)
    for wtype, gen in ((12, _rand_q4k), (14, _rand_q6k)):
        raw = gen(rng, 2)
        w = orc.dequant(raw, wtype, 512)
        for j in (0, 31, 32, 100, 255, 256, 300, 511):
            x = np.zeros(512, np.float32)
            x[j] = 1.0
            assert orc.dot_f32(raw, wtype, x, 512) == w[j]
