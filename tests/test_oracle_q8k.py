"""Pins of the oracle's Q8_K quantizer and int8 dots (q8k.c:34-262).

Known answers from the definition (zero block, spikes, exact .5 ties, the
clamp), the independent numpy restatement (bit-exact), brute-force integer
sums in int64, and fp64 closed forms for the fp32 epilogue."""
import numpy as np
import pytest

import oracle_np as onp


def test_q8k_zero_block(orc):
    xq, xd, xs = orc.q8k_quant(np.zeros(512, np.float32))
    assert np.all(xq == 0) and np.all(xd == 1.0) and np.all(xs == 0)


def test_q8k_spike_and_ties(orc):
    x = np.zeros(256, np.float32)
    x[3] = 127.0                       # amax 127 -> d = 1, inv = 1
    x[10], x[11], x[12], x[13] = 2.5, -3.5, 0.5, -0.5
    x[20], x[21] = 126.5, -126.4999
    xq, xd, xs = orc.q8k_quant(x)
    assert xd[0] == np.float32(1.0)
    assert xq[3] == 127
    assert list(xq[10:14]) == [3, -4, 1, -1]          # half away from zero
    assert list(xq[20:22]) == [127, -126]
    x2 = -x
    xq2, _, _ = orc.q8k_quant(x2)
    assert np.array_equal(xq2, -xq)


def test_q8k_scale_is_ieee_division(orc):
    rng = np.random.default_rng(3)
    for _ in range(50):
        x = rng.standard_normal(256).astype(np.float32) * np.float32(rng.uniform(1e-3, 1e3))
        _, xd, _ = orc.q8k_quant(x)
        amax = np.max(np.abs(x))
        assert xd[0] == np.float32(amax) / np.float32(127.0)


@pytest.mark.parametrize("seed", range(6))
def test_q8k_matches_numpy_restatement(orc, seed):
    rng = np.random.default_rng(100 + seed)
    scale = [1.0, 1e-3, 1e3, 0.02, 1e-20, 3e30][seed]
    x = (rng.standard_normal(256 * 16) * scale).astype(np.float32)
    x[:5] = 0.0
    a = orc.q8k_quant(x)
    b = onp.q8k_quant(x)
    for u, v in zip(a, b):
        assert u.dtype == v.dtype and np.array_equal(u, v)
    assert np.all(np.abs(a[0].astype(int)) <= 127)
    assert np.array_equal(a[2], a[0].astype(np.int64).reshape(-1, 16).sum(axis=1))


def _rand_q4k(rng, nb):
    raw = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    h = (rng.integers(0x2000, 0x3C00, size=(nb, 2))).astype(np.uint16)
    raw[:, 0:4] = h.view(np.uint8).reshape(nb, 4)
    return raw.reshape(-1)


def _rand_q6k(rng, nb):
    raw = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    h = rng.integers(0x2000, 0x3C00, size=nb).astype(np.uint16)
    raw[:, 208:210] = h.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


@pytest.mark.parametrize("nb", [1, 2, 4, 8])
def test_q4k_subsums_bruteforce(orc, nb):
    rng = np.random.default_rng(nb)
    raw = _rand_q4k(rng, nb)
    xq = rng.integers(-127, 128, size=256 * nb).astype(np.int8)
    got = orc.q4k_subsums(raw, xq, 256 * nb)
    # brute force straight from the bytes: element 64g+l <- low nibble of
    # qs[32g+l], element 64g+32+l <- high nibble
    blocks = raw.reshape(nb, 144)
    want = np.zeros(nb * 8, dtype=np.int64)
    for i in range(nb):
        for e in range(256):
            g, r = divmod(e, 64)
            byte = int(blocks[i, 16 + 32 * g + (r % 32)])
            q = (byte & 15) if r < 32 else (byte >> 4)
            want[8 * i + e // 32] += q * int(xq[256 * i + e])
    assert np.array_equal(got.astype(np.int64), want)
    assert np.array_equal(onp.q4k_subsums(raw, xq), want)


@pytest.mark.parametrize("nb", [1, 2, 8])
def test_q6k_blocksums_bruteforce(orc, nb):
    rng = np.random.default_rng(50 + nb)
    raw = _rand_q6k(rng, nb)
    xq = rng.integers(-127, 128, size=256 * nb).astype(np.int8)
    got = orc.q6k_blocksums(raw, xq, 256 * nb)
    blocks = raw.reshape(nb, 210)
    want = np.zeros(nb, dtype=np.int64)
    for i in range(nb):
        ql, qh = blocks[i, :128].astype(int), blocks[i, 128:192].astype(int)
        sc = blocks[i, 192:208].view(np.int8).astype(int)
        for e in range(256):
            n, r = divmod(e, 128)
            Q, l = divmod(r, 32)
            byte = ql[64 * n + (Q & 1) * 32 + l]
            lo = (byte & 15) if Q < 2 else (byte >> 4)
            q = (lo | (((qh[32 * n + l] >> (2 * Q)) & 3) << 4)) - 32
            want[i] += sc[e // 16] * q * int(xq[256 * i + e])
    assert np.array_equal(got.astype(np.int64), want)
    assert np.array_equal(onp.q6k_blocksums(raw, xq), want)


def _epilogue_bound(raw, wtype, xq, xd):
    w = onp.q4k_dequant(raw) if wtype == 12 else onp.q6k_dequant(raw)
    xf = xq.astype(np.float64) * np.repeat(xd.astype(np.float64), 256)
    return np.sum(np.abs(w * xf)) * 2.0 ** -20 + 1e-30


@pytest.mark.parametrize("wtype,nb", [(12, 1), (12, 8), (14, 2), (14, 8)])
def test_q8k_dot_vs_fp64_closed_form(orc, wtype, nb):
    rng = np.random.default_rng(wtype * 10 + nb)
    for _ in range(20):
        raw = _rand_q4k(rng, nb) if wtype == 12 else _rand_q6k(rng, nb)
        x = rng.standard_normal(256 * nb).astype(np.float32)
        xq, xd, xs = orc.q8k_quant(x)
        got = orc.q8k_dot(raw, wtype, xq, xd, xs, 256 * nb)
        ref = onp.q8k_dot_f64(raw, wtype, xq, xd)
        assert abs(got - ref) <= _epilogue_bound(raw, wtype, xq, xd)


def test_q8k_dot_unknown_type_is_zero(orc):
    rng = np.random.default_rng(0)
    raw = _rand_q4k(rng, 1)
    xq, xd, xs = orc.q8k_quant(rng.standard_normal(256).astype(np.float32))
    assert orc.q8k_dot(raw, 0, xq, xd, xs, 256) == 0.0
    assert orc.q8k_dot(raw, 13, xq, xd, xs, 256) == 0.0


def test_gateup_equals_two_dots(orc):
    rng = np.random.default_rng(4)
    g, u = _rand_q4k(rng, 8), _rand_q4k(rng, 8)
    xq, xd, xs = orc.q8k_quant(rng.standard_normal(2048).astype(np.float32))
    go, uo = orc.q8k_gateup(g, u, xq, xd, xs, 2048)
    assert go == orc.q8k_dot(g, 12, xq, xd, xs, 2048)
    assert uo == orc.q8k_dot(u, 12, xq, xd, xs, 2048)


@pytest.mark.parametrize("wtype", [12, 14])
def test_q8k_path_close_to_fp32_path(orc, wtype):
    """The int8 path differs from the fp32 dequant path only by the
    activation quantisation (q8k.c:8-10): within ~1% on N(0,1) inputs."""
    rng = np.random.default_rng(9)
    W = orc.fill_normal(21, 64 * 2048, 0.0, 0.02)
    Wq = orc.quantize(W, wtype)
    rb = len(Wq) // 64
    x = rng.standard_normal(2048).astype(np.float32)
    xq, xd, xs = orc.q8k_quant(x)
    a = np.array([orc.q8k_dot(Wq[r * rb:(r + 1) * rb], wtype, xq, xd, xs, 2048) for r in range(64)])
    b = np.array([orc.dot_f32(Wq[r * rb:(r + 1) * rb], wtype, x, 2048) for r in range(64)])
    assert np.linalg.norm(a - b) / np.linalg.norm(b) < 0.01


def test_matmul_driver_rows(orc):
    """matmul (nn.c:307-345): quantise each token once, one dot per row."""
    rng = np.random.default_rng(5)
    n_in, n_out, T = 512, 96, 3
    for wtype in (12, 14):
        W = orc.quantize(orc.fill_normal(77, n_in * n_out, 0.0, 0.02), wtype)
        x = rng.standard_normal(T * n_in).astype(np.float32)
        for threads in (1, 4):
            orc.set_threads(threads)
            out = orc.matmul_q8k(x, W, n_in, n_out, T, wtype)
            rb = len(W) // n_out
            for t in range(T):
                xq, xd, xs = orc.q8k_quant(x[t * n_in:(t + 1) * n_in])
                want = [orc.q8k_dot(W[r * rb:(r + 1) * rb], wtype, xq, xd, xs, n_in)
                        for r in range(n_out)]
                assert np.array_equal(out[t], np.array(want, dtype=np.float32))
    orc.set_threads(1)


def special_blocks():
    """Blocks of special values, each 256 long: a NaN among finite values,
    all NaN, NaN beside +Inf, +Inf, -Inf, subnormal values (amax/127 still
    subnormal), values so small that amax/127 underflows to 0, tiny normal
    values, near-overflow values, the largest finite values, +0 and -0."""
    rng = np.random.default_rng(5)
    f = np.float32
    out = {}
    for kind in ("nan", "allnan", "nan_inf", "pinf", "ninf", "sub", "underflow", "tiny", "huge", "max",
                 "zero", "negzero"):
        x = rng.standard_normal(256).astype(f)
        if kind == "nan":
            x[17] = np.nan
        elif kind == "allnan":
            x[:] = np.nan
        elif kind == "nan_inf":
            x[3], x[9] = np.inf, np.nan
        elif kind == "pinf":
            x[3] = np.inf
        elif kind == "ninf":
            x[200] = -np.inf
        elif kind == "sub":
            x = (x * f(1e-40)).astype(f)
        elif kind == "underflow":
            x = (x * f(1e-44)).astype(f)
        elif kind == "tiny":
            x = (x * f(1e-36)).astype(f)
        elif kind == "huge":
            x = (x * f(1e37)).astype(f)
        elif kind == "max":
            x[5], x[6] = f(3.4028235e38), -f(3.4028235e38)
        elif kind == "zero":
            x[:] = 0.0
        elif kind == "negzero":
            x[:] = -0.0
        out[kind] = x
    return out


def neon_q8k_block(x):
    """quantize_row_q8k for one block by the NEON instructions' definitions
    (q8k.c:41-80): vmaxq_f32 / vmaxvq_f32 return NaN when an operand is NaN;
    s = amax/127 unless !(amax > 0), then 1; vcvtaq_s32_f32 rounds half away
    from zero, saturates to int32 and gives 0 for NaN; then the clamp to
    +-127 and the 16-lane sums."""
    a = np.abs(x.astype(np.float32))
    amax = np.float32(np.nan) if np.isnan(a).any() else np.float32(max(0.0, float(a.max())))
    s = amax / np.float32(127.0) if amax > 0 else np.float32(1.0)
    inv = np.float32(1.0) / np.float32(s)
    v = (x.astype(np.float32) * inv).astype(np.float64)
    r = np.where(np.isnan(v), 0.0, np.sign(v) * np.floor(np.abs(v) + 0.5))
    q = np.clip(np.clip(r, -2.0 ** 31, 2.0 ** 31 - 1), -127, 127).astype(np.int8)
    return q, np.float32(s), q.astype(np.int32).reshape(16, 16).sum(axis=1).astype(np.int16)


def test_q8k_special_values_follow_neon_semantics(orc):
    for kind, x in special_blocks().items():
        with np.errstate(over="ignore", invalid="ignore"):
            eq, ed, es = neon_q8k_block(x)
        q, d, s = orc.q8k_quant(x)
        assert np.array_equal(q, eq), kind
        assert d.view(np.uint32)[0] == np.array([ed], np.float32).view(np.uint32)[0], kind
        assert np.array_equal(s, es), kind
    # the cases that pin the NaN rule: a NaN gives d = 1, x itself rounded
    x = special_blocks()["nan"]
    q, d, _ = orc.q8k_quant(x)
    assert d[0] == 1.0 and q[17] == 0 and q[0] == np.clip(np.round(x[0]), -127, 127)
