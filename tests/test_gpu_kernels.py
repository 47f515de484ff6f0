"""GPU parity: Q8_K quantisation, Q4_K/Q6_K matvecs and the build's quantiser,
each called through the C-ABI and checked against the CPU oracle.

Bars: Q8_K bit-exact; integer dot paths bit-exact (exact-integer pin below);
fp32 outputs within 1e-4 relative to max|y|."""
import numpy as np
import pytest

from conftest import max_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _q8_dev(qm, x, n, T):
    xb = qm.DBuf.from_array(x.astype(np.float32))
    xq = qm.DBuf(T * n)
    xd = qm.DBuf(4 * T * (n // 256))
    xs = qm.DBuf(2 * T * (n // 16))
    qm.q8k_quant_dev(xb, n, T, xq, xd, xs)
    return xb, xq, xd, xs


@pytest.mark.parametrize("n,T,scale", [(256, 1, 1.0), (2048, 1, 1.0), (512, 7, 1e-3),
                                       (8192, 3, 1e3), (2048, 64, 0.02)])
def test_q8k_quant_bit_exact(qm, orc, n, T, scale):
    rng = np.random.default_rng(n + T)
    x = (rng.standard_normal(n * T) * scale).astype(np.float32)
    x[:256] = 0.0 if T > 1 else x[:256]                # a zero block
    x[-1] = np.float32(127.0 * 2.5) if scale == 1.0 else x[-1]
    _, xq, xd, xs = _q8_dev(qm, x, n, T)
    gq, gd, gs = xq.download(np.int8), xd.download(np.float32), xs.download(np.int16)
    for t in range(T):
        oq, od, os_ = orc.q8k_quant(x[t * n:(t + 1) * n])
        assert np.array_equal(gq[t * n:(t + 1) * n], oq)
        assert np.array_equal(gd[t * (n // 256):(t + 1) * (n // 256)].view(np.uint32), od.view(np.uint32))
        assert np.array_equal(gs[t * (n // 16):(t + 1) * (n // 16)], os_)


def test_q8k_ties_and_spikes(qm, orc):
    x = np.zeros(256, np.float32)
    x[3] = 127.0
    x[10:14] = [2.5, -3.5, 0.5, -0.5]
    x[20:22] = [126.5, -126.4999]
    _, xq, xd, xs = _q8_dev(qm, x, 256, 1)
    assert list(xq.download(np.int8)[[3, 10, 11, 12, 13, 20, 21]]) == [127, 3, -4, 1, -1, 127, -126]
    assert xd.download(np.float32)[0] == 1.0


def test_q8k_special_values(qm, orc):
    """Blocks with NaN (alone, all, beside +Inf), +-Inf, subnormal values,
    amax/127 underflowing to 0, tiny, near-overflow and the largest finite
    values, +0 and -0: bytes, scales and sums bit for bit the oracle's (which
    a CPU test pins to the NEON instructions' definitions: a NaN anywhere in
    a block makes amax NaN and so d = 1).  The one-launch T = 1 matmul, which
    quantises x in LDS, gives the two-step form's outputs on the same x."""
    from test_oracle_q8k import special_blocks
    blocks = special_blocks()
    x = np.concatenate(list(blocks.values()))
    n = x.size
    xb, xq, xd, xs = _q8_dev(qm, x, n, 1)
    gq, gd, gs = xq.download(np.int8), xd.download(np.float32), xs.download(np.int16)
    oq, od, os_ = orc.q8k_quant(x)
    for i, kind in enumerate(blocks):
        assert np.array_equal(gq[256 * i:256 * (i + 1)], oq[256 * i:256 * (i + 1)]), kind
        assert gd.view(np.uint32)[i] == od.view(np.uint32)[i], kind
        assert np.array_equal(gs[16 * i:16 * (i + 1)], os_[16 * i:16 * (i + 1)]), kind
    n_mv = 4096                                      # the first 16 blocks: a tiled one-launch instance
    W = qm.DBuf.from_array(orc.quantize_q4k(orc.fill_normal(3, n_mv * 64, 0.0, 0.02)))
    o1, o2 = qm.DBuf(4 * 64), qm.DBuf(4 * 64)
    x16 = qm.DBuf.from_array(np.resize(x, n_mv).astype(np.float32))
    _, q16, d16, s16 = _q8_dev(qm, np.resize(x, n_mv), n_mv, 1)
    qm.matmul_dev(x16, W, n_mv, 64, 1, 12, o1)
    qm.matmul_q8k_dev(q16, d16, s16, W, n_mv, 64, 1, 12, o2)
    assert np.array_equal(o1.download(np.float32), o2.download(np.float32), equal_nan=True)


def _exact_q4k_rows(rng, n_out, nb):
    """Blocks with d = 1, dmin = 1 (fp16), random 6-bit scales/mins and
    nibbles: with xd = 1 every row dot is an integer below 2^24, so the fp32
    result is exact and must equal the integer closed form."""
    raw = rng.integers(0, 256, size=(n_out * nb, 144), dtype=np.uint8)
    one = np.array([1.0], np.float16).view(np.uint8)
    raw[:, 0:2] = one
    raw[:, 2:4] = one
    return raw.reshape(-1)


def test_q4k_integer_path_exact(qm, orc):
    import oracle_np as onp
    rng = np.random.default_rng(0)
    for nb in (1, 2, 8):
        n, n_out = 256 * nb, 96
        W = _exact_q4k_rows(rng, n_out, nb)
        # |xq| <= 31 keeps every partial sum far below 2^24
        xq = rng.integers(-31, 32, size=n).astype(np.int8)
        xd = np.ones(nb, np.float32)
        xs = xq.astype(np.int64).reshape(-1, 16).sum(axis=1).astype(np.int16)
        out = qm.DBuf(4 * n_out)
        qm.matmul_q8k_dev(qm.DBuf.from_array(xq), qm.DBuf.from_array(xd), qm.DBuf.from_array(xs),
                          qm.DBuf.from_array(W), n, n_out, 1, 12, out)
        got = out.download(np.float32).astype(np.float64)
        rb = 144 * nb
        _, _, sc, m, _ = onp.q4k_fields(W)
        for r in range(n_out):
            P = onp.q4k_subsums(W[r * rb:(r + 1) * rb], xq).reshape(nb, 8)
            sx = xs.astype(np.int64).reshape(nb, 8, 2).sum(axis=2)
            want = int(np.sum(sc[r * nb:(r + 1) * nb] * P) - np.sum(m[r * nb:(r + 1) * nb] * sx))
            assert got[r] == want


def test_q6k_integer_path_exact(qm, orc):
    import oracle_np as onp
    rng = np.random.default_rng(1)
    for nb in (1, 2, 8):
        n, n_out = 256 * nb, 64
        raw = rng.integers(0, 256, size=(n_out * nb, 210), dtype=np.uint8)
        raw[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
        raw[:, 192:208] = rng.integers(-8, 9, size=(n_out * nb, 16)).astype(np.int8).view(np.uint8)
        W = raw.reshape(-1)
        xq = rng.integers(-127, 128, size=n).astype(np.int8)
        xd = np.ones(nb, np.float32)
        xs = xq.astype(np.int64).reshape(-1, 16).sum(axis=1).astype(np.int16)
        out = qm.DBuf(4 * n_out)
        qm.matmul_q8k_dev(qm.DBuf.from_array(xq), qm.DBuf.from_array(xd), qm.DBuf.from_array(xs),
                          qm.DBuf.from_array(W), n, n_out, 1, 14, out)
        got = out.download(np.float32).astype(np.float64)
        rb = 210 * nb
        for r in range(n_out):
            want = int(onp.q6k_blocksums(W[r * rb:(r + 1) * rb], xq).sum())
            assert got[r] == want


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("n_in,n_out,T", [(256, 1, 1), (512, 2048, 1), (2048, 2048, 1),
                                          (2048, 37, 1), (4096, 300, 1), (8192, 65, 1),
                                          (2048, 129, 4), (512, 513, 3),
                                          # the engine's projection shapes (qma.h:196-199): wq, wk/wv, wo
                                          (2048, 8192, 1), (2048, 512, 1), (4096, 2048, 1)])
def test_matvec_vs_oracle(qm, orc, wtype, n_in, n_out, T):
    W = orc.quantize(orc.fill_normal(1000 + n_in + n_out, n_in * n_out, 0.0, 0.02), wtype)
    x = orc.fill_normal(7 + T, n_in * T, 0.0, 1.0)
    xb = qm.DBuf.from_array(x)
    Wb = qm.DBuf.from_array(W)
    out = qm.DBuf(4 * n_out * T)
    qm.matmul_dev(xb, Wb, n_in, n_out, T, wtype, out)
    got = out.download(np.float32).reshape(T, n_out)
    ref = orc.matmul_q8k(x, W, n_in, n_out, T, wtype)
    assert max_rel_err(got, ref) < TOL


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("n_in,n_out", [(256, 33), (2048, 2048), (8192, 65)])
def test_matmul_one_launch_equals_two_step(qm, orc, wtype, n_in, n_out):
    """At T = 1 the matmul seam is one launch (the matvec quantises x in LDS
    with the routine of the Q8_K kernel); its output must equal, bit for bit,
    the two-step form: Q8_K kernel, then the matvec on the stored operand.
    x carries exact .5 ties and a spike so the rounding paths are exercised."""
    W = orc.quantize(orc.fill_normal(2000 + n_in + n_out, n_in * n_out, 0.0, 0.02), wtype)
    x = orc.fill_normal(11 + n_in, n_in, 0.0, 1.0)
    x[::97] = np.float32(2.5)
    x[5] = np.float32(-9.0)
    xb, xq, xd, xs = _q8_dev(qm, x, n_in, 1)
    Wb = qm.DBuf.from_array(W)
    one = qm.DBuf(4 * n_out)
    two = qm.DBuf(4 * n_out)
    qm.matmul_dev(xb, Wb, n_in, n_out, 1, wtype, one)
    qm.matmul_q8k_dev(xq, xd, xs, Wb, n_in, n_out, 1, wtype, two)
    a = one.download(np.float32)
    b = two.download(np.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_lm_head_shape_q6k(qm, orc):
    """C2 shape (151,936 x 2048, Q6_K) generated on the GPU; the full output
    vector is checked against the oracle run on the downloaded bytes."""
    n_in, n_out = 2048, 151936
    rb = n_in // 256 * 210
    Wb = qm.DBuf(rb * n_out)
    qm.synth_weights(42, n_in * n_out, 0.02, 14, Wb.ptr)
    x = orc.fill_normal(3, n_in, 0.0, 1.0)
    out = qm.DBuf(4 * n_out)
    qm.matmul_dev(qm.DBuf.from_array(x), Wb, n_in, n_out, 1, 14, out)
    got = out.download(np.float32)
    W = Wb.download(np.uint8)
    orc.set_threads(8)
    ref = orc.matmul_q8k(x, W, n_in, n_out, 1, 14)[0]
    orc.set_threads(1)
    assert max_rel_err(got, ref) < TOL


def test_compat_entries_host_pointers(qm, orc):
    """qma_q8k_quant / qma_q8k_dot / qma_q8k_gateup with host buffers, as the
    engine calls them from its pool (nn.c:276-289, 423-437)."""
    import ctypes as C
    L = qm.lib()
    assert L.qma_q8k_available() == 1
    x = orc.fill_normal(5, 2048, 0.0, 1.0)
    xq = np.empty(2048, np.int8)
    xd = np.empty(8, np.float32)
    xs = np.empty(128, np.int16)
    p = lambda a: a.ctypes.data_as(C.c_void_p)
    L.qma_q8k_quant(p(x), 2048, p(xq), p(xd), p(xs))
    oq, od, os_ = orc.q8k_quant(x)
    assert np.array_equal(xq, oq) and np.array_equal(xd, od) and np.array_equal(xs, os_)
    g = orc.quantize(orc.fill_normal(6, 2048, 0.0, 0.02), 12)
    u = orc.quantize(orc.fill_normal(7, 2048, 0.0, 0.02), 12)
    d6 = orc.quantize(orc.fill_normal(8, 512, 0.0, 0.02), 14)
    ref_g = orc.q8k_dot(g, 12, xq, xd, xs, 2048)
    ref_u = orc.q8k_dot(u, 12, xq, xd, xs, 2048)
    got = L.qma_q8k_dot(p(g), 12, p(xq), p(xd), p(xs), 2048)
    assert abs(got - ref_g) <= TOL * abs(ref_g)
    go, uo = C.c_float(), C.c_float()
    L.qma_q8k_gateup(p(g), p(u), p(xq), p(xd), p(xs), 2048, C.byref(go), C.byref(uo))
    assert abs(go.value - ref_g) <= TOL * abs(ref_g) and abs(uo.value - ref_u) <= TOL * abs(ref_u)
    hq, hd, hs = orc.q8k_quant(orc.fill_normal(9, 512, 0.0, 1.0))
    ref6 = orc.q8k_dot(d6, 14, hq, hd, hs, 512)
    assert abs(L.qma_q8k_dot(p(d6), 14, p(hq), p(hd), p(hs), 512) - ref6) <= TOL * abs(ref6)
    assert L.qma_q8k_dot(p(g), 13, p(xq), p(xd), p(xs), 2048) == 0.0   # unknown type


@pytest.mark.parametrize("wtype", [12, 14])
def test_device_quantizer_matches_oracle(qm, orc, wtype):
    x = orc.fill_normal(77, 256 * 512, 0.0, 0.02)
    x[:256] = np.abs(x[:256])                  # all-non-negative block (min = 0 path)
    x[256:512] = 0.0                           # all-zero block
    xb = qm.DBuf.from_array(x)
    ob = qm.DBuf(x.size // 256 * (144 if wtype == 12 else 210))
    qm.quantize_dev(xb.ptr, x.size, wtype, ob.ptr)
    assert np.array_equal(ob.download(np.uint8), orc.quantize(x, wtype))


@pytest.mark.parametrize("wtype", [12, 14])
def test_synth_weights_deterministic_and_scaled(qm, orc, wtype):
    n = 256 * 4096
    bb = 144 if wtype == 12 else 210
    a, b = qm.DBuf(n // 256 * bb), qm.DBuf(n // 256 * bb)
    qm.synth_weights(123, n, 0.02, wtype, a.ptr)
    qm.synth_weights(123, n, 0.02, wtype, b.ptr)
    ra, rb_ = a.download(np.uint8), b.download(np.uint8)
    assert np.array_equal(ra, rb_)
    w = orc.dequant(ra, wtype, n)
    assert abs(w.std() - 0.02) < 0.002 and abs(w.mean()) < 0.002
