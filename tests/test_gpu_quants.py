"""GPU parity of the rest of the boundary, through the C-ABI, against the CPU
oracle on the same bytes:

* dequantisation (quants.c:29-75) bit-exact, also for fp16 block scales that
  are subnormal, infinite or NaN (the GPU decodes fp16 in hardware);
* the fp32 dequantise-then-dot matvec and the quants.c row entries
  (quants.c:80-133) within 1e-4 of max|y|;
* the q8k entries at row lengths that are not powers of two (q8k.c:92 takes
  any whole number of super-blocks), and called from 8 host threads at once
  as the engine's pool does (nn.c:276-289, 652-706);
* the matmul seam at the engine's other projection shapes (qma.h:186-199:
  wq / wqkv 2048 -> 8192, attn_gate 2048 -> 4096, wk / wv 2048 -> 512,
  ssm_beta / ssm_alpha 2048 -> 32, wo / ssm_out 4096 -> 2048; the types of
  wv and wqkv vary);
* Q6_K rows repacked by qmag_repack_q6k_dev (a layout of this library):
  bit-identical matmul results to the block layout through every matmul
  entry, the oracle's within 1e-4, and the documented byte order;
* qmag_matmul_group_dev (the projections of one x in one launch): each
  matrix's output bit-identical to a separate call, the oracle's within 1e-4.
"""
import ctypes as C
import threading

import numpy as np
import pytest

from conftest import max_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _rand_blocks(rng, wtype, nb, special=False):
    """Random-byte blocks (every bit pattern is a legal block) with fp16
    scales drawn from normal magnitudes or, with special, from the edge
    cases: subnormals, zero, +-Inf, NaN."""
    size = 144 if wtype == 12 else 210
    raw = rng.integers(0, 256, size=(nb, size), dtype=np.uint8)
    if special:
        pool = np.array([0x0001, 0x03FF, 0x8200, 0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x3C00, 0x0400],
                        np.uint16)
        d = pool[rng.integers(0, pool.size, nb)]
        dm = pool[rng.integers(0, pool.size, nb)]
    else:
        d = rng.uniform(1e-4, 1e-2, nb).astype(np.float16).view(np.uint16)
        dm = rng.uniform(1e-4, 1e-2, nb).astype(np.float16).view(np.uint16)
    if wtype == 12:
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    else:
        raw[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def _same_bits_or_both_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("special", [False, True])
def test_dequant_dev_bit_exact(qm, orc, wtype, special):
    rng = np.random.default_rng(wtype * 7 + special)
    nb = 600
    raw = _rand_blocks(rng, wtype, nb, special)
    y = qm.DBuf(4 * 256 * nb)
    qm.dequant_dev(qm.DBuf.from_array(raw), wtype, 256 * nb, y)
    got = y.download(np.float32)
    ref = orc.dequant(raw, wtype, 256 * nb)
    assert _same_bits_or_both_nan(got, ref)


@pytest.mark.parametrize("wtype", [12, 14])
def test_dequant_row_entries(qm, orc, wtype):
    """dequantize_row_q4_K / dequantize_row_q6_K with host pointers."""
    L = qm.lib()
    rng = np.random.default_rng(40 + wtype)
    raw = _rand_blocks(rng, wtype, 8)
    fn = L.dequantize_row_q4_K if wtype == 12 else L.dequantize_row_q6_K
    y = np.full(2048 + 16, 7.0, np.float32)
    fn(_p(raw), _p(y), 2048 + 100)          # only whole super-blocks (k / 256)
    assert _same_bits_or_both_nan(y[:2048], orc.dequant(raw, wtype, 2048))
    assert np.all(y[2048:] == 7.0)


def test_q8k_dot_subnormal_scales(qm, orc):
    """The int8 path with fp16 subnormal d / dmin (finite results)."""
    rng = np.random.default_rng(3)
    n_in, n_out = 2048, 256
    for wtype in (12, 14):
        raw = _rand_blocks(rng, wtype, n_out * 8)
        b = raw.reshape(n_out * 8, -1)
        sub = rng.integers(1, 0x400, (2, n_out * 8)).astype(np.uint16)     # fp16 subnormals
        if wtype == 12:
            b[:, 0:2] = sub[0].view(np.uint8).reshape(-1, 2)
            b[:, 2:4] = sub[1].view(np.uint8).reshape(-1, 2)
        else:
            b[:, 208:210] = sub[0].view(np.uint8).reshape(-1, 2)
        x = orc.fill_normal(9, n_in, 0.0, 1.0)
        out = qm.DBuf(4 * n_out)
        qm.matmul_dev(qm.DBuf.from_array(x), qm.DBuf.from_array(raw), n_in, n_out, 1, wtype, out)
        ref = orc.matmul_q8k(x, raw, n_in, n_out, 1, wtype)[0]
        assert max_rel_err(out.download(np.float32), ref) < TOL


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("n_in,n_out,T", [(256, 100, 1), (2048, 512, 1), (512, 2048, 3), (8192, 64, 2),
                                          (768, 77, 1), (12288, 40, 3), (16640, 33, 2), (24576, 17, 1)])
def test_matmul_f32_dev(qm, orc, wtype, n_in, n_out, T):
    """The QMA_NOQ8K dequantise-then-dot path against the oracle's
    dot_q4_K_f32 / dot_q6_K_f32 per row (quants.c:80-133), including rows
    longer than one 8192-value LDS chunk (a whole number of chunks, a
    ragged last chunk), whose partial sums are added in chunk order."""
    W = orc.quantize(orc.fill_normal(500 + n_in + n_out, n_in * n_out, 0.0, 0.02), wtype)
    x = orc.fill_normal(600 + T, T * n_in, 0.0, 1.0)
    out = qm.DBuf(4 * T * n_out)
    qm.matmul_f32_dev(qm.DBuf.from_array(x), qm.DBuf.from_array(W), n_in, n_out, T, wtype, out)
    got = out.download(np.float32).reshape(T, n_out)
    rb = W.size // n_out
    for t in range(T):
        ref = np.array([orc.dot_f32(W[r * rb:(r + 1) * rb], wtype, x[t * n_in:(t + 1) * n_in], n_in)
                        for r in range(n_out)], np.float32)
        assert max_rel_err(got[t], ref) < TOL


@pytest.mark.parametrize("wtype", [12, 14])
def test_dot_f32_entries(qm, orc, wtype):
    """dot_q4_K_f32 / dot_q6_K_f32 with host pointers, over 64 rows (the
    1e-4 bar is relative to the largest of the 64 results), including a row
    longer than one 8192-value chunk."""
    L = qm.lib()
    fn = L.dot_q4_K_f32 if wtype == 12 else L.dot_q6_K_f32
    for n in (2048, 512, 12288):
        W = orc.quantize(orc.fill_normal(70 + n, 64 * n, 0.0, 0.02), wtype)
        x = orc.fill_normal(71, n, 0.0, 1.0)
        rb = W.size // 64
        got = np.array([fn(_p(W[r * rb:]), _p(x), n) for r in range(64)], np.float32)
        ref = np.array([orc.dot_f32(W[r * rb:(r + 1) * rb], wtype, x, n) for r in range(64)], np.float32)
        assert max_rel_err(got, ref) < TOL


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("n_in", [768, 1280, 3072])
def test_matmul_non_power_of_two_rows(qm, orc, wtype, n_in):
    n_out, T = 300, 2
    W = orc.quantize(orc.fill_normal(900 + n_in, n_in * n_out, 0.0, 0.02), wtype)
    x = orc.fill_normal(901, T * n_in, 0.0, 1.0)
    out = qm.DBuf(4 * T * n_out)
    Wb = qm.DBuf.from_array(W)
    for T_ in (1, T):
        qm.matmul_dev(qm.DBuf.from_array(x[:T_ * n_in]), Wb, n_in, n_out, T_, wtype, out)
        got = out.download(np.float32, T_ * n_out).reshape(T_, n_out)
        ref = orc.matmul_q8k(x[:T_ * n_in], W, n_in, n_out, T_, wtype)
        for t in range(T_):
            assert max_rel_err(got[t], ref[t]) < TOL


def test_compat_dot_any_length(qm, orc):
    """qma_q8k_dot / qma_q8k_gateup at n = 768 and 1280 (not powers of two)."""
    L = qm.lib()
    for n in (768, 1280):
        xq, xd, xs = orc.q8k_quant(orc.fill_normal(n, n, 0.0, 1.0))
        rows = orc.quantize(orc.fill_normal(n + 1, 16 * n, 0.0, 0.02), 12).reshape(16, -1)
        got = np.array([L.qma_q8k_dot(_p(r), 12, _p(xq), _p(xd), _p(xs), n) for r in rows], np.float32)
        ref = np.array([orc.q8k_dot(r, 12, xq, xd, xs, n) for r in rows], np.float32)
        assert max_rel_err(got, ref) < TOL
        go, uo = C.c_float(), C.c_float()
        L.qma_q8k_gateup(_p(rows[0]), _p(rows[1]), _p(xq), _p(xd), _p(xs), n, C.byref(go), C.byref(uo))
        assert abs(go.value - ref[0]) <= TOL * np.abs(ref).max()
        assert abs(uo.value - ref[1]) <= TOL * np.abs(ref).max()


def test_compat_entries_concurrent_threads(qm, orc):
    """Eight host threads call qma_q8k_dot, qma_q8k_gateup and dot_q4_K_f32
    at once, as the pool workers do; every result matches the oracle."""
    L = qm.lib()
    n, rows_per = 2048, 24
    xq, xd, xs = orc.q8k_quant(orc.fill_normal(5, n, 0.0, 1.0))
    xf = orc.fill_normal(6, n, 0.0, 1.0)
    W = orc.quantize(orc.fill_normal(7, 8 * 2 * rows_per * n, 0.0, 0.02), 12).reshape(8, 2 * rows_per, -1)
    ref_q = np.array([[orc.q8k_dot(r, 12, xq, xd, xs, n) for r in W[k]] for k in range(8)], np.float32)
    ref_f = np.array([[orc.dot_f32(r, 12, xf, n) for r in W[k]] for k in range(8)], np.float32)
    got_q = np.zeros_like(ref_q)
    got_g = np.zeros_like(ref_q)
    got_f = np.zeros_like(ref_f)
    errors = []
    start = threading.Barrier(8)

    def work(k):
        try:
            start.wait()
            for i in range(2 * rows_per):
                got_q[k, i] = L.qma_q8k_dot(_p(W[k, i]), 12, _p(xq), _p(xd), _p(xs), n)
                got_f[k, i] = L.dot_q4_K_f32(_p(W[k, i]), _p(xf), n)
            for i in range(0, 2 * rows_per, 2):
                go, uo = C.c_float(), C.c_float()
                L.qma_q8k_gateup(_p(W[k, i]), _p(W[k, i + 1]), _p(xq), _p(xd), _p(xs), n,
                                 C.byref(go), C.byref(uo))
                got_g[k, i], got_g[k, i + 1] = go.value, uo.value
        except Exception as e:      # surfaced below
            errors.append(e)

    ts = [threading.Thread(target=work, args=(k,)) for k in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errors
    assert max_rel_err(got_q, ref_q) < TOL
    assert max_rel_err(got_g, ref_q) < TOL
    assert max_rel_err(got_f, ref_f) < TOL


@pytest.mark.parametrize("name,n_in,n_out,wtype", [
    ("wq", 2048, 8192, 12), ("wk", 2048, 512, 12), ("wv_q4k", 2048, 512, 12), ("wv_q6k", 2048, 512, 14),
    ("wo", 4096, 2048, 12), ("wo_q6k", 4096, 2048, 14),
    # the recurrent (gated delta net) layers' projections, qma.h:186-194
    ("wqkv_q6k", 2048, 8192, 14), ("attn_gate", 2048, 4096, 12), ("ssm_beta", 2048, 32, 12),
    ("ssm_out", 4096, 2048, 12)])
def test_matmul_projection_shapes(qm, orc, name, n_in, n_out, wtype):
    """The other matmul() call sites of qma_eval (nn.c:2111-2113, 2162,
    2165-2170, 2243) at the engine's shapes (qma.h:196-199), T = 1 (decode)
    and T = 5 (a prefill chunk)."""
    W = orc.quantize(orc.fill_normal(sum(map(ord, name)) + n_in, n_in * n_out, 0.0, 0.02), wtype)
    Wb = qm.DBuf.from_array(W)
    orc.set_threads(8)
    for T in (1, 5):
        x = orc.fill_normal(T + n_in, T * n_in, 0.0, 1.0)
        out = qm.DBuf(4 * T * n_out)
        qm.matmul_dev(qm.DBuf.from_array(x), Wb, n_in, n_out, T, wtype, out)
        got = out.download(np.float32).reshape(T, n_out)
        ref = orc.matmul_q8k(x, W, n_in, n_out, T, wtype)
        for t in range(T):
            assert max_rel_err(got[t], ref[t]) < TOL, (name, T, t)
    orc.set_threads(1)


def _repack_layout(W, n_in, n_out):
    """The row layout qmag_repack_q6k_dev documents (include/qma_gpu.h), from
    the block bytes: per row, every super-block's low ql task pieces, then the
    high ones, then the qh bytes, scales and d of every super-block."""
    nb = n_in // 256
    B = W.reshape(n_out, nb, 210)
    ql, qh, sc, d = B[:, :, :128], B[:, :, 128:192], B[:, :, 192:208], B[:, :, 208:210]
    lo = np.concatenate([ql[:, :, 0:32], ql[:, :, 64:96]], axis=2)
    hi = np.concatenate([ql[:, :, 32:64], ql[:, :, 96:128]], axis=2)
    return np.concatenate([x.reshape(n_out, -1) for x in (lo, hi, qh, sc, d)], axis=1).reshape(-1)


@pytest.mark.parametrize("n_in,n_out", [(2048, 1000), (4096, 777), (6144, 300)])
def test_q6k_repacked_rows_match_block_layout(qm, orc, n_in, n_out):
    """Q6_K rows repacked for the matvec (QMAG_TYPE_Q6_K_R) give the block
    layout's results bit for bit through every matmul entry (one-launch
    T = 1, two-step T = 3, pre-quantised, allocation-free; n_in = 6144 runs
    the one-wave-per-row kernel), and the oracle's within 1e-4; the
    repacked bytes follow the documented plane order."""
    W = orc.quantize(orc.fill_normal(7000 + n_in, n_in * n_out, 0.0, 0.02), 14)
    Wb = qm.DBuf.from_array(W)
    Rb = qm.DBuf(W.nbytes)
    qm.repack_q6k_dev(Wb, Rb, n_in, n_out)
    assert np.array_equal(Rb.download(np.uint8), _repack_layout(W, n_in, n_out))
    Ib = qm.DBuf.from_array(W)
    qm.repack_q6k_dev(Ib, Ib, n_in, n_out)                 # in place: the same bytes
    assert np.array_equal(Ib.download(np.uint8), Rb.download(np.uint8))
    L = qm.lib()
    for T in (1, 3):
        x = orc.fill_normal(7100 + T, T * n_in, 0.0, 1.0)
        xb = qm.DBuf.from_array(x)
        a, b, c = (qm.DBuf(4 * T * n_out) for _ in range(3))
        qm.matmul_dev(xb, Wb, n_in, n_out, T, qm.TYPE_Q6_K, a)
        qm.matmul_dev(xb, Rb, n_in, n_out, T, qm.TYPE_Q6_K_R, b)
        qm.check(L.qmag_matmul_noalloc_dev(xb.ptr, Rb.ptr, n_in, n_out, T, qm.TYPE_Q6_K_R, c.ptr))
        ga = a.download(np.float32)
        assert np.array_equal(ga.view(np.uint32), b.download(np.uint32)), T
        assert np.array_equal(ga.view(np.uint32), c.download(np.uint32)), T
        ref = orc.matmul_q8k(x, W, n_in, n_out, T, 14)
        for t in range(T):
            assert max_rel_err(ga.reshape(T, n_out)[t], ref[t]) < TOL
    xq, xd, xs = orc.q8k_quant(orc.fill_normal(7200, n_in, 0.0, 1.0))
    a, b = qm.DBuf(4 * n_out), qm.DBuf(4 * n_out)
    args = (qm.DBuf.from_array(xq), qm.DBuf.from_array(xd), qm.DBuf.from_array(xs))
    qm.matmul_q8k_dev(*args, Wb, n_in, n_out, 1, qm.TYPE_Q6_K, a)
    qm.matmul_q8k_dev(*args, Rb, n_in, n_out, 1, qm.TYPE_Q6_K_R, b)
    assert np.array_equal(a.download(np.uint32), b.download(np.uint32))


def test_q6k_repack_in_place_longest_row(qm, orc):
    """In place, the longest row the LDS staging takes (n_in 79,872: 65,520
    bytes) and a few rows: the documented layout, byte for byte."""
    n_in, n_out = 39 * 2048, 3
    W = orc.quantize(orc.fill_normal(7300, n_in * n_out, 0.0, 0.02), 14)
    Ib = qm.DBuf.from_array(W)
    qm.repack_q6k_dev(Ib, Ib, n_in, n_out)
    assert np.array_equal(Ib.download(np.uint8), _repack_layout(W, n_in, n_out))


def test_q6k_repacked_lm_head_shape(qm, orc):
    """The C2 shape (151,936 x 2048) repacked in place (no second copy of the
    255 MB matrix): bit-identical to the block layout's output."""
    n_in, n_out = 2048, 151936
    Wb = qm.DBuf(n_in // 256 * 210 * n_out)
    qm.synth_weights(42, n_in * n_out, 0.02, 14, Wb.ptr)
    Rb = qm.DBuf(Wb.nbytes)
    qm.synth_weights(42, n_in * n_out, 0.02, 14, Rb.ptr)
    qm.repack_q6k_dev(Rb, Rb, n_in, n_out)
    xb = qm.DBuf.from_array(orc.fill_normal(3, n_in, 0.0, 1.0))
    a, b = qm.DBuf(4 * n_out), qm.DBuf(4 * n_out)
    qm.matmul_dev(xb, Wb, n_in, n_out, 1, qm.TYPE_Q6_K, a)
    qm.matmul_dev(xb, Rb, n_in, n_out, 1, qm.TYPE_Q6_K_R, b)
    assert np.array_equal(a.download(np.uint32), b.download(np.uint32))


def test_q6k_repack_rejects_bad_arguments(qm):
    """Row lengths that are not a multiple of 2048, unaligned buffers, buffers
    that overlap without being the same one, rows too long to repack in place,
    and the repacked type at such lengths are argument errors."""
    L = qm.lib()
    W = qm.DBuf(8 * 210 * 64)
    R = qm.DBuf(8 * 210 * 64 + 64)
    x, out = qm.DBuf(4 * 2048), qm.DBuf(4 * 64)
    assert L.qmag_repack_q6k_dev(W.ptr, R.ptr, 1024, 64) == -2
    assert L.qmag_repack_q6k_dev(W.ptr, R.ptr + 8, 2048, 64) == -2
    assert L.qmag_repack_q6k_dev(W.ptr, W.ptr + 16, 2048, 63) == -2
    assert L.qmag_repack_q6k_dev(W.ptr, W.ptr, 40 * 2048, 1) == -2
    assert L.qmag_matmul_dev(x.ptr, W.ptr, 1024, 64, 1, qm.TYPE_Q6_K_R, out.ptr) == -2
    assert L.qmag_matmul_dev(x.ptr, R.ptr + 8, 2048, 64, 1, qm.TYPE_Q6_K_R, out.ptr) == -2
    assert L.qmag_repack_q6k_dev(W.ptr, R.ptr, 2048, 64) == 0


GROUPS = [
    # q, k, v of an attention layer (nn.c:2111-2113; wv's type varies)
    (2048, [(8192, 12), (512, 12), (512, 14)]),
    # qkv, gate, beta, alpha of a recurrent layer (nn.c:2162, 2165-2170)
    (2048, [(8192, 14), (4096, 12), (32, 12), (32, 12)]),
    # ragged row counts, a repacked Q6_K matrix, other row lengths
    (2048, [(300, 14), (77, 270), (5, 12)]),
    (4096, [(2048, 12), (33, 14)]),
    (512, [(100, 12), (3, 14)]),
    (8192, [(64, 14), (70, 12)]),
]


@pytest.mark.parametrize("n_in,mats", GROUPS)
def test_matmul_group_matches_separate_calls(qm, orc, n_in, mats):
    """qmag_matmul_group_dev (several matrices over one x, one launch) gives
    each matrix the bits of a separate qmag_matmul_dev call, and the oracle's
    result within 1e-4."""
    x = orc.fill_normal(8000 + n_in, n_in, 0.0, 1.0)
    xb = qm.DBuf.from_array(x)
    bufs, hosts = [], []
    for i, (n_out, t) in enumerate(mats):
        W = orc.quantize(orc.fill_normal(8100 + 7 * i + n_in, n_in * n_out, 0.0, 0.02), 14 if t == 270 else t)
        b = qm.DBuf.from_array(W)
        if t == 270:
            r = qm.DBuf(W.nbytes)
            qm.repack_q6k_dev(b, r, n_in, n_out)
            b = r
        bufs.append(b)
        hosts.append((W, 14 if t == 270 else t))
    outs = [qm.DBuf(4 * n_out) for n_out, _ in mats]
    qm.matmul_group_dev(xb, n_in, [(b, n, t) for b, (n, t) in zip(bufs, mats)], outs)
    for b, o, (n_out, t), (W, th) in zip(bufs, outs, mats, hosts):
        want = qm.DBuf(4 * n_out)
        qm.matmul_dev(xb, b, n_in, n_out, 1, t, want)
        got = o.download(np.float32)
        assert np.array_equal(got.view(np.uint32), want.download(np.uint32)), (n_out, t)
        ref = orc.matmul_q8k(x, W, n_in, n_out, 1, th)[0]
        assert max_rel_err(got, ref) < TOL


def test_matmul_group_rejects_bad_arguments(qm):
    """Group sizes outside 1..4, row lengths without a tiled form, unknown
    types and empty matrices are argument errors."""
    L = qm.lib()
    x, W, y = qm.DBuf(4 * 2048), qm.DBuf(144 * 8 * 64), qm.DBuf(4 * 64)

    def call(n_in, n, n_out=64, wtype=12):
        Ws = (C.c_void_p * max(n, 1))(*([W.ptr] * max(n, 1)))
        no = (C.c_int * max(n, 1))(*([n_out] * max(n, 1)))
        wt = (C.c_int * max(n, 1))(*([wtype] * max(n, 1)))
        ys = (C.c_void_p * max(n, 1))(*([y.ptr] * max(n, 1)))
        return L.qmag_matmul_group_dev(x.ptr, n_in, n, Ws, no, wt, ys)

    assert call(2048, 0) == -2
    assert call(2048, 5) == -2
    assert call(768, 1) == -2
    assert call(2048, 1, wtype=13) == -2
    assert call(2048, 1, n_out=0) == -2
    assert call(1024, 1, wtype=270) == -2
    assert call(2048, 2) == 0


def test_matmul_random_shapes_vs_oracle(qm, orc):
    """Seeded random shapes through the matmul seam: row lengths of 1-48
    super-blocks (powers of two take the tiled kernels, the others the
    per-row one), 1-3,000 rows, T 1-8, Q4_K, Q6_K and repacked Q6_K rows,
    the one-launch x form, the pre-quantised Q8_K form and the fp32 form,
    each within 1e-4 of the oracle per token."""
    rng = np.random.default_rng(77)
    for case in range(24):
        k = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 24, 32, 33, 48]))
        n_in = 256 * k
        n_out = int(rng.integers(1, min(3000, (1 << 22) // n_in) + 1))
        T = int(rng.choice([1, 1, 2, 3, 5, 8]))
        wt = int(rng.choice([12, 14, qm.TYPE_Q6_K_R])) if n_in % 2048 == 0 else int(rng.choice([12, 14]))
        form = str(rng.choice(["x", "q8k"] if wt == qm.TYPE_Q6_K_R else ["x", "q8k", "f32"]))
        wo = 14 if wt == qm.TYPE_Q6_K_R else wt
        Wh = orc.quantize(orc.fill_normal(900 + case, n_in * n_out, 0.0, 0.02), wo)
        x = orc.fill_normal(950 + case, T * n_in, 0.0, 1.0)
        W = qm.DBuf.from_array(Wh)
        if wt == qm.TYPE_Q6_K_R:
            qm.repack_q6k_dev(W, W, n_in, n_out)
        xb, out = qm.DBuf.from_array(x), qm.DBuf(4 * T * n_out)
        if form == "x":
            qm.matmul_dev(xb, W, n_in, n_out, T, wt, out)
        elif form == "q8k":
            xq, xd, xs = qm.DBuf(T * n_in), qm.DBuf(4 * T * n_in // 256), qm.DBuf(2 * T * n_in // 16)
            qm.q8k_quant_dev(xb, n_in, T, xq, xd, xs)
            qm.matmul_q8k_dev(xq, xd, xs, W, n_in, n_out, T, wt, out)
        else:
            qm.matmul_f32_dev(xb, W, n_in, n_out, T, wt, out)
        got = out.download(np.float32).reshape(T, n_out)
        if form == "f32":
            rb = Wh.size // n_out
            ref = np.array([[orc.dot_f32(Wh[r * rb:(r + 1) * rb], wo, x[t * n_in:(t + 1) * n_in], n_in)
                             for r in range(n_out)] for t in range(T)], np.float32)
        else:
            ref = orc.matmul_q8k(x, Wh, n_in, n_out, T, wo).reshape(T, n_out)
        for t in range(T):
            assert max_rel_err(got[t], ref[t]) < TOL, (case, n_in, n_out, T, wt, form, t)
        W.close()
