"""The allocation-free matmul entry (qmag_matmul_noalloc_dev) against the
ordinary matmul seam it mirrors (qmag_matmul_dev): same results bit for bit,
through the C-ABI, on two calls in a row (the second smaller, so it runs over
what the first left in the shared fixed scratch), and a clear error beyond the
scratch's size."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(qm, fn, x, Wb, n_in, n_out, T, wtype):
    out = qm.DBuf(4 * T * n_out)
    qm.check(fn(x.ptr, Wb.ptr, n_in, n_out, T, wtype, out.ptr))
    return out.download(np.float32)


@pytest.mark.parametrize("wtype", [12, 14])
def test_noalloc_matmul_matches_matmul(qm, orc, wtype):
    L = qm.lib()
    cases = [(2048, 1024, 64), (2048, 300, 5), (768, 200, 1)]    # large, then smaller; tiled and not
    for n_in, n_out, T in cases:
        W = orc.quantize(orc.fill_normal(31 + n_in + n_out, n_in * n_out, 0.0, 0.02), wtype)
        Wb = qm.DBuf.from_array(W)
        x = qm.DBuf.from_array(orc.fill_normal(17 + T, T * n_in, 0.0, 1.0))
        a = _run(qm, L.qmag_matmul_noalloc_dev, x, Wb, n_in, n_out, T, wtype)
        b = _run(qm, L.qmag_matmul_dev, x, Wb, n_in, n_out, T, wtype)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (n_in, n_out, T)
        ref = orc.matmul_q8k(x.download(np.float32), W, n_in, n_out, T, wtype)
        assert np.max(np.abs(a.reshape(T, n_out) - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_noalloc_matmul_rejects_oversize(qm):
    L = qm.lib()
    x = qm.DBuf(16)
    W = qm.DBuf(16)
    out = qm.DBuf(16)
    st = L.qmag_matmul_noalloc_dev(x.ptr, W.ptr, 4096, 8, 513, 12, out.ptr)     # 513 * 4096 > 2^21
    assert st == -2
    assert b"exceeds" in L.qmag_last_error()
