"""Pins of the CPU oracle's format code (fp16, Q4_K/Q6_K layouts).

Checks against numpy's float16 conversion (exact), the GGUF k-quant layout
stated from its spec (packing written independently of the unpacker), and
the independent numpy restatement in oracle/oracle_np.py."""
import ctypes as C

import numpy as np
import pytest

import oracle_np as onp


def test_half_to_float_exhaustive(orc):
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([L.orc_half_to_float(int(b)) for b in bits], dtype=np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_rne(orc):
    L = orc.lib()
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.01),
        rng.standard_normal(2000).astype(np.float32) * np.float32(1e-6),   # fp16 subnormals
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 8.940697e-08], dtype=np.float32),
        # exact ties between two fp16 values: 1 + (2k+1)*2^-11
        (np.float32(1.0) + (2 * np.arange(50, dtype=np.float32) + 1) * np.float32(2.0 ** -11)),
    ])
    got = np.array([L.orc_float_to_half(float(x)) for x in xs], dtype=np.uint16)
    ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def _pack_scales(sc, m):
    """GGUF Q4_K scale packing written from the format description: bytes
    0-3 hold scales 0-3 (6 bits) plus the top 2 bits of scales 4-7, bytes 4-7
    mins 0-3 plus the top 2 bits of mins 4-7, bytes 8-11 the low nibbles of
    scales 4-7 (low) and mins 4-7 (high)."""
    out = bytearray(12)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(out)


@pytest.mark.parametrize("j", range(8))
def test_scale_min_k4_exhaustive(orc, j):
    """All 64x64 (scale, min) values of sub-block j survive pack -> unpack,
    with the other sub-blocks' fields set to varied values."""
    L = orc.lib()
    rng = np.random.default_rng(j)
    s_out = C.c_uint8()
    m_out = C.c_uint8()
    buf = (C.c_uint8 * 12)()
    for s in range(64):
        for m in range(64):
            sc = [int(v) for v in rng.integers(0, 64, 8)]
            mm = [int(v) for v in rng.integers(0, 64, 8)]
            sc[j], mm[j] = s, m
            packed = _pack_scales(sc, mm)
            C.memmove(buf, packed, 12)
            L.orc_scale_min_k4(j, buf, C.byref(s_out), C.byref(m_out))
            assert (s_out.value, m_out.value) == (s, m)


def _random_blocks(rng, nb, bsize, d_offsets):
    raw = rng.integers(0, 256, size=(nb, bsize), dtype=np.uint8)
    # finite fp16 scales (random bit patterns, exponent < 31), including subnormals
    for off in d_offsets:
        h = rng.integers(0, 0x7C00, size=nb).astype(np.uint16)
        h |= (rng.integers(0, 2, size=nb).astype(np.uint16) << 15)
        raw[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def test_dequant_q4k_matches_numpy(orc):
    rng = np.random.default_rng(7)
    raw = _random_blocks(rng, 64, 144, (0, 2))
    got = orc.dequant(raw, orc.TYPE_Q4_K, 64 * 256).astype(np.float64)
    ref = onp.q4k_dequant(raw)
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) <= 4e-7 * scale


def test_dequant_q6k_matches_numpy(orc):
    rng = np.random.default_rng(8)
    raw = _random_blocks(rng, 64, 210, (208,))
    got = orc.dequant(raw, orc.TYPE_Q6_K, 64 * 256).astype(np.float64)
    ref = onp.q6k_dequant(raw)
    scale = np.abs(ref).max()
    assert np.max(np.abs(got - ref)) <= 4e-7 * scale


def test_q4k_element_layout_known_answer(orc):
    """One nibble set at a time: element 64g+l is the low nibble of
    qs[32g+l]; element 64g+32+l the high nibble (quants.c:37-44)."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([np.float16(1.0)]).view(np.uint8)       # d = 1
    blk[4:16] = np.frombuffer(_pack_scales([1] * 8, [0] * 8), dtype=np.uint8)
    for g in range(4):
        for l in (0, 7, 31):
            for hi in (0, 1):
                b = blk.copy()
                b[16 + 32 * g + l] = (5 << 4) if hi else 5
                y = orc.dequant(b, orc.TYPE_Q4_K, 256)
                e = 64 * g + 32 * hi + l
                assert y[e] == 5.0 and np.count_nonzero(y) == 1


def test_q6k_element_layout_known_answer(orc):
    """Element 128n+32Q+l takes ql[64n+l] (Q=0 low, Q=2 high nibble) or
    ql[64n+32+l] (Q=1 low, Q=3 high) and qh[32n+l] bits 2Q..2Q+1, scaled by
    sc[e/16] (quants.c:57-73)."""
    base = np.zeros(210, dtype=np.uint8)
    base[208:210] = np.array([np.float16(1.0)]).view(np.uint8)
    base[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    # all-zero quants mean q6 = 0 -> value -32 * sc
    y0 = orc.dequant(base, orc.TYPE_Q6_K, 256)
    assert np.array_equal(y0, -32.0 * np.repeat(np.arange(1, 17), 16).astype(np.float32))
    for n in range(2):
        for Q in range(4):
            for l in (0, 17, 31):
                b = base.copy()
                qli = 64 * n + (Q & 1) * 32 + l
                b[qli] = (9 << 4) if Q >= 2 else 9
                b[128 + 32 * n + l] = 2 << (2 * Q)
                e = 128 * n + 32 * Q + l
                y = orc.dequant(b, orc.TYPE_Q6_K, 256)
                want = y0.copy()
                want[e] = (9 + 32 - 32) * (e // 16 + 1)
                assert np.array_equal(y, want)


def test_quantizer_roundtrip(orc):
    """The build's fp32 -> Q4_K/Q6_K quantizers stay within their step."""
    x = orc.fill_normal(11, 256 * 32, 0.0, 0.02)
    for wtype, tol in ((orc.TYPE_Q4_K, 0.6), (orc.TYPE_Q6_K, 0.6)):
        q = orc.quantize(x, wtype)
        y = orc.dequant(q, wtype, x.size)
        # error bounded by ~half a quantisation step of each group
        step = np.abs(x).reshape(-1, 16).max(axis=1).repeat(16) / (7.5 if wtype == 12 else 31)
        assert np.all(np.abs(y - x) <= tol * step * 2 + 1e-7)
        rel = np.linalg.norm(y - x) / np.linalg.norm(x)
        assert rel < (0.08 if wtype == 12 else 0.02)
