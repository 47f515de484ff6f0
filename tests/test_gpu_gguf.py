"""GGUF -> HBM residency on the GPU: a two-layer qwen35moe-shaped FFN stack
(hidden 2048, expert ff 512, 16 experts, top-8 from expert_used_count; layer
0's down tensors Q6_K, layer 1's Q4_K, the per-layer down type of
qma.h:206, 212) and an LM head written by the test writer from the oracle's
quantised tensors, uploaded with qmag_gguf_upload_moe_layer /
qmag_gguf_upload_tensor, and run through the device entries against the
oracle on the same bytes."""
import types

import numpy as np
import pytest

import gguf_writer as gw
from conftest import max_rel_err
from moe_fixtures import make_host_layer
from test_gpu_moe import check_layer, check_layer_staged

pytestmark = pytest.mark.gpu

TOL = 1e-4
N, F, E, K = 2048, 512, 16, 8


@pytest.fixture(scope="module")
def model(orc, tmp_path_factory):
    layers = [make_host_layer(orc, seed=150 + i, n_embd=N, n_ff=F, n_expert=E, n_used=K,
                              t_down=(14 if i == 0 else 12)) for i in range(2)]
    head = orc.quantize_q6k(orc.fill_normal(151, N * 1000, 0.0, 0.02))
    tensors = gw.moe_model_tensors(layers) + [("output.weight", gw.T_Q6_K, [N, 1000], head)]
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    gw.write_gguf(path, gw.qwen35moe_metadata(2, N, E, K, F), tensors)
    return path, layers, head


def test_gguf_moe_layers_vs_oracle(qm, orc, model):
    path, layers, _ = model
    g = qm.Gguf(str(path))
    dev = [g.upload_moe_layer(il) for il in range(2)]
    try:
        for il, (L, hl) in enumerate(zip(dev, layers)):
            assert (L.n_embd, L.n_ff, L.n_expert, L.n_used) == (N, F, E, K)
            assert L.t_down_exps == L.t_down_shexp == hl.t_down_exps
            rl = types.SimpleNamespace(c=L, n_embd=N)
            for T in (1, 3):                     # persistent decode kernel, launch sequence
                x = orc.fill_normal(40 + il * 7 + T, T * N, 0.0, 1.0)
                check_layer(qm, orc, rl, hl, x, T)
            x = orc.fill_normal(60 + il, 16 * N, 0.0, 1.0)
            check_layer_staged(qm, orc, rl, hl, x, 16)        # grouped prefill
        # the stack over both layers (down types differ: each layer is its own
        # one-layer persistent launch) equals the layers chained one call at a
        # time, bit for bit
        x = orc.fill_normal(77, 2 * N, 0.0, 1.0)
        xb = qm.DBuf.from_array(x)
        qm.moe_stack_dev(dev, xb.ptr, 2)
        got = xb.download(np.float32).reshape(2, N)
        for t in range(2):
            xl = x[t * N:(t + 1) * N].copy()
            for L in dev:
                b = qm.DBuf.from_array(xl)
                qm.moe_stack_dev([L], b.ptr, 1)
                xl = b.download(np.float32)
            assert np.array_equal(got[t].view(np.uint32), xl.view(np.uint32)), f"token {t}"
    finally:
        for L in dev:
            qm.Gguf.free_moe_layer(L)
        g.close()


def test_gguf_lm_head_vs_oracle(qm, orc, model):
    path, _, head = model
    g = qm.Gguf(str(path))
    d, t, ne = g.upload_tensor("output.weight")
    try:
        assert t == 14 and ne == (N, 1000, 1)
        x = orc.fill_normal(5, N, 0.0, 1.0)
        out = qm.DBuf(4 * 1000)
        qm.check(qm.lib().qmag_matmul_dev(qm.DBuf.from_array(x).ptr, d, N, 1000, 1, t, out.ptr))
        ref = orc.matmul_q8k(x, head, N, 1000, 1, 14)[0]
        assert max_rel_err(out.download(np.float32), ref) < TOL
    finally:
        qm.check(qm.lib().qmag_free(d))
        g.close()
