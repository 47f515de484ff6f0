"""Pins of the oracle's MoE layer (nn.c:509-707) on small layers.

The router against an fp64 recomputation with its top-8 margin (tie rule =
stable sort on -p), the expert stage h = silu(g)*u against fp64 closed
forms, the combine order, and thread-count independence."""
import numpy as np
import pytest

import oracle_np as onp
from moe_fixtures import make_host_layer


@pytest.fixture(scope="module")
def small(orc):
    return make_host_layer(orc, seed=5, n_embd=512, n_ff=256, n_expert=16, n_used=4)


def test_route_vs_fp64(orc, small):
    rng = np.random.default_rng(0)
    for t in range(20):
        x = rng.standard_normal(small.n_embd).astype(np.float32)
        sel, w, logits = orc.moe_route(small, x)
        s64, w64, p64, margin = onp.route_f64(small.gate_inp.reshape(small.n_expert, -1), x,
                                              small.n_used)
        if margin > 1e-6:
            assert list(sel) == list(s64)
            assert np.allclose(w, w64, rtol=1e-5, atol=1e-7)
        assert abs(w.sum() - 1.0) < 1e-6


def test_route_tie_lowest_index(orc):
    """Equal probabilities: the lowest index wins (strict > scan, nn.c:531)."""
    lay = make_host_layer(orc, seed=1, n_embd=256, n_ff=256, n_expert=8, n_used=4,
                          zero_router=True)
    x = np.ones(256, np.float32)
    sel, w, _ = orc.moe_route(lay, x)
    assert list(sel) == [0, 1, 2, 3]
    assert np.allclose(w, 0.25)


def test_expert_h_vs_fp64(orc, small):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(small.n_embd).astype(np.float32)
    xq, xd, xs = orc.q8k_quant(x)
    N, F = small.n_embd, small.n_ff
    gb = small.gate_exps.size // small.n_expert
    for ex in (0, 7, 15):
        ge = small.gate_exps[ex * gb:(ex + 1) * gb]
        ue = small.up_exps[ex * gb:(ex + 1) * gb]
        h = orc.moe_expert_h(ge, ue, N, F, xq, xd, xs)
        rb = gb // F
        g = np.array([onp.q8k_dot_f64(ge[i * rb:(i + 1) * rb], 12, xq, xd) for i in range(F)])
        u = np.array([onp.q8k_dot_f64(ue[i * rb:(i + 1) * rb], 12, xq, xd) for i in range(F)])
        h64 = g / (1 + np.exp(-g)) * u
        assert np.max(np.abs(h - h64)) <= 1e-5 * np.max(np.abs(h64))


def test_moe_ffn_composition(orc, small):
    """out = sum_k w_k * down_k(Q8_K(h_k)) + sigmoid(gs) * down_sh(...), with
    every stage recomputed here from the oracle's own primitives, in order."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(small.n_embd).astype(np.float32)
    out = orc.moe_ffn(small, x, 1)[0]
    sel, w, _ = orc.moe_route(small, x)
    N, F = small.n_embd, small.n_ff
    xq, xd, xs = orc.q8k_quant(x)
    gb = small.gate_exps.size // small.n_expert
    db = small.down_exps.size // small.n_expert
    acc = np.zeros(N, np.float32)
    for k in range(small.n_used):
        ex = sel[k]
        h = orc.moe_expert_h(small.gate_exps[ex * gb:(ex + 1) * gb],
                             small.up_exps[ex * gb:(ex + 1) * gb], N, F, xq, xd, xs)
        hq, hd, hs = orc.q8k_quant(h)
        de = small.down_exps[ex * db:(ex + 1) * db]
        rb = db // N
        part = np.array([np.float32(w[k]) * np.float32(orc.q8k_dot(de[r * rb:(r + 1) * rb],
                         small.t_down_exps, hq, hd, hs, F)) for r in range(N)], np.float32)
        acc = (acc + part).astype(np.float32)
    gs = orc.moe_shared_gate(small.gate_inp_shexp, xq, xd, N)
    h = orc.moe_expert_h(small.gate_shexp, small.up_shexp, N, F, xq, xd, xs)
    hq, hd, hs = orc.q8k_quant(h)
    rb = small.down_shexp.size // N
    sh = np.array([orc.q8k_dot(small.down_shexp[r * rb:(r + 1) * rb], small.t_down_shexp,
                               hq, hd, hs, F) for r in range(N)], np.float32)
    acc = (acc + np.float32(gs) * sh).astype(np.float32)
    assert np.array_equal(out, acc)


def test_moe_ffn_thread_independent(orc, small):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(3 * small.n_embd).astype(np.float32)
    orc.set_threads(1)
    a = orc.moe_ffn(small, x, 3)
    orc.set_threads(4)
    b = orc.moe_ffn(small, x, 3)
    orc.set_threads(1)
    assert np.array_equal(a, b)
    # batched tokens equal single-token calls
    for t in range(3):
        assert np.array_equal(a[t], orc.moe_ffn(small, x[t * small.n_embd:(t + 1) * small.n_embd], 1)[0])


def test_moe_stack_is_residual_chain(orc):
    layers = [make_host_layer(orc, seed=40 + i, n_embd=256, n_ff=256, n_expert=8, n_used=2)
              for i in range(3)]
    x = orc.fill_normal(9, 256, 0.0, 1.0)
    got = orc.moe_stack(layers, x)
    y = x.copy()
    for L in layers:
        y = (orc.moe_ffn(L, y, 1)[0] + y).astype(np.float32)
    assert np.array_equal(got, y)


def _f64_layer_f32(hl, x, sel, w, gate_on_q8k=False, swap_gate_up=False):
    """The QMA_NOQ8K layer (nn.c:393-407, 475-492, 576-629) in fp64 from the
    closed-form dequantised weights; the two flags plant plausible mistakes
    (the q8k path's shared gate on Q8_K(x); silu taken of the up dot)."""
    N, F, E = hl.n_embd, hl.n_ff, hl.n_expert
    x64 = x.astype(np.float64)

    def deq(raw, wtype, rows, cols):
        f = onp.q4k_dequant if wtype == 12 else onp.q6k_dequant
        return f(raw).astype(np.float64).reshape(rows, cols)

    def expert(ge, ue, de, dt):
        g = deq(ge, 12, F, N) @ x64
        u = deq(ue, 12, F, N) @ x64
        if swap_gate_up:
            g, u = u, g
        h = g / (1.0 + np.exp(-g)) * u
        return deq(de, dt, N, F) @ h

    gb, db = hl.gate_exps.size // E, hl.down_exps.size // E
    out = np.zeros(N)
    for k, e in enumerate(sel):
        out += np.float64(w[k]) * expert(hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb],
                                         hl.down_exps[e * db:(e + 1) * db], hl.t_down_exps)
    if gate_on_q8k:
        xq, xd, _ = onp.q8k_quant(x)
        xin = xq.astype(np.float64) * np.repeat(xd.astype(np.float64), 256)
    else:
        xin = x64
    gs = 1.0 / (1.0 + np.exp(-(hl.gate_inp_shexp.astype(np.float64) @ xin)))
    return out + gs * expert(hl.gate_shexp, hl.up_shexp, hl.down_shexp, hl.t_down_shexp)


@pytest.mark.parametrize("t_down", [14, 12])
def test_moe_ffn_f32_vs_fp64(orc, t_down):
    """orc_moe_ffn_f32 (the fp32 twin) against its fp64 closed form on the
    oracle's own routing, within 2e-5 of max|out| (fp32 dots of 512 and 256
    terms); the shared gate on Q8_K(x) and silu of the wrong dot each move the
    output well beyond that bound, so the check tells them apart.  Also the
    known distance to the q8k layer (activation quantisation, ~1e-2 here)."""
    hl = make_host_layer(orc, seed=21, n_embd=512, n_ff=256, n_expert=16, n_used=4, t_down=t_down)
    x = orc.fill_normal(8, 2 * 512, 0.0, 1.0)
    got = orc.moe_ffn_f32(hl, x, 2)
    for t in range(2):
        xt = x[t * 512:(t + 1) * 512]
        sel, w, _ = orc.moe_route(hl, xt)
        ref = _f64_layer_f32(hl, xt, sel, w)
        scale = np.max(np.abs(ref))
        err = np.max(np.abs(got[t] - ref)) / scale
        assert err < 2e-5, err
        for wrong in (dict(gate_on_q8k=True), dict(swap_gate_up=True)):
            alt = _f64_layer_f32(hl, xt, sel, w, **wrong)
            assert np.max(np.abs(alt - ref)) / scale > 10 * 2e-5, wrong
        q8 = orc.moe_ffn(hl, xt, 1)[0]
        assert 1e-4 < np.max(np.abs(q8 - got[t])) / scale < 5e-2
