"""GPU parity of the MoE FFN layer (nn.c:509-707) and the decode layer stack,
through the C-ABI, against the CPU oracle on the same bytes.

Stage-wise: router logits (fp32, 1e-4 of max|logit|), the top-n_used
selection (the set exact whenever the oracle's n_used-th / next probability
gap is not a near-tie, the slot order whenever no gap among the selected is),
renormalised weights, shared gate, h = silu(g)*u per slot, and the layer
output (1e-4 of max|y|)."""
import numpy as np
import pytest

from conftest import max_rel_err
from moe_fixtures import make_host_layer

pytestmark = pytest.mark.gpu

TOL = 1e-4
TIE = 1e-5        # relative probability gap below which a selection flip is a near-tie


def route_margin(logits, n_used):
    lg = logits.astype(np.float64)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    s = np.sort(p)[::-1]
    if n_used >= s.size:          # every expert is selected: no boundary to flip
        return np.inf
    return (s[n_used - 1] - s[n_used]) / s[n_used - 1]


def order_margin(logits, n_used):
    """Smallest relative gap between consecutive probabilities among the
    n_used largest: route_margin's boundary gap decides which experts are
    selected, these gaps decide the order of the slots among them."""
    lg = logits.astype(np.float64)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    s = np.sort(p)[::-1][:n_used]
    return np.inf if s.size < 2 else float(np.min((s[:-1] - s[1:]) / s[:-1]))


def check_selection(sel, w, sel_o, w_o, logits_o, K, where, weights=True):
    """The GPU's selected experts equal the oracle's whenever the boundary gap
    is above the near-tie margin, and their slot order too whenever every gap
    among them is (two selected experts a near-tie apart may take each
    other's slot: the set, and so the output up to fp32 association, is the
    same); each expert's weight within 1e-5."""
    if route_margin(logits_o, K) <= TIE:
        return
    assert sorted(int(e) for e in sel) == sorted(int(e) for e in sel_o), f"selection, {where}"
    if order_margin(logits_o, K) > TIE:
        assert list(sel) == list(sel_o), f"selection order, {where}"
    if weights:
        wg = {int(e): v for e, v in zip(sel, w)}
        for e, v in zip(sel_o, w_o):
            assert np.isclose(wg[int(e)], v, rtol=1e-5, atol=1e-7), f"weights, {where}"


def host_of(orc, rl):
    a = rl.host_arrays()
    return orc.HostLayer(rl.n_embd, rl.n_ff, rl.n_expert, rl.n_used, a["gate_inp"], a["gate_exps"],
                         a["up_exps"], a["down_exps"], rl.t_down, a["gate_inp_shexp"],
                         a["gate_shexp"], a["up_shexp"], a["down_shexp"], rl.t_down,
                         router_bias=a.get("router_bias"))


def run_layer(qm, rl, x, T):
    xb = qm.DBuf.from_array(x)
    ob = qm.DBuf(4 * T * rl.n_embd)
    qm.moe_ffn_dev(rl.c, xb.ptr, ob.ptr, T)
    return ob.download(np.float32).reshape(T, rl.n_embd)


def check_layer(qm, orc, rl, hl, x, T, run=None):
    """Stage by stage against the oracle on hl's bytes.  `run(x, T)` computes
    the layer on the device (default: qmag_moe_ffn_dev on rl) and leaves the
    stage buffers of its last call for moe_last_stage."""
    N, F, E, K = hl.n_embd, hl.n_ff, hl.n_expert, hl.n_used
    got = run(x, T) if run else run_layer(qm, rl, x, T)
    st = qm.moe_last_stage(E, K, F)
    # stage checks on token 0
    x0 = x[:N]
    sel_o, w_o, logits_o = orc.moe_route(hl, x0)
    assert max_rel_err(st["logits"], logits_o) < TOL
    check_selection(st["sel"], st["w"], sel_o, w_o, logits_o, K, "token 0")
    xq, xd, xs = orc.q8k_quant(x0)
    assert abs(st["gs"] - orc.moe_shared_gate(hl.gate_inp_shexp, xq, xd, N)) < 1e-6
    gb = hl.gate_exps.size // E
    for k in range(K):
        e = int(st["sel"][k])
        h = orc.moe_expert_h(hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb],
                             N, F, xq, xd, xs)
        assert max_rel_err(st["h"][k], h) < TOL
    hsh = orc.moe_expert_h(hl.gate_shexp, hl.up_shexp, N, F, xq, xd, xs)
    assert max_rel_err(st["h"][K], hsh) < TOL
    # full outputs, per token; near-tie tokens are run with the GPU routing
    ref = orc.moe_ffn(hl, x, T)
    compared = 0
    for t in range(T):
        _, _, lg = orc.moe_route(hl, x[t * N:(t + 1) * N])
        if route_margin(lg, K) > TIE:
            assert max_rel_err(got[t], ref[t]) < TOL, f"token {t}"
            compared += 1
    assert compared >= max(1, T - 1)
    return got


@pytest.mark.parametrize("cfg", [
    dict(n_embd=512, n_ff=256, n_expert=16, n_used=4, t_down=14),
    dict(n_embd=256, n_ff=512, n_expert=12, n_used=8, t_down=12),
    dict(n_embd=1024, n_ff=1024, n_expert=64, n_used=6, t_down=14),
    dict(n_embd=2048, n_ff=512, n_expert=32, n_used=8, t_down=12),
    dict(n_embd=4096, n_ff=256, n_expert=16, n_used=4, t_down=14),
])
def test_moe_layer_small_shapes(qm, orc, cfg):
    hl = make_host_layer(orc, seed=11, **cfg)
    rl = qm.ResidentLayer.from_host(hl)
    for T in (1, 3):
        x = orc.fill_normal(100 + T, T * cfg["n_embd"], 0.0, 1.0)
        check_layer(qm, orc, rl, hl, x, T)
    rl.close()


@pytest.fixture(params=["fused", "sequence"])
def decode_path(request, qm):
    """Batch-1 decode runs as the persistent fused kernel or as the
    per-stage launch sequence; both must meet the same bar."""
    qm.set_fused(request.param == "fused")
    yield request.param
    qm.set_fused(True)


@pytest.mark.parametrize("t_down", [14, 12])
def test_moe_layer_qwen35moe_shape(qm, orc, t_down, decode_path):
    """C3: hidden 2048, 256 experts, top-8, expert ff 512, shared expert,
    Q4_K gate/up, Q6_K (or Q4_K) down; weights generated in HBM."""
    rl = qm.ResidentLayer(seed=3, layer=0, t_down=t_down)
    hl = host_of(orc, rl)
    for s in (5, 6, 7):
        x = orc.fill_normal(s, 2048, 0.0, 1.0)
        check_layer(qm, orc, rl, hl, x, 1)
    x4 = orc.fill_normal(6, 4 * 2048, 0.0, 1.0)
    check_layer(qm, orc, rl, hl, x4, 4)
    rl.close()


@pytest.mark.parametrize("n_used,n_expert", [(1, 256), (6, 40), (8, 8)])
def test_moe_layer_fused_small_routing(qm, orc, n_used, n_expert):
    """The fused kernel with fewer experts / fewer routed slots than the
    qwen35moe defaults (hidden 2048 and ff 512 kept)."""
    hl = make_host_layer(orc, seed=23, n_embd=2048, n_ff=512, n_expert=n_expert, n_used=n_used)
    rl = qm.ResidentLayer.from_host(hl)
    x = orc.fill_normal(8, 2048, 0.0, 1.0)
    check_layer(qm, orc, rl, hl, x, 1)
    rl.close()


def random_cases(seed, n):
    """Seeded random layer configurations within what every path accepts:
    hidden 256..4096, ff 256..1024, 8..256 experts, 1..8 routed, either down
    type for the routed and the shared expert, an optional router bias, T
    from 1 to 31, the persistent kernel and the grouped prefill each on or
    off (layers whose shape or T they do not take use the launch sequence)."""
    rng = np.random.default_rng(seed)
    for _ in range(n):
        N = int(rng.choice([256, 512, 1024, 2048, 4096]))
        F = int(rng.choice([256, 512, 1024]))
        E = int(rng.integers(8, 257))
        while E * N * F > (1 << 25):
            E = max(8, E // 2)
        yield dict(N=N, F=F, E=E, K=int(rng.integers(1, min(8, E) + 1)), td=int(rng.choice([12, 14])),
                   tds=int(rng.choice([12, 14])), bias=None if rng.random() < 0.5 else 1.0,
                   T=int(rng.choice([1, 1, 2, 3, 5, 8, 9, 16, 31])), fused=bool(rng.random() < 0.7),
                   grouped=bool(rng.random() < 0.7), seed=int(rng.integers(1, 1 << 30)))
    # the persistent decode kernel's shape (hidden 2048, ff 512, one token,
    # one down type), with random expert counts and routing widths
    for _ in range(n // 2):
        td = int(rng.choice([12, 14]))
        yield dict(N=2048, F=512, E=int(rng.integers(8, 33)), K=int(rng.integers(1, 9)), td=td, tds=td,
                   bias=None if rng.random() < 0.5 else 1.0, T=1, fused=True, grouped=True,
                   seed=int(rng.integers(1, 1 << 30)))


def test_moe_random_configs_end_to_end(qm, orc):
    """Random shapes, routing widths, down types, token counts and paths,
    each token's output compared with the oracle's whole layer (not teacher
    forced), with the cause of any difference identified:
      - the output from the GPU's own h through the oracle's Q8_K(h), down
        projection and combine is within 1e-4 for every token;
      - a token whose Q8_K(h) bytes all equal the oracle's is within 1e-4
        end to end;
      - where they differ, at most two bytes differ, each by one step.
    h itself differs from the oracle's only in its last bits (the fp32
    epilogue of the gate/up dots is associated differently, and SiLU uses
    the device's expf): a value on a rounding boundary of the second
    quantization then moves one step, and the output by up to ~2e-3 of
    max|y| -- the sensitivity of the reference's own two-stage quantisation,
    which a build of the reference with other fp32 association shows too."""
    flips = compared = 0
    try:
        for c in random_cases(2024, 14):
            N, F, E, K, T = c["N"], c["F"], c["E"], c["K"], c["T"]
            qm.set_fused(c["fused"])
            qm.set_grouped(c["grouped"])
            hl = make_host_layer(orc, c["seed"], N, F, E, K, c["td"], router_bias_std=c["bias"],
                                 t_down_sh=c["tds"])
            rl = qm.ResidentLayer.from_host(hl)
            x = orc.fill_normal(c["seed"] + 1, T * N, 0.0, 1.0)
            got = run_layer(qm, rl, x, T)
            st = qm.moe_last_stage(E, K, F, n_tok=T)
            ref = orc.moe_ffn(hl, x, T).reshape(T, N)
            gb, db = hl.gate_exps.size // E, hl.down_exps.size // E
            for t in range(T):
                xt = x[t * N:(t + 1) * N]
                if route_margin(orc.moe_route(hl, xt)[2], K) <= TIE:
                    continue
                xq, xd, xs = orc.q8k_quant(xt)
                acc = np.zeros(N, np.float32)
                steps = []
                for s in range(K + 1):
                    if s < K:
                        e = int(st["sel"][t][s])
                        ge, ue = hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb]
                        dn, wt, scale = hl.down_exps[e * db:(e + 1) * db], hl.t_down_exps, st["w"][t][s]
                    else:
                        ge, ue = hl.gate_shexp, hl.up_shexp
                        dn, wt, scale = hl.down_shexp, hl.t_down_shexp, st["gs"][t]
                    hg = st["h"][t][s]
                    ho = orc.moe_expert_h(ge, ue, N, F, xq, xd, xs)
                    assert max_rel_err(hg, ho) < TOL, (c, t, s)
                    qg, qo = orc.q8k_quant(hg)[0].astype(np.int32), orc.q8k_quant(ho)[0].astype(np.int32)
                    steps += list(np.abs(qg - qo)[qg != qo])
                    y = orc.matmul_q8k(hg, dn, F, N, 1, wt)[0]
                    acc = (acc + (np.float32(scale) * y).astype(np.float32)).astype(np.float32)
                assert max_rel_err(got[t], acc) < TOL, ("teacher forced", c, t)
                compared += 1
                if steps:
                    flips += 1
                    assert len(steps) <= 2 and all(d == 1 for d in steps), (c, t, steps)
                else:
                    assert max_rel_err(got[t], ref[t]) < TOL, ("end to end", c, t)
            rl.close()
    finally:
        qm.set_fused(True)
        qm.set_grouped(True)
    assert compared >= 100
    assert flips <= compared // 10


def selected_layer(orc, rl, sel):
    """A host layer holding only what one token's layer needs from the GPU
    copy: the selected experts (renumbered 0..K-1 in pick order), the shared
    expert and its gate; its router rows are those of the selected experts.
    Downloads ~18 MB instead of a whole 526 MB layer."""
    N, F, E = rl.n_embd, rl.n_ff, rl.n_expert
    gb = rl.bytes_gate_slab
    db = rl.bytes_down_slab
    pick = lambda buf, e, nb: buf.download(np.uint8, nb, offset=int(e) * nb)
    ge = np.concatenate([pick(rl.gate_exps, e, gb) for e in sel])
    ue = np.concatenate([pick(rl.up_exps, e, gb) for e in sel])
    de = np.concatenate([pick(rl.down_exps, e, db) for e in sel])
    wr = np.concatenate([rl.gate_inp.download(np.float32, N, offset=4 * N * int(e)) for e in sel])
    return orc.HostLayer(N, F, len(sel), len(sel), wr, ge, ue, de, rl.t_down,
                         rl.gate_inp_shexp.download(np.float32), rl.gate_shexp.download(np.uint8),
                         rl.up_shexp.download(np.uint8), rl.down_shexp.download(np.uint8), rl.t_down)


def check_layer_vs_oracle(qm, orc, rl, Wr, xl, got, st, where):
    """One decode layer on x_l, stage by stage against independent forms:
    logits, selection (outside near-ties) and weights against the fp64 router;
    the shared gate and every slot's h against the oracle on the same Q8_K(x);
    the output against the oracle's down projection and combine with the
    GPU's routing (nn.c:509-649)."""
    import oracle_np as onp
    K, F, N = rl.n_used, rl.n_ff, rl.n_embd
    s64, w64, _, _ = onp.route_f64(Wr, xl, K)
    lg64 = Wr.astype(np.float64) @ xl.astype(np.float64)
    assert max_rel_err(st["logits"], lg64) < TOL, f"logits, {where}"
    check_selection(st["sel"], st["w"], s64, w64, lg64, K, where)
    hl = selected_layer(orc, rl, st["sel"])
    xq, xd, xs = orc.q8k_quant(xl)
    assert abs(st["gs"] - orc.moe_shared_gate(hl.gate_inp_shexp, xq, xd, N)) < 1e-6, f"gate, {where}"
    gb = hl.gate_exps.size // K
    for k in range(K):
        h = orc.moe_expert_h(hl.gate_exps[k * gb:(k + 1) * gb], hl.up_exps[k * gb:(k + 1) * gb], N, F, xq, xd, xs)
        assert max_rel_err(st["h"][k], h) < TOL, f"h slot {k}, {where}"
    hsh = orc.moe_expert_h(hl.gate_shexp, hl.up_shexp, N, F, xq, xd, xs)
    assert max_rel_err(st["h"][K], hsh) < TOL, f"h shared, {where}"
    # the down projection and combine start from the GPU's own h (requantised
    # on the host): a last-bit difference in h that moves one Q8_K(h) value by
    # one step moves y by ~3e-4 of max|y| by itself, so a recomputed h could
    # neither confirm nor rule out an error here; the h check above bounds it
    db = hl.down_exps.size // K
    acc = np.zeros(N, np.float32)
    for k in range(K + 1):
        dn, scale = (hl.down_exps[k * db:(k + 1) * db], st["w"][k]) if k < K else (hl.down_shexp, st["gs"])
        y = orc.matmul_q8k(st["h"][k], dn, F, N, 1, rl.t_down)[0]
        acc = (acc + (np.float32(scale) * y).astype(np.float32)).astype(np.float32)
    assert max_rel_err(got, acc) < TOL, f"output, {where}"


def test_moe_decode_paths_agree_40_layers(qm, orc):
    """40 qwen35moe layers x 2 tokens (the C4 stack).

    1. Teacher-forced, layer by layer on the persistent kernel's own x_l
       (as qma_eval feeds moe_ffn, nn.c:2246-2252): every layer is checked
       stage by stage against the oracle and fp64 forms
       (check_layer_vs_oracle), and the persistent kernel and the launch
       sequence (independent kernels) agree to 1e-4 of max|y|.
    2. One 40-layer launch of the persistent kernel equals the same kernel
       applied one layer per launch bit for bit, so the hand-off of x between
       layers inside the kernel adds nothing.
    End to end the two paths are not compared at 1e-4: their fp32 sums are
    associated differently (router dot, softmax sum, shared gate), which
    moves h in the last bit and, rarely, one Q8_K(h) value by one step; over
    40 residual layers these steps reach ~1e-4 by themselves."""
    rls = [qm.ResidentLayer(seed=404, layer=l) for l in range(40)]
    cl = [r.c for r in rls]
    Wrs = [r.gate_inp.download(np.float32).reshape(r.n_expert, r.n_embd) for r in rls]
    x = orc.fill_normal(41, 2 * 2048, 0.0, 1.0)
    for t in range(2):
        xt = x[t * 2048:(t + 1) * 2048]
        # 1. layer-by-layer teacher forcing
        xl = xt.copy()
        for l in range(40):
            outs = []
            for fused in (True, False):
                qm.set_fused(fused)
                outs.append(run_layer(qm, rls[l], xl, 1)[0])
                if fused:
                    st = qm.moe_last_stage(256, 8, 512)
                    check_layer_vs_oracle(qm, orc, rls[l], Wrs[l], xl, outs[0], st, f"token {t} layer {l}")
            qm.set_fused(True)
            assert max_rel_err(outs[0], outs[1]) < TOL, f"token {t} layer {l}"
            xb = qm.DBuf.from_array(xl)
            qm.moe_stack_dev([cl[l]], xb.ptr, 1)          # x_{l+1} = x_l + moe_l(x_l)
            xl = xb.download(np.float32)
        # 2. one launch over all 40 layers
        xb = qm.DBuf.from_array(xt)
        qm.moe_stack_dev(cl, xb.ptr, 1)
        assert np.array_equal(xb.download(np.float32).view(np.uint32), xl.view(np.uint32))
    for r in rls:
        r.close()


def test_moe_layer_prefill_skewed_router(qm, orc):
    """C5 routing: router logits skewed by a seeded per-expert bias ~N(0,1)."""
    rl = qm.ResidentLayer(seed=9, layer=0, router_bias_std=1.0)
    hl = host_of(orc, rl)
    x = orc.fill_normal(15, 16 * 2048, 0.0, 1.0)
    check_layer_staged(qm, orc, rl, hl, x, 16)
    rl.close()


def check_layer_staged(qm, orc, rl, hl, x, T, stage1_tokens=None, run=None):
    """All T tokens, stage by stage with teacher forcing (for batches, where
    many tokens are compared):
      1. logits, selection (outside near-ties), weights and shared gate
         against the oracle's router on the same x;
      2. h per (token, slot) against the oracle's gate/up + SwiGLU of the
         expert the GPU selected;
      3. the output against the oracle's down projection (Q8_K of the GPU's
         own h, requantised on the host) and combine, with the GPU's weights.
    Stage 3 starts from the GPU's h so that a last-bit difference in h --
    the fp32 epilogues are associated differently -- which moves one Q8_K(h)
    value by one step cannot fake or mask an error in the down projection;
    stage 2 bounds that difference at the 1e-4 tolerance.  `run(x, T)`, if
    given, computes the layer in place of qmag_moe_ffn_dev on rl."""
    N, F, E, K = hl.n_embd, hl.n_ff, hl.n_expert, hl.n_used
    S = K + 1
    got = run(x, T) if run else run_layer(qm, rl, x, T)
    st = qm.moe_last_stage(E, K, F, n_tok=T)
    gb, db = hl.gate_exps.size // E, hl.down_exps.size // E
    tokens = range(T) if stage1_tokens is None else stage1_tokens
    for t in tokens:
        xt = x[t * N:(t + 1) * N]
        sel_o, w_o, lg_o = orc.moe_route(hl, xt)
        assert max_rel_err(st["logits"][t], lg_o) < TOL, f"logits, token {t}"
        check_selection(st["sel"][t], st["w"][t], sel_o, w_o, lg_o, K, f"token {t}")
        xq, xd, xs = orc.q8k_quant(xt)
        assert abs(st["gs"][t] - orc.moe_shared_gate(hl.gate_inp_shexp, xq, xd, N)) < 1e-6
        for s in range(S):
            if s < K:
                e = int(st["sel"][t][s])
                ge, ue = hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb]
            else:
                ge, ue = hl.gate_shexp, hl.up_shexp
            h = orc.moe_expert_h(ge, ue, N, F, xq, xd, xs)
            assert max_rel_err(st["h"][t][s], h) < TOL, f"h, token {t} slot {s}"
    for t in range(T):
        acc = np.zeros(N, np.float32)
        for s in range(S):
            if s < K:
                e = int(st["sel"][t][s])
                dn, wt, scale = hl.down_exps[e * db:(e + 1) * db], hl.t_down_exps, st["w"][t][s]
            else:
                dn, wt, scale = hl.down_shexp, hl.t_down_shexp, st["gs"][t]
            y = orc.matmul_q8k(st["h"][t][s], dn, F, N, 1, wt)[0]
            acc = (acc + (np.float32(scale) * y).astype(np.float32)).astype(np.float32)
        assert max_rel_err(got[t], acc) < TOL, f"output, token {t}"
    return got


@pytest.mark.parametrize("cfg", [
    dict(n_embd=512, n_ff=256, n_expert=16, n_used=4, t_down=14),
    dict(n_embd=256, n_ff=512, n_expert=12, n_used=8, t_down=12),
    dict(n_embd=1024, n_ff=1024, n_expert=64, n_used=6, t_down=14),
    dict(n_embd=2048, n_ff=512, n_expert=32, n_used=8, t_down=12),
    dict(n_embd=4096, n_ff=256, n_expert=16, n_used=4, t_down=14),
])
def test_moe_grouped_small_shapes(qm, orc, cfg):
    """Batches of >= 8 tokens run the grouped int8-MFMA expert GEMM; ragged
    counts (37 tokens) leave partial 16-pair blocks in most buckets."""
    hl = make_host_layer(orc, seed=13, **cfg)
    rl = qm.ResidentLayer.from_host(hl)
    for T in (8, 37):
        x = orc.fill_normal(300 + T, T * cfg["n_embd"], 0.0, 1.0)
        check_layer_staged(qm, orc, rl, hl, x, T)
    rl.close()


def test_moe_grouped_sequence_option(qm, orc):
    """QMAG_OPT_GROUPED = 0 sends a batch through the per-token launch
    sequence, which is checked against the oracle the same way."""
    hl = make_host_layer(orc, seed=17, n_embd=512, n_ff=256, n_expert=16, n_used=4, t_down=14)
    rl = qm.ResidentLayer.from_host(hl)
    x = orc.fill_normal(77, 12 * 512, 0.0, 1.0)
    qm.set_grouped(False)
    try:
        check_layer_staged(qm, orc, rl, hl, x, 12)
    finally:
        qm.set_grouped(True)
    rl.close()


def test_moe_prefill_c5_shape(qm, orc):
    """C5: 512 tokens, router skewed by a per-expert bias ~N(0,1) (4096
    routed pairs over a skewed set of experts), against the oracle: every
    token's output (stage 3), the router and h of every 8th token."""
    rl = qm.ResidentLayer(seed=55, layer=0, router_bias_std=1.0)
    hl = host_of(orc, rl)
    x = orc.fill_normal(512, 512 * 2048, 0.0, 1.0)
    orc.set_threads(8)
    try:
        check_layer_staged(qm, orc, rl, hl, x, 512, stage1_tokens=range(0, 512, 8))
    finally:
        orc.set_threads(1)
    rl.close()


def test_moe_grouped_repeatable(qm):
    """The grouped prefill gives the same bits on every call: bucket positions
    come from LDS atomics, but each pair's h and y are computed apart from the
    others, the router's k-chunk partials are summed in a fixed order, and the
    combine follows the reference's slot order.  Two calls on the C5 shape and
    one on a ragged batch, each repeated, compared bit for bit."""
    rl = qm.ResidentLayer(seed=57, layer=0, router_bias_std=1.0)
    for T, seed in ((512, 5), (37, 6)):
        x = np.random.default_rng(seed).standard_normal((T, 2048)).astype(np.float32)
        a = run_layer(qm, rl, x, T)
        b = run_layer(qm, rl, x, T)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"T={T}"
    rl.close()


def test_moe_prefill_large_ragged_batch(qm, orc):
    """A batch three times C5's and not a multiple of the 64-token router
    tile (T = 1500: 12,000 routed pairs, about 400 chunks, a partial router
    tile row), against the oracle: every token's output (stage 3), the router
    and h of every 50th token."""
    rl = qm.ResidentLayer(seed=58, layer=0, router_bias_std=1.0)
    hl = host_of(orc, rl)
    T = 1500
    x = orc.fill_normal(1500, T * 2048, 0.0, 1.0)
    orc.set_threads(8)
    try:
        check_layer_staged(qm, orc, rl, hl, x, T, stage1_tokens=range(0, T, 50))
    finally:
        orc.set_threads(1)
    rl.close()


@pytest.mark.parametrize("t_down,t_down_sh", [(14, 12), (12, 14)])
def test_moe_layer_mixed_down_types(qm, orc, t_down, t_down_sh):
    """The shared expert's down tensor in another type than the routed ones
    (GGUF files mix Q4_K and Q6_K per tensor): one token (the fused decode
    takes only one down type, so this runs the launch sequence), 3 tokens
    (the launch sequence) and 37 (the grouped prefill, whose down kernel picks
    the type per bucket), against the oracle."""
    hl = make_host_layer(orc, seed=71, n_embd=2048, n_ff=512, n_expert=32, n_used=8, t_down=t_down,
                         t_down_sh=t_down_sh)
    rl = qm.ResidentLayer.from_host(hl)
    for T in (1, 3, 37):
        x = orc.fill_normal(900 + T, T * 2048, 0.0, 1.0)
        check_layer_staged(qm, orc, rl, hl, x, T)
    rl.close()


def test_moe_stack_small(qm, orc):
    cfg = dict(n_embd=512, n_ff=256, n_expert=16, n_used=4)
    hls = [make_host_layer(orc, seed=60 + i, **cfg) for i in range(4)]
    rls = [qm.ResidentLayer.from_host(h) for h in hls]
    n_tok = 3
    x = orc.fill_normal(21, n_tok * 512, 0.0, 1.0)
    xb = qm.DBuf.from_array(x)
    qm.moe_stack_dev([r.c for r in rls], xb.ptr, n_tok)
    got = xb.download(np.float32).reshape(n_tok, 512)
    for t in range(n_tok):
        ref = orc.moe_stack(hls, x[t * 512:(t + 1) * 512])
        assert max_rel_err(got[t], ref) < TOL


def test_moe_stack_qwen35moe_shape(qm, orc, decode_path):
    rls = [qm.ResidentLayer(seed=77, layer=l) for l in range(2)]
    hls = [host_of(orc, r) for r in rls]
    x = orc.fill_normal(31, 2 * 2048, 0.0, 1.0)
    xb = qm.DBuf.from_array(x)
    qm.moe_stack_dev([r.c for r in rls], xb.ptr, 2)
    got = xb.download(np.float32).reshape(2, 2048)
    for t in range(2):
        ref = orc.moe_stack(hls, x[t * 2048:(t + 1) * 2048])
        assert max_rel_err(got[t], ref) < TOL


def test_moe_layer_descriptor_reuse(qm):
    """One-layer decode calls keep each distinct layer descriptor resident on
    the device, found by content: alternating layers must give the same
    bits as the first call on each, and a descriptor rewritten in place at
    the same host address must be seen with its new contents."""
    rls = [qm.ResidentLayer(seed=91, layer=l) for l in range(2)]
    x = qm.DBuf.from_array(np.random.default_rng(5).standard_normal(2048).astype(np.float32))
    outs = [qm.DBuf(4 * 2048) for _ in range(4)]

    def run(desc, o):
        qm.moe_ffn_dev(desc, x.ptr, o.ptr, 1)
        qm.sync()
        return o.download(np.float32).view(np.uint32).copy()

    a0 = run(rls[0].c, outs[0])
    a1 = run(rls[1].c, outs[1])
    a2 = run(rls[0].c, outs[2])
    assert np.array_equal(a0, a2)
    assert not np.array_equal(a0, a1)
    desc = type(rls[1].c).from_buffer_copy(rls[1].c)
    assert np.array_equal(run(desc, outs[3]), a1)
    for name, _ in type(desc)._fields_:
        setattr(desc, name, getattr(rls[0].c, name))
    assert np.array_equal(run(desc, outs[3]), a0)
    for r in rls:
        r.close()


def test_moe_prefill_concentrated_router(qm, orc):
    """Every token routed to the same 8 experts (a +40 logit bias on experts
    3, 17, ..): 8 buckets of 256 pairs plus the shared one, so the grouped
    GEMMs run only full 64-pair chunks, four per expert -- the case where
    one expert's rows are read by several chunks and the chunk list holds
    no partial chunk."""
    rl = qm.ResidentLayer(seed=123, layer=0, router_bias_std=1.0)
    hot = [3, 17, 60, 61, 99, 128, 200, 255]
    bias = np.random.default_rng(9).standard_normal(256).astype(np.float32) * 0.1
    bias[hot] += np.float32(40.0) + np.arange(8, dtype=np.float32)
    rl.router_bias.upload(bias)
    hl = host_of(orc, rl)
    T = 256
    x = orc.fill_normal(808, T * 2048, 0.0, 1.0)
    orc.set_threads(8)
    try:
        check_layer_staged(qm, orc, rl, hl, x, T, stage1_tokens=range(0, T, 16))
    finally:
        orc.set_threads(1)
    st = qm.moe_last_stage(256, 8, 512, n_tok=T)
    assert sorted(set(st["sel"].ravel().tolist())) == sorted(hot)
    rl.close()


LEAD = [12, 140, 77, 205]                          # biases 53, 52, 51, 50
TIED = [250, 7, 71, 135, 199, 3, 67, 131, 195, 100]  # all 40.0


@pytest.mark.parametrize("path,T", [("fused", 1), ("sequence", 1), ("sequence", 3), ("grouped", 16)])
def test_moe_route_exact_ties_lowest_index(qm, orc, path, T):
    """Logits tied exactly (a zero router, so the logits are the biases):
    among equal probabilities the reference's strict-> scan keeps the lowest
    expert index (nn.c:526-533).  Four experts lead; ten more share one
    bias, spread over the lanes and list positions of the top-K (expert e
    sits in lane e % 64, position e // 64; lanes 3 and 7 each hold four of
    them), so the last four slots go to 3, 7, 67, 71 in that order."""
    rl = qm.ResidentLayer(seed=321, layer=0, router_bias_std=1.0)
    rl.gate_inp.upload(np.zeros(256 * 2048, np.float32))
    bias = (np.random.default_rng(5).standard_normal(256) * 0.1).astype(np.float32)
    bias[LEAD] = np.array([53.0, 52.0, 51.0, 50.0], np.float32)
    bias[TIED] = np.float32(40.0)
    rl.router_bias.upload(bias)
    hl = host_of(orc, rl)
    x = orc.fill_normal(909 + T, T * 2048, 0.0, 1.0)
    qm.set_fused(path == "fused")
    try:
        got = run_layer(qm, rl, x, T)
        st = qm.moe_last_stage(256, 8, 512, n_tok=T)
    finally:
        qm.set_fused(True)
    want = LEAD + [3, 7, 67, 71]
    for t in range(T):
        sel_o, w_o, _ = orc.moe_route(hl, x[t * 2048:(t + 1) * 2048])
        assert list(sel_o) == want                 # the oracle keeps the same rule
        assert st["sel"][t].tolist() == want, f"token {t}"
        assert np.allclose(st["w"][t], w_o, rtol=1e-5, atol=1e-7), f"token {t}"
    ref = orc.moe_ffn(hl, x, T)
    for t in range(T):
        assert max_rel_err(got[t], ref[t]) < TOL, f"token {t}"
    rl.close()


def test_fused_launch_options_bit_identical(qm):
    """The persistent decode kernel gives the same bits launched
    cooperatively (QMAG_OPT_COOP) and with phase tracing on (QMAG_OPT_TRACE,
    which only adds timestamp stores) as in its default ordinary launch; the
    trace holds the launch's phase stamps (100 MHz counter, one launch well
    under a second)."""
    rls = [qm.ResidentLayer(seed=77, layer=l) for l in range(4)]
    cl = [r.c for r in rls]
    x = np.random.default_rng(3).standard_normal(2048).astype(np.float32)

    def run():
        xb = qm.DBuf.from_array(x)
        qm.moe_stack_dev(cl, xb.ptr, 1)
        return xb.download(np.float32)

    base = run()
    qm.set_coop(True)
    try:
        coop = run()
    finally:
        qm.set_coop(False)
    qm.set_trace(True)
    try:
        traced = run()
        tr = qm.trace_read(4)
    finally:
        qm.set_trace(False)
    again = run()
    for other in (coop, traced, again):
        assert np.array_equal(base.view(np.uint32), other.view(np.uint32))
    stamps = tr[tr > 0]
    assert stamps.size > 512
    assert int(stamps.max() - stamps.min()) < 100_000_000
    for r in rls:
        r.close()


def test_fused_abort_recovery_one_layer(qm, orc):
    """A persistent launch that finds its abort word set (as after an expired
    wait) writes no output; the next qmag_d2h re-runs the call through the
    launch sequence, so the caller reads the sequence path's result, and the
    next call runs the persistent kernel normally again."""
    rl = qm.ResidentLayer(seed=3, layer=0)
    hl_route = rl.gate_inp.download(np.float32).reshape(256, 2048)
    x = orc.fill_normal(12, 2048, 0.0, 1.0)
    qm.set_fused(False)
    want = run_layer(qm, rl, x, 1)[0]
    qm.set_fused(True)
    n0 = qm.fused_recoveries()
    qm.arm_test_abort(1)
    got = run_layer(qm, rl, x, 1)[0]
    assert qm.fused_recoveries() == n0 + 1
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    st = qm.moe_last_stage(256, 8, 512)
    check_layer_vs_oracle(qm, orc, rl, hl_route, x, got, st, "recovered")
    again = run_layer(qm, rl, x, 1)[0]           # the persistent kernel, armed again
    assert qm.fused_recoveries() == n0 + 1
    st = qm.moe_last_stage(256, 8, 512)
    check_layer_vs_oracle(qm, orc, rl, hl_route, x, again, st, "after recovery")
    rl.close()


@pytest.mark.parametrize("nth", [1, 2, 3])
def test_fused_abort_recovery_stack(qm, orc, nth):
    """Stack calls update x in place: with the nth launch of a 3-token call
    aborted, the tokens before it keep the persistent kernel's result and the
    rest are restored from the copy taken before the call and re-run through
    the launch sequence."""
    rls = [qm.ResidentLayer(seed=90, layer=l) for l in range(4)]
    cl = [r.c for r in rls]
    x = orc.fill_normal(13, 3 * 2048, 0.0, 1.0)
    res = {}
    for fused in (True, False):
        qm.set_fused(fused)
        xb = qm.DBuf.from_array(x)
        qm.moe_stack_dev(cl, xb.ptr, 3)
        res[fused] = xb.download(np.float32).reshape(3, 2048)
    qm.set_fused(True)
    n0 = qm.fused_recoveries()
    qm.arm_test_abort(nth)
    xb = qm.DBuf.from_array(x)
    qm.moe_stack_dev(cl, xb.ptr, 3)
    got = xb.download(np.float32).reshape(3, 2048)
    assert qm.fused_recoveries() == n0 + 1
    for t in range(3):
        want = res[True][t] if t < nth - 1 else res[False][t]
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), f"token {t}"
    for r in rls:
        r.close()


MIXED = [(14, 14), (14, 14), (12, 12), (12, 12), (14, 12), (14, 14)]   # (routed, shared) down types


def _mixed_stack(qm, orc):
    hls = [make_host_layer(orc, seed=80 + i, n_embd=2048, n_ff=512, n_expert=64, n_used=8, t_down=td,
                           t_down_sh=ts) for i, (td, ts) in enumerate(MIXED)]
    return hls, [qm.ResidentLayer.from_host(h) for h in hls]


def test_moe_stack_mixed_down_types(qm, orc):
    """A stack whose down types change from layer to layer (GGUF quant mixes
    do) and with one layer whose shared expert is typed apart: the persistent
    kernel takes the runs of layers it can (here layers 0-1, 2-3 and 5), the
    launch sequence the rest.  Every token equals the layers applied one call
    at a time (each through the path that takes it alone) bit for bit, and
    each of those layers is checked against the oracle stage by stage on its
    own input (teacher forcing: end to end, a near-tie in one layer's routing
    may pick another expert on either side)."""
    hls, rls = _mixed_stack(qm, orc)
    n_tok = 3
    x = orc.fill_normal(33, n_tok * 2048, 0.0, 1.0)
    xb = qm.DBuf.from_array(x)
    qm.moe_stack_dev([r.c for r in rls], xb.ptr, n_tok)
    got = xb.download(np.float32).reshape(n_tok, 2048)
    for t in range(n_tok):
        xl = x[t * 2048:(t + 1) * 2048].copy()
        for r, h in zip(rls, hls):
            check_layer_staged(qm, orc, r, h, xl, 1)
            b = qm.DBuf.from_array(xl)
            qm.moe_stack_dev([r.c], b.ptr, 1)
            xl = b.download(np.float32)
        assert np.array_equal(got[t].view(np.uint32), xl.view(np.uint32)), f"token {t}"
    for r in rls:
        r.close()


@pytest.mark.parametrize("nth", [2, 5])
def test_fused_abort_recovery_mixed_stack(qm, orc, nth):
    """With the nth persistent launch of a mixed stack's call aborted (3 fused
    runs per token), the tokens before its token keep the mixed path's result
    and the rest are restored and re-run through the launch sequence."""
    hls, rls = _mixed_stack(qm, orc)
    cl = [r.c for r in rls]
    x = orc.fill_normal(14, 3 * 2048, 0.0, 1.0)
    res = {}
    for fused in (True, False):
        qm.set_fused(fused)
        xb = qm.DBuf.from_array(x)
        qm.moe_stack_dev(cl, xb.ptr, 3)
        res[fused] = xb.download(np.float32).reshape(3, 2048)
    qm.set_fused(True)
    n0 = qm.fused_recoveries()
    qm.arm_test_abort(nth)
    xb = qm.DBuf.from_array(x)
    qm.moe_stack_dev(cl, xb.ptr, 3)
    got = xb.download(np.float32).reshape(3, 2048)
    assert qm.fused_recoveries() == n0 + 1
    for t in range(3):
        want = res[True][t] if t < (nth - 1) // 3 else res[False][t]
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), f"token {t}"
    for r in rls:
        r.close()


@pytest.mark.parametrize("n_used", [1, 2, 3])
def test_stack_small_n_used(qm, orc, n_used):
    """Multi-layer decode with fewer than 4 routed experts per token (not
    eligible for a multi-layer persistent launch, whose one-slot hand-offs
    need every workgroup on each layer's dependency chain, so every layer
    runs as its own one-layer launch): 4 layers.  The stack equals its layers
    chained one call at a time bit for bit, and each layer is checked against
    the oracle stage by stage on the GPU's own x_l."""
    hls = [make_host_layer(orc, seed=70 + i, n_embd=2048, n_ff=512, n_expert=32, n_used=n_used)
           for i in range(4)]
    rls = [qm.ResidentLayer.from_host(h) for h in hls]
    x = orc.fill_normal(22, 2 * 2048, 0.0, 1.0)
    xb = qm.DBuf.from_array(x)
    qm.moe_stack_dev([r.c for r in rls], xb.ptr, 2)
    got = xb.download(np.float32).reshape(2, 2048)
    for t in range(2):
        xl = x[t * 2048:(t + 1) * 2048].copy()
        for l in range(4):
            check_layer_staged(qm, orc, rls[l], hls[l], xl, 1)
            b = qm.DBuf.from_array(xl)
            qm.moe_stack_dev([rls[l].c], b.ptr, 1)
            xl = b.download(np.float32)
        assert np.array_equal(got[t].view(np.uint32), xl.view(np.uint32)), f"token {t}"
    for r in rls:
        r.close()


@pytest.mark.parametrize("case", ["nan_row", "inf_bias", "all_below_1e30", "all_at_1e30"])
@pytest.mark.parametrize("path", ["fused", "sequence", "grouped"])
def test_route_degenerate_softmax(qm, orc, case, path):
    """When the reference's softmax is NaN throughout -- a NaN logit, a +Inf
    logit, or every logit strictly below its -1e30 starting maximum -- its
    top-K scan picks expert 0 for every slot with weight -1e30 / (K * -1e30)
    (nn.c:517-536).  Every logit at exactly -1e30 is not degenerate: the
    maximum stays at -1e30, every term is expf(0) = 1 and the scan picks
    experts 0..K-1 (equal probabilities, lowest index first) with weight 1/K.
    Every GPU path makes the same picks and weights, and the output matches
    the oracle stage by stage."""
    E, K, N, F = 32, 8, 2048, 512
    hl = make_host_layer(orc, seed=88, n_embd=N, n_ff=F, n_expert=E, n_used=K, router_bias_std=0.0)
    wr = hl.gate_inp.reshape(E, N)
    bias = hl.router_bias
    if case == "nan_row":
        wr[5, 100] = np.nan
    elif case == "inf_bias":
        bias[9] = np.inf
    elif case == "all_below_1e30":
        bias[:] = -2e30
    else:
        bias[:] = -1e30            # the dot (|.| ~ 1) is absorbed: every logit is exactly -1e30
    rl = qm.ResidentLayer.from_host(hl)
    T = 16 if path == "grouped" else 1
    x = orc.fill_normal(19, T * N, 0.0, 1.0)
    qm.set_fused(path == "fused")
    try:
        got = run_layer(qm, rl, x, T)
        st = qm.moe_last_stage(E, K, F, n_tok=T)
    finally:
        qm.set_fused(True)
    gb, db = hl.gate_exps.size // E, hl.down_exps.size // E
    for t in range(T):
        xt = x[t * N:(t + 1) * N]
        sel_o, w_o, _ = orc.moe_route(hl, xt)
        assert list(sel_o) == (list(range(K)) if case == "all_at_1e30" else [0] * K)
        assert list(st["sel"][t]) == list(sel_o), f"token {t}"
        assert np.array_equal(st["w"][t].view(np.uint32), w_o.view(np.uint32)), f"token {t}"
        xq, xd, xs = orc.q8k_quant(xt)
        acc = np.zeros(N, np.float32)
        for s in range(K + 1):
            if s < K:
                e = int(sel_o[s])
                h = orc.moe_expert_h(hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb],
                                     N, F, xq, xd, xs)
                assert max_rel_err(st["h"][t][s], h) < TOL
                dn, scale = hl.down_exps[e * db:(e + 1) * db], st["w"][t][s]
            else:
                dn, scale = hl.down_shexp, st["gs"][t]
            y = orc.matmul_q8k(st["h"][t][s], dn, F, N, 1, hl.t_down_exps)[0]
            acc = (acc + (np.float32(scale) * y).astype(np.float32)).astype(np.float32)
        assert max_rel_err(got[t], acc) < TOL, f"output, token {t}"
    rl.close()


@pytest.mark.parametrize("cfg", [
    dict(n_embd=512, n_ff=256, n_expert=16, n_used=4, t_down=14),
    dict(n_embd=2048, n_ff=512, n_expert=32, n_used=8, t_down=12),
    dict(n_embd=1024, n_ff=1024, n_expert=64, n_used=6, t_down=14),
    dict(n_embd=4096, n_ff=256, n_expert=16, n_used=8, t_down=12),
])
def test_moe_layer_f32_vs_oracle(qm, orc, cfg):
    """qmag_moe_ffn_f32_dev, the QMA_NOQ8K layer (nn.c:393-407, 475-492, 585),
    against orc_moe_ffn_f32 on the same bytes, stage by stage: the router as
    the q8k branch's, the fp32 shared gate on fp32 x, h of every slot (fp32
    dequantise-then-dot, 1e-4 of max|h|) and the output (1e-4 of max|y|; no
    activation is requantised on this path, so the output is compared whole)
    for every token whose selection is not a near-tie."""
    hl = make_host_layer(orc, seed=31, **cfg)
    rl = qm.ResidentLayer.from_host(hl)
    N, F, E, K = hl.n_embd, hl.n_ff, hl.n_expert, hl.n_used
    gb = hl.gate_exps.size // E
    for T in (1, 5):
        x = orc.fill_normal(60 + T, T * N, 0.0, 1.0)
        xb = qm.DBuf.from_array(x)
        ob = qm.DBuf(4 * T * N)
        qm.moe_ffn_f32_dev(rl.c, xb.ptr, ob.ptr, T)
        got = ob.download(np.float32).reshape(T, N)
        st = qm.moe_last_stage(E, K, F, n_tok=T)
        ref = orc.moe_ffn_f32(hl, x, T)
        compared = 0
        for t in range(T):
            xt = x[t * N:(t + 1) * N]
            sel_o, w_o, lg_o = orc.moe_route(hl, xt)
            assert max_rel_err(st["logits"][t], lg_o) < TOL, f"logits, token {t}"
            assert abs(st["gs"][t] - orc.moe_shared_gate_f32(hl.gate_inp_shexp, xt, N)) < 1e-6
            for s in range(K + 1):
                if s < K:
                    e = int(st["sel"][t][s])
                    ge, ue = hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb]
                else:
                    ge, ue = hl.gate_shexp, hl.up_shexp
                h = orc.moe_expert_h_f32(ge, ue, N, F, xt)
                assert max_rel_err(st["h"][t][s], h) < TOL, f"h, token {t} slot {s}"
            if route_margin(lg_o, K) > TIE:
                check_selection(st["sel"][t], None, sel_o, None, lg_o, K, f"token {t}", weights=False)
                assert max_rel_err(got[t], ref[t]) < TOL, f"output, token {t}"
                compared += 1
        assert compared >= max(1, T - 1)
    rl.close()


@pytest.mark.parametrize("T", [1, 5, 16, 512])
def test_moe_ffn_host_equals_device(qm, orc, T):
    """qmag_moe_ffn_host (x and out in host memory, the engine's moe_ffn call)
    gives the bits of qmag_moe_ffn_dev on the same input: the persistent
    one-layer kernel (T = 1), the launch sequence (T = 5) and the grouped
    prefill (T = 16, and T = 512, the C5 batch, after the smaller calls: the
    pinned staging grows from one to 512 rows), the stage buffers those of
    the same path."""
    rl = qm.ResidentLayer(seed=7, layer=1)
    x = orc.fill_normal(90 + T, T * 2048, 0.0, 1.0)
    want = run_layer(qm, rl, x, T).reshape(-1)
    got = qm.moe_ffn_host(rl.c, x, T)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    again = qm.moe_ffn_host(rl.c, x, T)                # the staging reused
    assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
    rl.close()


def test_moe_ffn_host_recovers_expired_wait(qm, orc):
    """The host call's persistent launch finds its abort word set (the test
    hook, as after an expired wait): the call itself re-runs the layer through
    the launch sequence before copying out, so it returns that path's result,
    and the next host call runs the persistent kernel again."""
    rl = qm.ResidentLayer(seed=3, layer=0)
    x = orc.fill_normal(13, 2048, 0.0, 1.0)
    qm.set_fused(False)
    want_seq = qm.moe_ffn_host(rl.c, x, 1)
    qm.set_fused(True)
    want_fused = run_layer(qm, rl, x, 1).reshape(-1)
    n0 = qm.fused_recoveries()
    qm.arm_test_abort(1)
    got = qm.moe_ffn_host(rl.c, x, 1)
    assert qm.fused_recoveries() == n0 + 1
    assert np.array_equal(got.view(np.uint32), want_seq.view(np.uint32))
    again = qm.moe_ffn_host(rl.c, x, 1)
    assert qm.fused_recoveries() == n0 + 1
    assert np.array_equal(again.view(np.uint32), want_fused.view(np.uint32))
    with pytest.raises(qm.QmagError):
        qm.check(qm.lib().qmag_moe_ffn_host(qm.C.byref(rl.c), None, None, 1))
    rl.close()


def test_grouped_prefill_random_large_batches(qm, orc):
    """Seeded random layers through the grouped prefill at T from 65 to 300
    (buckets of many 64-pair chunks, partial chunks of every size, biased and
    unbiased routers): every token's selection checked as check_selection
    does, every 16th token teacher-forced stage by stage (h per slot, then the
    output from the GPU's h through the oracle's down projection and
    combine)."""
    rng = np.random.default_rng(4242)
    qm.set_grouped(True)
    for case in range(3):
        N = int(rng.choice([256, 512, 1024])); F = int(rng.choice([256, 512, 1024]))
        E = int(rng.integers(16, 129)); K = int(rng.integers(1, 9)); T = int(rng.integers(65, 301))
        td, tds = int(rng.choice([12, 14])), int(rng.choice([12, 14]))
        bias = None if case == 0 else float(case)
        hl = make_host_layer(orc, 5000 + case, N, F, E, K, td, router_bias_std=bias, t_down_sh=tds)
        rl = qm.ResidentLayer.from_host(hl)
        x = orc.fill_normal(5100 + case, T * N, 0.0, 1.0)
        got = run_layer(qm, rl, x, T)
        st = qm.moe_last_stage(E, K, F, n_tok=T)
        gb, db = hl.gate_exps.size // E, hl.down_exps.size // E
        for t in range(T):
            xt = x[t * N:(t + 1) * N]
            sel_o, w_o, lg_o = orc.moe_route(hl, xt)
            assert max_rel_err(st["logits"][t], lg_o) < TOL, (case, t)
            check_selection(st["sel"][t], st["w"][t], sel_o, w_o, lg_o, K, f"case {case} token {t}")
            if t % 16:
                continue
            xq, xd, xs = orc.q8k_quant(xt)
            acc = np.zeros(N, np.float32)
            for s in range(K + 1):
                if s < K:
                    e = int(st["sel"][t][s])
                    ge, ue = hl.gate_exps[e * gb:(e + 1) * gb], hl.up_exps[e * gb:(e + 1) * gb]
                    dn, wt, scale = hl.down_exps[e * db:(e + 1) * db], hl.t_down_exps, st["w"][t][s]
                else:
                    ge, ue = hl.gate_shexp, hl.up_shexp
                    dn, wt, scale = hl.down_shexp, hl.t_down_shexp, st["gs"][t]
                assert max_rel_err(st["h"][t][s], orc.moe_expert_h(ge, ue, N, F, xq, xd, xs)) < TOL, (case, t, s)
                y = orc.matmul_q8k(st["h"][t][s], dn, F, N, 1, wt)[0]
                acc = (acc + (np.float32(scale) * y).astype(np.float32)).astype(np.float32)
            assert max_rel_err(got[t], acc) < TOL, (case, t)
        rl.close()
