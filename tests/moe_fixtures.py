"""Seeded synthetic MoE layers for the tests (weights ~N(0, 0.02) quantised by
the build's quantizers; router ~N(0, 0.02); shared gate ~N(0, 0.02))."""
import numpy as np


def tensor_seed(seed: int, tag: int) -> int:
    return (seed * 1000003 + tag * 7919 + 12345) & 0xFFFFFFFFFFFFFFFF


def make_host_layer(orc, seed, n_embd=2048, n_ff=512, n_expert=256, n_used=8,
                    t_down=14, zero_router=False, router_bias_std=None, t_down_sh=None):
    N, F, E = n_embd, n_ff, n_expert
    t_down_sh = t_down if t_down_sh is None else t_down_sh
    if zero_router:
        gate_inp = np.zeros(E * N, np.float32)
    else:
        gate_inp = orc.fill_normal(tensor_seed(seed, 1), E * N, 0.0, 0.02)
    gate_exps = orc.quantize_q4k(orc.fill_normal(tensor_seed(seed, 2), E * F * N, 0.0, 0.02))
    up_exps = orc.quantize_q4k(orc.fill_normal(tensor_seed(seed, 3), E * F * N, 0.0, 0.02))
    down_exps = orc.quantize(orc.fill_normal(tensor_seed(seed, 4), E * N * F, 0.0, 0.02), t_down)
    wsh = orc.fill_normal(tensor_seed(seed, 5), N, 0.0, 0.02)
    gate_sh = orc.quantize_q4k(orc.fill_normal(tensor_seed(seed, 6), F * N, 0.0, 0.02))
    up_sh = orc.quantize_q4k(orc.fill_normal(tensor_seed(seed, 7), F * N, 0.0, 0.02))
    down_sh = orc.quantize(orc.fill_normal(tensor_seed(seed, 8), N * F, 0.0, 0.02), t_down_sh)
    bias = None
    if router_bias_std is not None:
        bias = orc.fill_normal(tensor_seed(seed, 9), E, 0.0, router_bias_std)
    return orc.HostLayer(N, F, E, n_used, gate_inp, gate_exps, up_exps, down_exps, t_down,
                         wsh, gate_sh, up_sh, down_sh, t_down_sh, router_bias=bias)
