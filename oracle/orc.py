"""ctypes binding of the CPU oracle (oracle/liborc.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg.  The product library never
uses it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")

QK_K = 256
TYPE_Q4_K = 12
TYPE_Q6_K = 14
Q4K_BYTES = 144
Q6K_BYTES = 210


def build(force: bool = False) -> str:
    """Compile liborc.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-B" if force else "all", "-C", HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p


def _declare(L):
    L.orc_half_to_float.restype = C.c_float
    L.orc_half_to_float.argtypes = [C.c_uint16]
    L.orc_float_to_half.restype = C.c_uint16
    L.orc_float_to_half.argtypes = [C.c_float]
    L.orc_scale_min_k4.argtypes = [C.c_int, P, P, P]
    L.orc_dequant_q4k.argtypes = [P, P, C.c_int64]
    L.orc_dequant_q6k.argtypes = [P, P, C.c_int64]
    L.orc_dot_q4k_f32.restype = C.c_float
    L.orc_dot_q4k_f32.argtypes = [P, P, C.c_int]
    L.orc_dot_q6k_f32.restype = C.c_float
    L.orc_dot_q6k_f32.argtypes = [P, P, C.c_int]
    L.orc_q8k_quant.argtypes = [P, C.c_int, P, P, P]
    L.orc_q8k_dot.restype = C.c_float
    L.orc_q8k_dot.argtypes = [P, C.c_int, P, P, P, C.c_int]
    L.orc_q8k_gateup.argtypes = [P, P, P, P, P, C.c_int, P, P]
    L.orc_q4k_subsums.argtypes = [P, P, C.c_int, P]
    L.orc_q6k_blocksums.argtypes = [P, P, C.c_int, P]
    L.orc_pool_set_threads.argtypes = [C.c_int]
    L.orc_pool_threads.restype = C.c_int
    L.orc_matmul_q8k.argtypes = [P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]
    L.orc_moe_route.argtypes = [C.POINTER(MoeLayer), P, P, P, P]
    L.orc_moe_ffn.argtypes = [C.POINTER(MoeLayer), P, P, C.c_int]
    L.orc_moe_ffn_routed.argtypes = [C.POINTER(MoeLayer), P, P, C.c_int, P, P]
    L.orc_moe_expert_h.argtypes = [P, P, C.c_int, C.c_int, P, P, P, P]
    L.orc_moe_shared_gate.restype = C.c_float
    L.orc_moe_shared_gate.argtypes = [P, P, P, C.c_int]
    L.orc_moe_stack.argtypes = [C.POINTER(MoeLayer), C.c_int, P]
    L.orc_moe_expert_h_f32.argtypes = [P, P, C.c_int, C.c_int, P, P]
    L.orc_moe_shared_gate_f32.restype = C.c_float
    L.orc_moe_shared_gate_f32.argtypes = [P, P, C.c_int]
    L.orc_moe_ffn_f32.argtypes = [C.POINTER(MoeLayer), P, P, C.c_int]
    L.orc_fill_normal.argtypes = [C.c_uint64, C.c_int64, C.c_float, C.c_float, P]
    L.orc_sampler_candidates.restype = C.c_int
    L.orc_sampler_candidates.argtypes = [C.c_int, P, C.POINTER(Sampler), P, P, C.c_int]
    L.orc_ecache_create.restype = P
    L.orc_ecache_create.argtypes = [C.c_size_t, C.c_size_t, C.c_int, C.c_int, C.c_int]
    L.orc_ecache_destroy.argtypes = [P]
    L.orc_ecache_counters.argtypes = [P, P]
    L.orc_ecache_io_start.argtypes = [P, C.c_int, C.c_int]
    for f in ("orc_ecache_get", "orc_ecache_hold", "orc_ecache_lookup"):
        getattr(L, f).restype = C.c_int
        getattr(L, f).argtypes = [P, C.c_int, C.c_int]
    L.orc_ecache_release.argtypes = [P]
    L.orc_ecache_drain.argtypes = [P]
    L.orc_ecache_clear.argtypes = [P]
    L.orc_ecache_hint.argtypes = [P, C.c_int, P, C.c_int]
    L.orc_ecache_prefetch.argtypes = [P, C.c_int, P, C.c_int]
    L.orc_sampler_pick.restype = C.c_int
    L.orc_sampler_pick.argtypes = [C.POINTER(Sampler), P, P, C.c_int, C.c_float]
    L.orc_quantize_q4k.argtypes = [P, C.c_int64, P]
    L.orc_quantize_q6k.argtypes = [P, C.c_int64, P]


class Sampler(C.Structure):
    """sampler_t (qma.h:279-287)."""
    _fields_ = [("seed", C.c_uint64), ("temp", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repeat_penalty", C.c_float), ("last_tokens", C.c_int * 64), ("n_last", C.c_int)]


def make_sampler(seed=1, temp=0.7, top_k=20, top_p=0.95, repeat_penalty=1.0, last=()):
    s = Sampler()
    s.seed = seed if seed else 0x9E3779B97F4A7C15        # sampler_init, sampler.c:16-23
    s.temp, s.top_k, s.top_p, s.repeat_penalty = temp, top_k, top_p, repeat_penalty
    for i, t in enumerate(last[:64]):
        s.last_tokens[i] = t
    s.n_last = min(len(last), 64)
    return s


def sampler_candidates(logits, s: Sampler, max_k: int = 40):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(max(max_k, 1), np.int32)
    lgs = np.zeros(max(max_k, 1), np.float32)
    k = lib().orc_sampler_candidates(logits.size, _p(logits), C.byref(s), _p(ids), _p(lgs), max_k)
    return ids[:k].copy(), lgs[:k].copy()


def sampler_pick(s: Sampler, ids, lgs, top_p: float) -> int:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    lgs = np.ascontiguousarray(lgs, dtype=np.float32).copy()
    return int(lib().orc_sampler_pick(C.byref(s), _p(ids), _p(lgs), ids.size, top_p))


class ECacheModel:
    """The expert cache policy of ecache.c (oracle/ecache_oracle.c): methods
    return slot indices (-1 on failure) in place of record pointers."""
    FIELDS = ("hits", "misses", "bytes_read", "evictions", "prefetched", "spec_issued", "n_slots")

    def __init__(self, budget_bytes, rec_bytes, policy=0, n_layer=1 << 15, n_expert=1 << 16):
        self.h = lib().orc_ecache_create(budget_bytes, rec_bytes, policy, n_layer, n_expert)
        assert self.h

    def io_start(self, nthreads, depth):
        lib().orc_ecache_io_start(self.h, nthreads, depth)

    def get(self, layer, expert):
        return lib().orc_ecache_get(self.h, layer, expert)

    def hold(self, layer, expert):
        return lib().orc_ecache_hold(self.h, layer, expert)

    def release(self):
        lib().orc_ecache_release(self.h)

    def hint(self, layer, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        lib().orc_ecache_hint(self.h, layer, _p(a), a.size)

    def prefetch(self, layer, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        lib().orc_ecache_prefetch(self.h, layer, _p(a), a.size)

    def drain(self):
        lib().orc_ecache_drain(self.h)

    def clear(self):
        lib().orc_ecache_clear(self.h)

    def lookup(self, layer, expert):
        return lib().orc_ecache_lookup(self.h, layer, expert)

    def stats(self):
        out = np.zeros(7, np.uint64)
        lib().orc_ecache_counters(self.h, _p(out))
        return dict(zip(self.FIELDS, (int(v) for v in out)))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_ecache_destroy(self.h)
            self.h = None


class MoeLayer(C.Structure):
    _fields_ = [
        ("n_embd", C.c_int), ("n_ff", C.c_int), ("n_expert", C.c_int), ("n_used", C.c_int),
        ("gate_inp", P), ("router_bias", P),
        ("gate_exps", P), ("up_exps", P), ("down_exps", P), ("t_down_exps", C.c_int),
        ("gate_inp_shexp", P), ("gate_shexp", P), ("up_shexp", P), ("down_shexp", P),
        ("t_down_shexp", C.c_int),
    ]


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(P)


# --------------------------------------------------------------------------
# thin numpy-facing wrappers
# --------------------------------------------------------------------------

def fill_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(C.c_uint64(seed), n, mean, std, _p(out))
    return out


def quantize_q4k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % QK_K == 0
    out = np.empty(x.size // QK_K * Q4K_BYTES, dtype=np.uint8)
    lib().orc_quantize_q4k(_p(x), x.size, _p(out))
    return out


def quantize_q6k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % QK_K == 0
    out = np.empty(x.size // QK_K * Q6K_BYTES, dtype=np.uint8)
    lib().orc_quantize_q6k(_p(x), x.size, _p(out))
    return out


def quantize(x: np.ndarray, wtype: int) -> np.ndarray:
    return quantize_q4k(x) if wtype == TYPE_Q4_K else quantize_q6k(x)


def dequant(blocks: np.ndarray, wtype: int, k: int) -> np.ndarray:
    y = np.empty(k, dtype=np.float32)
    fn = lib().orc_dequant_q4k if wtype == TYPE_Q4_K else lib().orc_dequant_q6k
    fn(_p(np.ascontiguousarray(blocks)), _p(y), k)
    return y


def q8k_quant(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n = x.size
    xq = np.empty(n, dtype=np.int8)
    xd = np.empty(n // QK_K, dtype=np.float32)
    xs = np.empty(n // 16, dtype=np.int16)
    lib().orc_q8k_quant(_p(x), n, _p(xq), _p(xd), _p(xs))
    return xq, xd, xs


def q8k_dot(row: np.ndarray, wtype: int, xq, xd, xs, n: int) -> float:
    return float(lib().orc_q8k_dot(_p(np.ascontiguousarray(row)), wtype, _p(xq), _p(xd),
                                   _p(xs), n))


def q8k_gateup(g: np.ndarray, u: np.ndarray, xq, xd, xs, n: int):
    go = C.c_float()
    uo = C.c_float()
    lib().orc_q8k_gateup(_p(g), _p(u), _p(xq), _p(xd), _p(xs), n, C.byref(go), C.byref(uo))
    return go.value, uo.value


def q4k_subsums(row: np.ndarray, xq: np.ndarray, n: int) -> np.ndarray:
    P_ = np.empty(n // 32, dtype=np.int32)
    lib().orc_q4k_subsums(_p(np.ascontiguousarray(row)), _p(xq), n, _p(P_))
    return P_


def q6k_blocksums(row: np.ndarray, xq: np.ndarray, n: int) -> np.ndarray:
    S = np.empty(n // QK_K, dtype=np.int32)
    lib().orc_q6k_blocksums(_p(np.ascontiguousarray(row)), _p(xq), n, _p(S))
    return S


def dot_f32(row: np.ndarray, wtype: int, x: np.ndarray, n: int) -> float:
    fn = lib().orc_dot_q4k_f32 if wtype == TYPE_Q4_K else lib().orc_dot_q6k_f32
    return float(fn(_p(np.ascontiguousarray(row)), _p(np.ascontiguousarray(x, dtype=np.float32)), n))


def set_threads(n: int) -> None:
    lib().orc_pool_set_threads(int(n))


def matmul_q8k(x: np.ndarray, W: np.ndarray, n_in: int, n_out: int, T: int, wtype: int):
    out = np.empty(T * n_out, dtype=np.float32)
    lib().orc_matmul_q8k(_p(np.ascontiguousarray(x, dtype=np.float32)), _p(W), n_in, n_out, T,
                         wtype, _p(out))
    return out.reshape(T, n_out)


class HostLayer:
    """Host copies of one MoE layer's tensors, in the GGUF byte layout."""

    def __init__(self, n_embd, n_ff, n_expert, n_used, gate_inp, gate_exps, up_exps, down_exps,
                 t_down_exps, gate_inp_shexp, gate_shexp, up_shexp, down_shexp, t_down_shexp,
                 router_bias=None):
        self.arrays = dict(gate_inp=np.ascontiguousarray(gate_inp, dtype=np.float32),
                           gate_exps=np.ascontiguousarray(gate_exps),
                           up_exps=np.ascontiguousarray(up_exps),
                           down_exps=np.ascontiguousarray(down_exps),
                           gate_inp_shexp=np.ascontiguousarray(gate_inp_shexp, dtype=np.float32),
                           gate_shexp=np.ascontiguousarray(gate_shexp),
                           up_shexp=np.ascontiguousarray(up_shexp),
                           down_shexp=np.ascontiguousarray(down_shexp))
        if router_bias is not None:
            self.arrays["router_bias"] = np.ascontiguousarray(router_bias, dtype=np.float32)
        self.n_embd, self.n_ff, self.n_expert, self.n_used = n_embd, n_ff, n_expert, n_used
        self.t_down_exps, self.t_down_shexp = t_down_exps, t_down_shexp
        a = self.arrays
        self.c = MoeLayer(n_embd, n_ff, n_expert, n_used, _p(a["gate_inp"]),
                          _p(a["router_bias"]) if "router_bias" in a else None,
                          _p(a["gate_exps"]), _p(a["up_exps"]), _p(a["down_exps"]), t_down_exps,
                          _p(a["gate_inp_shexp"]), _p(a["gate_shexp"]), _p(a["up_shexp"]),
                          _p(a["down_shexp"]), t_down_shexp)

    def __getattr__(self, k):
        a = self.__dict__.get("arrays", {})
        if k in a:
            return a[k]
        raise AttributeError(k)


def moe_route(layer: HostLayer, x: np.ndarray):
    sel = np.empty(layer.n_used, dtype=np.int32)
    w = np.empty(layer.n_used, dtype=np.float32)
    logits = np.empty(layer.n_expert, dtype=np.float32)
    lib().orc_moe_route(C.byref(layer.c), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(sel),
                        _p(w), _p(logits))
    return sel, w, logits


def moe_ffn(layer: HostLayer, x: np.ndarray, T: int) -> np.ndarray:
    out = np.empty(T * layer.n_embd, dtype=np.float32)
    lib().orc_moe_ffn(C.byref(layer.c), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(out), T)
    return out.reshape(T, layer.n_embd)


def moe_ffn_routed(layer: HostLayer, x: np.ndarray, T: int, sel: np.ndarray, w: np.ndarray):
    out = np.empty(T * layer.n_embd, dtype=np.float32)
    sel = np.ascontiguousarray(sel, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib().orc_moe_ffn_routed(C.byref(layer.c), _p(np.ascontiguousarray(x, dtype=np.float32)),
                             _p(out), T, _p(sel), _p(w))
    return out.reshape(T, layer.n_embd)


def moe_expert_h(ge, ue, n_embd, n_ff, xq, xd, xs):
    h = np.empty(n_ff, dtype=np.float32)
    lib().orc_moe_expert_h(_p(ge), _p(ue), n_embd, n_ff, _p(xq), _p(xd), _p(xs), _p(h))
    return h


def moe_ffn_f32(layer: HostLayer, x: np.ndarray, T: int) -> np.ndarray:
    """The fp32 twin of moe_ffn (QMA_NOQ8K)."""
    out = np.empty(T * layer.n_embd, dtype=np.float32)
    lib().orc_moe_ffn_f32(C.byref(layer.c), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(out), T)
    return out.reshape(T, layer.n_embd)


def moe_expert_h_f32(ge, ue, n_embd, n_ff, x):
    h = np.empty(n_ff, dtype=np.float32)
    lib().orc_moe_expert_h_f32(_p(ge), _p(ue), n_embd, n_ff, _p(np.ascontiguousarray(x, dtype=np.float32)), _p(h))
    return h


def moe_shared_gate_f32(wsh, x, n_embd) -> float:
    return float(lib().orc_moe_shared_gate_f32(_p(wsh), _p(np.ascontiguousarray(x, dtype=np.float32)), n_embd))


def moe_shared_gate(wsh, xq, xd, n_embd) -> float:
    return float(lib().orc_moe_shared_gate(_p(wsh), _p(xq), _p(xd), n_embd))


def moe_stack(layers, x: np.ndarray) -> np.ndarray:
    arr = (MoeLayer * len(layers))(*[l.c for l in layers])
    xo = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().orc_moe_stack(arr, len(layers), _p(xo))
    return xo
