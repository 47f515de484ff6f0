"""Python host-side binding of libqmagpu.so (ctypes), mirroring the C-ABI in
include/qma_gpu.h: the reference-compatible qma_q8k_* entries (src/q8k.c)
and the device entries for the matmul / moe_ffn seams of src/nn.c.

There is no fallback: if libqmagpu.so is missing or no gfx950 device is
present, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqmagpu.so")

QK_K = 256
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_Q6_K_R = 270          # Q6_K rows repacked by qmag_repack_q6k_dev (same bytes per row)
BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q6_K_R: 210}

P = C.c_void_p

# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "qma_q8k_available": (C.c_int, []),
    "qma_q8k_quant": (None, [P, C.c_int, P, P, P]),
    "qma_q8k_dot": (C.c_float, [P, C.c_int, P, P, P, C.c_int]),
    "qma_q8k_gateup": (None, [P, P, P, P, P, C.c_int, P, P]),
    "dequantize_row_q4_K": (None, [P, P, C.c_int64]),
    "dequantize_row_q6_K": (None, [P, P, C.c_int64]),
    "dot_q4_K_f32": (C.c_float, [P, P, C.c_int]),
    "dot_q6_K_f32": (C.c_float, [P, P, C.c_int]),
    "qmag_init": (C.c_int, [C.c_int]),
    "qmag_last_error": (C.c_char_p, []),
    "qmag_device_info": (C.c_int, [P, P, P, C.c_char_p, C.c_int]),
    "qmag_malloc": (C.c_int, [C.POINTER(P), C.c_size_t]),
    "qmag_free": (C.c_int, [P]),
    "qmag_h2d": (C.c_int, [P, P, C.c_size_t]),
    "qmag_d2h": (C.c_int, [P, P, C.c_size_t]),
    "qmag_d2d": (C.c_int, [P, P, C.c_size_t]),
    "qmag_memset": (C.c_int, [P, C.c_int, C.c_size_t]),
    "qmag_sync": (C.c_int, []),
    "qmag_event_record": (C.c_int, [C.c_int]),
    "qmag_event_elapsed": (C.c_int, [C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "qmag_prof_enable": (C.c_int, [C.c_int]),
    "qmag_prof_read": (C.c_int, [C.c_int, C.POINTER(C.c_long), C.POINTER(C.c_double)]),
    "qmag_set_option": (C.c_int, [C.c_int, C.c_int]),
    "qmag_fused_recoveries": (C.c_int, [C.POINTER(C.c_long)]),
    "qmag_trace_read": (C.c_int, [P, C.c_size_t]),
    "qmag_q8k_quant_dev": (C.c_int, [P, C.c_int, C.c_int, P, P, P]),
    "qmag_matmul_q8k_dev": (C.c_int, [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "qmag_matmul_dev": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "qmag_repack_q6k_dev": (C.c_int, [P, P, C.c_int, C.c_int]),
    "qmag_matmul_group_dev": (C.c_int, [P, C.c_int, C.c_int, P, P, P, P]),
    "qmag_matmul_noalloc_dev": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "qmag_dequant_dev": (C.c_int, [P, C.c_int, C.c_int64, P]),
    "qmag_matmul_f32_dev": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "qmag_moe_ffn_dev": (C.c_int, [P, P, P, C.c_int]),
    "qmag_moe_ffn_host": (C.c_int, [P, P, P, C.c_int]),
    "qmag_moe_ffn_f32_dev": (C.c_int, [P, P, P, C.c_int]),
    "qmag_moe_stack_dev": (C.c_int, [P, C.c_int, P, C.c_int]),
    "qmag_moe_last_stage": (C.c_int, [C.POINTER(P)] * 5),
    "qmag_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
    "qmag_gguf_close": (None, [P]),
    "qmag_gguf_meta_u64": (C.c_int, [P, C.c_char_p, C.POINTER(C.c_uint64)]),
    "qmag_gguf_tensor": (C.c_int, [P, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int64), C.POINTER(P),
                                   C.POINTER(C.c_size_t)]),
    "qmag_gguf_upload_tensor": (C.c_int, [P, C.c_char_p, C.POINTER(P), C.POINTER(C.c_int), C.POINTER(C.c_int64)]),
    "qmag_gguf_upload_moe_layer": (C.c_int, [P, C.c_int, P]),
    "qmag_gguf_free_moe_layer": (C.c_int, [P]),
    "qmag_ecache_init": (C.c_int, [C.POINTER(P), C.c_size_t, C.c_size_t, C.c_int]),
    "qmag_ecache_free": (None, [P]),
    "qmag_ecache_clear": (None, [P]),
    "qmag_ecache_get": (P, [P, C.c_int, C.c_int, P, P]),
    "qmag_ecache_hold": (P, [P, C.c_int, C.c_int, P, P]),
    "qmag_ecache_release": (None, [P]),
    "qmag_ecache_io_start": (C.c_int, [P, P, P, C.c_int, C.c_int]),
    "qmag_ecache_io_stop": (None, [P]),
    "qmag_ecache_hint": (None, [P, C.c_int, P, C.c_int]),
    "qmag_ecache_prefetch": (None, [P, C.c_int, P, C.c_int]),
    "qmag_ecache_drain": (C.c_int, [P]),
    "qmag_ecache_stats": (C.c_int, [P, P]),
    "qmag_ecache_slot_of": (C.c_int, [P, C.c_int, C.c_int]),
    "qmag_ecache_slot_ptr": (P, [P, C.c_int]),
    "qmag_moe_ffn_paged_dev": (C.c_int, [P, P, C.c_int, P, P, P, P, C.c_int]),
    "qmag_gguf_fetch_expert": (C.c_int, [P, C.c_int, C.c_int, P]),
    "qmag_gguf_expert_record_bytes": (C.c_int, [P, C.POINTER(C.c_size_t)]),
    "qmag_sampler_candidates_dev": (C.c_int, [C.c_int, P, P, P, P, C.c_int]),
    "qmag_sampler_sample_dev": (C.c_int, [C.c_int, P, P, C.c_int, C.c_float, P]),
    "qmag_synth_normal": (C.c_int, [C.c_uint64, C.c_size_t, C.c_float, C.c_float, P]),
    "qmag_synth_weights": (C.c_int, [C.c_uint64, C.c_size_t, C.c_float, C.c_int, P]),
    "qmag_quantize_dev": (C.c_int, [P, C.c_size_t, C.c_int, P]),
}


class QmagError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QmagError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise QmagError(f"qmag status {status}: {lib().qmag_last_error().decode()}")


def init(device: int = 0) -> None:
    check(lib().qmag_init(device))


def device_info():
    n_cu, clk, hbm = C.c_int(), C.c_int(), C.c_size_t()
    arch = C.create_string_buffer(64)
    check(lib().qmag_device_info(C.byref(n_cu), C.byref(clk), C.byref(hbm), arch, 64))
    return dict(n_cu=n_cu.value, clock_khz=clk.value, hbm_bytes=hbm.value, arch=arch.value.decode())


def sync() -> None:
    check(lib().qmag_sync())


OPT_FUSED = 1


def set_fused(on: bool) -> None:
    """Select the persistent single-launch decode kernel (default) or the
    per-stage launch sequence for batch-1 MoE decode."""
    check(lib().qmag_set_option(OPT_FUSED, 1 if on else 0))


OPT_TRACE = 2
TRACE_PHASES = ("start", "hopA", "router", "hopB", "gu_start", "gu_done", "hopC", "down_done")


def set_trace(on: bool) -> None:
    check(lib().qmag_set_option(OPT_TRACE, 1 if on else 0))


OPT_COOP = 3


def set_coop(on: bool) -> None:
    """Launch the fused decode kernel cooperatively, or (default) as an
    ordinary kernel after the occupancy check that makes it eligible."""
    check(lib().qmag_set_option(OPT_COOP, 1 if on else 0))


OPT_GROUPED = 4


def set_grouped(on: bool) -> None:
    """Batches of >= 8 tokens: the grouped int8-MFMA expert GEMM (default) or
    the per-token launch sequence."""
    check(lib().qmag_set_option(OPT_GROUPED, 1 if on else 0))


OPT_TEST_ABORT = 5


def arm_test_abort(nth: int = 1) -> None:
    """Make the nth persistent decode launch from now find its abort word set
    (tests of the recovery path)."""
    check(lib().qmag_set_option(OPT_TEST_ABORT, nth))


def fused_recoveries() -> int:
    n = C.c_long()
    check(lib().qmag_fused_recoveries(C.byref(n)))
    return n.value


def trace_read(n_layer: int) -> np.ndarray:
    """Phase timestamps of the last fused launch: uint64 [512][n_layer][8],
    device real-time counter at 100 MHz."""
    out = np.empty((512, n_layer, 8), dtype=np.uint64)
    check(lib().qmag_trace_read(out.ctypes.data_as(P), out.nbytes))
    return out


class DBuf:
    """A device allocation owned by Python (freed on close / GC)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = P()
        check(lib().qmag_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DBuf":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().qmag_h2d(self.ptr + offset, a.ctypes.data_as(P), a.nbytes))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(lib().qmag_d2h(out.ctypes.data_as(P), self.ptr + offset, out.nbytes))
        return out

    def at(self, offset: int) -> int:
        return self.ptr + offset

    def close(self) -> None:
        if getattr(self, "ptr", None):
            try:
                lib().qmag_free(self.ptr)
            finally:
                self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def d2h_ptr(ptr: int, dtype, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.dtype(dtype))
    check(lib().qmag_d2h(out.ctypes.data_as(P), ptr, out.nbytes))
    return out


class MoeLayer(C.Structure):
    """struct qmag_moe_layer (include/qma_gpu.h)."""
    _fields_ = [
        ("n_embd", C.c_int), ("n_ff", C.c_int), ("n_expert", C.c_int), ("n_used", C.c_int),
        ("gate_inp", P), ("router_bias", P),
        ("gate_exps", P), ("up_exps", P), ("down_exps", P), ("t_down_exps", C.c_int),
        ("gate_inp_shexp", P), ("gate_shexp", P), ("up_shexp", P), ("down_shexp", P),
        ("t_down_shexp", C.c_int),
    ]


# --------------------------------------------------------------- entries --

def q8k_quant_dev(x: DBuf, n: int, T: int, xq: DBuf, xd: DBuf, xs: DBuf) -> None:
    check(lib().qmag_q8k_quant_dev(x.ptr, n, T, xq.ptr, xd.ptr, xs.ptr))


def matmul_q8k_dev(xq, xd, xs, W: DBuf, n_in, n_out, T, wtype, out: DBuf) -> None:
    check(lib().qmag_matmul_q8k_dev(xq.ptr, xd.ptr, xs.ptr if xs is not None else None, W.ptr,
                                    n_in, n_out, T, wtype, out.ptr))


def matmul_dev(x: DBuf, W: DBuf, n_in, n_out, T, wtype, out: DBuf) -> None:
    check(lib().qmag_matmul_dev(x.ptr, W.ptr, n_in, n_out, T, wtype, out.ptr))


def matmul_group_dev(x: DBuf, n_in: int, mats, outs) -> None:
    """mats: [(W DBuf, n_out, wtype)], outs: [DBuf]; one launch for all."""
    n = len(mats)
    W = (P * n)(*[m[0].ptr for m in mats])
    no = (C.c_int * n)(*[m[1] for m in mats])
    wt = (C.c_int * n)(*[m[2] for m in mats])
    out = (P * n)(*[o.ptr for o in outs])
    check(lib().qmag_matmul_group_dev(x.ptr, n_in, n, W, no, wt, out))


def repack_q6k_dev(src: DBuf, dst: DBuf, n_in: int, n_out: int) -> None:
    check(lib().qmag_repack_q6k_dev(src.ptr, dst.ptr, n_in, n_out))


def dequant_dev(W: DBuf, wtype: int, n: int, y: DBuf) -> None:
    check(lib().qmag_dequant_dev(W.ptr, wtype, n, y.ptr))


def matmul_f32_dev(x: DBuf, W: DBuf, n_in, n_out, T, wtype, out: DBuf) -> None:
    check(lib().qmag_matmul_f32_dev(x.ptr, W.ptr, n_in, n_out, T, wtype, out.ptr))


def moe_ffn_dev(layer: MoeLayer, x_ptr: int, out_ptr: int, T: int) -> None:
    check(lib().qmag_moe_ffn_dev(C.byref(layer), x_ptr, out_ptr, T))


def moe_ffn_host(layer: MoeLayer, x: np.ndarray, T: int) -> np.ndarray:
    """One MoE layer on host buffers (qmag_moe_ffn_host): x f32 [T * n_embd]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    check(lib().qmag_moe_ffn_host(C.byref(layer), x.ctypes.data_as(P), out.ctypes.data_as(P), T))
    return out


def moe_ffn_f32_dev(layer: MoeLayer, x_ptr: int, out_ptr: int, T: int) -> None:
    """The fp32 twin of the layer (QMA_NOQ8K)."""
    check(lib().qmag_moe_ffn_f32_dev(C.byref(layer), x_ptr, out_ptr, T))


def moe_stack_dev(layers, x_ptr: int, n_tok: int) -> None:
    arr = (MoeLayer * len(layers))(*layers)
    check(lib().qmag_moe_stack_dev(arr, len(layers), x_ptr, n_tok))


def moe_last_stage(n_expert: int, n_used: int, n_ff: int, n_tok: int = 0):
    """Stage outputs of the last MoE call for token 0 (n_tok = 0), or, after
    a multi-token qmag_moe_ffn_dev call, for its first n_tok tokens (arrays
    gain a leading token axis)."""
    ptrs = [P() for _ in range(5)]
    check(lib().qmag_moe_last_stage(*[C.byref(p) for p in ptrs]))
    T = max(n_tok, 1)
    logits = d2h_ptr(ptrs[0].value, np.float32, T * n_expert).reshape(T, n_expert)
    sel = d2h_ptr(ptrs[1].value, np.int32, T * n_used).reshape(T, n_used)
    w = d2h_ptr(ptrs[2].value, np.float32, T * n_used).reshape(T, n_used)
    gs = d2h_ptr(ptrs[3].value, np.float32, T)
    h = d2h_ptr(ptrs[4].value, np.float32, T * (n_used + 1) * n_ff).reshape(T, n_used + 1, n_ff)
    if n_tok == 0:
        return dict(logits=logits[0], sel=sel[0], w=w[0], gs=gs[0], h=h[0])
    return dict(logits=logits, sel=sel, w=w, gs=gs, h=h)


def synth_normal(seed: int, n: int, mean: float, std: float, out_ptr: int) -> None:
    check(lib().qmag_synth_normal(C.c_uint64(seed), n, mean, std, out_ptr))


def synth_weights(seed: int, n: int, std: float, wtype: int, out_ptr: int) -> None:
    check(lib().qmag_synth_weights(C.c_uint64(seed), n, std, wtype, out_ptr))


def quantize_dev(x_ptr: int, n: int, wtype: int, out_ptr: int) -> None:
    check(lib().qmag_quantize_dev(x_ptr, n, wtype, out_ptr))


PROF_IDS = {"router": 0, "topk": 1, "gateup": 2, "hquant": 3, "down": 4, "fused": 5, "matvec": 6,
            "q8k": 7, "group": 8, "combine": 9}


def prof_enable(on: bool) -> None:
    check(lib().qmag_prof_enable(1 if on else 0))


def prof_read(name: str):
    n, ms = C.c_long(), C.c_double()
    check(lib().qmag_prof_read(PROF_IDS[name], C.byref(n), C.byref(ms)))
    return n.value, ms.value


class Timer:
    """HIP events on the library stream (the stream every qmag_* kernel runs on)."""

    def __init__(self, a: int = 0, b: int = 1):
        self.a, self.b = a, b

    def start(self) -> None:
        check(lib().qmag_event_record(self.a))

    def stop_ms(self) -> float:
        check(lib().qmag_event_record(self.b))
        ms = C.c_float()
        check(lib().qmag_event_elapsed(self.a, self.b, C.byref(ms)))
        return float(ms.value)


# ------------------------------------------------------- resident layers --

def tensor_seed(seed: int, layer: int, tag: int) -> int:
    return (seed * 0x100000001B3 + layer * 1000003 + tag * 7919 + 1) & 0xFFFFFFFFFFFFFFFF


class ResidentLayer:
    """One MoE layer's tensors generated directly in HBM (GGUF layout):
    router f32 ~N(0, .02), experts ~N(0, .02) quantised to Q4_K (gate/up)
    and Q4_K/Q6_K (down), shared gate f32 ~N(0, .02)."""

    def __init__(self, seed: int, layer: int = 0, n_embd=2048, n_ff=512, n_expert=256, n_used=8,
                 t_down=TYPE_Q6_K, router_bias_std: float | None = None):
        N, F, E = n_embd, n_ff, n_expert
        self.n_embd, self.n_ff, self.n_expert, self.n_used, self.t_down = N, F, E, n_used, t_down
        gu = N // QK_K * BLOCK_BYTES[TYPE_Q4_K] * F
        dn = F // QK_K * BLOCK_BYTES[t_down] * N
        self.bytes_gate_slab, self.bytes_down_slab = gu, dn
        self.gate_inp = DBuf(4 * E * N)
        self.gate_exps = DBuf(gu * E)
        self.up_exps = DBuf(gu * E)
        self.down_exps = DBuf(dn * E)
        self.gate_inp_shexp = DBuf(4 * N)
        self.gate_shexp = DBuf(gu)
        self.up_shexp = DBuf(gu)
        self.down_shexp = DBuf(dn)
        self.router_bias = DBuf(4 * E) if router_bias_std is not None else None
        ts = lambda tag: tensor_seed(seed, layer, tag)
        synth_normal(ts(1), E * N, 0.0, 0.02, self.gate_inp.ptr)
        synth_weights(ts(2), E * F * N, 0.02, TYPE_Q4_K, self.gate_exps.ptr)
        synth_weights(ts(3), E * F * N, 0.02, TYPE_Q4_K, self.up_exps.ptr)
        synth_weights(ts(4), E * N * F, 0.02, t_down, self.down_exps.ptr)
        synth_normal(ts(5), N, 0.0, 0.02, self.gate_inp_shexp.ptr)
        synth_weights(ts(6), F * N, 0.02, TYPE_Q4_K, self.gate_shexp.ptr)
        synth_weights(ts(7), F * N, 0.02, TYPE_Q4_K, self.up_shexp.ptr)
        synth_weights(ts(8), N * F, 0.02, t_down, self.down_shexp.ptr)
        if self.router_bias is not None:
            synth_normal(ts(9), E, 0.0, router_bias_std, self.router_bias.ptr)
        self.c = MoeLayer(N, F, E, n_used, self.gate_inp.ptr,
                          self.router_bias.ptr if self.router_bias else None,
                          self.gate_exps.ptr, self.up_exps.ptr, self.down_exps.ptr, t_down,
                          self.gate_inp_shexp.ptr, self.gate_shexp.ptr, self.up_shexp.ptr,
                          self.down_shexp.ptr, t_down)

    @classmethod
    def from_host(cls, hl) -> "ResidentLayer":
        """Upload an oracle HostLayer (tests)."""
        self = cls.__new__(cls)
        self.n_embd, self.n_ff, self.n_expert, self.n_used = hl.n_embd, hl.n_ff, hl.n_expert, hl.n_used
        self.t_down = hl.t_down_exps
        for k in ("gate_inp", "gate_exps", "up_exps", "down_exps", "gate_inp_shexp", "gate_shexp",
                  "up_shexp", "down_shexp"):
            setattr(self, k, DBuf.from_array(getattr(hl, k)))
        self.router_bias = DBuf.from_array(hl.router_bias) if "router_bias" in hl.arrays else None
        self.c = MoeLayer(hl.n_embd, hl.n_ff, hl.n_expert, hl.n_used, self.gate_inp.ptr,
                          self.router_bias.ptr if self.router_bias else None,
                          self.gate_exps.ptr, self.up_exps.ptr, self.down_exps.ptr, hl.t_down_exps,
                          self.gate_inp_shexp.ptr, self.gate_shexp.ptr, self.up_shexp.ptr,
                          self.down_shexp.ptr, hl.t_down_shexp)
        return self

    def host_arrays(self) -> dict:
        """Download every tensor (for the CPU oracle)."""
        N, F, E = self.n_embd, self.n_ff, self.n_expert
        out = dict(
            gate_inp=self.gate_inp.download(np.float32),
            gate_exps=self.gate_exps.download(np.uint8),
            up_exps=self.up_exps.download(np.uint8),
            down_exps=self.down_exps.download(np.uint8),
            gate_inp_shexp=self.gate_inp_shexp.download(np.float32),
            gate_shexp=self.gate_shexp.download(np.uint8),
            up_shexp=self.up_shexp.download(np.uint8),
            down_shexp=self.down_shexp.download(np.uint8),
        )
        if self.router_bias is not None:
            out["router_bias"] = self.router_bias.download(np.float32)
        return out

    def close(self) -> None:
        for k in ("gate_inp", "gate_exps", "up_exps", "down_exps", "gate_inp_shexp", "gate_shexp",
                  "up_shexp", "down_shexp", "router_bias"):
            b = getattr(self, k, None)
            if b is not None:
                b.close()


# ---------------------------------------------------------- expert cache --

FETCH_FN = C.CFUNCTYPE(C.c_int, P, C.c_int, C.c_int, P)


class ECacheCounters(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("bytes_read", C.c_uint64),
                ("evictions", C.c_uint64), ("prefetched", C.c_uint64), ("spec_issued", C.c_uint64),
                ("n_slots", C.c_int), ("rec_bytes", C.c_size_t), ("slot_bytes", C.c_size_t)]


class ECache:
    """The HBM expert cache (qmag_ecache_*).  fetch: a C function pointer
    (e.g. the GGUF fetch) or a Python callable (user, layer, expert, dst) ->
    int, wrapped and kept alive here; user: a pointer value or None."""

    def __init__(self, budget_bytes: int, rec_bytes: int, policy: int = 0, fetch=None, user=None):
        h = P()
        check(lib().qmag_ecache_init(C.byref(h), budget_bytes, rec_bytes, policy))
        self.h = h.value
        self.set_fetch(fetch, user)

    def set_fetch(self, fetch, user=None):
        if fetch is None or isinstance(fetch, int):
            self._cb = None
            self.fetch = fetch
        else:
            self._cb = fetch if isinstance(fetch, FETCH_FN) else FETCH_FN(fetch)
            self.fetch = C.cast(self._cb, P).value
        self.user = user

    def io_start(self, nthreads: int, depth: int) -> None:
        check(lib().qmag_ecache_io_start(self.h, self.fetch, self.user, nthreads, depth))

    def io_stop(self) -> None:
        lib().qmag_ecache_io_stop(self.h)

    def get(self, layer: int, expert: int) -> int:
        return lib().qmag_ecache_get(self.h, layer, expert, self.fetch, self.user) or 0

    def hold(self, layer: int, expert: int) -> int:
        return lib().qmag_ecache_hold(self.h, layer, expert, self.fetch, self.user) or 0

    def release(self) -> None:
        lib().qmag_ecache_release(self.h)

    def hint(self, layer: int, ids) -> None:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        lib().qmag_ecache_hint(self.h, layer, a.ctypes.data, a.size)

    def prefetch(self, layer: int, ids) -> None:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        lib().qmag_ecache_prefetch(self.h, layer, a.ctypes.data, a.size)

    def drain(self) -> None:
        check(lib().qmag_ecache_drain(self.h))

    def clear(self) -> None:
        lib().qmag_ecache_clear(self.h)

    def stats(self) -> dict:
        c = ECacheCounters()
        check(lib().qmag_ecache_stats(self.h, C.byref(c)))
        return {k: getattr(c, k) for k, _ in ECacheCounters._fields_}

    def slot_of(self, layer: int, expert: int) -> int:
        return lib().qmag_ecache_slot_of(self.h, layer, expert)

    def slot_ptr(self, slot: int) -> int:
        return lib().qmag_ecache_slot_ptr(self.h, slot) or 0

    def moe_ffn_paged(self, layer: "MoeLayer", il: int, x_ptr: int, out_ptr: int, T: int) -> None:
        check(lib().qmag_moe_ffn_paged_dev(C.byref(layer), self.h, il, self.fetch, self.user, x_ptr, out_ptr, T))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().qmag_ecache_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gguf_fetch_fn() -> int:
    """Address of qmag_gguf_fetch_expert, for ECache(fetch=...)."""
    return C.cast(lib().qmag_gguf_fetch_expert, P).value


# --------------------------------------------------------------- sampler --

class Sampler(C.Structure):
    """qmag_sampler: the layout of sampler_t (qma.h:279-287)."""
    _fields_ = [("seed", C.c_uint64), ("temp", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repeat_penalty", C.c_float), ("last_tokens", C.c_int * 64), ("n_last", C.c_int)]

    @classmethod
    def init(cls, seed=0, temp=0.7, top_k=40, top_p=0.95, repeat_penalty=1.0, last=()):
        """sampler_init (sampler.c:16-23) plus an optional token history."""
        s = cls()
        s.seed = seed if seed else 0x9E3779B97F4A7C15
        s.temp, s.top_k, s.top_p, s.repeat_penalty = temp, top_k, top_p, repeat_penalty
        for i, t in enumerate(list(last)[:64]):
            s.last_tokens[i] = t
        s.n_last = min(len(last), 64)
        return s


def sampler_candidates_dev(logits_ptr: int, n_vocab: int, s: Sampler, max_k: int = 40):
    """sampler_candidates on device logits: (ids, values), k of each."""
    ids = np.zeros(max_k, np.int32)
    lgs = np.zeros(max_k, np.float32)
    k = lib().qmag_sampler_candidates_dev(n_vocab, logits_ptr, C.addressof(s), ids.ctypes.data,
                                          lgs.ctypes.data, max_k)
    check(min(k, 0))
    return ids[:k].copy(), lgs[:k].copy()


def sampler_sample_dev(logits_ptr: int, n_vocab: int, s: Sampler, max_k: int = 40, top_p: float = None) -> int:
    """sampler_candidates + sampler_pick on the device; s is updated."""
    tok = C.c_int()
    check(lib().qmag_sampler_sample_dev(n_vocab, logits_ptr, C.addressof(s), max_k,
                                        s.top_p if top_p is None else top_p, C.byref(tok)))
    return tok.value


# ------------------------------------------------------------------ GGUF --

class Gguf:
    """An opened GGUF file (qmag_gguf_open); tensor queries need no GPU,
    uploads do."""

    def __init__(self, path: str):
        h = P()
        check(lib().qmag_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h.value

    def meta(self, key: str) -> int:
        v = C.c_uint64()
        check(lib().qmag_gguf_meta_u64(self.h, key.encode(), C.byref(v)))
        return v.value

    def tensor(self, name: str):
        """(type, (ne0, ne1, ne2), bytes as a numpy uint8 view copy)."""
        t, ne, data, nb = C.c_int(), (C.c_int64 * 3)(), P(), C.c_size_t()
        check(lib().qmag_gguf_tensor(self.h, name.encode(), C.byref(t), ne, C.byref(data), C.byref(nb)))
        buf = (C.c_uint8 * nb.value).from_address(data.value)
        return t.value, tuple(ne), np.frombuffer(buf, dtype=np.uint8).copy()

    def upload_tensor(self, name: str):
        """Device pointer (free with qmag_free), type, dims."""
        d, t, ne = P(), C.c_int(), (C.c_int64 * 3)()
        check(lib().qmag_gguf_upload_tensor(self.h, name.encode(), C.byref(d), C.byref(t), ne))
        return d.value, t.value, tuple(ne)

    def upload_moe_layer(self, il: int) -> MoeLayer:
        L = MoeLayer()
        check(lib().qmag_gguf_upload_moe_layer(self.h, il, C.byref(L)))
        return L

    def expert_record_bytes(self) -> int:
        r = C.c_size_t()
        check(lib().qmag_gguf_expert_record_bytes(self.h, C.byref(r)))
        return r.value

    @staticmethod
    def free_moe_layer(L: MoeLayer) -> None:
        check(lib().qmag_gguf_free_moe_layer(C.byref(L)))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().qmag_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
