"""Benchmark: MoE FFN decode on one MI355X (BASELINE.json metric).

Workload: a 40-layer qwen35moe MoE FFN stack,
all experts resident in HBM, decoding 256 tokens one after another at batch
1.  Per layer: router f32 2048->256, softmax top-8 renormalised, 8 routed
experts + 1 shared expert (gate/up 2048->512 Q4_K, down 512->2048 Q6_K),
SwiGLU, sigmoid-gated shared expert, residual add.  One step = the 256-token
sequence; weights (21.05 GB) and inputs are synthetic (seeded, generated in
HBM) and resident before the timed region.

Prints one JSON line.  value = tokens/s; HBM GB/s uses the algorithmic bytes
of one token through 40 layers (818,544,640 B).  "aux" carries the other
configurations, each with its CPU baseline (the oracle, timed on this host):
C1 / C2 (the matmul seam at 2048x2048 Q4_K and the 151936x2048 Q6_K LM head),
C3 (one layer per call), C5 (a 512-token prefill chunk), the engine's other
projection shapes at T = 1, and device sampling over the vocabulary.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-mobile-agent_amd"))

import ctypes as C

import numpy as np  # noqa: E402

import qmag  # noqa: E402

N_EMBD, N_FF, N_EXPERT, N_USED, N_LAYER, N_TOK = 2048, 512, 256, 8, 40, 256
HBM_PEAK = 8.0e12
Q4K_ROW = N_EMBD // 256 * 144          # 1152 B gate/up row
Q6K_ROW = N_FF // 256 * 210            # 420 B down row
EXPERT_BYTES = 2 * N_FF * Q4K_ROW + N_EMBD * Q6K_ROW          # 2,039,808
LAYER_TOKEN_BYTES = 4 * N_EXPERT * N_EMBD + 4 * N_EMBD + (N_USED + 1) * EXPERT_BYTES  # 20,463,616
TOKEN_BYTES = N_LAYER * LAYER_TOKEN_BYTES                      # 818,544,640
GATEUP_LAUNCH_BYTES = (N_USED + 1) * 2 * N_FF * Q4K_ROW + N_EMBD + 32 + 256 + (N_USED + 1) * N_FF * 4
DOWN_LAUNCH_BYTES = (N_USED + 1) * N_EMBD * Q6K_ROW + (N_USED + 1) * (N_FF + 8 + 64) + 4 * N_EMBD * 2
METRIC = "MoE FFN decode tokens/s + achieved HBM GB/s (% of peak), Q4_K/Q6_K, 1 GPU"
# HBM bytes per launch of the fused decode kernel, from two rocprofv3 counter
# passes over bench.py (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000, the factors
# read off a 1 GiB copy kernel in the same runs), with the profile holding
# them and the SHA-256 (first 16 hex digits) of the kernel's sources they were
# taken on: the kernel file and the headers it is compiled with, hashed in
# this order.  The figure is reported only while those sources are unchanged:
# an edit needs new counter passes (and a new entry here).
FUSED_TRAFFIC = {"bytes": 869.4e6, "profile": "profiles/moe_decode_kernel_c4_hbm_counters.md",
                 "sources": ["qwen-mobile-agent_amd/csrc/qmag_fused.hip", "qwen-mobile-agent_amd/csrc/qmag_device.h",
                             "qwen-mobile-agent_amd/csrc/qmag_internal.h"],
                 "source_sha16": "4b9c5003ac8317ef"}


def fused_source_sha16():
    h = hashlib.sha256()
    for rel in FUSED_TRAFFIC["sources"]:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def fused_traffic() -> tuple:
    """(HBM bytes per decode launch or None, where the figure comes from)."""
    try:
        sha = fused_source_sha16()
    except OSError:
        sha = None
    same = sha == FUSED_TRAFFIC["source_sha16"]
    info = {"profile": FUSED_TRAFFIC["profile"], "measured_on_source_sha16": FUSED_TRAFFIC["source_sha16"],
            "current_source_sha16": sha}
    if not same:
        info["note"] = "kernel source changed since the counter passes: traffic not reported"
    return (FUSED_TRAFFIC["bytes"] if same else None), info


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_info() -> dict:
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu": cpu}


def _orc():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc
    return orc


def gpu_loop(fn, seconds: float, min_iters: int = 3) -> tuple[float, int]:
    """Calls fn() back to back on the library stream for about `seconds`
    (iteration count calibrated on a short first pass); returns (ms per
    call from HIP events around the timed calls, calls)."""
    qmag.sync()
    timer = qmag.Timer(2, 3)
    timer.start()
    for _ in range(min_iters):
        fn()
    ms = timer.stop_ms() / min_iters
    iters = max(min_iters, int(seconds * 1e3 / max(ms, 1e-3)))
    timer.start()
    for _ in range(iters):
        fn()
    return timer.stop_ms() / iters, iters


def cpu_loop(fn, seconds: float, min_iters: int = 2) -> tuple[float, int]:
    """Wall time per call of a CPU function run for about `seconds`."""
    done = 0
    t0 = time.perf_counter()
    while True:
        fn()
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds and done >= min_iters:
            return el / done, done


def cpu_baseline(layers, seconds: float, n_layer_sample: int = 8):
    """Oracle (C restatement of the reference's q8k path, pool_run threads)
    on a bounded sample: the first n_layer_sample layers' bytes copied to the
    host, tokens decoded until `seconds` have elapsed; scaled to 40 layers."""
    orc = _orc()
    threads = min(os.cpu_count() or 1, 8)       # batch-1 MoE: 8 expert tasks (nn.c:162)
    hls = []
    for rl in layers[:n_layer_sample]:
        a = rl.host_arrays()
        hls.append(orc.HostLayer(N_EMBD, N_FF, N_EXPERT, N_USED, a["gate_inp"], a["gate_exps"],
                                 a["up_exps"], a["down_exps"], rl.t_down, a["gate_inp_shexp"],
                                 a["gate_shexp"], a["up_shexp"], a["down_shexp"], rl.t_down))
    orc.set_threads(threads)
    rng = np.random.default_rng(0)
    xs = [rng.standard_normal(N_EMBD).astype(np.float32) for _ in range(8)]
    it = [0]

    def one():
        orc.moe_stack(hls, xs[it[0] % len(xs)])
        it[0] += 1

    sec, done = cpu_loop(one, seconds)
    orc.set_threads(1)
    tok_s = n_layer_sample / N_LAYER / sec
    ci = cpu_info()
    return {"value": tok_s, "unit": "tokens/s (40-layer equivalent)", "cores": threads,
            "kind": "port", "us_per_layer_token": sec / n_layer_sample * 1e6,
            "sample": f"{done} tokens x {n_layer_sample} of 40 layers ({done * sec:.1f} s), scaled to 40 "
                      f"layers; nproc={ci['nproc']}, cpu={ci['cpu']}"}


def matvec_bytes(n_in: int, n_out: int, wtype: int) -> int:
    """Algorithmic bytes of one matmul-seam call at T = 1: weights, the
    fp32 input, its Q8_K form and the fp32 output."""
    rb = n_in // 256 * (144 if wtype == 12 else 210)
    return rb * n_out + 4 * n_in + (n_in + 4 * (n_in // 256) + 2 * (n_in // 16)) + 4 * n_out


def aux_matvec(name: str, n_in: int, n_out: int, wtype: int, copies: int, seconds: float,
               cpu_seconds: float, repack: bool = False) -> dict:
    """Configs C1/C2: the matmul seam at T = 1 (one launch: the matvec
    quantises x to Q8_K itself), rotating over `copies` distinct weight
    matrices so the working set exceeds the 256 MB last-level cache; the CPU
    baseline is the oracle's matmul (mm_worker rows over min(nproc, 16)
    pool threads, nn.c:276-303) on the first copy's bytes.  With `repack`
    the Q6_K matrices are repacked once (qmag_repack_q6k_dev, outside the
    timed region, in place) and timed as QMAG_TYPE_Q6_K_R: the same bytes and
    results."""
    rb = n_in // 256 * (144 if wtype == 12 else 210)
    Ws = [qmag.DBuf(rb * n_out) for _ in range(copies)]
    for i, w in enumerate(Ws):
        qmag.synth_weights(0xC100 + i, n_in * n_out, 0.02, wtype, w.ptr)
    if repack:
        for w in Ws:
            qmag.repack_q6k_dev(w, w, n_in, n_out)          # in place
        wtype = qmag.TYPE_Q6_K_R
    x = qmag.DBuf(4 * n_in)
    qmag.synth_normal(0xC1, n_in, 0.0, 1.0, x.ptr)
    out = qmag.DBuf(4 * n_out)

    def rotation():
        for w in Ws:
            qmag.matmul_dev(x, w, n_in, n_out, 1, wtype, out)

    rotation()
    ms, iters = gpu_loop(rotation, seconds)
    calls = iters * copies
    qmag.prof_enable(True)
    rotation()
    qmag.sync()
    n_mv, t_mv = qmag.prof_read("matvec")
    qmag.prof_enable(False)
    nbytes = matvec_bytes(n_in, n_out, wtype)
    call_us = ms * 1e3 / copies
    mv_us = t_mv * 1e3 / max(n_mv, 1)
    res = {"config": name, "bytes_per_call": nbytes, "us_per_call": call_us, "calls": calls,
           "gbps_per_call": nbytes / (call_us * 1e-6) / 1e9,
           "frac_of_peak_per_call": nbytes / (call_us * 1e-6) / HBM_PEAK,
           "matvec_kernel_us_event_pair": mv_us, "weight_copies": copies}
    log(f"{name}: {call_us:.2f} us/call ({res['gbps_per_call']:.0f} GB/s, "
        f"{100 * res['frac_of_peak_per_call']:.1f}% of peak), event-pair kernel {mv_us:.2f} us")
    if cpu_seconds > 0:
        orc = _orc()
        W0 = Ws[0].download(np.uint8)
        xh = x.download(np.float32)
        threads = min(os.cpu_count() or 1, 16)
        orc.set_threads(threads)
        sec, done = cpu_loop(lambda: orc.matmul_q8k(xh, W0, n_in, n_out, 1, wtype), cpu_seconds)
        orc.set_threads(1)
        ci = cpu_info()
        res["cpu_baseline"] = {"us_per_call": sec * 1e6, "gbps": nbytes / sec / 1e9, "cores": threads,
                               "kind": "port", "sample": f"{done} calls, nproc={ci['nproc']}, cpu={ci['cpu']}"}
        log(f"{name} cpu: {sec * 1e6:.0f} us/call on {threads} threads")
    for w in Ws:
        w.close()
    return res


# the engine's other matmul() call sites at decode (T = 1), qma.h:186-199,
# nn.c:2111-2113, 2162, 2165-2170, 2243
PROJECTIONS = [("wq", 2048, 8192, 12), ("wk", 2048, 512, 12), ("wv_q6k", 2048, 512, 14),
               ("wo", 4096, 2048, 12), ("wqkv_q6k", 2048, 8192, 14), ("attn_gate", 2048, 4096, 12),
               ("ssm_beta", 2048, 32, 12), ("ssm_out", 4096, 2048, 12)]


def aux_projections(seconds: float) -> dict:
    """Per-call time of each projection shape at T = 1, rotating over enough
    weight copies to exceed the last-level cache (>= 512 MB per shape)."""
    out = {}
    for name, n_in, n_out, wtype in PROJECTIONS:
        rb = n_in // 256 * (144 if wtype == 12 else 210)
        copies = max(2, min(256, (512 << 20) // (rb * n_out) + 1))
        Ws = [qmag.DBuf(rb * n_out) for _ in range(copies)]
        for i, w in enumerate(Ws):
            qmag.synth_weights(0xF200 + i, n_in * n_out, 0.02, wtype, w.ptr)
        x = qmag.DBuf(4 * n_in)
        qmag.synth_normal(0xF2, n_in, 0.0, 1.0, x.ptr)
        y = qmag.DBuf(4 * n_out)

        def rotation():
            for w in Ws:
                qmag.matmul_dev(x, w, n_in, n_out, 1, wtype, y)

        rotation()
        ms, _ = gpu_loop(rotation, seconds)
        us = ms * 1e3 / copies
        nb = matvec_bytes(n_in, n_out, wtype)
        out[name] = {"n_in": n_in, "n_out": n_out, "wtype": wtype, "us_per_call": us,
                     "gbps": nb / (us * 1e-6) / 1e9, "weight_copies": copies}
        for w in Ws:
            w.close()
    log("projections: " + ", ".join(f"{k} {v['us_per_call']:.2f} us ({v['gbps']:.0f} GB/s)" for k, v in out.items()))
    out["groups"] = aux_projection_groups(seconds)
    return out


# projections the engine computes from one x, timed as one qmag_matmul_group_dev
# launch against separate qmag_matmul_dev calls: q/k/v (nn.c:2111-2113) and the
# recurrent layer's qkv, gate, beta and alpha (nn.c:2162, 2165-2170)
PROJECTION_GROUPS = [("attn_qkv", 2048, [("wq", 8192, 12), ("wk", 512, 12), ("wv_q6k", 512, 14)]),
                     ("ssm_in", 2048, [("wqkv_q6k", 8192, 14), ("attn_gate", 4096, 12), ("ssm_beta", 32, 12),
                                       ("ssm_alpha", 32, 12)])]


def aux_projection_groups(seconds: float) -> dict:
    L = qmag.lib()
    res = {}
    for gname, n_in, mats in PROJECTION_GROUPS:
        rbs = [n_in // 256 * (144 if t == 12 else 210) for _, _, t in mats]
        gbytes = sum(rb * n for rb, (_, n, _) in zip(rbs, mats))
        copies = max(2, min(256, (512 << 20) // gbytes + 1))
        Ws = [[qmag.DBuf(rb * n) for rb, (_, n, _) in zip(rbs, mats)] for _ in range(copies)]
        for c, ws in enumerate(Ws):
            for w, (_, n, t) in zip(ws, mats):
                qmag.synth_weights(0xF300 + c, n_in * n, 0.02, t, w.ptr)
        x = qmag.DBuf(4 * n_in)
        qmag.synth_normal(0xF3, n_in, 0.0, 1.0, x.ptr)
        ys = [qmag.DBuf(4 * n) for _, n, _ in mats]
        k = len(mats)
        no = (C.c_int * k)(*[n for _, n, _ in mats])
        wt = (C.c_int * k)(*[t for _, _, t in mats])
        yp = (C.c_void_p * k)(*[y.ptr for y in ys])
        wps = [(C.c_void_p * k)(*[w.ptr for w in ws]) for ws in Ws]

        def grouped():
            for wp in wps:
                L.qmag_matmul_group_dev(x.ptr, n_in, k, wp, no, wt, yp)

        def separate():
            for ws in Ws:
                for w, y, (_, n, t) in zip(ws, ys, mats):
                    L.qmag_matmul_dev(x.ptr, w.ptr, n_in, n, 1, t, y.ptr)

        grouped()
        separate()
        ms_g, _ = gpu_loop(grouped, seconds)
        ms_s, _ = gpu_loop(separate, seconds)
        res[gname] = {"matrices": [m[0] for m in mats], "n_in": n_in, "weight_bytes": gbytes,
                      "us_one_launch": ms_g * 1e3 / copies, "us_separate_calls": ms_s * 1e3 / copies,
                      "weight_copies": copies}
        for ws in Ws:
            for w in ws:
                w.close()
    log("projection groups: " + ", ".join(f"{k} one launch {v['us_one_launch']:.2f} us vs separate "
                                          f"{v['us_separate_calls']:.2f} us" for k, v in res.items()))
    return res


def aux_sampler(seconds: float, cpu_seconds: float) -> dict:
    """Device sampling over the 151,936-entry vocabulary (the
    sampler_candidates + sampler_pick pair, agent.c:935-955, top_k 20 of
    max 40, temp 1.0, top_p 0.95, repeat penalty 1.1 over a 64-token
    history): per call on the GPU (logits resident; the token id comes
    back), and the oracle's pair on one host thread (the reference's
    sampler is single-threaded)."""
    V = 151936
    logits = qmag.DBuf(4 * V)
    qmag.synth_normal(0x5A, V, 0.0, 3.0, logits.ptr)
    hist = list(range(100, 164))
    s = qmag.Sampler.init(seed=1, temp=1.0, top_k=20, top_p=0.95, repeat_penalty=1.1, last=hist)
    qmag.sampler_sample_dev(logits.ptr, V, s, 40)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds or n < 10:
        qmag.sampler_sample_dev(logits.ptr, V, s, 40)
        n += 1
    gpu_us = (time.perf_counter() - t0) / n * 1e6
    res = {"config": "sampler: 151,936 logits, top_k 20 (max 40), temp 1, top_p 0.95, repeat penalty 1.1",
           "gpu_us_per_token": gpu_us, "gpu_calls": n,
           "note": "host wall time per call: the launch, the kernel and the wait for its result in pinned host memory"}
    if cpu_seconds > 0:
        orc = _orc()
        lh = logits.download(np.float32)
        so = orc.make_sampler(seed=1, temp=1.0, top_k=20, top_p=0.95, repeat_penalty=1.1, last=hist)

        def one():
            ids, lgs = orc.sampler_candidates(lh, so, 40)
            orc.sampler_pick(so, ids, lgs, 0.95)

        sec, done = cpu_loop(one, cpu_seconds)
        res["cpu_baseline"] = {"us_per_token": sec * 1e6, "cores": 1, "kind": "port", "sample": f"{done} calls"}
    log(f"sampler: gpu {gpu_us:.1f} us/token" +
        (f", cpu {res['cpu_baseline']['us_per_token']:.0f} us/token" if "cpu_baseline" in res else ""))
    return res


def aux_layer(cl, seconds: float, cpu_us_per_layer: float | None) -> dict:
    """Config C3: one MoE layer per call (T = 1, qmag_moe_ffn_dev), rotating
    over the 40 resident layers.  CPU baseline: the oracle's per layer-token
    time from the C4 sample (8 expert tasks on min(nproc, 8) threads)."""
    x = qmag.DBuf(4 * N_EMBD)
    out = qmag.DBuf(4 * N_EMBD)
    qmag.synth_normal(0xC3, N_EMBD, 0.0, 1.0, x.ptr)

    def rotation():
        for c in cl:
            qmag.moe_ffn_dev(c, x.ptr, out.ptr, 1)

    rotation()
    ms, _ = gpu_loop(rotation, seconds)
    us = ms * 1e3 / len(cl)
    res = {"config": "C3: one qwen35moe MoE FFN layer, batch-1 decode, one call per layer "
                     "rotating over 40 resident layers",
           "bytes_per_call": LAYER_TOKEN_BYTES, "us_per_call": us,
           "gbps": LAYER_TOKEN_BYTES / (us * 1e-6) / 1e9}
    res["frac_of_peak"] = res["gbps"] * 1e9 / HBM_PEAK
    # the same calls with x and out in host memory (qmag_moe_ffn_host, the
    # engine's own moe_ffn call): the PCIe-inclusive rate, each call
    # synchronous; wall time on the host, never the bench value
    hx = np.zeros(N_EMBD, np.float32)
    hx[:] = qmag.d2h_ptr(x.ptr, np.float32, N_EMBD)
    for c in cl:
        qmag.moe_ffn_host(c, hx, 1)
    t0 = time.perf_counter()
    n_host = 0
    while time.perf_counter() - t0 < seconds / 4 or n_host < len(cl):
        for c in cl:
            qmag.moe_ffn_host(c, hx, 1)
        n_host += len(cl)
    res["host_buffers_us_per_call"] = (time.perf_counter() - t0) / n_host * 1e6
    if cpu_us_per_layer:
        res["cpu_baseline"] = {"us_per_call": cpu_us_per_layer, "kind": "port",
                               "cores": min(os.cpu_count() or 1, 8),
                               "sample": "per layer-token time of the C4 CPU sample"}
    log(f"C3 layer: {us:.2f} us/call, {res['gbps']:.0f} GB/s; "
        f"with x and out in host memory {res['host_buffers_us_per_call']:.2f} us/call")
    return res


INT8_PEAK = 5.03e15       # dense int8 MFMA op/s, 256 CU x 2.4 GHz x 8192


def aux_prefill(seconds: float, cpu_seconds: float, T: int = 512, n_layers: int = 3) -> dict:
    """Config C5: one MoE layer over a 512-token prefill chunk (grouped
    int8-MFMA expert GEMM), router logits skewed by a seeded per-expert bias
    ~N(0,1); rotating over n_layers layers so one layer's experts are not
    still in the 256 MB last-level cache on the next call."""
    rls = [qmag.ResidentLayer(seed=0xC5, layer=l, router_bias_std=1.0) for l in range(n_layers)]
    x = qmag.DBuf(4 * T * N_EMBD)
    out = qmag.DBuf(4 * T * N_EMBD)
    qmag.synth_normal(0xC5, T * N_EMBD, 0.0, 1.0, x.ptr)
    distinct = []
    for rl in rls:
        qmag.moe_ffn_dev(rl.c, x.ptr, out.ptr, T)
        st = qmag.moe_last_stage(N_EXPERT, N_USED, N_FF, n_tok=T)
        distinct.append(len(np.unique(st["sel"])))
    def rotation():
        for rl in rls:
            qmag.moe_ffn_dev(rl.c, x.ptr, out.ptr, T)

    ms, _ = gpu_loop(rotation, seconds)
    us = ms * 1e3 / n_layers
    qmag.prof_enable(True)
    for rl in rls:
        qmag.moe_ffn_dev(rl.c, x.ptr, out.ptr, T)
    qmag.sync()
    kern = {k: qmag.prof_read(k) for k in ("router", "topk", "group", "gateup", "hquant", "down", "combine")}
    qmag.prof_enable(False)
    cpu = None
    if cpu_seconds > 0:
        # the oracle's moe_ffn over the same chunk: T * 8 (token, expert)
        # tasks on min(nproc, 16) pool threads (nn.c:576-612)
        orc = _orc()
        a = rls[0].host_arrays()
        hl = orc.HostLayer(N_EMBD, N_FF, N_EXPERT, N_USED, a["gate_inp"], a["gate_exps"], a["up_exps"],
                           a["down_exps"], rls[0].t_down, a["gate_inp_shexp"], a["gate_shexp"], a["up_shexp"],
                           a["down_shexp"], rls[0].t_down, router_bias=a["router_bias"])
        xh = x.download(np.float32)
        threads = min(os.cpu_count() or 1, 16)
        orc.set_threads(threads)
        sec, done = cpu_loop(lambda: orc.moe_ffn(hl, xh, T), cpu_seconds, min_iters=1)
        orc.set_threads(1)
        ci = cpu_info()
        cpu = {"us_per_layer": sec * 1e6, "tokens_per_s": T / sec, "cores": threads, "kind": "port",
               "sample": f"{done} x one {T}-token layer ({T * N_USED} pair tasks); nproc={ci['nproc']}, "
                         f"cpu={ci['cpu']}"}
        log(f"C5 cpu: {sec * 1e3:.0f} ms/layer on {threads} threads")
    for rl in rls:
        rl.close()
    n_pairs = T * N_USED
    # int8 ops: every (token, expert) pair runs gate + up (2 x 512 x 2048) and
    # down (2048 x 512) multiply-adds; the shared expert on every token
    ops = 2 * (n_pairs + T) * (2 * N_FF * N_EMBD + N_EMBD * N_FF)
    d = float(np.mean(distinct))
    nbytes = d * EXPERT_BYTES + EXPERT_BYTES + 4 * N_EXPERT * N_EMBD + 4 * N_EMBD
    per_k = {k: t / max(n, 1) * 1e3 for k, (n, t) in kern.items() if n}
    gemm_us = per_k.get("gateup", 0.0) + per_k.get("down", 0.0)
    res = {"config": f"C5: {T}-token prefill chunk, one MoE layer, router bias ~N(0,1), grouped int8-MFMA "
                     f"expert GEMM, rotating over {n_layers} layers",
           "us_per_layer": us, "tokens_per_s": T / (us * 1e-6), "distinct_experts": d,
           "int8_ops": ops, "mfma_tops": ops / (us * 1e-6) / 1e12, "mfma_frac_of_peak": ops / (us * 1e-6) / INT8_PEAK,
           "weight_bytes": nbytes, "hbm_gbps": nbytes / (us * 1e-6) / 1e9,
           "hbm_frac_of_peak": nbytes / (us * 1e-6) / HBM_PEAK, "per_kernel_us": per_k,
           "per_kernel_note": "HIP event pair around each launch on the library stream, one extra pass; "
                              "each pair adds a few us of its own, so short kernels read high (a kernel "
                              "trace gives their own durations; the sum exceeds us_per_layer)",
           "gemm_kernels_mfma_frac": ops / (gemm_us * 1e-6) / INT8_PEAK if gemm_us else None,
           "cpu_baseline": cpu}
    log(f"C5 prefill: {us:.1f} us/layer ({res['tokens_per_s']:.0f} tok/s), {d:.0f} distinct experts, "
        f"int8 {res['mfma_tops']:.1f} TOP/s ({100 * res['mfma_frac_of_peak']:.1f}% of peak), "
        f"weights {res['hbm_gbps']:.0f} GB/s; kernels " + ", ".join(f"{k} {v:.1f}" for k, v in per_k.items()))
    return res


AUX_LEGS = ("c1", "c2", "c3", "c5", "projections", "sampler")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU-baseline sample length of the headline (C4); the other CPU legs take a quarter")
    ap.add_argument("--aux-seconds", type=float, default=1.5,
                    help="GPU time per auxiliary configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--tokens", type=int, default=N_TOK)
    ap.add_argument("--decode", choices=("fused", "sequence"), default="fused",
                    help="persistent single-launch decode (default) or the per-stage launch sequence")
    ap.add_argument("--launch", choices=("coop", "plain"), default="plain",
                    help="fused kernel: ordinary launch (default) or cooperative launch")
    ap.add_argument("--probe-copy-mb", type=int, default=0,
                    help="after the run, one device-to-device copy of this many MiB between two "
                         "fresh buffers: a copy kernel of known size for scaling HBM counters")
    ap.add_argument("--aux", default="c1,c2,c3,c5,projections,sampler",
                    help="comma-separated auxiliary configurations to run (a profile of one of them "
                         "names only its kernels)")
    ap.add_argument("--no-aux", action="store_true",
                    help="skip the auxiliary configurations (C1, C2, C3, C5, projections, sampler)")
    args = ap.parse_args()
    unknown = [a for a in args.aux.split(",") if a and a not in AUX_LEGS]
    if unknown:
        print(f"unknown --aux entries {unknown}; known: {list(AUX_LEGS)}", file=sys.stderr)
        return 2
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build runs on a single MI355X; across GPUs the experts would shard by id, "
              "with one 8 KB reduction of the layer output per layer)",
              file=sys.stderr)
        return 2

    qmag.init(0)
    qmag.set_fused(args.decode == "fused")
    qmag.set_coop(args.launch == "coop")
    info = qmag.device_info()
    log(f"device {info}")
    t0 = time.perf_counter()
    layers = [qmag.ResidentLayer(seed=2026, layer=l) for l in range(N_LAYER)]
    x0 = qmag.DBuf(4 * args.tokens * N_EMBD)
    x = qmag.DBuf(4 * args.tokens * N_EMBD)
    qmag.synth_normal(0xC4, args.tokens * N_EMBD, 0.0, 1.0, x0.ptr)
    qmag.sync()
    log(f"generated {N_LAYER} resident layers in {time.perf_counter() - t0:.1f} s")
    cl = [l.c for l in layers]

    def step():
        qmag.check(qmag.lib().qmag_d2d(x.ptr, x0.ptr, x.nbytes))
        qmag.moe_stack_dev(cl, x.ptr, args.tokens)

    for _ in range(args.warmup):
        step()
    qmag.sync()
    timer = qmag.Timer(0, 1)
    timer.start()
    w0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    qmag.sync()
    wall = time.perf_counter() - w0
    ms = timer.stop_ms()
    ms_step = ms / args.steps
    tok_s = args.steps * args.tokens / (ms / 1e3)
    gbps = tok_s * TOKEN_BYTES / 1e9
    log(f"{ms_step:.2f} ms/step, {tok_s:.1f} tok/s, {gbps:.1f} GB/s (wall {wall:.2f} s)")
    out = qmag.d2h_ptr(x.ptr, np.float32, N_EMBD)
    if not np.all(np.isfinite(out)):
        log("non-finite output")
        return 1

    # per-kernel launch durations, HIP events on the library stream (the
    # stream every kernel runs on) around each launch, over one extra step:
    # per-launch events perturb the step total, so this pass is separate
    qmag.prof_enable(True)
    step()
    qmag.sync()
    prof = {k: qmag.prof_read(k) for k in ("router", "topk", "gateup", "hquant", "down", "fused")}
    qmag.prof_enable(False)
    log("per-kernel: " + ", ".join(f"{k}={n} launches {t / max(n, 1) * 1e3:.2f} us"
                                   for k, (n, t) in prof.items() if n))
    dom = max(prof, key=lambda k: prof[k][1])
    n_d, t_d = prof[dom]
    if dom == "fused":
        # one launch = one token through all 40 layers; the timed-region
        # average (events bracketing all launches) includes launch gaps
        kname = "moe_decode_kernel<Q6_K> (persistent; one token x 40 layers per launch)"
        bytes_launch = TOKEN_BYTES
        avg_us = ms / (args.steps * args.tokens) * 1e3
    else:
        kname = {"gateup": "gateup_kernel<8>", "down": "down_kernel<2,Q6_K,Q6_K>",
                 "router": "router_kernel", "topk": "topk_kernel", "hquant": "q8k_quant_kernel"}[dom]
        bytes_launch = {"gateup": GATEUP_LAUNCH_BYTES, "down": DOWN_LAUNCH_BYTES,
                        "router": 4 * N_EXPERT * N_EMBD + 4 * N_EMBD}.get(dom, 0)
        avg_us = t_d / n_d * 1e3
    roofline = {"bound": "hbm", "kernel": kname,
                "achieved": bytes_launch / (avg_us * 1e-6) / 1e9, "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "traffic": fused_traffic()[0] if dom == "fused" else None,
                "bytes_per_launch": bytes_launch,
                "avg_launch_us": avg_us, "avg_launch_us_event_pairs": t_d / n_d * 1e3}
    roofline["frac"] = roofline["achieved"] / roofline["peak"]
    if dom == "fused":
        roofline["traffic_source"] = fused_traffic()[1]

    if args.probe_copy_mb > 0:
        nb = args.probe_copy_mb << 20
        src, dst = qmag.DBuf(nb), qmag.DBuf(nb)
        qmag.synth_normal(7, nb // 4, 0.0, 1.0, src.ptr)
        qmag.check(qmag.lib().qmag_d2d(dst.ptr, src.ptr, nb))
        qmag.sync()
        del src, dst
        log(f"probe copy of {args.probe_copy_mb} MiB done")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(layers, args.cpu_seconds)
        log(f"cpu baseline {cpu['value']:.3f} tok/s")

    aux = None
    if not args.no_aux:
        cs = 0.0 if args.no_cpu else args.cpu_seconds / 4
        legs = {
            "c1": lambda: aux_matvec("C1: Q4_K matvec 2048x2048, matmul seam, T=1", 2048, 2048, 12, 128,
                                     args.aux_seconds, cs),
            "c2": lambda: {**aux_matvec("C2: Q6_K LM head 151936x2048, matmul seam, T=1", 2048, 151936, 14, 2,
                                        args.aux_seconds, cs),
                           "repacked": aux_matvec("C2 repacked: the same Q6_K LM head as QMAG_TYPE_Q6_K_R rows",
                                                  2048, 151936, 14, 2, args.aux_seconds, 0.0, repack=True)},
            "c3": lambda: aux_layer(cl, args.aux_seconds, cpu["us_per_layer_token"] if cpu else None),
            "c5": lambda: aux_prefill(args.aux_seconds, cs),
            "projections": lambda: aux_projections(args.aux_seconds / 4),
            "sampler": lambda: aux_sampler(args.aux_seconds / 2, cs / 2),
        }
        aux = {k: legs[k]() for k in args.aux.split(",") if k}

    line = {
        "metric": METRIC, "value": tok_s, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantised in HBM, x ~ N(0,1))",
        "config": {"workload": "C4: 40-layer qwen35moe MoE FFN stack decode, 256 tokens "
                               "sequential at batch 1, all experts resident",
                   "n_layer": N_LAYER, "tokens_per_step": args.tokens, "n_embd": N_EMBD,
                   "n_expert": N_EXPERT, "n_used": N_USED, "n_ff": N_FF,
                   "gate_up": "Q4_K", "down": "Q6_K", "parallelism": "single GPU",
                   "decode": args.decode, "launch": args.launch},
        "hbm_gbps": gbps, "hbm_frac_of_peak": gbps * 1e9 / HBM_PEAK,
        "bytes_per_token": TOKEN_BYTES,
        "roofline": roofline, "cpu_baseline": cpu,
        "per_kernel_us": {k: t / n * 1e3 for k, (n, t) in prof.items() if n},
        "aux": aux,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
