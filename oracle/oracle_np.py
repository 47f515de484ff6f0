"""Second, independent restatement of the reference arithmetic in numpy.

TEST INFRASTRUCTURE ONLY (used by tests/ to pin the C oracle).  Written from
the struct definitions and closed forms rather than from the C oracle:

* fp16 via numpy's own float16 (exact conversion);
* Q4_K / Q6_K element values from vectorised bit extraction
  (qma.h:77-90, quants.c:18-75);
* Q8_K with float32 division/multiply and explicit half-away-from-zero
  rounding done in float64 (q8k.c:34-85; np.round is half-even and is not
  used);
* integer sub-block sums in int64, fp32 results as fp64 closed forms.
"""
from __future__ import annotations

import numpy as np

QK_K = 256


def half_to_float(u16: np.ndarray) -> np.ndarray:
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- Q4_K ----

def q4k_fields(raw: np.ndarray):
    """Split Q4_K bytes into (d, dmin, sc[nb,8], m[nb,8], q[nb,256]) with q in
    element order (0..15)."""
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 144)
    d = half_to_float(b[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = half_to_float(b[:, 2:4].copy().view(np.uint16)[:, 0])
    s = b[:, 4:16].astype(np.int64)
    sc = np.empty((b.shape[0], 8), dtype=np.int64)
    m = np.empty((b.shape[0], 8), dtype=np.int64)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            m[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            m[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = b[:, 16:144].astype(np.int64).reshape(-1, 4, 32)
    q = np.concatenate([np.stack([qs[:, g] & 0xF, qs[:, g] >> 4], axis=1) for g in range(4)],
                       axis=1).reshape(-1, 256)
    return d, dmin, sc, m, q


def q4k_dequant(raw: np.ndarray) -> np.ndarray:
    d, dmin, sc, m, q = q4k_fields(raw)
    sub = np.repeat(np.arange(8), 32)
    w = (d[:, None].astype(np.float64) * sc[:, sub] * q
         - dmin[:, None].astype(np.float64) * m[:, sub])
    return w.reshape(-1)


# ---------------------------------------------------------------- Q6_K ----

def q6k_fields(raw: np.ndarray):
    """Split Q6_K bytes into (d, sc[nb,16], q[nb,256] in -32..31)."""
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 210)
    ql = b[:, 0:128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = half_to_float(b[:, 208:210].copy().view(np.uint16)[:, 0])
    q = np.empty((b.shape[0], 256), dtype=np.int64)
    for e in range(256):
        half, r = divmod(e, 128)
        Q, l = divmod(r, 32)
        byte = ql[:, 64 * half + (Q & 1) * 32 + l]
        lo = (byte & 0xF) if Q < 2 else (byte >> 4)
        hi = (qh[:, 32 * half + l] >> (2 * Q)) & 3
        q[:, e] = (lo | (hi << 4)) - 32
    return d, sc, q


def q6k_dequant(raw: np.ndarray) -> np.ndarray:
    d, sc, q = q6k_fields(raw)
    w = d[:, None].astype(np.float64) * sc[:, np.arange(256) // 16] * q
    return w.reshape(-1)


# ---------------------------------------------------------------- Q8_K ----

def q8k_quant(x: np.ndarray):
    x = np.asarray(x, dtype=np.float32).reshape(-1, QK_K)
    amax = np.max(np.abs(x), axis=1)
    d = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / d).astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32).astype(np.float64)
    r = np.trunc(v + np.copysign(0.5, v))
    q = np.clip(r, -127, 127).astype(np.int8)
    xs = q.astype(np.int64).reshape(-1, 16).sum(axis=1).astype(np.int16)
    return q.reshape(-1), d, xs


# ------------------------------------------------------ integer dots ----

def q4k_subsums(raw: np.ndarray, xq: np.ndarray) -> np.ndarray:
    """Per 32-lane sub-block int sums sum(q * xq) (q8k.c:117-120)."""
    _, _, _, _, q = q4k_fields(raw)
    x = np.asarray(xq, dtype=np.int64).reshape(-1, 256)
    return (q * x).reshape(-1, 8, 32).sum(axis=2).reshape(-1)


def q6k_blocksums(raw: np.ndarray, xq: np.ndarray) -> np.ndarray:
    """Per super-block sum(sc * (q6-32) * xq) (q8k.c:250-259)."""
    _, sc, q = q6k_fields(raw)
    x = np.asarray(xq, dtype=np.int64).reshape(-1, 256)
    return (sc[:, np.arange(256) // 16] * q * x).sum(axis=1)


def q8k_dot_f64(raw: np.ndarray, wtype: int, xq, xd) -> float:
    """Closed form sum_j deq(W)_j * (xq_j * xd) in fp64."""
    w = q4k_dequant(raw) if wtype == 12 else q6k_dequant(raw)
    xf = np.asarray(xq, dtype=np.float64) * np.repeat(np.asarray(xd, dtype=np.float64), QK_K)
    return float(np.dot(w, xf))


def route_f64(Wr: np.ndarray, x: np.ndarray, n_used: int, bias=None):
    """fp64 router: returns (sel, w, probs, margin between the n_used-th and
    (n_used+1)-th probabilities).  Tie rule = stable sort on -p (nn.c:529-533)."""
    lg = Wr.astype(np.float64) @ x.astype(np.float64)
    if bias is not None:
        lg = lg + bias.astype(np.float64)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    sel = order[:n_used]
    w = p[sel] / p[sel].sum()
    margin = p[order[n_used - 1]] - p[order[n_used]]
    return sel, w, p, margin
